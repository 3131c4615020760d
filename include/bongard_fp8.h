/*
 * bongard_fp8.h - C ABI of the MI355X (gfx950) FP8 linear path.
 *
 * Built as libbongard_fp8.so from the HIP sources in bongard_amd/csrc. Every entry point:
 *   - returns 0 on success, a non-zero BF8_E* code otherwise; bf8_last_error() then
 *     gives a thread-local message;
 *   - takes raw device pointers allocated by the caller (PyTorch), never allocates,
 *     frees or synchronises, and enqueues its kernels on the given HIP stream
 *     (`stream` is a hipStream_t; NULL means the legacy default stream);
 *   - keeps no mutable global state besides the error message, so calls on different
 *     streams are independent (except bf8_quantize_bf16_noalloc, which uses a
 *     library-owned scratch array per GPU instead of a caller workspace).
 *
 * Formats are OCP FP8: BF8_E4M3 (max 448, no inf, NaN = 0x7F/0xFF) and BF8_E5M2
 * (max 57344, IEEE-like inf/NaN). Payloads are one byte per element.
 *
 * A "meta" record is four fp32 values in device memory: {amax, scale, scale_inv, 0}.
 * scale = fp32(fp8_max / max(f64(amax), 1e-12)) (correctly rounded),
 * scale_inv = fp32(1 / scale); the quantized value is q = fp8(clamp(f32(x) * scale)).
 *
 * The reference (AgentBull/bongard) has no native FFI for this path: it reaches the same
 * arithmetic through torchao's Float8Linear and TransformerEngine's te.Linear /
 * te.LayerNormMLP from Python. Each declaration names the reference call site whose
 * arithmetic it replaces; the Python binding is bongard_amd/_lib.py (ctypes).
 */
#ifndef BONGARD_FP8_H
#define BONGARD_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BF8_E4M3 = 0, BF8_E5M2 = 1 };
/* Flag OR'ed into the fmt of a current-scaling entry point (bf8_scale_from_partials,
 * bf8_cast_partials_bf16, bf8_quantize_bf16, bf8_quantize_axiswise_bf16): the scale is
 * rounded down to a power of two by clearing its mantissa (torchao
 * round_scales_to_power_of_2, set by its rowwise recipes). */
enum { BF8_SCALE_POW2 = 0x10 };
enum { BF8_OUT_BF16 = 0, BF8_OUT_F32 = 1 };
enum {
  BF8_OK = 0,
  BF8_EINVAL = 1,   /* bad argument: shape, alignment, format, null pointer */
  BF8_ELAUNCH = 2,  /* a kernel launch failed (hipGetLastError after launch) */
  BF8_ESIZE = 3     /* caller-provided workspace too small */
};

/* Thread-local message for the last non-zero return code on this thread. */
const char* bf8_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int bf8_abi_version(void);

/* ---------------------------------------------------------------------------------
 * Per-tensor amax and scale (current scaling).
 * Replaces torchao tensor_to_amax + amax_to_scale, reached from TrainingLinear.forward
 * (bongard/float8_training.py:22, Float8Linear.forward) and the amax step of TE's
 * Float8CurrentScaling quantizer used by TELinear / TEMLP (bongard/te_linear.py:73-74)
 * and FusedMLP (bongard/fused_mlp.py:76-78).
 * ------------------------------------------------------------------------------- */

/* Number of uint32 partial-amax slots bf8_amax_bf16 writes for n elements. */
int64_t bf8_amax_partials(int64_t n);

/* partials[i] = fp32 bit pattern of max|x| over block i's share of x (NaN sorts above
 * inf). x: bf16 [n], 16-byte aligned. partials: uint32 [bf8_amax_partials(n)]. */
int bf8_amax_bf16(const void* x, int64_t n, uint32_t* partials, void* stream);

/* meta = {amax, scale, scale_inv, 0} from n_partials partial-amax slots. */
int bf8_scale_from_partials(const uint32_t* partials, int64_t n_partials, int fmt,
                            float* meta, void* stream);


/* ---------------------------------------------------------------------------------
 * Saturating cast bf16 -> e4m3/e5m2, optional transposed copy.
 * Replaces torchao to_fp8_saturated (+ the .t().contiguous() layouts fed to
 * torch._scaled_mm) and TE's cast / cast-transpose kernels
 * (bongard/te_linear.py:73-74, bongard/fused_mlp.py:76-78).
 * x: bf16 [rows, cols] row-major, cols % 16 == 0. scale: device fp32 (meta + 1).
 * out: fp8 [rows, cols] (nullable if out_t given); out_t: fp8 [cols, rows] or NULL.
 * ------------------------------------------------------------------------------- */
int bf8_cast_bf16(const void* x, int64_t rows, int64_t cols, const float* scale, int fmt,
                  uint8_t* out, uint8_t* out_t, void* stream);

/* Cast with the scale derived from amax partials (as written by bf8_amax_bf16,
 * bf8_gemm_geglu or bf8_geglu_bwd; n_partials <= 4096): every block reduces them to the
 * scale before casting, and meta receives {amax, scale, scale_inv, 0}. */
int bf8_cast_partials_bf16(const void* x, int64_t rows, int64_t cols, const uint32_t* partials,
                           int64_t n_partials, int fmt, float* meta, uint8_t* out,
                           uint8_t* out_t, void* stream);

/* amax -> scale -> cast (two kernels: bf8_amax_bf16, bf8_cast_partials_bf16); meta gets
 * {amax, scale, scale_inv, 0}. partials: uint32 [bf8_amax_partials(rows * cols)]. */
int bf8_quantize_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                      uint8_t* out_t, float* meta, uint32_t* partials, void* stream);

/* bf8_quantize_bf16 without the partials argument: allocates nothing and takes no
 * workspace. No counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The amax partials live in a library-owned device array of 1024 uint32 slots
 * (4 KB per GPU, held until the process ends; any tensor needs at most 1024, larger needs
 * are refused with BF8_EINVAL). The array is shared by every call on a GPU and keeps the
 * last call's contents, so calls that overlap on one GPU (different streams, or host
 * threads) race; serialize them. Results equal bf8_quantize_bf16's bit for bit. */
int bf8_quantize_bf16_noalloc(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                              uint8_t* out_t, float* meta, void* stream);

/* bf8_quantize_bf16 (rowwise output only) of 1-8 tensors in two launches: one amax pass
 * over all of them, one cast pass. Tensor t (x[t]: bf16 [n[t]], out[t]: fp8 [n[t]], both
 * 16-byte aligned; fmt[t] may carry BF8_SCALE_POW2) gets the bytes and meta[t] that its
 * own bf8_quantize_bf16 call would give; tensors with n[t] == 0 are skipped (meta
 * untouched). The arrays are host memory. partials: uint32
 * [bf8_quantize_many_partials(count, n)].
 * Replaces the back-to-back per-tensor casts of one forward: input and weight of
 * Float8Linear (bongard/float8_training.py:22) and TELinear (bongard/te_linear.py:73-74),
 * input, fc1 and fc2 weights of TEMLP / FusedMLP (bongard/te_linear.py:98-103,
 * bongard/fused_mlp.py:76-78). */
int64_t bf8_quantize_many_partials(int count, const int64_t* n);
int bf8_quantize_many_bf16(int count, const void* const* x, const int64_t* n, const int* fmt,
                           uint8_t* const* out, float* const* meta, uint32_t* partials,
                           void* stream);

/* ---------------------------------------------------------------------------------
 * FP8 GEMM, TN: C[m, n] = (sum_k A[m, k] * B[n, k]) * a_scale_inv * b_scale_inv(n)
 *                          (+ bias[n]), fp32 accumulation, bf16 or fp32 output.
 * Replaces torch._scaled_mm (cuBLASLt) under torchao Float8Linear (forward, and the
 * dgrad/wgrad GEMMs of its backward) and TE's FP8 GEMM under te.Linear
 * (bongard/te_linear.py:73-74); the emulated form is
 * ((Aq.float() / sa) @ (Bq.float() / sb).T).to(out_dtype).
 * A: fp8 [M, K] (row stride lda bytes), B: fp8 [N, K] (row stride ldb bytes),
 * K % 16 == 0, lda % 16 == ldb % 16 == 0, N % 8 == 0.
 * b_scale_inv: n_seg fp32 values at stride b_scale_stride floats; seg_ends (host array,
 * n_seg <= 4, ascending, last == N) assigns column n to the first segment whose end
 * exceeds n (fused QKV keeps one weight scale per projection). seg_ends may be NULL when
 * n_seg == 1. bias: bf16 [N] or NULL. C: [M, N] with row stride ldc elements.
 * ws: fp32 workspace for split-K partial sums (or, for a shape whose tiles leave a short
 * last round, the partials of the tail tiles' K pieces), bf8_gemm_workspace(M, N, K)
 * bytes (0 when the shape runs without either; ws may then be NULL). A smaller ws makes
 * the call choose a plan that fits it; results do not depend on the plan beyond fp32
 * summation order.
 * ------------------------------------------------------------------------------- */
size_t bf8_gemm_workspace(int64_t M, int64_t N, int64_t K);
int bf8_gemm(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b,
             int64_t ldb, int64_t M, int64_t N, int64_t K, const float* a_scale_inv,
             const float* b_scale_inv, int b_scale_stride, const int64_t* seg_ends,
             int n_seg, const void* bias, void* C, int out_dtype, int64_t ldc, void* ws,
             size_t ws_bytes, void* stream);

/* bf8_gemm for the training backward's dgrad and wgrad GEMMs on operands kept in the
 * layout that produced them, so no transposed fp8 copy is needed: B is given as
 * B^T [K, N] (row stride ldb >= N bytes, N % 16 == 0) and, when a_kmajor is 1, A as
 * A^T [K, M] (lda >= M, M % 16 == 0), else A [M, K] as in bf8_gemm. e5m2 A x e4m3 B,
 * one scale each, no bias; ws: bf8_gemm_kmajor_workspace(M, N, K) bytes. The products
 * and their fp32 sums are those of bf8_gemm on the transposed copies, bit for bit (same K
 * order). On small outputs, where the K-major tiles would leave most CUs idle, a call with
 * a_kmajor == 0 may transpose B into ws and run bf8_gemm's plan on it (the workspace size
 * covers that; with a smaller ws the call stays K-major). Replaces the dgrad (dX = dY . W) and wgrad (dW = dY^T . X) GEMMs of torchao's
 * Float8Linear and TE's Linear backward (bongard/float8_training.py:22;
 * bongard/te_linear.py:73-74), which transposes their operands' fp8 copies instead. */
size_t bf8_gemm_kmajor_workspace(int64_t M, int64_t N, int64_t K);
int bf8_gemm_kmajor(const uint8_t* A, int fmt_a, int64_t lda, int a_kmajor, const uint8_t* B,
                    int fmt_b, int64_t ldb, int64_t M, int64_t N, int64_t K,
                    const float* a_scale_inv, const float* b_scale_inv, void* C, int out_dtype,
                    int64_t ldc, void* ws, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * Gate/up GEMM with the gated-GELU(tanh) epilogue.
 * Replaces TEMLP.forward's gate_up GEMM + F.gelu(gate, approximate='tanh') * up
 * (bongard/te_linear.py:98-103; HF T5Gemma2MLP.forward) and TE LayerNormMLP's
 * fc1 + geglu (bongard/fused_mlp.py:25-30). Rounding chain, per element:
 *   g = bf16(acc_g * sx_inv * sg_inv), u = bf16(acc_u * sx_inv * su_inv),
 *   h = bf16(f32(bf16(gelu_tanh(f32(g)))) * f32(u)).
 * X: fp8 [M, K]; W: fp8 [2I, K] = [W_gate; W_up] (up rows start at row I).
 * w_scale_inv[0] scales gate rows, w_scale_inv[w_scale_stride] up rows
 * (w_scale_stride == 0: one shared scale, as TE's stacked gate_up weight).
 * H: bf16 [M, I] (row stride ldh). GU: bf16 [M, 2I] (gate | up, bf16-rounded
 * pre-activations kept for the backward) or NULL. h_partials: uint32
 * [bf8_geglu_partials(M, I)] per-tile amax of |H| (fp32 bits), for
 * bf8_cast_partials_bf16. I % 128 == 0.
 * bf16(gelu_tanh(g)) is torch's CPU gelu(approximate='tanh') on bf16 bit for bit (a
 * table over 2^-16 <= |g| < 8 taken from it at build time, closed rules outside), so H
 * equals the reference chain given g and u; a NaN H is 0xFFFF.
 * ------------------------------------------------------------------------------- */
int64_t bf8_geglu_partials(int64_t M, int64_t I);
int bf8_gemm_geglu(const uint8_t* X, int64_t ldx, const uint8_t* W, int64_t ldw, int64_t M,
                   int64_t I, int64_t K, const float* x_scale_inv, const float* w_scale_inv,
                   int w_scale_stride, void* H, int64_t ldh, void* GU,
                   uint32_t* h_partials, void* stream);

/* ---------------------------------------------------------------------------------
 * The gated GELU on its own: H bf16 [M, I] = bf16(bf16(gelu_tanh(g)) * u) from GU bf16
 * [M, 2I] (gate | up, the bf16 pre-activations), the step between the gate/up and down
 * GEMMs of TEMLP.forward, F.gelu(gate, approximate='tanh') * up (bongard/te_linear.py:103),
 * for pre-activations produced without the fused epilogue. Per-block amax partials of |H|
 * go to partials [bf8_geglu_partials_elementwise(M, I)] (for bf8_cast_partials_bf16).
 * gelu_tanh is torch's CPU function bit for bit (tables taken from it at build time), as
 * in bf8_gemm_geglu's epilogue; NaN results are 0xFFFF. I % 8 == 0, 16-byte aligned.
 * ------------------------------------------------------------------------------- */
int64_t bf8_geglu_partials_elementwise(int64_t M, int64_t I);
int bf8_geglu_bf16(const void* GU, int64_t M, int64_t I, void* H, uint32_t* partials,
                   void* stream);

/* ---------------------------------------------------------------------------------
 * Backward of the gated GELU: given dH bf16 [M, I] and GU bf16 [M, 2I] (from the
 * forward), write dGU bf16 [M, 2I] with
 *   d_gate = bf16(bf16(dH * u) * gelu'(g)), d_up = bf16(dH * bf16(gelu(g)))
 * following autograd of F.gelu(g, approximate='tanh') * u in bf16
 * (bongard/te_linear.py:103) bit for bit (gelu and its derivative factor are torch's CPU
 * values), and per-block amax partials of |dGU| into partials
 * [bf8_geglu_bwd_partials(M, I)] for its e5m2 cast (bf8_cast_partials_bf16).
 * ------------------------------------------------------------------------------- */
int64_t bf8_geglu_bwd_partials(int64_t M, int64_t I);
int bf8_geglu_bwd(const void* dH, const void* GU, int64_t M, int64_t I, void* dGU,
                  uint32_t* partials, void* stream);

/* ---------------------------------------------------------------------------------
 * Delayed scaling with an amax history (no counterpart in the reference, which uses
 * only current scaling: bongard/te_linear.py:38-39, bongard/fused_mlp.py:31-33).
 * Semantics (TE DelayedScaling, margin 0, amax_compute_algo "max"):
 *   the scale used at step t is fp8_max / max(history before step t) (1.0 while the
 *   history is all zero); after the step, amax_t (reduced from partials) is written
 *   into the ring at *pos and pos advances modulo len.
 * state: fp32 [len + 4] = {history[len], amax_t, scale, scale_inv, pos}; the last
 * three live at state + len + 1 .. + 3 so that state + len is a meta record.
 * bf8_delayed_scale_begin writes meta = state + len (scale for this step) before the
 * cast; bf8_delayed_scale_end pushes this step's amax after it.
 * ------------------------------------------------------------------------------- */
int bf8_delayed_scale_begin(float* state, int len, int fmt, void* stream);
int bf8_delayed_scale_end(float* state, int len, const uint32_t* partials,
                          int64_t n_partials, void* stream);

/* The scale step of bf8_cast_delayed_bf16 alone (same state / len / pos / prev_partials /
 * meta_out semantics, meta_out nullable): for a producer that then quantizes its own
 * output with the published scale (bf8_gemm_geglu_quant reading meta_out + 1) and writes
 * the new amax partials itself. Replaces the scale update of TE's DelayedScaling cast of
 * the fc2 input (bongard/te_linear.py:98-103; bongard/fused_mlp.py:25-30). */
int bf8_delayed_scale_fold(float* state, int len, int pos, const uint32_t* prev_partials,
                           int64_t n_prev, int fmt, float* meta_out, void* stream);

/* Delayed-scaling cast in one pass (the begin / cast / amax / end sequence above fused):
 * the kernel first pushes the previous step's amax (max of prev_partials, n_prev of them,
 * n_prev = 0 on the first step) into slot pos (0 <= pos < len) of the history, derives
 * this step's scale from the history, publishes {amax, scale, scale_inv, next slot} at
 * state + len and {history max, scale, scale_inv, 0} at meta_out (nullable; a copy the
 * next step does not overwrite, for a backward pass that runs after it), casts x like
 * bf8_cast_bf16, and writes this step's amax partials of |x|
 * into partials_out [bf8_cast_amax_partials(rows, cols, out_t != NULL)] (NULL when the
 * producer of x supplies them, as the gated-GELU GEMM does for H). Keep partials_out
 * until the next step's call, which reads it as prev_partials. */
int64_t bf8_cast_amax_partials(int64_t rows, int64_t cols, int transpose);
int bf8_cast_delayed_bf16(const void* x, int64_t rows, int64_t cols, float* state, int len,
                          int pos, const uint32_t* prev_partials, int64_t n_prev, int fmt,
                          float* meta_out, uint8_t* out, uint8_t* out_t, uint32_t* partials_out,
                          void* stream);

/* Up to 8 bf8_cast_delayed_bf16 calls in one launch (one training step's forward
 * quantizes x, [W_gate; W_up] and W_down at once, as TE casts one forward's operands
 * together: bongard/te_linear.py:73-74). Entry t takes
 * the arguments of the single call as element t of each array (out[t] or out_t[t] may be
 * NULL, partials_out[t] too); n_prev[t] <= 2048. Each tensor runs on the grid of its own
 * call, so bytes, metas, histories and partials equal those of the calls made one by one
 * in array order. Tensors with no elements are skipped (their state is left unchanged). */
int bf8_cast_delayed_many_bf16(int count, const void* const* x, const int64_t* rows,
                               const int64_t* cols, float* const* state, const int* len,
                               const int* pos, const uint32_t* const* prev_partials,
                               const int64_t* n_prev, const int* fmt, float* const* meta_out,
                               uint8_t* const* out, uint8_t* const* out_t,
                               uint32_t* const* partials_out, void* stream);

/* bf8_geglu_bwd fused with the delayed-scaling cast of its output (bf8_cast_delayed_bf16
 * semantics for state / len / pos / prev_partials / meta_out): for the 'fp8_delayed'
 * recipe, whose dGU scale is known before dGU exists. Writes dGU in fp8 directly, as
 * out [M, 2I] and/or out_t [2I, M], and this step's amax partials of |dGU| into
 * partials_out [bf8_geglu_bwd_delayed_partials(M, I)]; no bf16 dGU round trip. Bytes
 * equal bf8_geglu_bwd followed by bf8_cast_delayed_bf16. I % 64 == 0, M % 16 == 0,
 * n_prev <= 4096. Replaces the dGU cast of TE's delayed-scaling backward under TEMLP /
 * FusedMLP (bongard/te_linear.py:98-103; bongard/fused_mlp.py:25-30). */
int64_t bf8_geglu_bwd_delayed_partials(int64_t M, int64_t I);
int bf8_geglu_bwd_delayed(const void* dH, const void* GU, int64_t M, int64_t I, float* state,
                          int len, int pos, const uint32_t* prev_partials, int64_t n_prev, int fmt,
                          float* meta_out, uint8_t* out, uint8_t* out_t, uint32_t* partials_out,
                          void* stream);

/* ---------------------------------------------------------------------------------
 * Axiswise (per-row / per-column) quantization, torchao AXISWISE scaling granularity.
 * Replaces torchao hp_tensor_to_float8_dynamic(x, ..., scaling_granularity=AXISWISE,
 * axiswise_dim=-1 or 0, round_scales_to_power_of_2) under TrainingLinear.forward
 * (bongard/float8_training.py:22) for the rowwise recipes (bongard/float8_training.py:9).
 * x: bf16 [rows, cols] row-major, cols % 16 == 0, cols <= 16384. fmt may carry
 * BF8_SCALE_POW2 (the rowwise recipes set it).
 *   out [rows, cols], row_scale_inv [rows]: one scale per row (axiswise_dim -1);
 *   out_t [cols, rows], col_scale_inv [cols]: one scale per column (axiswise_dim 0),
 *   stored transposed (row c of out_t = column c of x).
 * Either pair may be NULL (not both). scale = fp32(fp8_max / max(f64(amax), 1e-12))
 * (then rounded down to a power of two), scale_inv = fp32(1 / scale).
 * ws: bf8_axiswise_workspace(rows, cols) bytes, 256-byte aligned, when out_t is given.
 * ------------------------------------------------------------------------------- */
size_t bf8_axiswise_workspace(int64_t rows, int64_t cols);
int bf8_quantize_axiswise_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                               float* row_scale_inv, uint8_t* out_t, float* col_scale_inv,
                               void* ws, size_t ws_bytes, void* stream);

/* FP8 GEMM with axiswise dequant scales, TN like bf8_gemm:
 *   C[m, n] = (sum_k A[m, k] * B[n, k]) * (a_scale_inv[a_vec ? m : 0] *
 *             b_scale_inv[b_vec ? n : 0]) (+ bias[n]).
 * Replaces torch._scaled_mm with row-wise scales (scale_a [M, 1], scale_b [1, N]) as
 * torchao's addmm_float8_unwrapped issues it for the rowwise recipes (a tensorwise
 * operand's scale is broadcast along its axis). Shapes, alignment and the split-K
 * workspace as bf8_gemm; a per-column b_scale_inv is 16-byte aligned. */
int bf8_gemm_axiswise(const uint8_t* A, int fmt_a, int64_t lda, const uint8_t* B, int fmt_b,
                      int64_t ldb, int64_t M, int64_t N, int64_t K, const float* a_scale_inv,
                      int a_vec, const float* b_scale_inv, int b_vec, const void* bias, void* C,
                      int out_dtype, int64_t ldc, void* ws, size_t ws_bytes, void* stream);

/* bf8_gemm_geglu with H quantized in the epilogue: H8 = e4m3(clamp(H * h_scale)) [M, I]
 * (8-byte aligned) and optionally H8t = its transpose [I, M] (16-byte aligned, M % 32 ==
 * 0), bytes identical to bf8_cast_bf16 of the bf16 H with the scale at h_scale (a device
 * fp32, e.g. meta_out + 1 of bf8_delayed_scale_fold). H (bf16) and GU are optional; the
 * amax partials of |H| are written as by bf8_gemm_geglu. The activation-and-cast ahead of
 * fc2 in TE LayerNormMLP / te.Linear under delayed scaling (bongard/te_linear.py:98-103,
 * bongard/fused_mlp.py:25-30). */
int bf8_gemm_geglu_quant(const uint8_t* X, int64_t ldx, const uint8_t* W, int64_t ldw,
                         int64_t M, int64_t I, int64_t K, const float* x_scale_inv,
                         const float* w_scale_inv, int w_scale_stride, const float* h_scale,
                         void* H, int64_t ldh, uint8_t* H8, uint8_t* H8t, void* GU,
                         uint32_t* h_partials, void* stream);

/* ---------------------------------------------------------------------------------
 * MXFP8 (OCP microscaling: 32-element blocks, one E8M0 scale byte each).
 * Replaces TE's MXFP8BlockScaling recipe (bongard/te_linear.py:17,38-39;
 * bongard/fused_mlp.py:9,31-33): its quantizer and its block-scaled FP8 GEMM.
 * Per block: amax = max |x|, e = E8M0 of fp32(amax * fp32(1 / fp8_max)) rounded up to a
 * power of two (NaN amax -> 0xFF, capped at 0xFE), q = fp8(clamp(x * 2^(127 - e))).
 * Scale arrays are [rows, bf8_mx_scale_ld(K)] bytes: byte b of a row is block b (K
 * elements b*32 .. b*32+31); bytes past the last block are 127 (= 1.0).
 * ------------------------------------------------------------------------------- */
int64_t bf8_mx_scale_ld(int64_t K);

/* x: bf16 [rows, cols]. out [rows, cols] + out_scales [rows, bf8_mx_scale_ld(cols)]:
 * blocks along rows (cols % 32 == 0). out_t [cols, rows] + out_t_scales
 * [cols, bf8_mx_scale_ld(rows)]: blocks along columns, stored transposed (rows % 32 == 0).
 * Either pair may be NULL (not both). */
int bf8_quantize_mx_bf16(const void* x, int64_t rows, int64_t cols, int fmt, uint8_t* out,
                         uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                         void* stream);

/* bf8_quantize_mx_bf16's rowwise output for 1-8 tensors in one launch: tensor t (x[t]:
 * bf16 [rows[t], cols[t]], cols[t] % 32 == 0) gets the bytes out[t] and scales
 * out_scales[t] ([rows[t], bf8_mx_scale_ld(cols[t])]) of its own call; empty tensors are
 * skipped. The arrays are host memory.
 * Replaces the per-tensor MXFP8 quantizations of one TE forward under 'mxfp8' (input and
 * weights of TELinear / TEMLP / FusedMLP: bongard/te_linear.py:98-103,
 * bongard/fused_mlp.py:25-33) when no columnwise copies are needed. */
int bf8_quantize_mx_many_bf16(int count, const void* const* x, const int64_t* rows,
                              const int64_t* cols, const int* fmt, uint8_t* const* out,
                              uint8_t* const* out_scales, void* stream);

/* ---------------------------------------------------------------------------------
 * NVFP4 (TE NVFP4BlockScaling under the 'nvfp4' recipe: bongard/te_linear.py:17,38,
 * bongard/fused_mlp.py:9,32). Round to nearest even everywhere, 1-D blocks of 16 along
 * the GEMM's reduction dimension; TE's random Hadamard transform, stochastic rounding of
 * gradients and 2-D weight blocks are not implemented.
 *   meta = {amax, S_enc = fp32(2688 / max(amax, 1e-12)), S_dec = fp32(1 / S_enc), 0}
 *   per block of 16 with b = max |x|: s = e4m3(fp32(fp32(b / 6) * S_enc)) (the scale
 *   byte), mult = s ? fp32(S_enc / s) : 0, code = e2m1_rne(fp32(x * mult)) saturating at
 *   6 (sign bit 3; two codes a byte, the even element in the low nibble)
 * bf8_quantize_nvfp4_bf16: amax pass into partials [bf8_amax_partials(rows * cols)], then
 * out [rows, cols / 2] + out_scales [rows, cols / 16] (rowwise, cols % 16 == 0) and/or
 * out_t [cols, rows / 2] + out_t_scales [cols, rows / 16] (the rowwise quantization of x^T,
 * rows % 16 == 0). bf8_dequant_nvfp4: bf16 [rows, cols] = e2m1(code) * s (exact; S_dec is
 * left to the GEMM). bf8_gemm_bf16: C = (A . B^T accumulated in fp32) * a_scale_inv *
 * b_scale_inv on bf16 A [M, K], B [N, K] (row strides lda, ldb elements, K % 8 == 0) on
 * the bf16 MFMA (gfx950's block-scaled MFMA takes FP4 only with power-of-two scales per 32
 * values, so NVFP4 runs as these exact bf16 operands with the two S_dec in the epilogue);
 * ws: bf8_gemm_bf16_workspace(M, N, K) bytes or 0.
 * ------------------------------------------------------------------------------- */
int bf8_quantize_nvfp4_bf16(const void* x, int64_t rows, int64_t cols, uint8_t* out,
                            uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                            float* meta, uint32_t* partials, void* stream);
/* bf8_quantize_nvfp4_bf16 without its amax pass: the per-tensor amax is the maximum of
 * n_partials amax partials of |x| (fp32 bits) that x's producer already wrote (the gated
 * GELU's backward for dGU, the fused RMSNorm for its output, the gate/up epilogue for H),
 * as NVFP4BlockScaling's quantizer takes the amax of the same tensor (bongard/te_linear.py:
 * 17,38; bongard/fused_mlp.py:9,32). Same outputs, bit for bit. */
int bf8_quantize_nvfp4_partials_bf16(const void* x, int64_t rows, int64_t cols,
                                     const uint32_t* partials, int64_t n_partials, uint8_t* out,
                                     uint8_t* out_scales, uint8_t* out_t, uint8_t* out_t_scales,
                                     float* meta, void* stream);
/* The NVFP4 quantizer whose rowwise copy is written as its exact bf16 dequantization deq
 * [rows, cols] (e2m1(code) * block scale, S_dec left to the GEMM: bf8_dequant_nvfp4's output
 * bit for bit) in place of the codes and scale bytes, for a tensor whose rowwise copy only
 * feeds the next GEMM (the forward's input, H, the backward's gradients under
 * NVFP4BlockScaling: bongard/te_linear.py:17,38; bongard/fused_mlp.py:9,32); out_t /
 * out_t_scales: the columnwise codes as in bf8_quantize_nvfp4_bf16, or NULL.
 * n_partials > 0: the amax comes from that many producer partials (as
 * bf8_quantize_nvfp4_partials_bf16); n_partials == 0: an amax pass writes partials
 * [bf8_amax_partials(rows * cols)] first. */
int bf8_quantize_nvfp4_dequant_bf16(const void* x, int64_t rows, int64_t cols,
                                    uint32_t* partials, int64_t n_partials, void* deq,
                                    uint8_t* out_t, uint8_t* out_t_scales, float* meta,
                                    void* stream);
int bf8_dequant_nvfp4(const uint8_t* q, const uint8_t* scales, int64_t rows, int64_t cols,
                      void* out, void* stream);
size_t bf8_gemm_bf16_workspace(int64_t M, int64_t N, int64_t K);
int bf8_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                  int64_t K, const float* a_scale_inv, const float* b_scale_inv, void* C,
                  int out_dtype, int64_t ldc, void* ws, size_t ws_bytes, void* stream);
/* bf8_gemm_geglu on bf16 operands: the NVFP4 gate/up projection (X^ [M, K] and
 * [W_gate; W_up]^ [2I, K], exactly dequantized, row strides ldx, ldw elements, K % 8 == 0)
 * with the gated GELU of TEMLP / LayerNormMLP (bongard/te_linear.py:98-103,
 * bongard/fused_mlp.py:25-30, under NVFP4BlockScaling: bongard/te_linear.py:17,38) in its
 * epilogue: g and u are the bf16 roundings of the fp32 sums times x_scale * w_scale (the two
 * S_dec), H = bf16(bf16(gelu_tanh(g)) * u) [M, I], GU the bf16 [g | u] [M, 2I] or NULL,
 * h_partials the amax partials of |H| [bf8_geglu_partials(M, I)]; I % 128 == 0. H and GU
 * equal bf8_gemm_bf16's bf16 output followed by bf8_geglu_bf16, bit for bit, where that
 * GEMM runs unsplit. */
int bf8_gemm_geglu_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw, int64_t M,
                        int64_t I, int64_t K, const float* x_scale, const float* w_scale,
                        void* H, int64_t ldh, void* GU, uint32_t* h_partials, void* stream);

/* C[m, n] = sum_b 2^(ea[m,b] + eb[n,b] - 254) * sum_{k in block b} A[m, k] * B[n, k]
 * (+ bias[n]), e4m3 operands, fp32 accumulation; TN like bf8_gemm, K % 32 == 0. Scale
 * arrays 4-byte aligned with row strides >= bf8_mx_scale_ld(K), multiples of 4.
 * ws: bf8_gemm_mx_workspace(M, N, K) bytes (split-K partials) or 0. */
size_t bf8_gemm_mx_workspace(int64_t M, int64_t N, int64_t K);
int bf8_gemm_mx(const uint8_t* A, int64_t lda, const uint8_t* A_scales, int64_t lda_sc,
                const uint8_t* B, int64_t ldb, const uint8_t* B_scales, int64_t ldb_sc,
                int64_t M, int64_t N, int64_t K, const void* bias, void* C, int out_dtype,
                int64_t ldc, void* ws, size_t ws_bytes, void* stream);

/* The gate/up GEMM with the gated-GELU epilogue (as bf8_gemm_geglu) on MXFP8 operands:
 * X [M, K] + scales, W [2I, K] = [W_gate; W_up] + scales. H, GU as bf8_gemm_geglu; no
 * amax partials (H's own MX quantization needs none). */
int bf8_gemm_geglu_mx(const uint8_t* X, int64_t ldx, const uint8_t* X_scales, int64_t ldx_sc,
                      const uint8_t* W, int64_t ldw, const uint8_t* W_scales, int64_t ldw_sc,
                      int64_t M, int64_t I, int64_t K, void* H, int64_t ldh, void* GU,
                      void* stream);

/* bf8_gemm_geglu_mx with H's MXFP8 (e4m3) quantization fused into the epilogue: the
 * activation-and-cast step ahead of fc2 in TE LayerNormMLP / te.Linear under
 * MXFP8BlockScaling (bongard/fused_mlp.py:25-33, bongard/te_linear.py:98-103), with
 * bytes and scales identical to bf8_quantize_mx_bf16 of the bf16 H.
 * H8 [M, I] (8-byte aligned) + H8_scales [M, ldh8_sc >= I / 32]: blocks along I (bytes
 * past I / 32 untouched). H8t [I, M] (16-byte aligned, M % 32 == 0) + H8t_scales
 * [I, ldh8t_sc >= bf8_mx_scale_ld(M)]: blocks along M, padded with 127 to
 * bf8_mx_scale_ld(M); NULL for none. H (bf16, ldh) and GU are optional (NULL = not
 * written). I % 128 == 0. */
int bf8_gemm_geglu_mx_quant(const uint8_t* X, int64_t ldx, const uint8_t* X_scales,
                            int64_t ldx_sc, const uint8_t* W, int64_t ldw,
                            const uint8_t* W_scales, int64_t ldw_sc, int64_t M, int64_t I,
                            int64_t K, void* H, int64_t ldh, uint8_t* H8, uint8_t* H8_scales,
                            int64_t ldh8_sc, uint8_t* H8t, uint8_t* H8t_scales,
                            int64_t ldh8t_sc, void* GU, void* stream);

/* ---------------------------------------------------------------------------------
 * RMSNorm fused with the amax pass of the quantization that follows it.
 * Replaces the RMSNorm (zero-centred gamma) of TE LayerNormMLP built at
 * bongard/fused_mlp.py:25-30 (HF T5Gemma2RMSNorm in evaluation, bongard/fused_mlp.py:64-65):
 *   r = 1 / sqrt(mean(f32(x)^2) + eps),  y = bf16((f32(x) * r) * (1 + f32(gamma)))
 * (gamma unchanged when zero_centered == 0). x, y: bf16 [rows, cols] row-major, cols % 8
 * == 0, cols <= 4096; gamma: bf16 [cols]; rstd: fp32 [rows] (r per row) or NULL.
 * partials: uint32 [bf8_rmsnorm_partials(rows)] amax keys of |y| per block, to pass to
 * bf8_cast_partials_bf16 (the cast then needs no amax pass over y).
 * ------------------------------------------------------------------------------- */
int64_t bf8_rmsnorm_partials(int64_t rows);
int bf8_rmsnorm_bf16(const void* x, int64_t rows, int64_t cols, const void* gamma, float eps,
                     int zero_centered, void* y, float* rstd, uint32_t* partials,
                     void* stream);

/* Backward of bf8_rmsnorm_bf16 for the bf16 gradient dy [rows, cols] of y, the autograd of
 * the fp32 formula above (the backward of TE LayerNormMLP's norm, bongard/fused_mlp.py:25-30,
 * as FusedMLP trains it): with n = x r, g = f32(dy), dn = g (z + gamma) (z = 1 when
 * zero_centered, else 0):
 *   dx = bf16(r (dn - n * sum_j(dn_j n_j) / cols))          per row
 *   dgamma = bf16(sum over rows of g n)                      per column
 * r is recomputed as the forward computes it. dx [rows, cols] and dgamma [cols] (bf16) are
 * each optional (not both NULL); dgamma needs ws: bf8_rmsnorm_bwd_workspace(rows, cols)
 * bytes of fp32 block partials, added in a fixed order (deterministic). Same shape limits
 * as the forward. */
size_t bf8_rmsnorm_bwd_workspace(int64_t rows, int64_t cols);
int bf8_rmsnorm_bwd_bf16(const void* x, const void* dy, int64_t rows, int64_t cols,
                         const void* gamma, float eps, int zero_centered, void* dx,
                         void* dgamma, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BONGARD_FP8_H */
