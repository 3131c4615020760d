"""Tensor-level FP8 ops on top of libbongard_fp8.so (gfx950 HIP kernels).

Every op runs on the caller's current HIP stream, allocates its outputs with PyTorch's
caching allocator, and never synchronises with the host. Inputs must be CUDA (HIP)
tensors; there is no CPU path.

Quantized tensors are returned as :class:`Fp8Tensor`: fp8 payload(s) plus a 4-float
device "meta" record ``{amax, scale, scale_inv, 0}`` with
``scale = fp32(fp8_max / max(f64(amax), 1e-12))`` and ``q = fp8(clamp(x * scale))``,
the semantics of torchao's tensorwise recipe (tensor_to_amax / amax_to_scale /
to_fp8_saturated) behind bongard/float8_training.py:22 and of TE's
Float8CurrentScaling behind bongard/te_linear.py:38-39,73-74.
"""

import ctypes
import functools
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from . import _lib

E4M3 = 0
E5M2 = 1
FP8_MAX = {E4M3: 448.0, E5M2: 57344.0}
TORCH_FP8 = {E4M3: torch.float8_e4m3fn, E5M2: torch.float8_e5m2}
OUT_BF16 = 0
OUT_F32 = 1
SCALE_POW2 = 0x10  # OR'ed into fmt: round the scale down to a power of two


@dataclass
class Fp8Tensor:
    """A per-tensor-scaled FP8 tensor: ``data`` [rows, cols] and/or ``data_t`` [cols, rows]."""

    data: Optional[torch.Tensor]
    data_t: Optional[torch.Tensor]
    meta: torch.Tensor  # float32 [4] (or a view into a larger buffer)
    fmt: int
    rows: int
    cols: int

    @property
    def scale(self):
        return self.meta[1]

    @property
    def scale_inv(self):
        return self.meta[2]

    @property
    def amax(self):
        return self.meta[0]


# Host cost matters at small shapes (eager forwards of a few microseconds of GPU work):
# pointers and streams go to the C ABI as plain integers (ctypes converts them for the
# void* parameters), the current stream is read through torch's raw-handle accessor, and
# the plan-dependent counts are cached per shape.
def _ptr(t):
    return t.data_ptr() if t is not None else None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _dev_index(device=None):
    if device is None:
        return torch.cuda.current_device()
    if not isinstance(device, torch.device):
        device = torch.device(device)
    return device.index if device.index is not None else torch.cuda.current_device()


def _stream(device=None):
    """The caller's current HIP stream on ``device`` as an integer handle."""
    idx = _dev_index(device)
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def _stream_key(device):
    idx = _dev_index(device)
    return idx, _stream(idx)


def _tile_override():
    # the GEMM planner reads this variable on every call; cached counts follow it
    return os.environ.get("BONGARD_FP8_GEMM_TILE", "")


@functools.lru_cache(maxsize=4096)
def _amax_partials_cached(n):
    return int(_lib.lib().bf8_amax_partials(n))


@functools.lru_cache(maxsize=4096)
def _many_partials_cached(sizes):
    return int(_lib.lib().bf8_quantize_many_partials(
        len(sizes), (ctypes.c_int64 * len(sizes))(*sizes)))


@functools.lru_cache(maxsize=4096)
def _gemm_ws_cached(M, N, K, override):
    return int(_lib.lib().bf8_gemm_workspace(M, N, K))


@functools.lru_cache(maxsize=4096)
def _geglu_partials_cached(M, I, override):
    return int(_lib.lib().bf8_geglu_partials(M, I))


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("bongard_amd FP8 ops need tensors on the HIP device (no CPU path)")


def _byte_matrix(who, **tensors):
    """FP8 payloads and E8M0 scale arrays reach the kernels as row-major byte matrices
    (row stride = stride(0), elements contiguous within a row): reject anything else
    rather than let the kernel read a transposed view's bytes in the wrong order."""
    for name, t in tensors.items():
        if t is None:
            continue
        if t.dim() != 2 or t.element_size() != 1 or (t.shape[1] > 1 and t.stride(1) != 1):
            raise ValueError(f"{who}: {name} must be a 2-D one-byte tensor with contiguous rows "
                             f"(got {t.dtype} {tuple(t.shape)} strides {t.stride()})")


def _out_matrix(who, out, shape, dtype):
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or (shape[1] > 1 and out.stride(1) != 1):
        raise ValueError(f"{who}: out must be {dtype} {tuple(shape)} with contiguous rows")


def _check_cast_outputs(who, out, out_t, rows, cols):
    """Caller-supplied cast outputs: contiguous one-byte [rows, cols] / [cols, rows]."""
    for name, t, shape in (("out", out, (rows, cols)), ("out_t", out_t, (cols, rows))):
        if t is not None and (tuple(t.shape) != shape or t.element_size() != 1
                              or not t.is_contiguous()):
            raise ValueError(f"{who}: {name} must be a contiguous one-byte tensor of shape "
                             f"{shape} (got {t.dtype} {tuple(t.shape)})")


def _gu_operand(who, GU, M, I):
    """The forward's saved [gate | up] pre-activations: bf16 [M, 2I], contiguous."""
    if GU.dtype != torch.bfloat16 or tuple(GU.shape) != (M, 2 * I):
        raise ValueError(f"{who}: GU must be bf16 [{M}, {2 * I}] (got {GU.dtype} {tuple(GU.shape)})")
    return GU.contiguous()


def _bf16_2d(x):
    if x.dtype != torch.bfloat16:
        raise TypeError(f"expected a bfloat16 tensor, got {x.dtype}")
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    if not x.is_contiguous():
        x = x.contiguous()
    return x


def amax_partials_count(n):
    return _amax_partials_cached(int(n))


def new_meta(device, count=1):
    """Uninitialised meta record(s): float32 [count, 4] (or [4] when count == 1); the
    kernels that produce a meta write all four words."""
    return torch.empty((count, 4) if count > 1 else (4,), dtype=torch.float32, device=device)


# Per-(device, stream) scratch for amax partials, reused in stream order.
_PARTIALS = {}


def partials_buffer(count, device):
    key = _stream_key(device)
    buf = _PARTIALS.get(key)
    if buf is None or buf.numel() < count:
        buf = torch.empty(max(int(count), 4096), dtype=torch.int32, device=device)
        _PARTIALS[key] = buf
    return buf


# Per-(device, stream) split-K workspace of bf8_gemm (fp32 partial sums), reused in
# stream order.
_GEMM_WS = {}


def gemm_workspace(nbytes, device):
    key = _stream_key(device)
    buf = _GEMM_WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=device)
        _GEMM_WS[key] = buf
    return buf


def quantize(x, fmt=E4M3, *, rowwise=True, transpose=False, meta=None, out=None, out_t=None,
             pow2=False):
    """Current-scaling quantization of a bf16 tensor (flattened to 2-D [rows, cols]).

    Returns an :class:`Fp8Tensor` whose ``data`` is [rows, cols] (if ``rowwise``) and
    ``data_t`` [cols, rows] (if ``transpose``), both as torch float8 tensors. ``pow2``
    rounds the scale down to a power of two (torchao round_scales_to_power_of_2).
    """
    _require_gpu(x)
    x = _bf16_2d(x)
    rows, cols = x.shape
    dev = x.device
    if meta is None:
        meta = new_meta(dev)
    if rowwise and out is None:
        out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=dev)
    if transpose and out_t is None:
        out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=dev)
    _check_cast_outputs("quantize", out if rowwise else None, out_t if transpose else None,
                        rows, cols)
    L = _lib.lib()
    parts = partials_buffer(_amax_partials_cached(rows * cols), dev)
    _lib.check(L.bf8_quantize_bf16(_ptr(x), rows, cols, fmt | (SCALE_POW2 if pow2 else 0),
                                   _ptr(out if rowwise else None),
                                   _ptr(out_t if transpose else None), _ptr(meta),
                                   _ptr(parts), _stream(dev)), "bf8_quantize_bf16")
    return Fp8Tensor(out if rowwise else None, out_t if transpose else None, meta, fmt, rows, cols)


def quantize_many(xs, fmts=None, *, pow2=False, metas=None):
    """:func:`quantize` (rowwise output, current scaling) of up to 8 bf16 tensors in two
    launches: one amax pass over all of them, one cast pass. Each result equals that
    tensor's own ``quantize(x, fmt, pow2=pow2)``, bytes and meta. ``fmts``: one format
    for all tensors or one per tensor (default e4m3); ``metas``: optional meta rows to
    write (as ``quantize(meta=...)``)."""
    xs = [_bf16_2d(x) for x in xs]
    count = len(xs)
    if not 1 <= count <= 8:
        raise ValueError(f"quantize_many: {count} tensors (1 to 8 supported)")
    _require_gpu(*xs)
    dev = xs[0].device
    if any(x.device != dev for x in xs):
        raise ValueError("quantize_many: tensors on different devices")
    if fmts is None or isinstance(fmts, int):
        fmts = [E4M3 if fmts is None else fmts] * count
    if len(fmts) != count:
        raise ValueError("quantize_many: one format per tensor")
    if metas is None:
        metas = new_meta(dev, count).unbind(0) if count > 1 else (new_meta(dev),)
    outs = [torch.empty(x.shape, dtype=TORCH_FP8[f], device=dev) for x, f in zip(xs, fmts)]
    L = _lib.lib()
    sizes = tuple(x.numel() for x in xs)
    n = (ctypes.c_int64 * count)(*sizes)
    parts = partials_buffer(max(1, _many_partials_cached(sizes)), dev)
    flag = SCALE_POW2 if pow2 else 0
    _lib.check(L.bf8_quantize_many_bf16(
        count, (ctypes.c_void_p * count)(*[x.data_ptr() for x in xs]), n,
        (ctypes.c_int * count)(*[f | flag for f in fmts]),
        (ctypes.c_void_p * count)(*[o.data_ptr() for o in outs]),
        (ctypes.c_void_p * count)(*[m.data_ptr() for m in metas]), _ptr(parts), _stream(dev)),
        "bf8_quantize_many_bf16")
    return [Fp8Tensor(o, None, m, f, x.shape[0], x.shape[1])
            for x, o, m, f in zip(xs, outs, metas, fmts)]


def amax(x):
    """Per-block partial amax keys (int32 view of fp32 bits) of a bf16 tensor."""
    _require_gpu(x)
    x = _bf16_2d(x)
    partials = torch.empty(amax_partials_count(x.numel()), dtype=torch.int32, device=x.device)
    _lib.check(_lib.lib().bf8_amax_bf16(_ptr(x), x.numel(), _ptr(partials), _stream(x.device)),
               "bf8_amax_bf16")
    return partials


def scale_from_partials(partials, fmt, meta=None):
    if meta is None:
        meta = new_meta(partials.device)
    _lib.check(_lib.lib().bf8_scale_from_partials(_ptr(partials), partials.numel(), fmt,
                                                  _ptr(meta), _stream(partials.device)),
               "bf8_scale_from_partials")
    return meta


def cast_partials(x, partials, fmt=E4M3, *, rowwise=True, transpose=False):
    """Cast whose scale comes from amax partials (as returned by ``gemm_geglu`` /
    ``geglu_bwd``); returns the Fp8Tensor with its freshly written meta."""
    _require_gpu(x, partials)
    x = _bf16_2d(x)
    rows, cols = x.shape
    meta = new_meta(x.device)
    out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=x.device) if rowwise else None
    out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=x.device) if transpose else None
    _lib.check(_lib.lib().bf8_cast_partials_bf16(_ptr(x), rows, cols, _ptr(partials),
                                                 partials.numel(), fmt, _ptr(meta), _ptr(out),
                                                 _ptr(out_t), _stream(x.device)),
               "bf8_cast_partials_bf16")
    return Fp8Tensor(out, out_t, meta, fmt, rows, cols)


def cast(x, meta, fmt=E4M3, *, rowwise=True, transpose=False, out=None, out_t=None):
    """Cast with an existing scale (``meta[1]``), e.g. delayed scaling."""
    _require_gpu(x, meta)
    x = _bf16_2d(x)
    rows, cols = x.shape
    if rowwise and out is None:
        out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=x.device)
    if transpose and out_t is None:
        out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=x.device)
    _check_cast_outputs("cast", out if rowwise else None, out_t if transpose else None,
                        rows, cols)
    scale_ptr = ctypes.c_void_p(meta.data_ptr() + 4)
    _lib.check(_lib.lib().bf8_cast_bf16(_ptr(x), rows, cols, scale_ptr, fmt,
                                        _ptr(out if rowwise else None),
                                        _ptr(out_t if transpose else None), _stream(x.device)),
               "bf8_cast_bf16")
    return Fp8Tensor(out if rowwise else None, out_t if transpose else None, meta, fmt, rows, cols)


def _sinv_ptr(meta):
    return meta.data_ptr() + 8


def gemm(a, a_fmt, a_meta, b, b_fmt, b_meta, *, out_dtype=torch.bfloat16, bias=None,
         seg_ends: Optional[Sequence[int]] = None, b_meta_stride=4, out=None):
    """``C = (a @ b.T) * a_scale_inv * b_scale_inv (+ bias)`` on fp8 operands.

    a: fp8 [M, K], b: fp8 [N, K] (row-major, K contiguous). ``b_meta`` is the meta of b,
    or for ``seg_ends`` (fused projections) the first of ``len(seg_ends)`` meta records
    ``b_meta_stride`` floats apart.
    """
    _require_gpu(a, b, a_meta, b_meta)
    _byte_matrix("gemm", a=a, b=b)
    M, K = a.shape
    N, Kb = b.shape
    if K != Kb:
        raise ValueError(f"gemm: inner dims differ ({K} vs {Kb})")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("gemm: out_dtype must be bfloat16 or float32")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    _out_matrix("gemm", out, (M, N), out_dtype)
    n_seg = 1
    seg = None
    if seg_ends is not None:
        n_seg = len(seg_ends)
        seg = (ctypes.c_int64 * n_seg)(*[int(s) for s in seg_ends])
    if bias is not None:
        if bias.dtype != torch.bfloat16:
            raise TypeError("gemm: bias must be bfloat16")
        bias = bias.contiguous()
    L = _lib.lib()
    ws_bytes = _gemm_ws_cached(M, N, K, _tile_override())
    ws = gemm_workspace(ws_bytes, a.device) if ws_bytes else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.check(L.bf8_gemm(_ptr(a), a_fmt, a.stride(0), _ptr(b), b_fmt, b.stride(0), M, N, K,
                          _sinv_ptr(a_meta), _sinv_ptr(b_meta), b_meta_stride, seg, n_seg,
                          _ptr(bias), _ptr(out), OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32,
                          out.stride(0), _ptr(ws), ws_bytes, _stream(a.device)), "bf8_gemm")
    return out


@functools.lru_cache(maxsize=256)
def _gemm_kmajor_ws_cached(M, N, K, override):
    return int(_lib.lib().bf8_gemm_kmajor_workspace(M, N, K))


def gemm_kmajor(a, a_fmt, a_meta, b_t, b_fmt, b_meta, *, a_kmajor=False,
                out_dtype=torch.bfloat16, out=None):
    """:func:`gemm` with B given as ``b_t`` = B^T [K, N] (and, when ``a_kmajor``, A as ``a``
    = A^T [K, M]): the backward's dgrad and wgrad GEMMs on the fp8 tensors as their
    producers wrote them, no transposed copies (bf8_gemm_kmajor; e5m2 x e4m3). Same
    products and fp32 sums as :func:`gemm` on the transposed operands."""
    _require_gpu(a, b_t, a_meta, b_meta)
    _byte_matrix("gemm_kmajor", a=a, b_t=b_t)
    if a_kmajor:
        K, M = a.shape
    else:
        M, K = a.shape
    Kb, N = b_t.shape
    if K != Kb:
        raise ValueError(f"gemm_kmajor: inner dims differ ({K} vs {Kb})")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("gemm_kmajor: out_dtype must be bfloat16 or float32")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    _out_matrix("gemm_kmajor", out, (M, N), out_dtype)
    ws_bytes = _gemm_kmajor_ws_cached(M, N, K, _tile_override())
    ws = gemm_workspace(ws_bytes, a.device) if ws_bytes else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.check(_lib.lib().bf8_gemm_kmajor(
        _ptr(a), a_fmt, a.stride(0), int(bool(a_kmajor)), _ptr(b_t), b_fmt, b_t.stride(0), M, N,
        K, _sinv_ptr(a_meta), _sinv_ptr(b_meta), _ptr(out),
        OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32, out.stride(0), _ptr(ws), ws_bytes,
        _stream(a.device)), "bf8_gemm_kmajor")
    return out


@dataclass
class AxisFp8Tensor:
    """An axiswise-scaled FP8 tensor (torchao AXISWISE granularity) of x [rows, cols]:
    ``data`` [rows, cols] with one scale per row (``row_sinv`` fp32 [rows], the inverse
    scales) and/or ``data_t`` [cols, rows] with one scale per column of x (``col_sinv``
    fp32 [cols])."""

    data: Optional[torch.Tensor]
    row_sinv: Optional[torch.Tensor]
    data_t: Optional[torch.Tensor]
    col_sinv: Optional[torch.Tensor]
    fmt: int
    rows: int
    cols: int


_AXIS_WS = {}


def quantize_axiswise(x, fmt=E4M3, *, rowwise=True, colwise=False, pow2=True):
    """Per-row (``rowwise``, torchao axiswise_dim=-1) and/or per-column (``colwise``,
    axiswise_dim=0, stored transposed) quantization of a bf16 tensor; ``pow2`` rounds the
    scales down to powers of two as torchao's rowwise recipes do."""
    _require_gpu(x)
    x = _bf16_2d(x)
    rows, cols = x.shape
    dev = x.device
    if not (rowwise or colwise):
        raise ValueError("quantize_axiswise: nothing requested")
    out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=dev) if rowwise else None
    rs = torch.empty(rows, dtype=torch.float32, device=dev) if rowwise else None
    out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=dev) if colwise else None
    cs = torch.empty(cols, dtype=torch.float32, device=dev) if colwise else None
    L = _lib.lib()
    ws, nbytes = None, 0
    if colwise:
        nbytes = int(L.bf8_axiswise_workspace(rows, cols))
        key = _stream_key(dev)
        ws = _AXIS_WS.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
            _AXIS_WS[key] = ws
        nbytes = ws.numel()
    _lib.check(L.bf8_quantize_axiswise_bf16(_ptr(x), rows, cols, fmt | (SCALE_POW2 if pow2 else 0),
                                            _ptr(out), _ptr(rs), _ptr(out_t), _ptr(cs), _ptr(ws),
                                            nbytes, _stream(dev)), "bf8_quantize_axiswise_bf16")
    return AxisFp8Tensor(out, rs, out_t, cs, fmt, rows, cols)


def gemm_axiswise(a, a_fmt, a_sinv, b, b_fmt, b_sinv, *, out_dtype=torch.bfloat16, bias=None,
                  out=None):
    """``C[m, n] = (a @ b.T)[m, n] * a_sinv[m] * b_sinv[n] (+ bias[n])`` on fp8 operands.

    a: fp8 [M, K], b: fp8 [N, K]. ``a_sinv`` is fp32 [M] (one inverse scale per row of a)
    or a single value (1-element tensor, e.g. a meta's ``scale_inv``); likewise ``b_sinv``
    with [N]."""
    _require_gpu(a, b, a_sinv, b_sinv)
    _byte_matrix("gemm_axiswise", a=a, b=b)
    M, K = a.shape
    N, Kb = b.shape
    if K != Kb:
        raise ValueError(f"gemm_axiswise: inner dims differ ({K} vs {Kb})")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("gemm_axiswise: out_dtype must be bfloat16 or float32")

    def vec_flag(sv, n, what):
        if sv.dtype != torch.float32 or not sv.is_contiguous():
            raise TypeError(f"gemm_axiswise: {what} must be contiguous float32")
        if sv.numel() == n and n != 1:
            return 1
        if sv.numel() == 1:
            return 0
        raise ValueError(f"gemm_axiswise: {what} must have 1 or {n} elements")

    a_vec = vec_flag(a_sinv, M, "a_sinv")
    b_vec = vec_flag(b_sinv, N, "b_sinv")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    _out_matrix("gemm_axiswise", out, (M, N), out_dtype)
    if bias is not None:
        if bias.dtype != torch.bfloat16:
            raise TypeError("gemm_axiswise: bias must be bfloat16")
        bias = bias.contiguous()
    L = _lib.lib()
    ws_bytes = _gemm_ws_cached(M, N, K, _tile_override())
    ws = gemm_workspace(ws_bytes, a.device) if ws_bytes else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.check(L.bf8_gemm_axiswise(_ptr(a), a_fmt, a.stride(0), _ptr(b), b_fmt, b.stride(0), M, N,
                                   K, _ptr(a_sinv), a_vec, _ptr(b_sinv), b_vec, _ptr(bias),
                                   _ptr(out), OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32,
                                   out.stride(0), _ptr(ws), ws_bytes, _stream(a.device)),
               "bf8_gemm_axiswise")
    return out


@dataclass
class MxFp8Tensor:
    """An MXFP8 tensor of x [rows, cols] (32-element blocks, one E8M0 byte each):
    ``data`` [rows, cols] with ``scales`` [rows, mx_scale_ld(cols)] (blocks along rows)
    and/or ``data_t`` [cols, rows] with ``scales_t`` [cols, mx_scale_ld(rows)] (blocks along
    columns of x, stored transposed)."""

    data: Optional[torch.Tensor]
    scales: Optional[torch.Tensor]
    data_t: Optional[torch.Tensor]
    scales_t: Optional[torch.Tensor]
    fmt: int
    rows: int
    cols: int


def mx_scale_ld(K):
    return int(_lib.lib().bf8_mx_scale_ld(int(K)))


def quantize_mx(x, fmt=E4M3, *, rowwise=True, colwise=False):
    """MXFP8 quantization of a bf16 tensor (TE MXFP8BlockScaling arithmetic)."""
    _require_gpu(x)
    x = _bf16_2d(x)
    rows, cols = x.shape
    dev = x.device
    if not (rowwise or colwise):
        raise ValueError("quantize_mx: nothing requested")
    out = sc = out_t = sc_t = None
    if rowwise:
        out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=dev)
        sc = torch.empty((rows, mx_scale_ld(cols)), dtype=torch.uint8, device=dev)
    if colwise:
        out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=dev)
        sc_t = torch.empty((cols, mx_scale_ld(rows)), dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().bf8_quantize_mx_bf16(_ptr(x), rows, cols, fmt, _ptr(out), _ptr(sc),
                                               _ptr(out_t), _ptr(sc_t), _stream(dev)),
               "bf8_quantize_mx_bf16")
    return MxFp8Tensor(out, sc, out_t, sc_t, fmt, rows, cols)


def quantize_mx_many(xs, fmts=None):
    """Rowwise :func:`quantize_mx` of up to 8 bf16 tensors in one launch; each result
    equals that tensor's own ``quantize_mx(x, fmt)`` (bytes and scales). ``fmts``: one
    format for all or one per tensor (default e4m3)."""
    xs = [_bf16_2d(x) for x in xs]
    count = len(xs)
    if not 1 <= count <= 8:
        raise ValueError(f"quantize_mx_many: {count} tensors (1 to 8 supported)")
    _require_gpu(*xs)
    dev = xs[0].device
    if any(x.device != dev for x in xs):
        raise ValueError("quantize_mx_many: tensors on different devices")
    if fmts is None or isinstance(fmts, int):
        fmts = [E4M3 if fmts is None else fmts] * count
    if len(fmts) != count:
        raise ValueError("quantize_mx_many: one format per tensor")
    outs = [torch.empty(x.shape, dtype=TORCH_FP8[f], device=dev) for x, f in zip(xs, fmts)]
    scs = [torch.empty((x.shape[0], mx_scale_ld(x.shape[1])), dtype=torch.uint8, device=dev)
           for x in xs]
    _lib.check(_lib.lib().bf8_quantize_mx_many_bf16(
        count, (ctypes.c_void_p * count)(*[x.data_ptr() for x in xs]),
        (ctypes.c_int64 * count)(*[x.shape[0] for x in xs]),
        (ctypes.c_int64 * count)(*[x.shape[1] for x in xs]), (ctypes.c_int * count)(*fmts),
        (ctypes.c_void_p * count)(*[o.data_ptr() for o in outs]),
        (ctypes.c_void_p * count)(*[c.data_ptr() for c in scs]), _stream(dev)),
        "bf8_quantize_mx_many_bf16")
    return [MxFp8Tensor(o, c, None, None, f, x.shape[0], x.shape[1])
            for x, o, c, f in zip(xs, outs, scs, fmts)]


def gemm_mx(a, a_scales, b, b_scales, *, out_dtype=torch.bfloat16, bias=None, out=None):
    """``C = a @ b.T`` on MXFP8 (e4m3) operands a [M, K], b [N, K] with their E8M0 block
    scales [M, >= mx_scale_ld(K)], [N, ...]."""
    _require_gpu(a, b, a_scales, b_scales)
    _byte_matrix("gemm_mx", a=a, b=b, a_scales=a_scales, b_scales=b_scales)
    M, K = a.shape
    N, Kb = b.shape
    if K != Kb:
        raise ValueError(f"gemm_mx: inner dims differ ({K} vs {Kb})")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("gemm_mx: out_dtype must be bfloat16 or float32")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    _out_matrix("gemm_mx", out, (M, N), out_dtype)
    if bias is not None:
        if bias.dtype != torch.bfloat16:
            raise TypeError("gemm_mx: bias must be bfloat16")
        bias = bias.contiguous()
    L = _lib.lib()
    ws_bytes = int(L.bf8_gemm_mx_workspace(M, N, K))
    ws = gemm_workspace(ws_bytes, a.device) if ws_bytes else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.check(L.bf8_gemm_mx(_ptr(a), a.stride(0), _ptr(a_scales), a_scales.stride(0), _ptr(b),
                             b.stride(0), _ptr(b_scales), b_scales.stride(0), M, N, K, _ptr(bias),
                             _ptr(out), OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32,
                             out.stride(0), _ptr(ws), ws_bytes, _stream(a.device)), "bf8_gemm_mx")
    return out


def gemm_geglu_mx(x8, x_scales, w8, w_scales, intermediate, *, keep_gu=False):
    """Gate/up GEMM + gated GELU on MXFP8 operands; returns ``(H bf16 [M, I], GU or None)``."""
    _require_gpu(x8, x_scales, w8, w_scales)
    _byte_matrix("gemm_geglu_mx", x8=x8, w8=w8, x_scales=x_scales, w_scales=w_scales)
    M, K = x8.shape
    I = int(intermediate)
    if w8.shape != (2 * I, K):
        raise ValueError(f"gemm_geglu_mx: W must be [{2 * I}, {K}]")
    H = torch.empty((M, I), dtype=torch.bfloat16, device=x8.device)
    GU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=x8.device) if keep_gu else None
    _lib.check(_lib.lib().bf8_gemm_geglu_mx(_ptr(x8), x8.stride(0), _ptr(x_scales),
                                            x_scales.stride(0), _ptr(w8), w8.stride(0),
                                            _ptr(w_scales), w_scales.stride(0), M, I, K, _ptr(H),
                                            H.stride(0), _ptr(GU), _stream(x8.device)),
               "bf8_gemm_geglu_mx")
    return H, GU


def gemm_geglu_mx_quant(x8, x_scales, w8, w_scales, intermediate, *, colwise=False,
                        keep_gu=False, keep_h=False):
    """:func:`gemm_geglu_mx` with H's MXFP8 (e4m3) quantization done in the GEMM epilogue.

    Returns ``(hq, GU or None, H or None)``: ``hq`` an :class:`MxFp8Tensor` of H with the
    rowwise copy and, if ``colwise`` (needs M % 32 == 0), the columnwise one, byte for byte
    what :func:`quantize_mx` gives for the bf16 H; ``H`` the bf16 H when ``keep_h``."""
    _require_gpu(x8, x_scales, w8, w_scales)
    _byte_matrix("gemm_geglu_mx_quant", x8=x8, w8=w8, x_scales=x_scales, w_scales=w_scales)
    M, K = x8.shape
    I = int(intermediate)
    if w8.shape != (2 * I, K):
        raise ValueError(f"gemm_geglu_mx_quant: W must be [{2 * I}, {K}]")
    dev = x8.device
    fp8 = TORCH_FP8[E4M3]
    h8 = torch.empty((M, I), dtype=fp8, device=dev)
    h8_sc = torch.empty((M, mx_scale_ld(I)), dtype=torch.uint8, device=dev)
    h8t = h8t_sc = None
    if colwise:
        h8t = torch.empty((I, M), dtype=fp8, device=dev)
        h8t_sc = torch.empty((I, mx_scale_ld(M)), dtype=torch.uint8, device=dev)
    H = torch.empty((M, I), dtype=torch.bfloat16, device=dev) if keep_h else None
    GU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=dev) if keep_gu else None
    _lib.check(_lib.lib().bf8_gemm_geglu_mx_quant(
        _ptr(x8), x8.stride(0), _ptr(x_scales), x_scales.stride(0), _ptr(w8), w8.stride(0),
        _ptr(w_scales), w_scales.stride(0), M, I, K, _ptr(H), I, _ptr(h8), _ptr(h8_sc),
        h8_sc.stride(0), _ptr(h8t), _ptr(h8t_sc), h8t_sc.stride(0) if colwise else 0, _ptr(GU),
        _stream(dev)), "bf8_gemm_geglu_mx_quant")
    return MxFp8Tensor(h8, h8_sc, h8t, h8t_sc, E4M3, M, I), GU, H


def geglu_partials_count(M, intermediate):
    return _geglu_partials_cached(int(M), int(intermediate), _tile_override())


def gemm_geglu(x8, x_meta, w8, w_meta, intermediate, *, w_meta_stride=0, keep_gu=False,
               partials=None):
    """Gate/up GEMM with the gated-GELU epilogue.

    x8: fp8 e4m3 [M, K]; w8: fp8 e4m3 [2I, K] (gate rows then up rows). Returns
    ``(H bf16 [M, I], GU bf16 [M, 2I] or None, h_partials int32 [tiles])``; the per-tile
    amax partials of |H| feed ``cast_partials`` (or a delayed scaler). ``partials``: an
    optional caller-owned buffer of at least ``geglu_partials_count(M, I)`` entries.
    """
    _require_gpu(x8, w8, x_meta, w_meta)
    _byte_matrix("gemm_geglu", x8=x8, w8=w8)
    M, K = x8.shape
    I = int(intermediate)
    if w8.shape != (2 * I, K):
        raise ValueError(f"gemm_geglu: weight must be [{2 * I}, {K}], got {tuple(w8.shape)}")
    L = _lib.lib()
    H = torch.empty((M, I), dtype=torch.bfloat16, device=x8.device)
    GU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=x8.device) if keep_gu else None
    count = _geglu_partials_cached(M, I, _tile_override())
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=x8.device)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"gemm_geglu: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(L.bf8_gemm_geglu(_ptr(x8), x8.stride(0), _ptr(w8), w8.stride(0), M, I, K,
                                _sinv_ptr(x_meta), _sinv_ptr(w_meta), w_meta_stride, _ptr(H),
                                H.stride(0), _ptr(GU), _ptr(parts), _stream(x8.device)),
               "bf8_gemm_geglu")
    return H, GU, parts


def gemm_geglu_quant(x8, x_meta, w8, w_meta, intermediate, h_meta, *, w_meta_stride=0,
                     transpose=False, keep_gu=False, keep_h=False, partials=None):
    """:func:`gemm_geglu` with H cast to e4m3 in the epilogue with the scale ``h_meta[1]``
    (a device meta record, e.g. from :func:`delayed_scale_fold`), byte for byte what
    :func:`cast` gives for the bf16 H. Returns ``(hq, GU or None, H or None, h_partials)``:
    ``hq`` the :class:`Fp8Tensor` of H (``data`` [M, I], ``data_t`` [I, M] when
    ``transpose``, which needs M % 32 == 0) with meta ``h_meta``."""
    _require_gpu(x8, w8, x_meta, w_meta, h_meta)
    _byte_matrix("gemm_geglu_quant", x8=x8, w8=w8)
    M, K = x8.shape
    I = int(intermediate)
    if w8.shape != (2 * I, K):
        raise ValueError(f"gemm_geglu_quant: weight must be [{2 * I}, {K}], got {tuple(w8.shape)}")
    dev = x8.device
    L = _lib.lib()
    h8 = torch.empty((M, I), dtype=TORCH_FP8[E4M3], device=dev)
    h8t = torch.empty((I, M), dtype=TORCH_FP8[E4M3], device=dev) if transpose else None
    H = torch.empty((M, I), dtype=torch.bfloat16, device=dev) if keep_h else None
    GU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=dev) if keep_gu else None
    count = _geglu_partials_cached(M, I, _tile_override())
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=dev)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"gemm_geglu_quant: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(L.bf8_gemm_geglu_quant(
        _ptr(x8), x8.stride(0), _ptr(w8), w8.stride(0), M, I, K, _sinv_ptr(x_meta),
        _sinv_ptr(w_meta), w_meta_stride, ctypes.c_void_p(h_meta.data_ptr() + 4), _ptr(H), I,
        _ptr(h8), _ptr(h8t), _ptr(GU), _ptr(parts), _stream(dev)), "bf8_gemm_geglu_quant")
    return Fp8Tensor(h8, h8t, h_meta, E4M3, M, I), GU, H, parts


def delayed_scale_fold(state, length, pos, prev_partials, fmt=E4M3, meta_out=None):
    """The scale step of :func:`cast_delayed` alone: pushes ``prev_partials`` (the previous
    step's amax partials, or None) into history slot ``pos``, derives this step's scale and
    returns it as a meta record (``meta_out``, allocated when None)."""
    _require_gpu(state)
    if meta_out is None:
        meta_out = new_meta(state.device)
    n_prev = 0 if prev_partials is None else prev_partials.numel()
    _lib.check(_lib.lib().bf8_delayed_scale_fold(_ptr(state), int(length), int(pos),
                                                 _ptr(prev_partials), n_prev, fmt,
                                                 _ptr(meta_out), _stream(state.device)),
               "bf8_delayed_scale_fold")
    return meta_out


def geglu(GU, *, partials=None):
    """H bf16 [M, I] = gelu_tanh(gate) * up from the bf16 pre-activations GU [M, 2I]
    (gate | up), bit for bit the reference's bf16 chain, and the per-block amax partials
    of |H| (for ``cast_partials``)."""
    _require_gpu(GU)
    if GU.dtype != torch.bfloat16 or GU.dim() != 2 or GU.shape[1] % 2:
        raise ValueError(f"geglu: GU must be bf16 [M, 2I] (got {GU.dtype} {tuple(GU.shape)})")
    GU = GU.contiguous()
    M, I = GU.shape[0], GU.shape[1] // 2
    L = _lib.lib()
    H = torch.empty((M, I), dtype=torch.bfloat16, device=GU.device)
    count = int(L.bf8_geglu_partials_elementwise(M, I))
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=GU.device)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"geglu: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(L.bf8_geglu_bf16(_ptr(GU), M, I, _ptr(H), _ptr(parts), _stream(GU.device)),
               "bf8_geglu_bf16")
    return H, parts


def geglu_bwd_partials_count(M, intermediate):
    return int(_lib.lib().bf8_geglu_bwd_partials(int(M), int(intermediate)))


def geglu_bwd(dH, GU, *, partials=None):
    """dGU bf16 [M, 2I] (d_gate | d_up) from dH [M, I] and the forward's GU, and the
    per-block amax partials of |dGU| (for ``cast_partials`` or a delayed scaler;
    ``partials``: an optional caller-owned buffer)."""
    _require_gpu(dH, GU)
    dH = dH.contiguous()
    M, I = dH.shape
    GU = _gu_operand("geglu_bwd", GU, M, I)
    L = _lib.lib()
    dGU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=dH.device)
    count = int(L.bf8_geglu_bwd_partials(M, I))
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=dH.device)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"geglu_bwd: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(L.bf8_geglu_bwd(_ptr(dH), _ptr(GU), M, I, _ptr(dGU), _ptr(parts),
                               _stream(dH.device)), "bf8_geglu_bwd")
    return dGU, parts


RMSNORM_MAX_COLS = 4096


def rmsnorm_supported(cols):
    """Whether the fused RMSNorm kernel takes rows of ``cols`` elements."""
    return cols % 8 == 0 and 0 < cols <= RMSNORM_MAX_COLS


def rmsnorm_partials_count(rows):
    return int(_lib.lib().bf8_rmsnorm_partials(int(rows)))


def rmsnorm(x, weight, eps, *, zero_centered=True, want_rstd=False, partials=None):
    """RMSNorm of bf16 rows (HF T5Gemma2RMSNorm arithmetic) fused with the amax of its output.

    Returns ``(y bf16 [rows, cols], rstd fp32 [rows] or None, partials int32)``; pass the
    partials to :func:`cast_partials` (current scaling) to quantize y without an amax pass.
    ``partials``: an optional caller-owned buffer of at least ``rmsnorm_partials_count``
    entries (e.g. a delayed scaler's producer buffer).
    """
    _require_gpu(x, weight)
    x = _bf16_2d(x)
    rows, cols = x.shape
    if weight.dtype != torch.bfloat16 or weight.numel() != cols:
        raise ValueError(f"rmsnorm: weight must be bf16 [{cols}]")
    weight = weight.contiguous()
    L = _lib.lib()
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if want_rstd else None
    count = int(L.bf8_rmsnorm_partials(rows))
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=x.device)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"rmsnorm: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(L.bf8_rmsnorm_bf16(_ptr(x), rows, cols, _ptr(weight), float(eps),
                                  int(bool(zero_centered)), _ptr(y), _ptr(rstd), _ptr(parts),
                                  _stream(x.device)), "bf8_rmsnorm_bf16")
    return y, rstd, parts


def rmsnorm_backward(x, dy, weight, eps, *, zero_centered=True, need_dx=True, need_dw=True):
    """Gradients (dx bf16 [rows, cols] or None, dweight bf16 [cols] or None) of
    :func:`rmsnorm` for the bf16 gradient dy of its output."""
    _require_gpu(x, dy, weight)
    x = _bf16_2d(x)
    dy = _bf16_2d(dy)
    rows, cols = x.shape
    if tuple(dy.shape) != (rows, cols):
        raise ValueError(f"rmsnorm_backward: dy must be [{rows}, {cols}]")
    if weight.dtype != torch.bfloat16 or weight.numel() != cols:
        raise ValueError(f"rmsnorm_backward: weight must be bf16 [{cols}]")
    if not (need_dx or need_dw):
        return None, None
    weight = weight.contiguous()
    L = _lib.lib()
    dx = torch.empty_like(x) if need_dx else None
    dw = torch.empty(cols, dtype=torch.bfloat16, device=x.device) if need_dw else None
    ws, nbytes = None, 0
    if need_dw:
        nbytes = int(L.bf8_rmsnorm_bwd_workspace(rows, cols))
        ws = gemm_workspace(nbytes, x.device)
        nbytes = ws.numel()
    _lib.check(L.bf8_rmsnorm_bwd_bf16(_ptr(x), _ptr(dy), rows, cols, _ptr(weight), float(eps),
                                      int(bool(zero_centered)), _ptr(dx), _ptr(dw), _ptr(ws),
                                      nbytes, _stream(x.device)), "bf8_rmsnorm_bwd_bf16")
    return dx, dw


def geglu_bwd_delayed_partials_count(M, intermediate):
    return int(_lib.lib().bf8_geglu_bwd_delayed_partials(int(M), int(intermediate)))


def geglu_bwd_delayed(dH, GU, state, length, pos, prev_partials, fmt=E5M2, *, rowwise=True,
                      transpose=False, partials_out, meta_out=None):
    """dGU of the gated GELU quantized at once with a delayed scale (``cast_delayed``
    semantics for state / pos / prev_partials / meta_out); returns the :class:`Fp8Tensor`
    of dGU [M, 2I] (``data`` and/or ``data_t``). ``partials_out`` receives this step's
    amax partials (``geglu_bwd_delayed_partials_count`` entries)."""
    _require_gpu(dH, GU, state)
    dH = dH.contiguous()
    M, I = dH.shape
    GU = _gu_operand("geglu_bwd_delayed", GU, M, I)
    dev = dH.device
    if meta_out is None:
        meta_out = new_meta(dev)
    out = torch.empty((M, 2 * I), dtype=TORCH_FP8[fmt], device=dev) if rowwise else None
    out_t = torch.empty((2 * I, M), dtype=TORCH_FP8[fmt], device=dev) if transpose else None
    n_prev = 0 if prev_partials is None else prev_partials.numel()
    _lib.check(_lib.lib().bf8_geglu_bwd_delayed(
        _ptr(dH), _ptr(GU), M, I, _ptr(state), int(length), int(pos), _ptr(prev_partials),
        n_prev, fmt, _ptr(meta_out), _ptr(out), _ptr(out_t), _ptr(partials_out), _stream(dev)),
        "bf8_geglu_bwd_delayed")
    return Fp8Tensor(out, out_t, meta_out, fmt, M, 2 * I)


def new_delayed_state(length, device):
    """Delayed-scaling state: float32 [length + 4] = history, {amax, scale, scale_inv, pos}."""
    st = torch.zeros(length + 4, dtype=torch.float32, device=device)
    st[length + 1] = 1.0
    st[length + 2] = 1.0
    return st


def delayed_scale_begin(state, length, fmt):
    _lib.check(_lib.lib().bf8_delayed_scale_begin(_ptr(state), length, fmt,
                                                  _stream(state.device)),
               "bf8_delayed_scale_begin")
    return state[length:length + 4]


def delayed_scale_end(state, length, partials):
    _lib.check(_lib.lib().bf8_delayed_scale_end(_ptr(state), length, _ptr(partials),
                                                partials.numel(), _stream(state.device)),
               "bf8_delayed_scale_end")


def cast_amax_partials_count(rows, cols, transpose):
    return int(_lib.lib().bf8_cast_amax_partials(int(rows), int(cols), int(bool(transpose))))


def cast_delayed(x, state, length, pos, prev_partials, fmt=E4M3, *, rowwise=True,
                 transpose=False, partials_out=None, meta_out=None):
    """One-pass delayed-scaling cast (bf8_cast_delayed_bf16).

    ``prev_partials``: the previous step's amax partials (None on the first step), pushed
    into history slot ``pos`` before the scale is derived. ``partials_out``: buffer for
    this step's amax partials of |x| (``cast_amax_partials_count`` entries), or None when
    the producer of x wrote them. Returns an :class:`Fp8Tensor` whose meta is
    ``meta_out`` (a fresh record if None): {history max, scale, scale_inv, 0}.
    """
    _require_gpu(x, state)
    x = _bf16_2d(x)
    rows, cols = x.shape
    dev = x.device
    if meta_out is None:
        meta_out = new_meta(dev)
    out = torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=dev) if rowwise else None
    out_t = torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=dev) if transpose else None
    n_prev = 0 if prev_partials is None else prev_partials.numel()
    _lib.check(_lib.lib().bf8_cast_delayed_bf16(
        _ptr(x), rows, cols, _ptr(state), int(length), int(pos), _ptr(prev_partials), n_prev,
        fmt, _ptr(meta_out), _ptr(out), _ptr(out_t), _ptr(partials_out), _stream(dev)),
        "bf8_cast_delayed_bf16")
    return Fp8Tensor(out, out_t, meta_out, fmt, rows, cols)


def cast_delayed_many(jobs):
    """Several :func:`cast_delayed` calls in one launch (bf8_cast_delayed_many_bf16).

    ``jobs``: up to 8 dicts with the keys x, state, length, pos, prev_partials, fmt,
    rowwise, transpose, partials_out, meta_out (the arguments of :func:`cast_delayed`).
    Returns one :class:`Fp8Tensor` per job; bytes, metas, histories and partials equal
    those of the calls made one by one in order."""
    count = len(jobs)
    if not 1 <= count <= 8:
        raise ValueError(f"cast_delayed_many: {count} tensors (1 to 8 supported)")
    fields = {k: [] for k in ("x", "rows", "cols", "state", "len", "pos", "prev", "n_prev",
                              "fmt", "meta", "out", "out_t", "parts")}
    results = []
    dev = None
    for j in jobs:
        x = _bf16_2d(j["x"])
        _require_gpu(x, j["state"])
        dev = x.device if dev is None else dev
        if x.device != dev:
            raise ValueError("cast_delayed_many: tensors on different devices")
        rows, cols = x.shape
        fmt = j.get("fmt", E4M3)
        meta = j.get("meta_out")
        if meta is None:
            meta = new_meta(dev)
        out = (torch.empty((rows, cols), dtype=TORCH_FP8[fmt], device=dev)
               if j.get("rowwise", True) else None)
        out_t = (torch.empty((cols, rows), dtype=TORCH_FP8[fmt], device=dev)
                 if j.get("transpose", False) else None)
        prev = j.get("prev_partials")
        for key, val in (("x", _ptr(x)), ("rows", rows), ("cols", cols),
                         ("state", _ptr(j["state"])), ("len", int(j["length"])),
                         ("pos", int(j["pos"])), ("prev", _ptr(prev)),
                         ("n_prev", 0 if prev is None else prev.numel()), ("fmt", fmt),
                         ("meta", _ptr(meta)), ("out", _ptr(out)), ("out_t", _ptr(out_t)),
                         ("parts", _ptr(j.get("partials_out")))):
            fields[key].append(val)
        results.append(Fp8Tensor(out, out_t, meta, fmt, rows, cols))
    P = ctypes.c_void_p * count
    I64 = ctypes.c_int64 * count
    I32 = ctypes.c_int * count
    _lib.check(_lib.lib().bf8_cast_delayed_many_bf16(
        count, P(*fields["x"]), I64(*fields["rows"]), I64(*fields["cols"]), P(*fields["state"]),
        I32(*fields["len"]), I32(*fields["pos"]), P(*fields["prev"]), I64(*fields["n_prev"]),
        I32(*fields["fmt"]), P(*fields["meta"]), P(*fields["out"]), P(*fields["out_t"]),
        P(*fields["parts"]), _stream(dev)), "bf8_cast_delayed_many_bf16")
    return results


# ---- NVFP4 (e2m1 in 16-blocks, e4m3 block scales, fp32 tensor scale) -------------------
@dataclass
class NvFp4Tensor:
    """An NVFP4 tensor of x [rows, cols]: ``data`` uint8 [rows, cols / 2] (two e2m1 codes a
    byte) with ``scales`` uint8 e4m3 [rows, cols / 16] (blocks along cols) and/or the
    columnwise copy ``data_t`` [cols, rows / 2] with ``scales_t`` [cols, rows / 16] (blocks
    along rows), and ``meta`` fp32 [4] = {amax, S_enc, S_dec, 0}. ``cache_dequant``: keep
    the exact bf16 dequantization of each copy on the object after its first use (a weight
    cached across microbatches: 2 bytes per element per copy, no dequantization pass per
    GEMM afterwards)."""

    data: Optional[torch.Tensor]
    scales: Optional[torch.Tensor]
    data_t: Optional[torch.Tensor]
    scales_t: Optional[torch.Tensor]
    meta: torch.Tensor
    rows: int
    cols: int
    cache_dequant: bool = False
    _deq: Optional[torch.Tensor] = field(default=None, repr=False)
    _deq_t: Optional[torch.Tensor] = field(default=None, repr=False)


def nvfp4_dequant(q, *, transpose=False):
    """bf16 = e2m1(code) * s of ``q``'s rowwise copy (or with ``transpose`` its columnwise
    copy), exact and without S_dec; kept on ``q`` when ``q.cache_dequant`` is set, or
    written by the quantizer itself (``quantize_nvfp4(dequant_rows=True)``)."""
    attr = "_deq_t" if transpose else "_deq"
    if getattr(q, attr) is None and not q.cache_dequant:
        return dequant_nvfp4(q.data_t, q.scales_t) if transpose else dequant_nvfp4(q.data, q.scales)
    d = getattr(q, attr)
    if d is None:
        d = dequant_nvfp4(q.data_t, q.scales_t) if transpose else dequant_nvfp4(q.data, q.scales)
        setattr(q, attr, d)
    return d


def quantize_nvfp4(x, *, rowwise=True, colwise=False, partials=None, dequant_rows=False):
    """NVFP4 quantization of a bf16 tensor (flattened to 2-D): an amax pass and the block
    quantization (rowwise needs cols % 16 == 0, columnwise rows % 16 == 0). ``partials``:
    the amax partials of |x| its producer wrote (int32 / uint32 fp32 bits: ``geglu_bwd``'s,
    the fused RMSNorm's, the gated-GELU GEMM's); the amax pass is then skipped
    (bf8_quantize_nvfp4_partials_bf16, the same outputs bit for bit). ``dequant_rows``: the
    rowwise copy is kept only as its exact bf16 dequantization (``nvfp4_dequant(q)``; data
    and scales None), for a tensor whose rowwise copy only feeds the next GEMM
    (bf8_quantize_nvfp4_dequant_bf16)."""
    _require_gpu(x, partials)
    x = _bf16_2d(x)
    rows, cols = x.shape
    dev = x.device
    meta = new_meta(dev)
    u8 = torch.uint8
    codes = rowwise and not dequant_rows
    out = torch.empty((rows, cols // 2), dtype=u8, device=dev) if codes else None
    sc = torch.empty((rows, cols // 16), dtype=u8, device=dev) if codes else None
    out_t = torch.empty((cols, rows // 2), dtype=u8, device=dev) if colwise else None
    sc_t = torch.empty((cols, rows // 16), dtype=u8, device=dev) if colwise else None
    L = _lib.lib()
    if partials is not None:
        if partials.dtype != torch.int32 or partials.dim() != 1 or partials.numel() < 1:
            raise ValueError("quantize_nvfp4: partials must be a non-empty 1-D int32 tensor")
    if dequant_rows and rowwise:
        deq = torch.empty((rows, cols), dtype=torch.bfloat16, device=dev)
        if partials is not None:
            parts, n_parts = partials.contiguous(), partials.numel()
        else:
            parts, n_parts = partials_buffer(max(1, int(L.bf8_amax_partials(rows * cols))), dev), 0
        _lib.check(L.bf8_quantize_nvfp4_dequant_bf16(
            _ptr(x), rows, cols, _ptr(parts), n_parts, _ptr(deq), _ptr(out_t), _ptr(sc_t),
            _ptr(meta), _stream(dev)), "bf8_quantize_nvfp4_dequant_bf16")
        return NvFp4Tensor(None, None, out_t, sc_t, meta, rows, cols, _deq=deq)
    if partials is not None:
        _lib.check(L.bf8_quantize_nvfp4_partials_bf16(
            _ptr(x), rows, cols, _ptr(partials.contiguous()), partials.numel(), _ptr(out),
            _ptr(sc), _ptr(out_t), _ptr(sc_t), _ptr(meta), _stream(dev)),
            "bf8_quantize_nvfp4_partials_bf16")
        return NvFp4Tensor(out, sc, out_t, sc_t, meta, rows, cols)
    parts = partials_buffer(max(1, int(L.bf8_amax_partials(rows * cols))), dev)
    _lib.check(L.bf8_quantize_nvfp4_bf16(_ptr(x), rows, cols, _ptr(out), _ptr(sc), _ptr(out_t),
                                         _ptr(sc_t), _ptr(meta), _ptr(parts), _stream(dev)),
               "bf8_quantize_nvfp4_bf16")
    return NvFp4Tensor(out, sc, out_t, sc_t, meta, rows, cols)


def dequant_nvfp4(data, scales):
    """bf16 [rows, 2 * data cols] = e2m1(code) * s per element (exact, without S_dec)."""
    _require_gpu(data, scales)
    rows, half = data.shape
    out = torch.empty((rows, 2 * half), dtype=torch.bfloat16, device=data.device)
    _lib.check(_lib.lib().bf8_dequant_nvfp4(_ptr(data.contiguous()), _ptr(scales.contiguous()),
                                            rows, 2 * half, _ptr(out), _stream(data.device)),
               "bf8_dequant_nvfp4")
    return out


def gemm_bf16(a, b, a_sinv, b_sinv, *, out_dtype=torch.bfloat16):
    """``C = (a @ b.T accumulated in fp32) * a_sinv * b_sinv`` on bf16 a [M, K], b [N, K]
    (row-major) with the bf16 MFMA; a_sinv, b_sinv: device fp32 scalars."""
    _require_gpu(a, b, a_sinv, b_sinv)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError("gemm_bf16: a and b must be bfloat16")
    if a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("gemm_bf16: a and b must be row-major")
    M, K = a.shape
    N, Kb = b.shape
    if K != Kb:
        raise ValueError(f"gemm_bf16: inner dims differ ({K} vs {Kb})")
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    L = _lib.lib()
    ws_bytes = int(L.bf8_gemm_bf16_workspace(M, N, K))
    ws = gemm_workspace(ws_bytes, a.device) if ws_bytes else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.check(L.bf8_gemm_bf16(_ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K,
                               _ptr(a_sinv), _ptr(b_sinv), _ptr(out),
                               OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32,
                               out.stride(0), _ptr(ws), ws_bytes, _stream(a.device)),
               "bf8_gemm_bf16")
    return out


def gemm_geglu_bf16(a, b, a_sinv, b_sinv, intermediate, *, keep_gu=False, partials=None):
    """:func:`gemm_geglu` on bf16 operands a [M, K], b [2I, K] (gate rows then up rows) with
    device fp32 scalars a_sinv, b_sinv applied to the sums (bf8_gemm_geglu_bf16). Returns
    ``(H bf16 [M, I], GU bf16 [M, 2I] or None, h_partials int32)``."""
    _require_gpu(a, b, a_sinv, b_sinv)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError("gemm_geglu_bf16: a and b must be bfloat16")
    if a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("gemm_geglu_bf16: a and b must be row-major")
    M, K = a.shape
    I = int(intermediate)
    if tuple(b.shape) != (2 * I, K):
        raise ValueError(f"gemm_geglu_bf16: weight must be [{2 * I}, {K}], got {tuple(b.shape)}")
    H = torch.empty((M, I), dtype=torch.bfloat16, device=a.device)
    GU = torch.empty((M, 2 * I), dtype=torch.bfloat16, device=a.device) if keep_gu else None
    count = _geglu_partials_cached(M, I, _tile_override())
    if partials is None:
        parts = torch.empty(count, dtype=torch.int32, device=a.device)
    else:
        if partials.numel() < count or partials.dtype != torch.int32:
            raise ValueError(f"gemm_geglu_bf16: partials must be int32 with >= {count} entries")
        parts = partials[:count]
    _lib.check(_lib.lib().bf8_gemm_geglu_bf16(
        _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, I, K, _ptr(a_sinv), _ptr(b_sinv),
        _ptr(H), H.stride(0), _ptr(GU), _ptr(parts), _stream(a.device)), "bf8_gemm_geglu_bf16")
    return H, GU, parts


def gemm_geglu_nvfp4(a_data, a_scales, a_meta, b_data, b_scales, b_meta, intermediate, *,
                     keep_gu=False, a_deq=None, b_deq=None):
    """The NVFP4 gate/up projection with the gated GELU in its epilogue: both operands
    dequantized exactly to bf16, then :func:`gemm_geglu_bf16` with the two S_dec.
    ``a_deq`` / ``b_deq``: an operand's bf16 dequantization when the caller holds it."""
    a = a_deq if a_deq is not None else dequant_nvfp4(a_data, a_scales)
    b = b_deq if b_deq is not None else dequant_nvfp4(b_data, b_scales)
    return gemm_geglu_bf16(a, b, a_meta[2:3], b_meta[2:3], intermediate, keep_gu=keep_gu)


def gemm_nvfp4(a_data, a_scales, a_meta, b_data, b_scales, b_meta, *, out_dtype=torch.bfloat16,
               a_deq=None, b_deq=None):
    """``C = (A^ @ B^.T) * S_dec(a) * S_dec(b)`` for NVFP4 operands A [M, K], B [N, K]
    (blocks along K): both dequantized exactly to bf16, then the bf16 MFMA GEMM.
    ``a_deq`` / ``b_deq``: an operand's bf16 dequantization when the caller holds it."""
    a = a_deq if a_deq is not None else dequant_nvfp4(a_data, a_scales)
    b = b_deq if b_deq is not None else dequant_nvfp4(b_data, b_scales)
    return gemm_bf16(a, b, a_meta[2:3], b_meta[2:3], out_dtype=out_dtype)
