// FP8 GEMM kernels for 256 x 128 block tiles (one translation unit per tile shape).
#include "gemm_kernel_impl.hpp"

namespace bf8 {
template int launch_gemm_tile<Tile256x128>(const GemmParams&, int, int, int, int, hipStream_t,
                                              bool);
}  // namespace bf8
