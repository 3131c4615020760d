// FP8 GEMM kernels for 128 x 64 block tiles with two K groups (one translation unit per tile shape).
#include "gemm_kernel_impl.hpp"

namespace bf8 {
template int launch_gemm_tile<Tile128x64k2>(const GemmParams&, int, int, int, int, hipStream_t,
                                              bool);
}  // namespace bf8
