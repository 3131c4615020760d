// FP8 GEMM kernels for 256 x 256 block tiles run by eight waves with a third B slot (linear
// epilogues), one translation unit per tile shape.
#include "gemm_kernel_impl.hpp"

namespace bf8 {
template int launch_gemm_tile<Tile256x256w8x>(const GemmParams&, int, int, int, int,
                                                 hipStream_t, bool);
}  // namespace bf8
