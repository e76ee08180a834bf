// The megakernel's instantiations for H = 256, I = 512 (bf16 and fp8 weights) with GEMM stages in passes for
// sources longer than the three-chunk cross-attention ring (Shape::LONG: the chunks beyond the third streamed
// into registers), in a translation unit of their own.
// (the second pair: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<256, 512, false, false, false, false, true>(Params);
template __global__ void mkx_megakernel<256, 512, true, false, false, false, true>(Params);
template __global__ void mkx_megakernel<256, 512, false, false, true, false, true>(Params);
template __global__ void mkx_megakernel<256, 512, true, false, true, false, true>(Params);
}  // namespace mkx
