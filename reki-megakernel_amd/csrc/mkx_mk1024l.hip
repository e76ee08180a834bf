// The megakernel's instantiations for H = 1024, I = 4096 (bf16 and fp8 weights) with GEMM stages in passes for
// sources longer than the three-chunk cross-attention ring (Shape::LONG: the chunks beyond the third streamed
// into registers), in a translation unit of their own.
// (the second pair: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<1024, 4096, false, false, false, false, true>(Params);
template __global__ void mkx_megakernel<1024, 4096, true, false, false, false, true>(Params);
template __global__ void mkx_megakernel<1024, 4096, false, false, true, false, true>(Params);
template __global__ void mkx_megakernel<1024, 4096, true, false, true, false, true>(Params);
}  // namespace mkx
