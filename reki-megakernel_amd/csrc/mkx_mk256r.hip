// The megakernel's instantiations for H = 256, I = 512 (bf16 and fp8 weights) with row-wise GEMM stages (the
// form for launches whose GEMM tasks cover more row tiles than one pass holds), in a translation unit of their own.
// (the second pair: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<256, 512, false, true>(Params);
template __global__ void mkx_megakernel<256, 512, true, true>(Params);
template __global__ void mkx_megakernel<256, 512, false, true, true>(Params);
template __global__ void mkx_megakernel<256, 512, true, true, true>(Params);
}  // namespace mkx
