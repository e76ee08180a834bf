// The megakernel's instantiations for H = 768, I = 3072 (bf16 and fp8 weights) with row-wise GEMM stages (the
// form for launches whose GEMM tasks cover more row tiles than one pass holds), in a translation unit of their own.
// (the second pair: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<768, 3072, false, true>(Params);
template __global__ void mkx_megakernel<768, 3072, true, true>(Params);
template __global__ void mkx_megakernel<768, 3072, false, true, true>(Params);
template __global__ void mkx_megakernel<768, 3072, true, true, true>(Params);
}  // namespace mkx
