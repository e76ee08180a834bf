// The megakernel's instantiations for H = 768, I = 3072 (bf16 and fp8 weights) with GEMM stages in passes,
// in a translation unit of their own so that the build can give them their own code-generation options.
// (the second pair: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<768, 3072, false, false>(Params);
template __global__ void mkx_megakernel<768, 3072, true, false>(Params);
template __global__ void mkx_megakernel<768, 3072, false, false, true>(Params);
template __global__ void mkx_megakernel<768, 3072, true, false, true>(Params);
}  // namespace mkx
