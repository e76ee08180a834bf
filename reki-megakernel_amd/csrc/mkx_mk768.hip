// The megakernel's instantiations for H = 768, I = 3072 (bf16 and fp8 weights), in a translation unit of their
// own so that the build can give them their own code-generation options (mkx/_build.py).
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<768, 3072, false>(Params);
template __global__ void mkx_megakernel<768, 3072, true>(Params);
}  // namespace mkx
