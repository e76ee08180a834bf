// The megakernel's instantiations for H = 256, I = 512 (bf16 and fp8 weights), in a translation unit of their
// own so that the build can give them their own code-generation options (mkx/_build.py).
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<256, 512, false>(Params);
template __global__ void mkx_megakernel<256, 512, true>(Params);
}  // namespace mkx
