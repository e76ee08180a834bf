// The megakernel's row-wise instantiations for H = 256, I = 512 with fp8 weights whose self-attention tasks
// run two query tiles each (Shape::PAIRS: launches whose one-tile attention tasks outnumber the workgroups),
// in a translation unit of their own. (The fp16-weight row-wise kernels run a second query tile of a
// sample-head with its keys and values still in LDS instead.)
// (the second: AdaRMS operands scaled, for launches with an operand shift)
#include "mkx_kernel.h"

namespace mkx {
template __global__ void mkx_megakernel<256, 512, true, true, false, true>(Params);
template __global__ void mkx_megakernel<256, 512, true, true, true, true>(Params);
}  // namespace mkx
