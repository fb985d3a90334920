// The single-sequence persistent kernels with fp8 weights (one translation unit per list, compiled in parallel).
#include "mk_device.h"

namespace mk {
MK_FUSED_SHAPES_FP8(MK_FUSED_KERNEL)
}  // namespace mk
