// The single-sequence persistent kernels with bf16 weights (one translation unit per list, compiled in parallel).
#include "mk_device.h"

namespace mk {
MK_FUSED_SHAPES_BF16(MK_FUSED_KERNEL)
}  // namespace mk
