// The batched persistent kernels with fp8 weights (one translation unit per list, compiled in parallel).
#define MK_LANE_OPAQUE 1   // lane_id() kept local to each phase (mk_device.h)
#include "mk_batch.h"

namespace mk {
MK_BATCH_SHAPES_FP8(MK_BATCH_KERNEL)
}  // namespace mk
