// The batched persistent kernels with bf16 weights (one translation unit per list, compiled in parallel).
#include "mk_batch.h"

namespace mk {
MK_BATCH_SHAPES_BF16(MK_BATCH_KERNEL)
}  // namespace mk
