// The DeepSeek-V2 (multi-head latent attention) persistent kernels (their own translation unit).
#include "mk_mla.h"

namespace mk {
MK_DS_SHAPES(MK_DS_KERNEL)
}  // namespace mk
