// Kernels of the quantised matrix path for one weight type.
#include "gemv_impl.h"

namespace llmhip {
LLMHIP_INSTANTIATE(LLMHIP_Q8_0)
}  // namespace llmhip
