// f16 attention-forward kernels for head_dim 64 (one translation unit per
// (dtype, head_dim) so the template variants compile in parallel).
#include "attn_kernel16.h"

namespace trinix {
TRINIX_ATTN16_LAUNCHER(launch_attn16_f16_d64, F16, 64)
}  // namespace trinix
