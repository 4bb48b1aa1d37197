// bf16 attention-forward kernels for head_dim 128 (one translation unit per
// (dtype, head_dim) so the template variants compile in parallel).
#include "attn_kernel16.h"

namespace trinix {
TRINIX_ATTN16_LAUNCHER(launch_attn16_bf16_d128, BF16, 128)
}  // namespace trinix
