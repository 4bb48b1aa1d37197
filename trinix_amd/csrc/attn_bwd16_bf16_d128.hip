// Backward kernels for bf16, head_dim 128 (one translation unit per
// instantiation keeps compile times parallel).
#include "attn_bwd16.h"

namespace trinix {
TRINIX_ATTN_BWD16_LAUNCHER(launch_bwd16_bf16_d128, BF16, 128)
}  // namespace trinix
