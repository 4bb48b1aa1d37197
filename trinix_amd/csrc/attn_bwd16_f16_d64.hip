// Backward kernels for f16, head_dim 64 (one translation unit per
// instantiation keeps compile times parallel).
#include "attn_bwd16.h"

namespace trinix {
TRINIX_ATTN_BWD16_LAUNCHER(launch_bwd16_f16_d64, F16, 64)
}  // namespace trinix
