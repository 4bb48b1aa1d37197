// Device-side dropout generator state for calls captured in HIP graphs.
//
// The attention kernels draw their keep masks from Philox4x32-10 with a
// seed and an offset (common.h keep_field).  Taken from the host, those two
// values would be frozen into a captured graph and every replay would drop
// the same elements.  Instead the caller keeps a generator {seed, offset} in
// device memory and, for each call, this kernel copies it to the call's own
// {seed, offset} and advances the generator's offset; the attention kernels
// of that call (forward and backward) read the call's copy
// (trinix_attn_fwd_args.dropout_state).  Captured, the copy and the advance
// run again on every replay, so each replay draws a new offset.  No
// counterpart in the reference: its eager F.dropout
// (trinix/layers/attention/base.py:395) takes the same from torch's
// graph-safe generator state.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "index_map.h"
#include "trinix_attn.h"

namespace {

// One lane reads both words and writes three: plain vector loads and stores.
__global__ __launch_bounds__(64) void dropout_state_advance_kernel(uint64_t* gen, uint64_t* call, uint64_t inc) {
  if (threadIdx.x == 0) {
    const uint64_t seed = gen[0], off = gen[1];
    call[0] = seed;
    call[1] = off;
    gen[1] = off + inc;
  }
}

}  // namespace

extern "C" int trinix_dropout_state_advance(uint64_t* generator, uint64_t* call_state, uint64_t increment,
                                            void* stream) {
  if (!generator || !call_state) return TRINIX_ERR_NULL_POINTER;
  if (((uintptr_t)generator & 7) || ((uintptr_t)call_state & 7)) return TRINIX_ERR_BAD_ARGUMENT;
  const hipError_t err = trinix::launch_kernel(&dropout_state_advance_kernel, dim3(1), dim3(64), 0,
                                               (hipStream_t)stream, generator, call_state, increment);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

// Size of the keep map a dropout forward writes for its backward
// (trinix_attn_fwd_args.dropout_keep_map; layout in index_map.h).
extern "C" int trinix_dropout_keep_map_bytes(int64_t batch, int64_t nheads_q, int64_t seqlen_q, int64_t seqlen_k,
                                             int64_t* bytes) {
  if (!bytes) return TRINIX_ERR_NULL_POINTER;
  if (batch <= 0 || nheads_q <= 0 || seqlen_q <= 0 || seqlen_k <= 0 || seqlen_q >= (1ll << 30) ||
      seqlen_k >= (1ll << 30) || batch >= (1 << 20) || nheads_q >= (1 << 20))
    return TRINIX_ERR_BAD_SHAPE;
  const int64_t blocks = trinix::keep_map_nbi(seqlen_q) * trinix::keep_map_nbj(seqlen_k);
  if (blocks > (INT64_MAX / 128) / (batch * nheads_q)) return TRINIX_ERR_BAD_SHAPE;
  *bytes = 128 * batch * nheads_q * blocks;
  return TRINIX_OK;
}
