// Host-only argument checks and launch planning of the attention library.
// Plain C++ (no HIP types): compiled into libtrinix_attn.so and, on its own,
// into the CPU sanitizer test (address + undefined-behaviour sanitizers).
#pragma once
#include <stdint.h>

#include "trinix_attn.h"

namespace trinix {

// Tile shape of one 16-bit forward kernel instantiation.
struct Cfg16 {
  int nw;   // wavefronts per workgroup (32 query rows per key split)
  int occ;  // target wavefronts per SIMD (register budget 512 / occ)
  int bn;   // keys per K/V tile
  int ks;   // key split: wavefronts sharing one 32-row group (rows per workgroup = 32 * nw / ks)
};

// Largest 16-bit K/V key-row stride (elements) the forward's 32-bit in-tile
// offsets address: 128 rows * 2 B * 2^22 = 2^30 bytes.
constexpr int64_t kMaxKvRowStride = 1ll << 22;

// Argument checks of trinix_attn_fwd (also the split-KV entry points) and of
// trinix_attn_bwd: TRINIX_OK or the status code to return, no launch.
int validate_fwd_args(const trinix_attn_fwd_args* a);
int validate_bwd_args(const trinix_attn_bwd_args* a);

// Tile configuration of the 16-bit forward for a problem: `banded` when
// causal or windowed, `plain` without a mask or dropout.
Cfg16 pick_cfg16(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool plain);
// Whether the 16-bit dQ backward runs 256-row workgroups with 128-key tiles.
bool pick_dq_wide(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool masked);

// Split-KV decode plan.
constexpr int kDecodeMaxSq = 16;
constexpr int kDecodeTargetWgs = 1024;  // 4 workgroups of 4 wavefronts per CU
constexpr int kDecodeMinChunk = 128;
struct SplitPlan {
  int n_splits, chunk, klo, khi, M, RG;
  int64_t ws_bytes;
};
// false if the split-KV kernel does not apply (then trinix_attn_fwd is the path).
bool make_split_plan(const trinix_attn_fwd_args* a, SplitPlan* pl);

}  // namespace trinix
