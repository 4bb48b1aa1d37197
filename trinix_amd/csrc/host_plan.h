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
  int ks;   // key split: wavefronts sharing one 32-row group (rows per workgroup = 32 * nw / ks);
            // 0: per work item, from plan_split_rows
};

// Work items of the per-item key split, at most kMaxRowItems per (batch, q-head).
constexpr int kMaxRowItems = 128;

// Largest 16-bit K/V key-row stride (elements) the forward's 32-bit in-tile
// offsets address: 128 rows * 2 B * 2^22 = 2^30 bytes.
constexpr int64_t kMaxKvRowStride = 1ll << 22;

// Argument checks of trinix_attn_fwd (also the split-KV entry points) and of
// trinix_attn_bwd: TRINIX_OK or the status code to return, no launch.
int validate_fwd_args(const trinix_attn_fwd_args* a);
int validate_bwd_args(const trinix_attn_bwd_args* a);

// Tile configuration of the 16-bit forward for a problem: `banded` when
// causal or windowed, `plain` without a mask or dropout, `split_ok` when the
// per-item key split applies (causal, no window, no mask, dropout or fused
// q norm).
Cfg16 pick_cfg16(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool plain,
                 bool split_ok = false);
// Work items of the per-item key split for a causal problem of `heads`
// (batch * q-heads) row sequences, row blocks of `rows` (= 32 * nw) rows and
// `bn`-key tiles: the longest row blocks (tile count above half the longest)
// run as two items (split, half 0 / 1) while the grid keeps one round of
// resident workgroups, the rest as one; items ordered by chain length (tiles
// per wavefront), longest first.  Writes `items` and returns their count, or
// 0 if more than `max`.
int plan_split_rows(int64_t sq, int64_t sk, int64_t heads, int rows, int bn, uint8_t* items, int max);
// Whether the 16-bit dQ backward runs 256-row workgroups with 128-key tiles.
bool pick_dq_wide(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool masked);

// Window bounds as the kernels take them: every |j - i| < 2^30 (seqlen_q,
// seqlen_k < 2^30), so a bound beyond +-2^30 selects the same keys as
// +-2^30, and the kernels' index arithmetic on it stays in 32 bits.
int64_t clamp_window(int64_t w);

// Launch plan of trinix_attn_fwd (the 16-bit kernels' tile shape, or the
// fp32 kernel's): row blocks per (batch, q-head), grid size and the per-item
// key split table.
constexpr int kWavesF32 = 4;
struct FwdPlan {
  Cfg16 cfg;           // 16-bit kernels; cfg.ks = 0 only with n_items > 0
  int num_mblk;        // work items per (batch, q-head)
  int64_t total_work;  // workgroups
  int n_items;         // entries of row_items (cfg.ks == 0)
  uint8_t row_items[kMaxRowItems];
};
// TRINIX_OK, or TRINIX_ERR_BAD_SHAPE when the grid exceeds 2^31 - 1
// workgroups.  For validated arguments.
int plan_fwd(const trinix_attn_fwd_args* a, FwdPlan* pl);

// Launch plan of trinix_attn_bwd's 16-bit kernels: 128-key blocks (dK/dV)
// and 128- or 256-row blocks (dQ).
struct BwdPlan {
  int num_kblk, num_mblk;
  bool dq_wide;
};
int plan_bwd(const trinix_attn_bwd_args* a, BwdPlan* pl);

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
