// Host-only argument checks and launch planning (declared in host_plan.h):
// plain C++, no HIP.  Every function only reads its arguments and returns a
// status, a plan or a tile shape.
#include "host_plan.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace trinix {
namespace {

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

int check_tensor(const void* ptr, const int64_t st[4], int esize) {
  if (!ptr) return TRINIX_ERR_NULL_POINTER;
  if (st[3] != 1) return TRINIX_ERR_BAD_STRIDE;
  if (esize == 2) {
    // 16-byte vector loads of 8 consecutive head_dim elements per row
    if (!aligned16(ptr)) return TRINIX_ERR_BAD_STRIDE;
    for (int a = 0; a < 3; ++a)
      if (st[a] % 8 != 0) return TRINIX_ERR_BAD_STRIDE;
  } else if (((uintptr_t)ptr & 3) != 0) {
    return TRINIX_ERR_BAD_STRIDE;
  }
  return TRINIX_OK;
}

// fp32 BSHD tensor (generic kernels, element loads): head_dim stride 1.
int check32(const void* ptr, const int64_t st[4]) {
  if (!ptr) return TRINIX_ERR_NULL_POINTER;
  if (st[3] != 1 || ((uintptr_t)ptr & 3) != 0) return TRINIX_ERR_BAD_STRIDE;
  return TRINIX_OK;
}

// 16-bit BSHD tensor: head_dim stride 1, 16-byte aligned rows, and a row
// stride the 32-bit in-tile offsets can address (tiles of up to 128 rows).
int check16(const void* ptr, const int64_t st[4]) {
  if (!ptr) return TRINIX_ERR_NULL_POINTER;
  if (st[3] != 1 || !aligned16(ptr)) return TRINIX_ERR_BAD_STRIDE;
  for (int a = 0; a < 3; ++a)
    if (st[a] % 8 != 0) return TRINIX_ERR_BAD_STRIDE;
  if (st[1] < 0 || st[1] >= kMaxKvRowStride) return TRINIX_ERR_BAD_STRIDE;
  return TRINIX_OK;
}

}  // namespace

// Tile configuration of the 16-bit kernel: 4 wavefronts x 32 query rows,
// 64-key tiles, 2 wavefronts per SIMD (1 for head_dim 256).  A small grid at
// head_dim 64 -- no more 128-row workgroups than CUs -- splits each 32-row
// group's keys between two wavefronts (ks = 2, 64 rows per workgroup): twice
// the workgroups, half the longest chain of tiles, at twice the K/V copies
// per flop.  Measured at head_dim 64, bf16: 128 workgroups at S = 4096..16384
// +50..62%, 64 workgroups at S = 1024 +2%, 384 workgroups (S = 1024) -3%.
// Head_dim 128 without a mask or dropout takes 8 wavefronts x 32 rows and
// 128-key tiles (one workgroup of 256 rows per CU, 128 KiB of LDS): half the
// barriers and tile bookkeeping per flop, once the grid holds enough 256-row
// workgroups -- 512 with causal / window bands (whose rows differ in length),
// 256 without.  Measured at bf16, graph-timed kernel: causal 512 workgroups
// +8%, 1024 +1.5..3% (C3), 2048 +2.7%, C4 +2..2.4%; full rows 256 workgroups
// +8%; below those counts it loses (causal 256 workgroups -9%, 128 -20%).
// TRINIX_ATTN_CFG="nw,occ,bn[,ks]" overrides the choice (tuning only; a
// configuration that is not built is rejected with TRINIX_ERR_BAD_ARGUMENT).
constexpr int64_t kSmallGrid = 256;  // CUs of an MI355X
// Enough 256-row workgroups for the wide shape: 512 with a causal / window
// band, 256 without (batch * hq * row blocks, without overflow: each factor
// < 2^31 here, and the product is formed only below 2^9 * 2^22).
static bool wide_grid(int64_t batch, int64_t hq, int64_t sq, bool banded) {
  const int64_t need = banded ? 2 * kSmallGrid : kSmallGrid;
  return batch * hq >= need || batch * hq * ((sq + 255) / 256) >= need;
}
Cfg16 pick_cfg16(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool plain,
                 bool split_ok) {
  Cfg16 c{4, head_dim == 256 ? 1 : 2, 64, 1};
  // batch * hq * row blocks, without overflow (each factor < 2^31 here)
  if (head_dim == 64 && batch * hq <= kSmallGrid && batch * hq * ((sq + 127) / 128) <= kSmallGrid) c.ks = 2;
  else if (head_dim == 64 && split_ok && batch * hq <= 2 * kSmallGrid &&
           batch * hq * ((sq + 127) / 128) <= 2 * kSmallGrid)
    c.ks = 0;
  if (head_dim == 128 && plain && wide_grid(batch, hq, sq, banded)) c = Cfg16{8, 2, 128, 1};
  if (const char* env = getenv("TRINIX_ATTN_CFG")) {
    int nw = 0, occ = 0, bn = 0, ks = 1;
    // ks 1 or 2: wavefronts per 32-row group; 0: the per-item split
    if (sscanf(env, "%d,%d,%d,%d", &nw, &occ, &bn, &ks) >= 3 && nw > 0 && ks >= 0 && ks <= 2 &&
        (ks == 0 || nw % ks == 0))
      c = Cfg16{nw, occ, bn, ks};
  }
  return c;
}

// Per-item key split for causal grids of up to two rounds of 128-row
// workgroups at head_dim 64 (C2: 384): the longest row blocks' chains of
// tiles set the kernel time there, so the longest blocks run as two 64-row
// items with two wavefronts per 32-row group (half the chain each), the
// others as one item.  Blocks are split longest first while the grid stays
// within one round of resident workgroups (two per CU: 2 * 256 for all
// (batch, q-head) pairs), since a workgroup of a second round pays its
// start-up and epilogue again after the first round.
int plan_split_rows(int64_t sq, int64_t sk, int64_t heads, int rows, int bn, uint8_t* items, int max) {
  const int64_t nb = (sq + rows - 1) / rows;
  if (nb <= 0 || nb > 63 || heads <= 0) return 0;  // row block in 6 bits
  auto tiles = [&](int64_t rb) {
    const int64_t keys = std::min(sk, (rb + 1) * rows);  // causal: row i sees keys j <= i
    return (keys + bn - 1) / bn;
  };
  const int64_t max_t = tiles(nb - 1);
  const int64_t budget = std::min<int64_t>(max, std::max<int64_t>(nb, 2 * kSmallGrid / heads));
  struct Item { int64_t chain; int rb, split, half; };
  Item list[2 * 64];
  int n = 0;
  int64_t count = nb;  // items so far: one per block, one more per split block
  for (int64_t rb = nb - 1; rb >= 0; --rb) {
    const int64_t t = tiles(rb);
    if (2 * t > max_t + 1 && count + 1 <= budget) {
      ++count;
      for (int h = 0; h < 2; ++h) list[n++] = Item{(t + 1) / 2, (int)rb, 1, h};
    } else {
      list[n++] = Item{t, (int)rb, 0, 0};
    }
  }
  if (n > max) return 0;
  std::stable_sort(list, list + n, [](const Item& a, const Item& b) { return a.chain > b.chain; });
  for (int k = 0; k < n; ++k) items[k] = (uint8_t)((list[k].rb << 2) | (list[k].split << 1) | list[k].half);
  return n;
}

// The dQ backward kernel takes the same wide shape (8 wavefronts x 32 rows,
// 128-key tiles) under the same rule, at head_dim 128 without a mask
// (dropout included).  Measured at C3 (bf16): forward + backward 2.297 ->
// 2.284 ms, dQ ~2% faster, gradients bit-identical.
// TRINIX_BWD_DQ_WIDE=0 / 1 overrides the grid rule (tuning and tests; the
// wide shape is still only taken where it is built).
bool pick_dq_wide(int64_t head_dim, int64_t batch, int64_t hq, int64_t sq, bool banded, bool masked) {
  if (head_dim != 128 || masked) return false;
  if (const char* env = getenv("TRINIX_BWD_DQ_WIDE")) {
    if (env[0] == '0') return false;
    if (env[0] == '1') return true;
  }
  return wide_grid(batch, hq, sq, banded);
}

// The kernels address a mask row with 32-bit element offsets (load_mask4):
// a key stride in [0, 2^31 / Sk).  A mask broadcast over keys has stride 0.
static bool mask_key_stride_ok(int64_t sj, int64_t sk) {
  return sj >= 0 && (sk <= 1 || sj <= ((1ll << 31) - 1) / (sk - 1));  // (sk - 1) * sj < 2^31, no overflow
}

// Every mask stride is a non-negative element count (0 = broadcast); the
// batch, head and row parts of an address are formed in 64 bits.  The dK/dV
// kernel reads the 32 rows of a query sub-tile at 32-bit offsets r * si from
// the sub-tile's first row (r < 32, and r <= Sq - 1).
static bool mask_strides_ok(const int64_t st[4], int64_t sq, int64_t sk) {
  if (st[0] < 0 || st[1] < 0 || st[2] < 0) return false;
  const int64_t rows = sq - 1 < 31 ? sq - 1 : 31;
  if (rows > 0 && st[2] > ((1ll << 31) - 1) / rows) return false;
  return mask_key_stride_ok(st[3], sk);
}

// A dropout keep map goes with dropout, the 16-bit kernels at head_dim 64
// or 128 (the MFMA backward that reads it), and a 16-byte aligned buffer.
static bool keep_map_ok(const void* map, float dropout_p, int32_t dtype, int64_t head_dim) {
  return dropout_p > 0.f && (dtype == TRINIX_BF16 || dtype == TRINIX_F16) && (head_dim == 64 || head_dim == 128) &&
         aligned16(map);
}

int validate_fwd_args(const trinix_attn_fwd_args* a) {
  if (!a) return TRINIX_ERR_NULL_POINTER;
  const int esize = a->dtype == TRINIX_F32 ? 4 : 2;
  if (a->dtype != TRINIX_F32 && a->dtype != TRINIX_F16 && a->dtype != TRINIX_BF16) return TRINIX_ERR_BAD_DTYPE;
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return TRINIX_ERR_BAD_HEAD_DIM;
  if (a->batch <= 0 || a->seqlen_q <= 0 || a->seqlen_k <= 0 || a->nheads_q <= 0 || a->nheads_kv <= 0)
    return TRINIX_ERR_BAD_SHAPE;
  if (a->nheads_q % a->nheads_kv != 0) return TRINIX_ERR_BAD_SHAPE;
  if (a->seqlen_q >= (1ll << 30) || a->seqlen_k >= (1ll << 30) || a->batch >= (1 << 20) || a->nheads_q >= (1 << 20))
    return TRINIX_ERR_BAD_SHAPE;
  int rc;
  if ((rc = check_tensor(a->q, a->q_stride, esize))) return rc;
  if ((rc = check_tensor(a->k, a->k_stride, esize))) return rc;
  if ((rc = check_tensor(a->v, a->v_stride, esize))) return rc;
  // 16-bit kernels address a K/V tile (up to 128 key rows) as one base plus
  // per-lane 32-bit byte offsets: the key-row stride must be in [0, 2^22).
  if (esize == 2 && (a->k_stride[1] < 0 || a->k_stride[1] >= kMaxKvRowStride || a->v_stride[1] < 0 ||
                     a->v_stride[1] >= kMaxKvRowStride))
    return TRINIX_ERR_BAD_STRIDE;
  if ((rc = check_tensor(a->out, a->out_stride, esize))) return rc;
  if (a->mask && a->mask_dtype != TRINIX_F32 && a->mask_dtype != TRINIX_F16 && a->mask_dtype != TRINIX_BF16 &&
      a->mask_dtype != TRINIX_U8)
    return TRINIX_ERR_BAD_DTYPE;
  if (a->mask_blockmap && !a->mask) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->mask && !mask_strides_ok(a->mask_stride, a->seqlen_q, a->seqlen_k)) return TRINIX_ERR_BAD_STRIDE;
  if (!(a->dropout_p >= 0.f && a->dropout_p < 1.f)) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->dropout_state && ((uintptr_t)a->dropout_state & 7)) return TRINIX_ERR_BAD_ARGUMENT;
  if ((a->rope_cos == nullptr) != (a->rope_sin == nullptr)) return TRINIX_ERR_NULL_POINTER;
  if (a->rope_cos && esize == 2 &&
      (!aligned16(a->rope_cos) || !aligned16(a->rope_sin) || a->rope_stride % 8 != 0))
    return TRINIX_ERR_BAD_STRIDE;
  if (a->q_norm_out && (!a->q_norm_weight || !aligned16(a->q_norm_out))) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->dropout_keep_map && !keep_map_ok(a->dropout_keep_map, a->dropout_p, a->dtype, a->head_dim))
    return TRINIX_ERR_BAD_ARGUMENT;
  if (a->q_norm_weight) {
    if (esize != 2) return TRINIX_ERR_BAD_DTYPE;
    if (a->mask || a->dropout_p > 0.f) return TRINIX_ERR_BAD_ARGUMENT;
    if (!aligned16(a->q_norm_weight)) return TRINIX_ERR_BAD_STRIDE;
    if (!(a->q_norm_eps >= 0.f)) return TRINIX_ERR_BAD_ARGUMENT;
  }

  return TRINIX_OK;
}

int validate_bwd_args(const trinix_attn_bwd_args* a) {
  if (!a) return TRINIX_ERR_NULL_POINTER;
  if (a->dtype != TRINIX_F16 && a->dtype != TRINIX_BF16 && a->dtype != TRINIX_F32) return TRINIX_ERR_BAD_DTYPE;
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return TRINIX_ERR_BAD_HEAD_DIM;
  if (!(a->dropout_p >= 0.f && a->dropout_p < 1.f)) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->dropout_state && ((uintptr_t)a->dropout_state & 7)) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->dropout_keep_map && !keep_map_ok(a->dropout_keep_map, a->dropout_p, a->dtype, a->head_dim))
    return TRINIX_ERR_BAD_ARGUMENT;
  if (a->batch <= 0 || a->seqlen_q <= 0 || a->seqlen_k <= 0 || a->nheads_q <= 0 || a->nheads_kv <= 0 ||
      a->nheads_q % a->nheads_kv != 0)
    return TRINIX_ERR_BAD_SHAPE;
  if (a->seqlen_q >= (1ll << 30) || a->seqlen_k >= (1ll << 30) || a->batch >= (1 << 20) || a->nheads_q >= (1 << 20))
    return TRINIX_ERR_BAD_SHAPE;
  if (!a->lse || !a->delta) return TRINIX_ERR_NULL_POINTER;
  int rc;
  auto check = a->dtype == TRINIX_F32 ? check32 : check16;
  if ((rc = check(a->q, a->q_stride)) || (rc = check(a->k, a->k_stride)) || (rc = check(a->v, a->v_stride)) ||
      (rc = check(a->out, a->out_stride)) || (rc = check(a->dout, a->dout_stride)) ||
      (rc = check(a->dq, a->dq_stride)) || (rc = check(a->dk, a->dk_stride)) || (rc = check(a->dv, a->dv_stride)))
    return rc;
  if (a->mask && a->mask_dtype != TRINIX_F32 && a->mask_dtype != TRINIX_F16 && a->mask_dtype != TRINIX_BF16 &&
      a->mask_dtype != TRINIX_U8)
    return TRINIX_ERR_BAD_DTYPE;
  if (a->mask_blockmap && !a->mask) return TRINIX_ERR_BAD_ARGUMENT;
  if (a->mask && !mask_strides_ok(a->mask_stride, a->seqlen_q, a->seqlen_k)) return TRINIX_ERR_BAD_STRIDE;
  return TRINIX_OK;
}

int64_t clamp_window(int64_t w) {
  const int64_t lim = 1ll << 30;
  return w < -lim ? -lim : (w > lim ? lim : w);
}

int plan_fwd(const trinix_attn_fwd_args* a, FwdPlan* pl) {
  const bool f32 = a->dtype == TRINIX_F32;
  const bool plain = !a->mask && !(a->dropout_p > 0.f);
  const bool split_ok = plain && a->causal && !a->has_window && !a->q_norm_weight;
  Cfg16 cfg = pick_cfg16(a->head_dim, a->batch, a->nheads_q, a->seqlen_q, a->causal || a->has_window, plain,
                         split_ok);
  if (a->q_norm_weight) cfg.ks = 1;  // the fused q RMSNorm is built without the key split
  pl->n_items = 0;
  pl->num_mblk = 0;
  if (cfg.ks == 0) {  // per-item key split: the item table, or no split
    const int n = split_ok ? plan_split_rows(a->seqlen_q, a->seqlen_k, a->batch * a->nheads_q, 32 * cfg.nw, cfg.bn,
                                             pl->row_items, kMaxRowItems) : 0;
    if (n > (a->seqlen_q + 32 * cfg.nw - 1) / (32 * cfg.nw)) {
      pl->num_mblk = n;
      pl->n_items = n;
    } else {
      cfg.ks = 1;  // no block split (or no plan): the plain shape, without the per-item decode
    }
  }
  if (f32 || cfg.ks != 0) {
    const int bm = f32 ? 32 * kWavesF32 : 32 * cfg.nw / cfg.ks;
    pl->num_mblk = (int)((a->seqlen_q + bm - 1) / bm);
  }
  pl->cfg = cfg;
  pl->total_work = a->batch * a->nheads_q * pl->num_mblk;
  if (pl->total_work >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  return TRINIX_OK;
}

int plan_bwd(const trinix_attn_bwd_args* a, BwdPlan* pl) {
  pl->num_kblk = (int)((a->seqlen_k + 127) / 128);
  pl->dq_wide = a->dtype != TRINIX_F32 && pick_dq_wide(a->head_dim, a->batch, a->nheads_q, a->seqlen_q,
                                                       a->causal || a->has_window, a->mask != nullptr);
  pl->num_mblk = (int)((a->seqlen_q + (pl->dq_wide ? 255 : 127)) / (pl->dq_wide ? 256 : 128));
  if (a->batch * a->nheads_q * pl->num_mblk >= (1ll << 31) || a->batch * a->nheads_kv * pl->num_kblk >= (1ll << 31))
    return TRINIX_ERR_BAD_SHAPE;
  return TRINIX_OK;
}

bool make_split_plan(const trinix_attn_fwd_args* a, SplitPlan* pl) {
  if (a->dtype != TRINIX_BF16 && a->dtype != TRINIX_F16) return false;
  if (a->dropout_p > 0.f || a->rope_cos || a->q_norm_weight) return false;
  if (a->seqlen_q > kDecodeMaxSq) return false;
  if (a->head_dim != 64 && a->head_dim != 128) return false;
  const int64_t Sq = a->seqlen_q, Sk = a->seqlen_k;
  const int64_t G = a->nheads_q / a->nheads_kv;
  const int64_t M = G * Sq;
  const int64_t RG = (M + 15) / 16;
  const int64_t wl = clamp_window(a->window_left), wr = clamp_window(a->window_right);
  // Keys some row i in [0, Sq) may see: lo(i) = max(0, i - wl) is smallest at
  // i = 0, hi(i) = min(Sk - 1, i (causal), i + wr (window)) largest at Sq - 1.
  int64_t klo = a->has_window ? -wl : 0;
  klo = klo < 0 ? 0 : (klo > Sk ? Sk : klo);
  int64_t hi = Sk - 1;
  if (a->causal) hi = hi < Sq - 1 ? hi : Sq - 1;
  if (a->has_window) hi = hi < Sq - 1 + wr ? hi : Sq - 1 + wr;
  int64_t khi = hi + 1;
  khi = khi < 0 ? 0 : (khi > Sk ? Sk : khi);
  if (khi <= klo) return false;  // no visible key: every row is NaN, leave it to trinix_attn_fwd
  const int64_t span = khi - klo;
  const int64_t items = a->batch * a->nheads_kv * RG;
  int64_t target = kDecodeTargetWgs, min_chunk = kDecodeMinChunk;
  if (const char* env = getenv("TRINIX_SPLITKV_CFG")) {  // "target_wgs,min_chunk" (tuning only)
    long long t = 0, c = 0;
    if (sscanf(env, "%lld,%lld", &t, &c) == 2 && t > 0 && c >= 64) {
      target = t;
      min_chunk = c;
    }
  }
  const int64_t max_splits = (span + min_chunk - 1) / min_chunk;
  int64_t n = (target + items - 1) / items;
  n = n < 1 ? 1 : (n > max_splits ? max_splits : n);
  int64_t chunk = (span + n - 1) / n;
  chunk = (chunk + 63) / 64 * 64;
  n = (span + chunk - 1) / chunk;
  if (items * n >= (1ll << 31)) return false;
  pl->n_splits = (int)n;
  pl->chunk = (int)chunk;
  pl->klo = (int)klo;
  pl->khi = (int)khi;
  pl->M = (int)M;
  pl->RG = (int)RG;
  pl->ws_bytes = n > 1 ? a->batch * a->nheads_kv * M * n * (a->head_dim + 1) * 4 : 0;
  return true;
}

}  // namespace trinix
