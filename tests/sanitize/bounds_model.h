// CPU bounds model of the attention kernels' memory accesses.
//
// For one argument set accepted by the C ABI's validation, and the launch
// plan the library computes for it (plan_fwd / plan_bwd / make_split_plan,
// host_plan.cpp), this model walks the kernels' work decomposition with
// the kernels' own index maps (trinix_amd/csrc/index_map.h: work items, row
// blocks, key-tile ranges, tile-copy rows and 32-bit lane offsets) and
// checks every address they form:
//   * each access names an element inside its tensor: batch, sequence, head
//     and head_dim indices in range (a K/V tile reaching past seqlen_k reads
//     its clamped rows, a q/dO tile past seqlen_q likewise);
//   * the 32-bit parts of an address (per-lane tile offsets, mask element
//     offsets) equal the same offset formed in 64 bits: nothing wraps;
//   * every work item is run by exactly one workgroup, every output row is
//     written by exactly one lane (when the grid is small enough to list);
//   * the key tiles a row block visits hold every key its rows may see
//     (causal / window), and the tiles it runs without a predicate hold only
//     allowed (row, key) pairs;
//   * split-KV chunks tile the visible keys and partial results stay inside
//     the workspace.
//   * with a dropout keep map, the words the forward writes and the 256-byte
//     copies the backward makes of it lie inside the map (index_map.h).
// The per-lane load formulas that are not in index_map.h (a row's q, K/V,
// mask and output addresses: base + b*sb + h*sh + row*ss) are restated here
// from the kernels, each next to the kernel line it follows.
//
// Built with g++ (the CPU sanitizer test): __host__ / __device__ are
// defined empty before index_map.h is included.
#pragma once
#include <cstdint>
#include <cstdio>
#include <vector>

#define __host__
#define __device__
#include "index_map.h"
#include "host_plan.h"

namespace bounds {

using namespace trinix;

struct Report {
  long checks = 0, failures = 0;
  void fail(const char* what, const char* fmt, long long a = 0, long long b = 0, long long c = 0,
            long long d = 0) {
    ++failures;
    if (failures <= 20) {
      std::fprintf(stderr, "bounds: %s: ", what);
      std::fprintf(stderr, fmt, a, b, c, d);
      std::fprintf(stderr, "\n");
    }
  }
  bool expect(bool ok, const char* what, const char* fmt, long long a = 0, long long b = 0, long long c = 0,
              long long d = 0) {
    ++checks;
    if (!ok) fail(what, fmt, a, b, c, d);
    return ok;
  }
};

// Sample of [0, n): all of it when n <= limit, else both ends and a spread
// of interior points (deterministic).
int g_sample_ends = 8, g_sample_inner = 24;  // sampled points of a large range (fewer in the fuzz)
inline std::vector<int64_t> sample(int64_t n, int64_t limit, int ends = -1, int inner = -1) {
  if (ends < 0) ends = g_sample_ends;
  if (inner < 0) inner = g_sample_inner;
  std::vector<int64_t> v;
  if (n <= 0) return v;
  if (n <= limit) {
    for (int64_t i = 0; i < n; ++i) v.push_back(i);
    return v;
  }
  for (int64_t i = 0; i < ends; ++i) v.push_back(i);
  for (int64_t i = 0; i < ends; ++i) v.push_back(n - 1 - i);
  uint64_t x = (uint64_t)n * 0x9E3779B97F4A7C15ull + 12345;
  for (int k = 0; k < inner; ++k) {
    x ^= x >> 12, x ^= x << 25, x ^= x >> 27;
    v.push_back((int64_t)((x * 0x2545F4914F6CDD1Dull) % (uint64_t)n));
  }
  return v;
}

// Keys row i may see with the caller's (unclamped) window: [lo, hi], empty
// when hi < lo.  Computed in 128 bits from the arguments, not from the
// kernels' clamped values.
inline void allowed_keys(const trinix_attn_fwd_args& a, int64_t i, int64_t& lo, int64_t& hi) {
  __int128 l = 0, h = (__int128)a.seqlen_k - 1;
  if (a.causal && h > i) h = i;
  if (a.has_window) {
    const __int128 wl = (__int128)i - a.window_left, wr = (__int128)i + a.window_right;
    if (wl > l) l = wl;
    if (wr < h) h = wr;
  }
  if (h < l) {
    lo = 1;
    hi = 0;
    return;
  }
  lo = (int64_t)l;
  hi = (int64_t)h;
}

inline int swz_of(int which, int D, int row) {  // 0: swz_k, 1: swz_v, 2: swz_kt
  switch (D) {
    case 64: return which == 0 ? swz_k<64>(row) : which == 1 ? swz_v<64>(row) : swz_kt<64>(row);
    case 128: return which == 0 ? swz_k<128>(row) : which == 1 ? swz_v<128>(row) : swz_kt<128>(row);
    default: return which == 0 ? swz_k<256>(row) : which == 1 ? swz_v<256>(row) : swz_kt<256>(row);
  }
}

// One BN-row tile of a 16-bit (B, S, H, D) tensor copied global -> LDS by NW
// wavefronts (attn_kernel16.h load_tile, attn_bwd16.h load_rows): the base
// is row n0 of (b, h), 64-bit; lane offsets are tile_copy_offset of the
// (clamped) tile row.  `clamp_always`: the backward clamps every tile (rows
// past `rows` read row rows-1); the forward clamps only a tile reaching past
// `rows`, and uses the precomputed offsets (ld_koff) otherwise.
inline void check_tile_copy(Report& R, const char* what, int64_t n0, int BN, int D, int NW, int swz, int64_t rows,
                            int64_t ss, bool clamp_always) {
  const int UPR = D / 8, LPW = BN * UPR / (64 * NW);
  if (!R.expect(n0 >= 0 && n0 < rows, what, "tile start %lld outside [0, %lld)", n0, rows)) return;
  for (int w = 0; w < NW; ++w)
    for (int l = 0; l < LPW; ++l)
      for (int lane = 0; lane < 64; ++lane) {
        const int row = tile_copy_row(w, LPW, l, lane, UPR);
        const int unit = (lane % UPR) ^ swz_of(swz, D, row);
        int64_t trow = row;
        if (clamp_always || n0 + BN > rows) {
          const int64_t last = rows - 1 - n0;  // >= 0 above
          trow = row < last ? row : last;
        }
        const uint32_t off = tile_copy_offset((uint32_t)trow, ss, (uint32_t)unit);
        const int64_t exact = trow * ss * 2 + (int64_t)unit * 16;
        R.expect((int64_t)off == exact, what, "32-bit lane offset %lld != %lld (row %lld, stride %lld)",
                 (long long)off, exact, trow, ss);
        R.expect(n0 + trow < rows && row < BN && unit >= 0 && unit < UPR, what,
                 "row %lld of %lld, unit %lld of %lld", n0 + trow, rows, unit, UPR);
      }
}

// ---- forward, 16-bit kernels (attn_kernel16.h) ------------------------------
inline void model_fwd16(Report& R, const trinix_attn_fwd_args& a, const FwdPlan& pl, int64_t item_limit) {
  const int D = (int)a.head_dim;
  const Cfg16 cfg = pl.cfg;
  const int NW = cfg.nw, BN = cfg.bn, KS = cfg.ks;
  const int B = (int)a.batch, Sq = (int)a.seqlen_q, Sk = (int)a.seqlen_k, Hq = (int)a.nheads_q,
            Hkv = (int)a.nheads_kv, G = Hq / Hkv;
  const int64_t wl = clamp_window(a.window_left), wr = clamp_window(a.window_right);
  const bool causal = a.causal != 0, win = a.has_window != 0;
  R.expect(BN * (D / 8) % (64 * NW) == 0, "fwd", "tile shape nw %lld bn %lld", NW, BN);
  if (KS == 0) R.expect(pl.n_items == pl.num_mblk && pl.n_items <= kMaxRowItems, "fwd", "split items %lld", pl.n_items);
  const int64_t total = pl.total_work;
  const bool all = total <= item_limit && (int64_t)B * Hq * Sq <= 4 * item_limit;
  std::vector<uint8_t> seen_item(all ? (size_t)total : 0), seen_row(all ? (size_t)B * Hq * Sq : 0);
  const int64_t bmap_rows = ((int64_t)Sq + 31) / 32, bmap_cols = ((int64_t)Sk + 63) / 64;
  for (int64_t blk : sample(total, all ? total : 0)) {
    const FwdItem it = fwd_item((int)blk, B, Hkv, G, pl.num_mblk, (int)total, causal, win);
    if (!R.expect(it.b >= 0 && it.b < B && it.hkv >= 0 && it.hkv < Hkv && it.gq >= 0 && it.gq < G && it.mi >= 0 &&
                      it.mi < pl.num_mblk,
                  "fwd item", "block %lld -> out of range (b %lld, hkv %lld, mi %lld)", blk, it.b, it.hkv, it.mi))
      continue;
    if (all) {
      const int64_t key = (((int64_t)it.b * Hkv + it.hkv) * pl.num_mblk + it.mi) * G + it.gq;
      R.expect(seen_item[key]++ == 0, "fwd item", "work item %lld run twice (block %lld)", key, blk);
    }
    const int hq = it.hkv * G + it.gq;
    const uint32_t item = KS == 0 ? pl.row_items[it.mi] : 0u;
    const RowBlock rb = fwd_row_block(KS, NW, it.mi, causal, pl.num_mblk, item);
    const int bm = NW * 32 / rb.ks;
    R.expect(rb.m0 >= 0 && rb.m0 < Sq, "fwd rows", "item first row %lld outside [0, %lld)", rb.m0, Sq);
    const TileRange tr = fwd_tile_range(rb.m0, bm, Sq, Sk, causal, win, wl, wr, BN);
    R.expect(tr.t_lo <= tr.t_flo && tr.t_flo <= tr.t_fhi && tr.t_fhi <= tr.t_hi, "fwd tiles",
             "ordering %lld %lld %lld %lld", tr.t_lo, tr.t_flo, tr.t_fhi, tr.t_hi);
    if (tr.t_lo < tr.t_hi)
      R.expect((int64_t)(tr.t_hi - 1) * BN < Sk, "fwd tiles", "last tile %lld starts past Sk %lld", tr.t_hi - 1, Sk);
    // every key a row of the item may see lies in the visited tiles (the
    // allowed keys' bounds grow with the row: check the first and last row)
    const int mlast = imin(rb.m0 + bm, Sq) - 1;
    for (int64_t i : {(int64_t)rb.m0, (int64_t)mlast}) {
      int64_t lo, hi;
      allowed_keys(a, i, lo, hi);
      if (lo <= hi)
        R.expect(lo >= (int64_t)tr.t_lo * BN && hi < (int64_t)tr.t_hi * BN, "fwd tiles",
                 "row %lld sees keys [%lld, %lld] outside the visited tiles (from key %lld)", i, lo, hi,
                 (int64_t)tr.t_lo * BN);
    }
    // full tiles: every (i, j) of the item allowed
    if (tr.t_flo < tr.t_fhi) {
      const int64_t j0 = (int64_t)tr.t_flo * BN, j1 = (int64_t)tr.t_fhi * BN - 1;
      for (int64_t i : {(int64_t)rb.m0, (int64_t)mlast}) {
        int64_t lo, hi;
        allowed_keys(a, i, lo, hi);
        R.expect(lo <= j0 && j1 <= hi, "fwd full tiles", "row %lld: keys [%lld, %lld] not all allowed (%lld)", i, j0,
                 j1, lo);
      }
    }
    // K / V tiles: the first two, the last two and the full range's edges
    for (int t : {tr.t_lo, tr.t_lo + 1, tr.t_flo, tr.t_fhi - 1, tr.t_fhi, tr.t_hi - 2, tr.t_hi - 1}) {
      if (t < tr.t_lo || t >= tr.t_hi) continue;
      check_tile_copy(R, "fwd K tile", (int64_t)t * BN, BN, D, NW, 0, Sk, a.k_stride[1], false);
      check_tile_copy(R, "fwd V tile", (int64_t)t * BN, BN, D, NW, 1, Sk, a.v_stride[1], false);
    }
    for (int w = 0; w < NW; ++w) {
      const int kp = w % rb.ks;
      const int iw0 = rb.m0 + (w / rb.ks) * 32;
      const bool live = iw0 < Sq;
      for (int r = 0; r < 32; ++r) {
        const int i = iw0 + r, ic = imin(i, Sq - 1);  // q row (attn_kernel16.h:133-134, 167)
        R.expect(ic >= 0 && ic < Sq, "fwd q row", "row %lld", ic);
        if (all && i < Sq && kp == 0) {
          const int64_t key = ((int64_t)it.b * Hq + hq) * Sq + i;
          R.expect(seen_row[key]++ == 0, "fwd out", "row %lld of head %lld written twice", i, hq);
        }
        if (a.mask && live) {
          // mask row ic (64-bit) + key j at 32-bit offset min(j, Sk-1)*sj (load_mask4)
          for (int t : {tr.t_lo, tr.t_hi - 1}) {
            if (t < tr.t_lo || t >= tr.t_hi) continue;
            for (int dj = 0; dj < BN; dj += BN - 1) {
              const int64_t j = (int64_t)t * BN + dj, jc = j < Sk - 1 ? j : Sk - 1;
              const uint32_t off = (uint32_t)jc * (uint32_t)a.mask_stride[3];
              R.expect((int64_t)off == jc * a.mask_stride[3] && off < (1u << 31), "fwd mask", "key %lld offset %lld",
                       jc, (long long)off);
            }
          }
        }
      }
      if (a.mask && a.mask_blockmap && live)
        R.expect(iw0 / 32 < bmap_rows, "fwd block map", "row block %lld of %lld", iw0 / 32, bmap_rows);
      (void)bmap_cols;
      if (a.dropout_keep_map && a.dropout_p > 0.f && live) {
        // half g of word r of block (iw0/32, tile*BN/32 + nb) (attn_kernel16.h softmax, DROP == 2)
        const int64_t nbi = keep_map_nbi(Sq), nbj = keep_map_nbj(Sk), words = (int64_t)B * Hq * nbi * nbj * 32;
        for (int t : {tr.t_lo, tr.t_hi - 1}) {
          if (t < tr.t_lo || t >= tr.t_hi || (t - tr.t_lo) % rb.ks != kp) continue;
          for (int nb = 0; nb < BN / 32; ++nb) {
            const int64_t bi = iw0 >> 5, bj = (((int64_t)t * BN) >> 5) + nb;
            R.expect(bi < nbi && bj < nbj, "fwd keep map", "block (%lld, %lld) of (%lld, %lld)", bi, bj, nbi, nbj);
            for (int r : {0, 31})
              for (int g : {0, 1}) {
                const int64_t half = 2 * (keep_map_block((int64_t)it.b * Hq + hq, bi, bj, nbi, nbj) + r) + g;
                R.expect(half >= 0 && half < 2 * words, "fwd keep map", "half-word %lld of %lld", half, 2 * words);
              }
          }
        }
      }
    }
  }
  if (all) {
    for (int64_t k = 0; k < total; ++k)
      if (!R.expect(seen_item[k] == 1, "fwd item", "work item %lld run %lld times", k, seen_item[k])) break;
    for (int64_t k = 0; k < (int64_t)B * Hq * Sq; ++k)
      if (!R.expect(seen_row[k] == 1, "fwd out", "output row %lld written %lld times", k, seen_row[k])) break;
  }
}

// ---- backward, 16-bit kernels (attn_bwd16.h) ----------------------------------
inline void model_bwd16(Report& R, const trinix_attn_bwd_args& a, const BwdPlan& pl, int64_t item_limit) {
  const int D = (int)a.head_dim;
  const int B = (int)a.batch, Sq = (int)a.seqlen_q, Sk = (int)a.seqlen_k, Hq = (int)a.nheads_q,
            Hkv = (int)a.nheads_kv, G = Hq / Hkv;
  int dlo, dhi;
  band_offsets(a.causal != 0, a.has_window != 0, clamp_window(a.window_left), clamp_window(a.window_right), dlo, dhi);
  trinix_attn_fwd_args f{};  // the forward's view of the same problem (allowed keys)
  f.seqlen_q = a.seqlen_q, f.seqlen_k = a.seqlen_k, f.causal = a.causal, f.has_window = a.has_window;
  f.window_left = a.window_left, f.window_right = a.window_right;

  // dK / dV: 8 wavefronts, 4 key groups of 32 keys, 64-row query tiles
  constexpr int BK = 128, BQ = 64, NWKV = 8;
  const int64_t nkv = (int64_t)B * Hkv * pl.num_kblk;
  const bool all = nkv <= item_limit;
  std::vector<uint8_t> seen(all ? (size_t)nkv : 0), seen_key(all ? (size_t)B * Hkv * Sk : 0);
  for (int64_t blk : sample(nkv, all ? nkv : 0)) {
    const KvItem it = bwd_kv_item((int)blk, B, Hkv, pl.num_kblk, a.causal != 0);
    if (!R.expect(it.b >= 0 && it.b < B && it.hkv >= 0 && it.hkv < Hkv && it.kblk >= 0 && it.kblk < pl.num_kblk,
                  "dkdv item", "block %lld out of range", blk))
      continue;
    if (all) {
      const int64_t key = ((int64_t)it.b * Hkv + it.hkv) * pl.num_kblk + it.kblk;
      R.expect(seen[key]++ == 0, "dkdv item", "item %lld twice", key);
    }
    const int kb0 = it.kblk * BK;
    R.expect(kb0 < Sk, "dkdv keys", "key block start %lld past Sk %lld", kb0, Sk);
    int qt_lo, qt_hi;
    bwd_query_tiles(kb0, BK, Sq, Sk, dlo, dhi, BQ, qt_lo, qt_hi);
    // every query that sees a key of the block lies in [qt_lo*BQ, qt_hi*BQ):
    // row i sees key j iff j in allowed_keys(i); scan the rows' bounds
    const int kmax = imin(kb0 + BK, Sk) - 1;
    for (int64_t i : sample(Sq, 512, 16, 32)) {
      int64_t lo, hi;
      allowed_keys(f, i, lo, hi);
      if (lo <= hi && lo <= kmax && hi >= kb0)
        R.expect(i >= (int64_t)qt_lo * BQ && i < (int64_t)qt_hi * BQ, "dkdv queries",
                 "row %lld sees the key block at %lld but lies outside query tiles [%lld, %lld)", i, kb0, qt_lo, qt_hi);
    }
    const int UPR = D / 8, LPW = BQ * UPR / (64 * NWKV);
    for (int qt : {qt_lo, qt_lo + 1, qt_hi - 1}) {
      if (qt < qt_lo || qt >= qt_hi) continue;
      const int i0 = qt * BQ;
      if (!R.expect(i0 < Sq, "dkdv queries", "query tile at %lld past Sq %lld", i0, Sq)) continue;
      check_tile_copy(R, "dkdv Q tile", i0, BQ, D, NWKV, 2, Sq, a.q_stride[1], true);
      check_tile_copy(R, "dkdv dO tile", i0, BQ, D, NWKV, 2, Sq, a.dout_stride[1], true);
      (void)LPW;
      for (int lane = 0; lane < 64; ++lane) {  // lse / delta: vo + i0 + min(lane, Sq-1-i0)
        const int64_t row = i0 + imin(lane, Sq - 1 - i0);
        R.expect(row >= 0 && row < Sq, "dkdv lse", "row %lld", row);
      }
      if (a.dropout_keep_map && a.dropout_p > 0.f) {
        // load_item: 4 copies of 64 words, block (qt*2 + c/2, kblk*4) + (c%2)*64 + lane
        const int64_t nbi = keep_map_nbi(Sq), nbj = keep_map_nbj(Sk), words = (int64_t)B * Hq * nbi * nbj * 32;
        for (int gh : {0, G - 1})
          for (int c = 0; c < 4; ++c) {
            const int64_t bi = (int64_t)qt * 2 + (c >> 1), bj = (int64_t)it.kblk * 4;
            R.expect(bi < nbi && bj + 3 < nbj, "dkdv keep map", "blocks (%lld, %lld..+3) of (%lld, %lld)", bi, bj, nbi,
                     nbj);
            const int64_t base = keep_map_block((int64_t)it.b * Hq + it.hkv * G + gh, bi, bj, nbi, nbj) + (c & 1) * 64;
            R.expect(base >= 0 && base + 63 < words, "dkdv keep map", "words [%lld, %lld] of %lld", base, base + 63,
                     words);
          }
      }
      if (a.mask) {
        for (int st = 0; st < BQ / 32; ++st) {  // attn_bwd16.h stage A, 64-bit sub-tile row + 32-bit offsets
          const int ia = i0 + st * 32;
          if (ia >= Sq) continue;  // sub_live
          const int rlast = imin(31, Sq - 1 - ia);
          R.expect(rlast >= 0, "dkdv mask", "sub-tile last row %lld", rlast);
          for (int r : {0, rlast}) {
            const uint32_t off = (uint32_t)r * (uint32_t)a.mask_stride[2];
            R.expect((int64_t)off == (int64_t)r * a.mask_stride[2] && off < (1u << 31), "dkdv mask",
                     "row offset %lld (row %lld, stride %lld)", (long long)off, r, a.mask_stride[2]);
          }
          if (a.mask_blockmap)
            R.expect(ia / 32 < ((int64_t)Sq + 31) / 32, "dkdv block map", "row block %lld", ia / 32);
        }
      }
    }
    for (int kg = 0; kg < 4; ++kg)
      for (int l = 0; l < 32; ++l) {
        const int j = kb0 + kg * 32 + l, jc = imin(j, Sk - 1);  // K / V row of the lane
        R.expect(jc >= 0 && jc < Sk, "dkdv K row", "key %lld", jc);
        if (all && j < Sk) {  // dK / dV rows written once (stage B / stage A)
          const int64_t key = ((int64_t)it.b * Hkv + it.hkv) * Sk + j;
          R.expect(seen_key[key]++ == 0, "dkdv out", "key row %lld written twice", j);
        }
      }
  }
  if (all) {
    for (int64_t k = 0; k < nkv; ++k)
      if (!R.expect(seen[k] == 1, "dkdv item", "item %lld run %lld times", k, seen[k])) break;
    for (int64_t k = 0; k < (int64_t)B * Hkv * Sk; ++k)
      if (!R.expect(seen_key[k] == 1, "dkdv out", "dK/dV row %lld written %lld times", k, seen_key[k])) break;
  }

  // dQ: the forward's decomposition
  const int NW = pl.dq_wide ? 8 : 4, BN = pl.dq_wide ? 128 : 64, BM = NW * 32;
  const int64_t nq = (int64_t)B * Hq * pl.num_mblk;
  const bool allq = nq <= item_limit && (int64_t)B * Hq * Sq <= 4 * item_limit;
  std::vector<uint8_t> seen_row(allq ? (size_t)B * Hq * Sq : 0);
  for (int64_t blk : sample(nq, allq ? nq : 0)) {
    const DqItem it = bwd_dq_item((int)blk, B, Hq, Hkv, G, pl.num_mblk, a.causal != 0, BM);
    if (!R.expect(it.b >= 0 && it.b < B && it.hkv >= 0 && it.hkv < Hkv && it.gq >= 0 && it.gq < G && it.m0 >= 0 &&
                      it.m0 < Sq,
                  "dq item", "block %lld out of range (m0 %lld)", blk, it.m0))
      continue;
    const int hq = it.hkv * G + it.gq;
    int t_lo, t_hi;
    bwd_key_tiles(it.m0, BM, Sq, Sk, dlo, dhi, BN, t_lo, t_hi);
    const int mlast = imin(it.m0 + BM, Sq) - 1;
    for (int64_t i : {(int64_t)it.m0, (int64_t)mlast}) {
      int64_t lo, hi;
      allowed_keys(f, i, lo, hi);
      if (lo <= hi)
        R.expect(lo >= (int64_t)t_lo * BN && hi < (int64_t)t_hi * BN, "dq tiles", "row %lld keys [%lld, %lld] missed",
                 i, lo, hi);
    }
    for (int t : {t_lo, t_lo + 1, t_hi - 2, t_hi - 1}) {
      if (t < t_lo || t >= t_hi) continue;
      check_tile_copy(R, "dq K tile", (int64_t)t * BN, BN, D, NW, 2, Sk, a.k_stride[1], true);
      check_tile_copy(R, "dq V tile", (int64_t)t * BN, BN, D, NW, 2, Sk, a.v_stride[1], true);
    }
    if (a.dropout_keep_map && a.dropout_p > 0.f) {
      // load_keep: the wavefront's NB/2 copies of 64 words, block (iw0/32, t*NB) + c*64 + lane
      const int NB = BN / 32;
      const int64_t nbi = keep_map_nbi(Sq), nbj = keep_map_nbj(Sk), words = (int64_t)B * Hq * nbi * nbj * 32;
      for (int t : {t_lo, t_hi - 1}) {
        if (t < t_lo || t >= t_hi) continue;
        for (int w = 0; w < NW; ++w) {
          const int iw0 = it.m0 + w * 32;
          if (iw0 >= Sq) continue;
          const int64_t bi = iw0 >> 5, bj = (int64_t)t * NB;
          R.expect(bi < nbi && bj + NB - 1 < nbj, "dq keep map", "blocks (%lld, %lld..) of (%lld, %lld)", bi, bj, nbi,
                   nbj);
          for (int c = 0; c < NB / 2; ++c) {
            const int64_t base = keep_map_block((int64_t)it.b * Hq + hq, bi, bj, nbi, nbj) + c * 64;
            R.expect(base >= 0 && base + 63 < words, "dq keep map", "words [%lld, %lld] of %lld", base, base + 63,
                     words);
          }
        }
      }
    }
    for (int w = 0; w < NW; ++w)
      for (int r = 0; r < 32; ++r) {
        const int i = it.m0 + w * 32 + r, ic = imin(i, Sq - 1);
        R.expect(ic >= 0 && ic < Sq, "dq q row", "row %lld", ic);
        if (allq && i < Sq) {
          const int64_t key = ((int64_t)it.b * Hq + hq) * Sq + i;
          R.expect(seen_row[key]++ == 0, "dq out", "dQ row %lld written twice", i);
        }
      }
  }
  if (allq)
    for (int64_t k = 0; k < (int64_t)B * Hq * Sq; ++k)
      if (!R.expect(seen_row[k] == 1, "dq out", "dQ row %lld written %lld times", k, seen_row[k])) break;
}

// ---- split-KV decode (attn_decode.hip) ----------------------------------------
inline void model_decode(Report& R, const trinix_attn_fwd_args& a, const SplitPlan& pl, int64_t item_limit) {
  const int D = (int)a.head_dim;
  const int B = (int)a.batch, Sq = (int)a.seqlen_q, Sk = (int)a.seqlen_k, Hq = (int)a.nheads_q,
            Hkv = (int)a.nheads_kv, G = Hq / Hkv;
  const int64_t nwg = (int64_t)B * Hkv * pl.RG * pl.n_splits;
  const int64_t nrows = (int64_t)B * Hkv * pl.M * pl.n_splits;  // partial slots
  if (pl.n_splits > 1)
    R.expect(pl.ws_bytes == nrows * (D + 1) * 4, "decode plan", "workspace %lld != %lld", pl.ws_bytes,
             nrows * (D + 1) * 4);
  R.expect(pl.M == G * Sq && pl.RG == (pl.M + 15) / 16, "decode plan", "rows %lld groups %lld", pl.M, pl.RG);
  std::vector<uint8_t> slot(nwg <= item_limit && pl.n_splits > 1 ? (size_t)nrows : 0);
  for (int64_t blk : sample(nwg, item_limit)) {
    const DecItem it = dec_item((int)blk, pl.RG, pl.n_splits);
    if (!R.expect(it.rg >= 0 && it.rg < pl.RG && it.split >= 0 && it.split < pl.n_splits && it.bh >= 0 &&
                      it.bh < B * Hkv,
                  "decode item", "block %lld out of range", blk))
      continue;
    int c0, c1;
    dec_chunk(pl.klo, pl.khi, pl.chunk, it.split, c0, c1);
    R.expect(0 <= pl.klo && c0 < c1 && c1 <= pl.khi && pl.khi <= Sk, "decode chunk",
             "chunk [%lld, %lld) of [%lld, %lld)", c0, c1, pl.klo, pl.khi);
    // K / V rows: min(j, Sk - 1) for keys j >= c0 (steps past the chunk end re-read clamped rows)
    R.expect(c0 >= 0 && c0 <= Sk - 1, "decode K row", "first key %lld", c0);
    for (int lr = 0; lr < 16; ++lr) {
      const int r = it.rg * 16 + lr;
      if (r >= pl.M) continue;  // padding row: reads row 0, writes nothing
      const int i = r / G, hq = (it.bh % Hkv) * G + r % G;
      R.expect(i >= 0 && i < Sq && hq >= 0 && hq < Hq, "decode row", "row %lld head %lld", i, hq);
      if (pl.n_splits > 1) {
        const int64_t idx = dec_partial_index(it.bh, pl.M, r, pl.n_splits, it.split);
        R.expect(idx >= 0 && idx < nrows && (idx + 1) * D <= nrows * D, "decode partial", "slot %lld of %lld", idx,
                 nrows);
        if (!slot.empty()) R.expect(slot[idx]++ == 0, "decode partial", "slot %lld written twice", idx);
      }
    }
  }
  if (!slot.empty())
    for (int64_t k = 0; k < nrows; ++k)
      if (!R.expect(slot[k] == 1, "decode partial", "slot %lld written %lld times", k, slot[k])) break;
  // merge: row `row` reads slots [row*n, row*n + n) and writes (b, i, hq)
  if (pl.n_splits > 1)
    for (int64_t row : sample((int64_t)B * Hkv * pl.M, 64)) {
      const int64_t bh = row / pl.M, r = row % pl.M;
      R.expect((row + 1) * pl.n_splits <= nrows && r / G < Sq && (bh % Hkv) * G + r % G < Hq, "decode merge",
               "row %lld", row);
    }
}

}  // namespace bounds
