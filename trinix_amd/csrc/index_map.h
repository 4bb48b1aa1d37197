// Index maps of the attention kernels: which work item a workgroup runs,
// which query rows and key tiles it covers, and the offsets of its tile
// copies.  Plain integer code with no HIP dependency, marked __host__
// __device__: the kernels inline it, and the CPU bounds model
// (tests/sanitize/bounds_model.h, built by g++ with the two attributes
// defined empty) runs the same functions over the launch plans of
// host_plan.cpp to check every address they produce against the tensors'
// extents.
#pragma once
#include <stdint.h>

namespace trinix {

// Workgroups are dispatched round-robin over the kXcds = 8 XCDs of an
// MI355X (WG x runs on XCD x % 8).  Give each XCD one contiguous range of the
// work list, so work items that read the same K/V (neighbouring items) share
// that XCD's L2.
constexpr int kXcds = 8;
__host__ __device__ inline int xcd_remap(int x, int total) {
  const int xcd = x % kXcds, idx = x / kXcds;
  const int per = total / kXcds, rem = total % kXcds;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }
__host__ __device__ inline int imax(int a, int b) { return a > b ? a : b; }
__host__ __device__ inline int64_t lmin(int64_t a, int64_t b) { return a < b ? a : b; }
__host__ __device__ inline int64_t lmax(int64_t a, int64_t b) { return a > b ? a : b; }

// Swizzle of the 16-byte units of a D-wide row-major tile row.  K rows are
// read 16 bytes per lane, 16 consecutive rows per access; V rows are read 8
// bytes per lane by ds_read_b64_tr_b16, 4 consecutive rows x 64 bytes per
// 32 lanes.  Rows of D >= 128 (256 or 512 bytes) all start on bank 0, so
// the unit index is XORed with the row (mod 16 units); 128-byte rows (D = 64)
// pair up first.
template <int D>
__host__ __device__ inline int swz_k(int row) {
  return D >= 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__host__ __device__ inline int swz_v(int row) {
  return D >= 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1);
}

// Swizzle of tiles read both ways: row-wise (ds_read_b128, 16 consecutive
// rows per access phase) and by ds_read_b64_tr_b16 (4 consecutive rows x 64
// bytes per 32 lanes).  Rows sharing a bank period need distinct units for
// the row reads (a bijection of the 16 rows onto the 16 units); the
// transpose reads need the 64-byte group (unit bits 2-3) to differ across
// any 4 consecutive rows.  Swapping the two 2-bit fields of the row index
// gives both (for D = 64, two 128-byte rows share a period: the same on
// (row >> 1) & 7 with fields of 1 and 2 bits).  swz_k alone conflicts 4-way
// on the transpose reads.
template <int D>
__host__ __device__ inline int swz_kt(int row) {
  if constexpr (D >= 128) {
    const int s = row & 15;
    return ((s & 3) << 2) | (s >> 2);
  } else {
    const int s = (row >> 1) & 7;
    return ((s & 1) << 2) | (s >> 1);
  }
}

// ---- tile copies (global -> LDS, 16 bytes per lane) ----------------------
// Copy l of wavefront `wave` fills LDS units [64*(wave*LPW + l), +64) of a
// tile of rows of UPR 16-byte units: lane `lane` takes unit u, tile row u / UPR.
__host__ __device__ inline int tile_copy_row(int wave, int lpw, int l, int lane, int upr) {
  return ((wave * lpw + l) * 64 + lane) / upr;
}
// Byte offset of (tile row `row`, 16-byte unit `unit`) from the tile's first
// row, in 32 bits, for a 16-bit tensor with row stride `ss` elements.  The
// host bounds ss (kMaxKvRowStride) so that every tile row of a copy fits.
__host__ __device__ inline uint32_t tile_copy_offset(uint32_t row, int64_t ss, uint32_t unit) {
  return row * (uint32_t)ss * 2u + unit * 16u;
}

// ---- forward (attn_fwd_mfma16) --------------------------------------------
// Work item of workgroup `blk`: (batch, kv-head, q-head within the group,
// row-block slot).  Each XCD owns whole KV-head groups, so the q-heads
// sharing a KV head run on one XCD and share its L2.  Causal row blocks are
// dispatched longest first across all the head groups of an XCD (when the
// groups split evenly over the 8 XCDs): the long chains then start first
// and run alone on their CUs, and the short blocks fill in behind them.
// With a causal window the row blocks have (nearly) one length and each
// reads a window of K/V: an XCD then runs its head groups one after the
// other, row blocks longest first within each, so that its resident
// workgroups read one group's window (C4: 16 groups, two per XCD; with
// both interleaved the XCD's 4 MB L2 held neither window).
struct FwdItem {
  int b, hkv, gq, mi;
};
__host__ __device__ inline FwdItem fwd_item(int blk, int B, int Hkv, int G, int num_mblk, int total_work,
                                            bool causal, bool windowed) {
  FwdItem it;
  const int groups = B * Hkv;
  if (causal && groups % kXcds == 0) {
    const int xcd = blk % kXcds, j = blk / kXcds;  // j: dispatch order in the XCD
    const int ng = groups / kXcds;
    int hg;
    if (windowed) {
      const int per = num_mblk * G;  // one head group's items
      hg = xcd * ng + j / per;
      it.mi = (j % per) / G;
      it.gq = j % G;
    } else {
      it.mi = j / (ng * G);
      const int rest = j % (ng * G);
      hg = xcd * ng + rest / G;
      it.gq = rest % G;
    }
    it.hkv = hg % Hkv;
    it.b = hg / Hkv;
  } else {
    int w = xcd_remap(blk, total_work);
    it.gq = w % G;
    w /= G;
    it.mi = w % num_mblk;
    w /= num_mblk;
    it.hkv = w % Hkv;
    it.b = w / Hkv;
  }
  return it;
}

// First query row of a work item and its wavefronts per 32-row group (ks).
// KS = 1 or 2: row block mi (causal: reversed, longest rows first) of
// NW*32/KS rows.  KS = 0: entry `item` of the per-item split table
// (row block << 2 | split << 1 | half): a whole block of NW*32 rows (ks 1)
// or one half of it (NW*16 rows, ks 2).
struct RowBlock {
  int m0, ks;
};
__host__ __device__ inline RowBlock fwd_row_block(int KS, int NW, int mi, bool causal, int num_mblk, uint32_t item) {
  RowBlock rb;
  if (KS == 0) {
    rb.ks = (item & 2u) ? 2 : 1;
    rb.m0 = (int)(item >> 2) * (NW * 32) + (int)(item & 1u) * (NW * 16);
  } else {
    const int mblk = causal ? (num_mblk - 1 - mi) : mi;  // longest rows first
    rb.ks = KS;
    rb.m0 = mblk * (NW * 32 / KS);
  }
  return rb;
}

// Key tiles of BN keys a workgroup of rows [m0, m0 + bm) visits,
// [t_lo, t_hi), and its full tiles [t_flo, t_fhi) (every (i, j) of the
// workgroup allowed): causal j <= i, window -wl <= j - i <= wr, j < Sk.
// wl and wr are at most 2^30 in magnitude (clamp_window, host_plan.cpp).
struct TileRange {
  int t_lo, t_hi, t_flo, t_fhi;
};
__host__ __device__ inline TileRange fwd_tile_range(int m0, int bm, int Sq, int Sk, bool causal, bool has_window,
                                                    int64_t wl, int64_t wr, int BN) {
  const int mlast = imin(m0 + bm, Sq) - 1;
  int64_t lo = 0, hi = Sk, flo = 0, fhi = Sk;
  if (causal) {
    hi = lmin(hi, (int64_t)mlast + 1);
    fhi = lmin(fhi, (int64_t)m0 + 1);
  }
  if (has_window) {
    lo = lmax(lo, (int64_t)m0 - wl);
    hi = lmin(hi, (int64_t)mlast + wr + 1);
    flo = lmax(flo, (int64_t)mlast - wl);
    fhi = lmin(fhi, (int64_t)m0 + wr + 1);
  }
  TileRange tr;
  tr.t_lo = (int)(lo / BN);
  tr.t_hi = hi > lo ? (int)((hi + BN - 1) / BN) : tr.t_lo;
  int t_flo = (int)((flo + BN - 1) / BN);
  int t_fhi = fhi > 0 ? (int)(fhi / BN) : 0;
  t_flo = imin(imax(t_flo, tr.t_lo), tr.t_hi);
  tr.t_flo = t_flo;
  tr.t_fhi = imin(imax(t_fhi, t_flo), tr.t_hi);
  return tr;
}

// ---- backward ---------------------------------------------------------------
// Allowed (i, j): j - i in [dlo, dhi] (causal: j <= i; window: -wl <= j-i <= wr),
// clamped to +-2^30 (every |j - i| < 2^30).
__host__ __device__ inline void band_offsets(bool causal, bool has_window, int64_t wl, int64_t wr, int& dlo,
                                             int& dhi) {
  int64_t lo = INT32_MIN / 2, hi = INT32_MAX / 2;
  if (causal) hi = 0;
  if (has_window) {
    lo = lo > -wl ? lo : -wl;
    hi = hi < wr ? hi : wr;
  }
  dlo = (int)(lo < INT32_MIN / 2 ? INT32_MIN / 2 : lo);
  dhi = (int)(hi > INT32_MAX / 2 ? INT32_MAX / 2 : hi);
}

// dK/dV: work item (batch, kv-head, block of BK keys) of workgroup `blk`.
// Each XCD owns whole (batch, kv-head) groups, whose Q / dO tiles it then
// reads from its own L2.  Causal: low key blocks see the most queries; when
// the groups split evenly over the XCDs, an XCD dispatches the key blocks of
// all its groups in ascending order (longest first), so that the short
// blocks fill in behind the long ones.
struct KvItem {
  int b, hkv, kblk;
};
__host__ __device__ inline KvItem bwd_kv_item(int blk, int B, int Hkv, int num_kblk, bool causal) {
  KvItem it;
  const int groups = B * Hkv;
  if (causal && groups % kXcds == 0) {
    const int xcd = blk % kXcds, j = blk / kXcds;  // j: dispatch order in the XCD
    const int ng = groups / kXcds;
    it.kblk = j / ng;
    const int hg = xcd * ng + j % ng;
    it.hkv = hg % Hkv;
    it.b = hg / Hkv;
    return it;
  }
  int w = xcd_remap(blk, groups * num_kblk);
  it.kblk = w % num_kblk;
  w /= num_kblk;
  it.hkv = w % Hkv;
  it.b = w / Hkv;
  return it;
}
// Query tiles of BQ rows [qt_lo, qt_hi) that see any key of [kb0, kb0 + BK):
// i - j in [-dhi, -dlo], 0 <= i < Sq.
__host__ __device__ inline void bwd_query_tiles(int kb0, int BK, int Sq, int Sk, int dlo, int dhi, int BQ,
                                                int& qt_lo, int& qt_hi) {
  const int kmax = imin(kb0 + BK, Sk) - 1;
  const int i_lo = (int)lmax((int64_t)0, (int64_t)kb0 - dhi);
  const int i_hi = (int)lmin((int64_t)Sq, (int64_t)kmax - dlo + 1);
  qt_lo = i_lo / BQ;
  qt_hi = i_hi > i_lo ? (i_hi + BQ - 1) / BQ : qt_lo;
}

// dQ: work item (batch, kv-head, q-head in the group, first row m0) of
// workgroup `blk`, rows in blocks of BM (causal: longest rows first).
struct DqItem {
  int b, hkv, gq, m0;
};
__host__ __device__ inline DqItem bwd_dq_item(int blk, int B, int Hq, int Hkv, int G, int num_mblk, bool causal,
                                              int BM) {
  int w = xcd_remap(blk, B * Hq * num_mblk);
  DqItem it;
  it.gq = w % G;
  w /= G;
  const int mi = w % num_mblk;
  w /= num_mblk;
  it.hkv = w % Hkv;
  it.b = w / Hkv;
  it.m0 = (causal ? (num_mblk - 1 - mi) : mi) * BM;
  return it;
}
// Key tiles [t_lo, t_hi) of BN keys that rows [m0, m0 + BM) may see.
__host__ __device__ inline void bwd_key_tiles(int m0, int BM, int Sq, int Sk, int dlo, int dhi, int BN, int& t_lo,
                                              int& t_hi) {
  const int mlast = imin(m0 + BM, Sq) - 1;
  const int64_t lo = lmax((int64_t)0, (int64_t)m0 + dlo);
  const int64_t hi = lmin((int64_t)Sk, (int64_t)mlast + dhi + 1);
  t_lo = (int)(lo / BN);
  t_hi = hi > lo ? (int)((hi + BN - 1) / BN) : t_lo;
}

// ---- dropout keep map ---------------------------------------------------------
// The keep decisions of a dropout forward, one bit per (row i, key j) of
// each (batch, q-head) bh, stored so that the backward reads them instead of
// regenerating them.  Blocks of 32 rows x 32 keys, KM_NBI row blocks by
// KM_NBJ key blocks per bh, padded to whole 64-row and 128-key tiles so that
// every tile copy of the backward stays inside the map.  A block is 32
// uint32 words, word i % 32 holding row i; its bit 16h + 4q + e is key
// 8q + 4h + e of the block (kept = 1), h = 0, 1, q, e = 0..3: the order in
// which a lane pair of the kernels holds a row's 32 keys (lane half h,
// element 4q + e).  The blocks of one row block are consecutive in j.
__host__ __device__ inline int64_t keep_map_nbi(int64_t Sq) { return 2 * ((Sq + 63) / 64); }
__host__ __device__ inline int64_t keep_map_nbj(int64_t Sk) { return 4 * ((Sk + 127) / 128); }
// Word index of the first word of block (bi, bj) of bh.
__host__ __device__ inline int64_t keep_map_block(int64_t bh, int64_t bi, int64_t bj, int64_t nbi, int64_t nbj) {
  return ((bh * nbi + bi) * nbj + bj) * 32;
}

// ---- split-KV decode (attn_decode16) --------------------------------------
// Work item of workgroup `blk`: 16 packed rows (row group rg), one key chunk,
// (batch, kv-head) bh.
struct DecItem {
  int rg, split, bh;
};
__host__ __device__ inline DecItem dec_item(int blk, int RG, int n_splits) {
  DecItem it;
  it.rg = blk % RG;
  blk /= RG;
  it.split = blk % n_splits;
  it.bh = blk / n_splits;
  return it;
}
// Keys [c0, c1) of chunk `split`.
__host__ __device__ inline void dec_chunk(int klo, int khi, int chunk, int split, int& c0, int& c1) {
  c0 = klo + split * chunk;
  c1 = imin(khi, c0 + chunk);
}
// Partial (O, lse) slot of packed row r of (batch, kv-head) bh, chunk split.
__host__ __device__ inline int64_t dec_partial_index(int bh, int M, int r, int n_splits, int split) {
  return ((int64_t)bh * M + r) * n_splits + split;
}

}  // namespace trinix
