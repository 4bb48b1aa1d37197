// Backward of the bf16/fp16 attention forward (head_dim 64/128), from the
// log-sum-exp the forward saves.  No counterpart in the reference: its
// Triton path returns a detached output (trinix/kernels/attention_kernel.py:
// 497-517); the gradients follow the eager path's softmax(scale*q k^T +
// bias + mask) v (trinix/layers/attention/base.py:347-400).
//
// With z = scale*q.k (+ ALiBi + mask), P = exp(z - lse), O = P V:
//   dV = P^T dO,  dP = dO V^T,  dZ = P * (dP - delta),  delta = rowsum(dO*O),
//   dK = scale * dZ^T Q,  dQ = scale * dZ K.
// Three launches, no atomics (deterministic):
//   bwd_delta  delta[b, h, i] = sum_d dO*O (fp32);
//   bwd_dkdv   one workgroup of 8 wavefronts per (batch, kv-head, 128
//              keys): per 32 keys one wavefront computes P and dV (K rows in
//              registers), a second one dP, dZ and dK (V rows in registers)
//              from the first one's P; both walk every q-head of the group
//              and every query tile of the band, so dK and dV of a KV head
//              are summed in registers (GQA included);
//   bwd_dq     one workgroup per (batch, q-head, 128 query rows), the
//              forward's shape: S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dZ^T;
//              at head_dim 128 without a mask on large grids, 256 rows and
//              128-key tiles per workgroup (dq_wide, as the forward).
// All products run on v_mfma_f32_32x32x16_{bf16,f16}; P and dZ are rounded to
// the input dtype for their products, as in the forward.  bwd_dkdv also takes
// dZ = P (dP - delta) from the rounded P (bwd_dq from the fp32 one).
#pragma once
#include <cfloat>
#include <climits>
#include <utility>

#include "attn_params.h"
#include "lds_tile.h"

namespace trinix {

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;  // (B, Hq, Sq), natural log
  float* delta;      // (B, Hq, Sq)
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh, do_sb, do_ss, do_sh;
  int64_t dq_sb, dq_ss, dq_sh, dk_sb, dk_ss, dk_sh, dv_sb, dv_ss, dv_sh;
  int B, Sq, Sk, Hq, Hkv, G;
  float scale, scale_log2;
  int causal, has_window;
  int64_t wl, wr;
  const float* alibi;
  int64_t al_sb, al_sh;
  const void* mask;
  int mask_dtype;
  int64_t mk_sb, mk_sh, mk_si, mk_sj;
  const uint8_t* bmap;
  int64_t bm_sb, bm_sh;
  int bm_cols;
  int num_kblk, num_mblk;  // 128-key blocks (dK/dV), 128- or 256-row blocks (dQ)
  int dq_wide;             // dQ in 256-row workgroups with 128-key tiles
  // dropout of the forward (common.h keep_field): same Philox stream
  int use_dropout;
  uint32_t drop_thresh;  // dropped when the 16-bit Philox field < drop_thresh
  float drop_scale;      // 1 / (1 - p)
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
  const uint64_t* drop_state;  // {seed, offset} in device memory, read in place of the four above; or null
  const uint32_t* keep_map;    // the forward's keep bits (index_map.h), read in place of Philox; or null
  int64_t km_nbi, km_nbj;      // its row / key blocks per (batch, q-head)
};

// Allowed (i, j): j - i in [dlo, dhi] (causal: j <= i; window: -wl <= j-i <= wr).
struct Band {
  int dlo, dhi;
  __device__ Band(const BwdParams& p) { band_offsets(p.causal != 0, p.has_window != 0, p.wl, p.wr, dlo, dhi); }
  __device__ bool ok(int i, int j) const { return j - i >= dlo && j - i <= dhi; }
};

// Allowed range [lo, lo + span] of one index as an unsigned interval test:
// (uint32_t)(x - lo) <= span is one subtract and one compare per element (an
// empty range gets lo = INT_MAX, which no x in [0, 2^30) passes).
struct Span {
  int lo;
  uint32_t span;
  __device__ Span(int64_t a, int64_t b) {
    if (b < a) {
      lo = INT_MAX;
      span = 0u;
    } else {
      lo = (int)a;
      span = (uint32_t)(b - a);
    }
  }
  __device__ bool ok(int x) const { return (uint32_t)(x - lo) <= span; }
};

// LDS operand reads of a row-major, D-wide 16-bit tile swizzled with
// swz_kt.  The per-lane parts of the addresses are computed once; each read
// adds its row-block offset as an immediate.  Adding a multiple of 16 rows
// leaves swz_kt unchanged (it depends on row bits 0-3), so:
//  * row read (A operand, row blk*32 + l%32, head_dim chunk ds):
//      byte offset blk*32*D*2 + (row_lane ^ 32*ds), as
//      16*((2ds + g) ^ swz) = 32*ds ^ 16*(g ^ swz) and the row part r*D*2
//      has no bits below bit 7;
//  * transpose read (A operand over 8 rows: rows t and t+8 of k-step kk of
//      sub-tile st, head_dim block db): (st*32 + kk*16)*D*2 + tr0[db] / tr1[db].
template <int D>
struct TileReader {
  static constexpr int DB = D / 32;
  uint32_t row_lane;
  uint32_t tr0[DB], tr1[DB];
  __device__ explicit TileReader(int lane) {
    const int r = lane & 31, g = lane >> 5;
    row_lane = (uint32_t)(r * D * 2 + 16 * (g ^ swz_kt<D>(r)));
    const int tr_G = lane >> 4, tr_s = lane & 15, tr_g = tr_G >> 1, tr_dh = tr_G & 1;
    const int row0 = tr_g * 4 + (tr_s >> 2), row1 = row0 + 8;
    const int c = tr_dh * 2 + ((tr_s & 3) >> 1), half = (tr_s & 1) * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      tr0[db] = (uint32_t)((row0 * D + (((db * 4) | c) ^ swz_kt<D>(row0)) * 8 + half) * 2);
      tr1[db] = (uint32_t)((row1 * D + (((db * 4) | c) ^ swz_kt<D>(row1)) * 8 + half) * 2);
    }
  }
  __device__ u32x4_t row(const uint16_t* tile, int blk, int ds) const {
    return *(const u32x4_t*)((const char*)tile + blk * 32 * D * 2 + (row_lane ^ (uint32_t)(ds << 5)));
  }
  __device__ u32x4_t tr(const uint16_t* tile, int st, int db, int kk) const {
    const char* base = (const char*)tile + (st * 32 + kk * 16) * D * 2;
    const s16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(base + tr0[db]));
    const s16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(base + tr1[db]));
    const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo4), h2 = __builtin_bit_cast(u32x2_t, hi4);
    return (u32x4_t){l2[0], l2[1], h2[0], h2[1]};
  }
};

// Dropout of the forward (common.h keep_field), regenerated: (row i, key j)
// is kept when 16-bit field j%8 of Philox(counter (j/8, i, b*Hq+h, off_lo),
// key (seed_lo ^ off_hi, seed_hi)) is at least drop_thresh.
//
// Lane q's value (q = 0..7 of each aligned 8-lane group) in every lane of
// the group: a quad broadcast of lane q % 4 (quad_perm [q,q,q,q] = q * 0x55)
// is right in q's own quad; the other quad takes it shifted by 4 lanes
// (row_shr:4 = 0x114 into banks 1 and 3 when q < 4, row_shl:4 = 0x104 into
// banks 0 and 2 when q >= 4).  DPP controls must be constants: q is a
// template argument.
template <int Q>
__device__ inline uint32_t bcast8(uint32_t x) {
  const int t = __builtin_amdgcn_mov_dpp((int)x, (Q & 3) * 0x55, 0xf, 0xf, false);
  return (uint32_t)__builtin_amdgcn_update_dpp(t, t, Q < 4 ? 0x114 : 0x104, 0xf, Q < 4 ? 0xa : 0x5, false);
}
// Bits e8 and 8 + e8 of lane q's `own`, q = 0..7, at result bits q and q + 8.
template <int... Q>
__device__ inline uint32_t gather_keep_bits(uint32_t own, int e8, std::integer_sequence<int, Q...>) {
  return ((((bcast8<Q>(own) >> e8) & 0x101u) << Q) | ...);
}

// keep_bits_of_key: for a lane that owns key j (lanes 8m'..8m'+7 of each
// half-wave hold 8 consecutive keys, 8-aligned; e8 = j % 8) and the 16 query
// rows r(v) = r0 + (v>>2)*8 + (v&3), v = 0..15, bit v of the result is set
// when (row r(v), j) is kept.  The forward draws one Philox call per (row, 8
// consecutive keys), so the eight lanes share every call: lane e8 makes the
// calls of rows v = e8 and e8 + 8 (one call per 8 elements, as in the
// forward) and the group hands out the keep bytes through DPP (bcast8).
__device__ inline uint32_t keep_bits_of_key(const DropKey& dkey, int bh, int j, int r0) {
  const int e8 = j & 7;
  uint32_t own = 0;  // bit 8h + k: row r(e8 + 8h), key 8*(j/8) + k
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int v = e8 + 8 * h;
    const u32x4_t c = {(uint32_t)(j >> 3), (uint32_t)(r0 + (v >> 2) * 8 + (v & 3)), (uint32_t)bh, dkey.off_lo};
    const u32x4_t w = Philox::run(c, dkey.k0, dkey.k1);
#pragma unroll
    for (int k = 0; k < 8; ++k) own |= (keep_field(w[k >> 1], k & 1, dkey.thresh) ? 1u : 0u) << (8 * h + k);
  }
  // rows v = q and q + 8 come from lane q of the group
  return gather_keep_bits(own, e8, std::make_integer_sequence<int, 8>{});
}

// x of lane l ^ S, within each 32-lane half (S = 1, 2: quad permutes; 4, 8:
// two row shifts into alternate banks; 16: v_permlane16_swap, which trades
// the odd 16-lane rows of its first operand with the even rows of its
// second, the partner's value then in the first result on odd rows).
template <int S>
__device__ inline uint32_t xor_lane(uint32_t x, int lane) {
  if constexpr (S == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xb1, 0xf, 0xf, false);  // [1,0,3,2]
  if constexpr (S == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4e, 0xf, 0xf, false);  // [2,3,0,1]
  if constexpr (S == 4 || S == 8) {
    // row_shl:S into the banks whose lane bit S is clear, row_shr:S into the others
    const int t = __builtin_amdgcn_update_dpp((int)x, (int)x, 0x100 | S, 0xf, S == 4 ? 0x5 : 0x3, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(t, (int)x, 0x110 | S, 0xf, S == 4 ? 0xa : 0xc, false);
  }
  if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  }
  return x;
}
// One stage of a bit transpose of a 32x32 block held a word per lane: lane
// index bit S trades places with word bit T.  Of lanes l and l ^ S, the one
// with lane bit S clear keeps its bits whose bit-T index is clear and takes
// the partner's such bits, moved up by T, into the others; the other lane
// keeps its bits with bit-T index set and takes the partner's moved down.
template <int S, int T>
__device__ inline uint32_t transpose_stage(uint32_t a, int lane) {
  constexpr uint32_t M = T == 16 ? 0x0000ffffu : T == 8 ? 0x00ff00ffu : T == 4 ? 0x0f0f0f0fu : T == 2 ? 0x33333333u : 0x55555555u;
  const uint32_t t = xor_lane<S>(a, lane);
  const bool up = (lane & S) != 0;
  const uint32_t y = __builtin_amdgcn_alignbit(t, t, up ? T : 32 - T);  // rotate right
  const uint32_t m = up ? ~M : M;
  return (a & m) | (y & ~m);
}
// Keep words of a 32x32 block, one row per lane (lane l: row l % 32, both
// lane halves alike), the row's keys in the keep map's order (bit
// 16h + 4q + e: key 8q + 4h + e).  Returns, for the lane's key l % 32, the
// rows in the same order: bit 16h + 4q + e for row 8q + 4h + e.  The five
// stages trade lane bits 4, 3, 2, 1, 0 with word bits 3, 2, 4, 1, 0, which
// turns the map's key order into the key index and the row index into that
// order.
__device__ inline uint32_t transpose_keep_block(uint32_t a, int lane) {
  a = transpose_stage<16, 8>(a, lane);
  a = transpose_stage<8, 4>(a, lane);
  a = transpose_stage<4, 16>(a, lane);
  a = transpose_stage<2, 2>(a, lane);
  return transpose_stage<1, 1>(a, lane);
}

// ---------------------------------------------------------------------------
// dK, dV: a two-stage pipeline over two wavefronts per 32-key group.  Lane l
// of either wavefront of group kg owns key j = kb0 + 32kg + l%32.  Per
// 32-query sub-tile, with the query rows on the MFMA rows (A operand: Q / dO
// rows read from LDS) and the keys on the columns (B operand: the lane's K /
// V row in registers):
//   stage A (waves 0..NG-1):   S = Q K^T, P = exp(scale*S + bias - lse),
//                              dV^T += dO^T P, and P (in the input dtype) to
//                              LDS;
//   stage B (waves NG..2NG-1): dP = dO V^T, dZ = P (dP - delta) with stage A's
//                              P, dK^T += Q^T dZ;
// stage B runs one item (one query tile of one q-head) behind stage A.  Wave
// w and w + NG share a SIMD (the 8 wavefronts of the workgroup go round-robin
// over its 4 SIMDs), so every SIMD holds one wavefront of each stage, 16
// MFMAs per sub-tile each, and one's softmax VALU work overlaps the other's
// MFMAs.  dO^T and Q^T come from LDS transpose reads.
// Q/dO/lse/delta tiles rotate through NSL = 3 LDS slots (stage A's item,
// stage B's item, the item being loaded) and P through 2; one barrier per
// item orders all of it.  The loop runs six steps per trip so that every slot
// index is a compile-time constant (LDS addresses as immediate offsets).
// With dropout (DROP = 1: regenerated from Philox; DROP = 2: the forward's
// keep map, whose words of the item's rows are copied to LDS with its tiles
// and transposed in registers, transpose_keep_block), stage A takes the keep
// bits of its sub-tile, dV^T += dO^T (keep ? P : 0), and hands the bits to
// stage B through LDS next to P; stage B takes dZ' = P (keep dP - delta
// (1-p)), the delta kernel having scaled delta = rowsum(dO*O) by 1-p.  The
// 1/(1-p) of Pd = keep P/(1-p) and of dZ = P (keep dP/(1-p) - delta) =
// dZ'/(1-p) is applied once per output element in the epilogue.
// ---------------------------------------------------------------------------
template <class E, int D, bool ALIBI, bool MASK, int DROP>
__global__ __launch_bounds__(512, 1) void attn_bwd_dkdv(const BwdParams p) {
  DropKey dkey{};
  if constexpr (DROP) dkey = drop_key(p);
  constexpr int NW = 8, NG = NW / 2, BK = NG * 32, BQ = 64, NSL = 3, NST = BQ / 32;
  constexpr int DS = D / 16, DB = D / 32, UPR = D / 8, TILE = BQ * D;
  constexpr int LPW = BQ * UPR / (64 * NW);  // 16-byte copies per wavefront per Q (or dO) tile
  constexpr int RPF = 4, TPF = 2;            // row / transpose operand reads issued ahead of their MFMA
  static_assert(LPW >= 1 && BQ * UPR % (64 * NW) == 0, "tile shape");

  __shared__ __attribute__((aligned(1024))) uint16_t lds_q[NSL * TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_o[NSL * TILE];
  __shared__ __attribute__((aligned(1024))) u32x4_t lds_p[2 * NG * NST * 2 * 64];
  __shared__ __attribute__((aligned(256))) float lds_l[NSL * BQ];
  __shared__ __attribute__((aligned(256))) float lds_d[NSL * BQ];
  __shared__ __attribute__((aligned(256))) uint32_t lds_m[DROP ? 2 * NG * NST * 64 : 1];  // keep bits
  // the item's rows of the keep map (slot, sub-tile st, key group kg, row): DROP == 2
  __shared__ __attribute__((aligned(256))) uint32_t lds_kw[DROP == 2 ? NSL * NST * NG * 32 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave % NG;
  const int g = lane >> 5;

  const KvItem wi = bwd_kv_item((int)blockIdx.x, p.B, p.Hkv, p.num_kblk, p.causal != 0);  // (index_map.h)
  const int kblk = wi.kblk, hkv = wi.hkv, b = wi.b;
  const int kb0 = kblk * BK;
  const int j0 = kb0 + kg * 32;
  const int j = j0 + (lane & 31);
  const int jc = min(j, p.Sk - 1);
  const Band band(p);
  // queries this lane's key may see: j - dhi <= i <= j - dlo, 0 <= i < Sq (none if j >= Sk)
  const Span qspan = j < p.Sk ? Span(max((int64_t)0, (int64_t)j - band.dhi), min((int64_t)p.Sq - 1, (int64_t)j - band.dlo))
                              : Span(1, 0);
  const float c = p.scale_log2;

  // Query range of the workgroup's keys [kb0, kb0 + BK): i - j in [-dhi, -dlo].
  int qt_lo, qt_hi;
  bwd_query_tiles(kb0, BK, p.Sq, p.Sk, band.dlo, band.dhi, BQ, qt_lo, qt_hi);
  const int nqt = qt_hi - qt_lo;
  const int n_items = nqt > 0 ? p.G * nqt : 0;  // item = (q-head of the group, query tile)

  // ---- tile copies: Q and dO rows (16-byte units, swizzled), lse and delta
  auto ld_row = [&](int l) __attribute__((always_inline)) { return tile_copy_row(wave, LPW, l, lane, UPR); };
  auto ld_unit = [&](int l) __attribute__((always_inline)) { return (lane % UPR) ^ swz_kt<D>(ld_row(l)); };
  const uint32_t wave_lds = __builtin_amdgcn_readfirstlane((uint32_t)(wave * LPW * 1024));
  auto load_rows = [&](const uint16_t* base, int64_t ss, uint16_t* lds_tile, int i0) __attribute__((always_inline)) {
    const uint64_t gb = uniform_ptr((const char*)base + (int64_t)i0 * ss * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds_tile + wave_lds;
    const int last = p.Sq - 1 - i0;  // rows past Sq load row Sq-1 (finite, masked out)
#pragma unroll
    for (int l = 0; l < LPW; ++l) {
      const uint32_t row = (uint32_t)min(ld_row(l), last);
      dma_16b_s(tile_copy_offset(row, ss, (uint32_t)ld_unit(l)), gb,
                __builtin_amdgcn_readfirstlane(lds0 + l * 1024));
    }
  };
  auto load_vec = [&](const float* base, float* lds_vec, int i0) __attribute__((always_inline)) {
    const uint64_t gb = uniform_ptr(base + i0);
    const uint32_t row = (uint32_t)min(lane, p.Sq - 1 - i0);
    dma_4b_s(row * 4u, gb, __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds_vec));
  };
  struct Item {
    int gh, qt;
  };
  // Wave 0 loads each item's lse into a register with the item's copies and
  // writes it to LDS, times log2 e, at the end of the step (before the wait
  // and barrier that publish the item).  A row with no allowed key has lse
  // -inf and every score -inf: the finite floor keeps exp2(score - lse2) at 0
  // instead of exp2(-inf + inf) = NaN.
  float lse_pend = 0.f;
  float* lse_dst = nullptr;
  auto write_lse = [&]() __attribute__((always_inline)) {
    if (wave == 0 && lse_dst) {
      *lse_dst = fmaxf(lse_pend * kLog2e, -0.5f * FLT_MAX);
      lse_dst = nullptr;
    }
  };
  auto next_item = [&](Item it) __attribute__((always_inline)) {
    return it.qt + 1 < qt_hi ? Item{it.gh, it.qt + 1} : Item{it.gh + 1, qt_lo};
  };
  auto load_item = [&](Item it, auto slot_c) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot_c)::value;
    const int hq = hkv * p.G + it.gh, i0 = it.qt * BQ;
    load_rows(p.q + b * p.q_sb + hq * p.q_sh, p.q_ss, lds_q + SL * TILE, i0);
    load_rows(p.dout + b * p.do_sb + hq * p.do_sh, p.do_ss, lds_o + SL * TILE, i0);
    const int64_t vo = ((int64_t)b * p.Hq + hq) * p.Sq;
    if (wave == 0) {
      // lse of the item's rows, written to LDS times log2 e by write_lse
      lse_pend = p.lse[vo + i0 + min(lane, p.Sq - 1 - i0)];
      lse_dst = lds_l + SL * BQ + lane;
    }
    if (wave == 1) load_vec(p.delta + vo, lds_d + SL * BQ, i0);
    if constexpr (DROP == 2) {
      // keep words of the item's two 32-row blocks and the workgroup's four
      // 32-key blocks: per row block 512 consecutive bytes, two copies of
      // 256 (waves 2..5, one each)
      if (wave >= 2 && wave < 6) {
        const int c = wave - 2, st = c >> 1;
        const uint64_t gb = uniform_ptr(p.keep_map + keep_map_block((int64_t)b * p.Hq + hq, it.qt * 2 + st, kblk * 4,
                                                                    p.km_nbi, p.km_nbj) + (c & 1) * 64);
        dma_4b_s((uint32_t)lane * 4u, gb,
                 __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(lds_kw + SL * NST * NG * 32 + c * 64)));
      }
    }
  };
  // Does sub-tile st of the item hold allowed pairs for this wavefront's keys
  // (band, bounds, block map)?  Both stages take the same decision, so stage
  // B reads P exactly where stage A wrote it.  `full`: no pair of the
  // sub-tile is outside the band or past Sq / Sk.
  auto sub_live = [&](Item it, int st, int& mcode, bool& full) __attribute__((always_inline)) {
    const int ia = it.qt * BQ + st * 32, ib = min(ia + 31, p.Sq - 1);
    if (ia >= p.Sq || j0 >= p.Sk) return false;
    const int jb = min(j0 + 31, p.Sk - 1);
    if (j0 - ib > band.dhi || jb - ia < band.dlo) return false;  // nothing allowed
    mcode = 1;
    if constexpr (MASK) {
      if (p.bmap) {
        const int hq = hkv * p.G + it.gh;
        const uint8_t code = p.bmap[b * p.bm_sb + hq * p.bm_sh + (int64_t)(ia / 32) * p.bm_cols + j0 / 64];
        if (code == 2) return false;
        mcode = code == 0 ? 0 : 1;
      }
    }
    full = ia + 31 < p.Sq && j0 + 31 < p.Sk && jb - ia <= band.dhi && j0 - ib >= band.dlo;
    return true;
  };

  const TileReader<D> tr(lane);
  // P of sub-tile st of P slot ps, k-step kk: the lane's 8 values, in the
  // register layout both stages share
  auto p_slot = [&](int ps, int st, int kk) __attribute__((always_inline)) {
    return lds_p + ((ps * NG + kg) * NST + st) * 2 * 64 + kk * 64 + lane;
  };
  // the lane's keep bits of sub-tile st of P slot ps (DROP)
  auto m_slot = [&](int ps, int st) __attribute__((always_inline)) {
    return lds_m + ((ps * NG + kg) * NST + st) * 64 + lane;
  };

  // One stage: operand rows, the step loop, the epilogue.  Both stages run
  // the same n_items + 1 steps and so the same barriers.
  auto run = [&](auto stage_c) __attribute__((always_inline)) {
    constexpr bool SB = decltype(stage_c)::value;  // stage B (dK)
    u32x4_t br[DS];                                 // the lane's K row (stage A) or V row (stage B)
    {
      const uint16_t* row = SB ? p.v + b * p.v_sb + hkv * p.v_sh + (int64_t)jc * p.v_ss
                               : p.k + b * p.k_sb + hkv * p.k_sh + (int64_t)jc * p.k_ss;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) br[ds] = *(const u32x4_t*)(row + ds * 16 + g * 8);
    }
    f32x16_t acc[DB];  // dV^T (stage A) or dK^T (stage B): lane row = key j, d = db*32 + vq*8 + 4g + e
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = (f32x16_t){};

    // S (stage A: Q rows) or dP (stage B: dO rows) of sub-tile st: DS
    // MFMAs whose A operands are read from LDS RPF MFMAs ahead, pinned with
    // sched_group_barrier.
    auto scores = [&](const uint16_t* rows, int st) __attribute__((always_inline)) {
      f32x16_t s = {};
      u32x4_t af[DS];
#pragma unroll
      for (int k = 0; k < RPF; ++k) af[k] = tr.row(rows, st, k);
#pragma unroll
      for (int k = 0; k < DS; ++k) {
        if (k + RPF < DS) af[k + RPF] = tr.row(rows, st, k + RPF);
        s = E::mfma(af[k], br[k], s);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, RPF, 0);
#pragma unroll
      for (int k = 0; k < DS; ++k) {
        if (k + RPF < DS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      return s;
    };
    // The first TPF transpose operands of `grad`, read before the softmax /
    // dZ VALU work so that their latency is hidden behind it.  The MFMA
    // phases run at wave priority 1 and the VALU phases at 0, so the SIMD
    // favours issuing the MFMAs of one stage while the other does VALU work.
    auto tpre = [&](const uint16_t* tt, int st, u32x4_t* t0) __attribute__((always_inline)) {
#pragma unroll
      for (int m = 0; m < TPF; ++m) t0[m] = tr.tr(tt, st, m / 2, m % 2);
    };
    // acc^T += T^T X for sub-tile st: T = dO (stage A) or Q (stage B) through
    // transpose reads, X = P or dZ from registers (k-step kk = m % 2).
    auto grad = [&](const uint16_t* tt, int st, const u32x4_t* xb, const u32x4_t* t0) __attribute__((always_inline)) {
      constexpr int NTR = 2 * DB;
      u32x4_t tf[NTR];
#pragma unroll
      for (int m = 0; m < TPF; ++m) tf[m] = t0[m];
#pragma unroll
      for (int m = 0; m < NTR; ++m) {
        if (m + TPF < NTR) tf[m + TPF] = tr.tr(tt, st, (m + TPF) / 2, (m + TPF) % 2);
        acc[m / 2] = E::mfma(tf[m], xb[m % 2], acc[m / 2]);
      }
#pragma unroll
      for (int m = 0; m < NTR; ++m) {
        if (m + TPF < NTR) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    };

    // element v of a lane's S / dP / P / dZ: query row st*32 + (v/4)*8 + 4g + v%4 of the item
    auto stage_a = [&](Item it, auto sl_c, auto ps_c) __attribute__((always_inline)) {
      constexpr int SL = decltype(sl_c)::value, PS = decltype(ps_c)::value;
      const int hq = hkv * p.G + it.gh, i0 = it.qt * BQ;
      float slope_l2 = 0.f;
      if constexpr (ALIBI) slope_l2 = -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e;
      const uint16_t* qt_lds = lds_q + SL * TILE;
      const uint16_t* ot_lds = lds_o + SL * TILE;
      const float* l_lds = lds_l + SL * BQ;
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        int mcode;
        bool full;
        if (!sub_live(it, st, mcode, full)) continue;
        __builtin_amdgcn_s_setprio(1);
        const f32x16_t s = scores(qt_lds, st);
        u32x4_t t0[TPF];
        tpre(ot_lds, st, t0);
        __builtin_amdgcn_s_setprio(0);
        const char* mrow = nullptr;
        if constexpr (MASK) {
          if (mcode > 0) {
            const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
            // the sub-tile's first row in 64 bits; its 32 rows then sit at
            // 32-bit offsets r * mk_si, r < 32 (the host bounds 31 * mk_si)
            mrow = (const char*)p.mask +
                   (b * p.mk_sb + hq * p.mk_sh + (int64_t)jc * p.mk_sj + (int64_t)(i0 + st * 32) * p.mk_si) * esz;
          }
        }
        float x[16];
        // |i - j| = |fj - (row offset in the sub-tile)| with fj = j - (first
        // row of the lane's group): one subtraction of an immediate and one
        // FMA per element (the distance is exact in fp32 below 2^24, as
        // (float)|i - j| is)
        const float fj = ALIBI ? (float)(j - (i0 + st * 32 + g * 4)) : 0.f;
        // scale * log2 e * S - lse * log2 e in one FMA per element (lse2: the
        // LDS copy, already times log2 e and floored)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const f32x4_t l4 = *(const f32x4_t*)(l_lds + st * 32 + vq * 8 + g * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) x[vq * 4 + e] = __builtin_fmaf(s[vq * 4 + e], c, -l4[e]);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if constexpr (ALIBI) x[v] = __builtin_fmaf(fabsf(fj - (float)((v >> 2) * 8 + (v & 3))), slope_l2, x[v]);
        if constexpr (MASK) {
          // rows vq*8 + 4g + 0..3 of the sub-tile: 4 consecutive rows per
          // load group, one dtype switch per group (rows past Sq read row
          // Sq-1; they are masked below).  A live sub-tile starts at a row
          // < Sq, so the last row's offset within it is in [0, 31].
          if (mcode > 0) {
            const int rlast = min(31, p.Sq - 1 - (i0 + st * 32));
#pragma unroll
            for (int vq = 0; vq < 4; ++vq) {
              float mv[4];
              load_mask4(mrow, p.mask_dtype, vq * 8 + g * 4, p.mk_si, rlast, mv);
#pragma unroll
              for (int e = 0; e < 4; ++e) x[vq * 4 + e] += mv[e] * kLog2e;
            }
          }
        }
        if (!full) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int i = i0 + st * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
            x[v] = qspan.ok(i) ? x[v] : -INFINITY;
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) x[v] = __builtin_amdgcn_exp2f(x[v]);
        u32x4_t pb[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          pb[kk] = (u32x4_t){E::pack(x[kk * 8 + 0], x[kk * 8 + 1]), E::pack(x[kk * 8 + 2], x[kk * 8 + 3]),
                             E::pack(x[kk * 8 + 4], x[kk * 8 + 5]), E::pack(x[kk * 8 + 6], x[kk * 8 + 7])};
          *p_slot(PS, st, kk) = pb[kk];
        }
        if constexpr (DROP) {
          // dV takes the dropped P of the forward's PV product.  Keep bits of
          // the lane's key, row r(v) at bit v: from the forward's keep map
          // (the block's row words, transposed), or regenerated
          uint32_t km;
          if constexpr (DROP == 2)
            km = transpose_keep_block(lds_kw[(SL * NST + st) * NG * 32 + kg * 32 + (lane & 31)], lane) >> (16 * g);
          else
            km = keep_bits_of_key(dkey, b * p.Hq + hq, j, i0 + st * 32 + g * 4);
          *m_slot(PS, st) = km;
#pragma unroll
          for (int v = 0; v < 16; ++v) x[v] = __uint_as_float(__float_as_uint(x[v]) & keep_word(km, v));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
            pb[kk] = (u32x4_t){E::pack(x[kk * 8 + 0], x[kk * 8 + 1]), E::pack(x[kk * 8 + 2], x[kk * 8 + 3]),
                               E::pack(x[kk * 8 + 4], x[kk * 8 + 5]), E::pack(x[kk * 8 + 6], x[kk * 8 + 7])};
        }
        __builtin_amdgcn_s_setprio(1);
        grad(ot_lds, st, pb, t0);
        __builtin_amdgcn_s_setprio(0);
      }
    };

    auto stage_b = [&](Item it, auto sl_c, auto ps_c) __attribute__((always_inline)) {
      constexpr int SL = decltype(sl_c)::value, PS = decltype(ps_c)::value;
      const uint16_t* qt_lds = lds_q + SL * TILE;
      const uint16_t* ot_lds = lds_o + SL * TILE;
      const float* d_lds = lds_d + SL * BQ;
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        int mcode;
        bool full;
        if (!sub_live(it, st, mcode, full)) continue;
        __builtin_amdgcn_s_setprio(1);
        const f32x16_t dp = scores(ot_lds, st);
        u32x4_t t0[TPF];
        tpre(qt_lds, st, t0);
        __builtin_amdgcn_s_setprio(0);
        u32x4_t zb[2];
        uint32_t km = 0;
        if constexpr (DROP) km = *m_slot(PS, st);
        // dP of the dropped P, without its 1/(1-p) (epilogue): keep ? dP : 0
        auto dpk = [&](int v) __attribute__((always_inline)) {
          if constexpr (DROP) return __uint_as_float(__float_as_uint(dp[v]) & keep_word(km, v));
          else return dp[v];
        };
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const u32x4_t pw = *p_slot(PS, st, kk);  // word w: elements kk*8 + 2w, kk*8 + 2w + 1
          float z[8];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int vq = kk * 2 + h;
            const f32x4_t d4 = *(const f32x4_t*)(d_lds + st * 32 + vq * 8 + g * 4);
            z[h * 4 + 0] = E::lo(pw[h * 2 + 0]) * (dpk(vq * 4 + 0) - d4[0]);
            z[h * 4 + 1] = E::hi(pw[h * 2 + 0]) * (dpk(vq * 4 + 1) - d4[1]);
            z[h * 4 + 2] = E::lo(pw[h * 2 + 1]) * (dpk(vq * 4 + 2) - d4[2]);
            z[h * 4 + 3] = E::hi(pw[h * 2 + 1]) * (dpk(vq * 4 + 3) - d4[3]);
          }
          zb[kk] = (u32x4_t){E::pack(z[0], z[1]), E::pack(z[2], z[3]), E::pack(z[4], z[5]), E::pack(z[6], z[7])};
        }
        __builtin_amdgcn_s_setprio(1);
        grad(qt_lds, st, zb, t0);
        __builtin_amdgcn_s_setprio(0);
      }
    };

    // Step s: stage A on item s (Q/dO slot s%3, P slot s%2), stage B on item
    // s - 1, item s + 1 loading into slot (s+1)%3.  The barrier at the top of
    // step s is where item s has landed, P of item s-1 is written, and slot
    // (s+1)%3 (last read in step s-1 by stage B) and P slot s%2 are free.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    if (n_items > 0) load_item(Item{0, qt_lo}, I0{});
    write_lse();
    Item ia{0, qt_lo}, ib{0, qt_lo};
    auto step = [&](auto sa_c, auto pa_c, int s) __attribute__((always_inline)) {
      constexpr int SA = decltype(sa_c)::value, PA = decltype(pa_c)::value;
      __builtin_amdgcn_s_waitcnt(0);  // this wavefront's copies and P writes landed
      __syncthreads();                // ... and every wavefront's
      const Item in = next_item(ia);
      if (s + 1 < n_items) load_item(in, std::integral_constant<int, (SA + 1) % NSL>{});
      if constexpr (!SB) {
        if (s < n_items) stage_a(ia, sa_c, pa_c);
        write_lse();
      } else {
        if (s > 0) stage_b(ib, std::integral_constant<int, (SA + NSL - 1) % NSL>{}, std::integral_constant<int, 1 - PA>{});
      }
      ib = ia;
      ia = in;
    };
    for (int s = 0; s <= n_items; s += 6) {
      step(I0{}, I0{}, s);
      if (s + 1 <= n_items) step(I1{}, I1{}, s + 1);
      if (s + 2 <= n_items) step(I2{}, I0{}, s + 2);
      if (s + 3 <= n_items) step(I0{}, I1{}, s + 3);
      if (s + 4 <= n_items) step(I1{}, I0{}, s + 4);
      if (s + 5 <= n_items) step(I2{}, I1{}, s + 5);
    }

    // ---- epilogue: dV, or dK = scale * dZ^T Q
    if (j < p.Sk) {
      uint16_t* row = SB ? p.dk + b * p.dk_sb + hkv * p.dk_sh + (int64_t)j * p.dk_ss
                         : p.dv + b * p.dv_sb + hkv * p.dv_sh + (int64_t)j * p.dv_ss;
      // with dropout the 1/(1-p) of Pd (dV) and of keep*dP (dK; delta comes
      // scaled by 1-p) is applied here, once per output element
      const float f = (SB ? p.scale : 1.f) * (DROP ? p.drop_scale : 1.f);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int d0 = db * 32 + vq * 8 + g * 4;
          *(u32x2_t*)(row + d0) = (u32x2_t){E::pack(acc[db][vq * 4 + 0] * f, acc[db][vq * 4 + 1] * f),
                                            E::pack(acc[db][vq * 4 + 2] * f, acc[db][vq * 4 + 3] * f)};
        }
    }
  };
  if (wave >= NG) run(std::true_type{});
  else run(std::false_type{});
}

// ---------------------------------------------------------------------------
// dQ.  The forward's decomposition: lane l of wavefront w owns query row
// i = m0 + 32w + l%32 (NW wavefronts, BN-key tiles: 4 and 64, or 8 and 128
// with dq_wide); per 32-key half of a tile S^T = K Q^T and dP^T = V dO^T (keys on
// the MFMA rows, A operands from the K / V tiles in LDS; B operands the
// lane's Q / dO rows in registers), dZ^T = P^T (dP^T - delta) in registers,
// dQ^T += K^T dZ^T with K^T from LDS transpose reads.  With dropout (DROP)
// dZ' = P (keep dP - delta (1-p)) (delta scaled by the delta kernel) and
// the 1/(1-p) of dZ = dZ'/(1-p) applied in the epilogue; the keep bits are
// drawn as the forward draws them (DROP = 1: the two lanes of a row share
// the calls of 8-key group pairs, philox_pair_words) or read from the
// forward's keep map (DROP = 2: each wavefront copies its rows' words of a
// key tile to LDS with the tile).
// ---------------------------------------------------------------------------
template <class E, int D, bool ALIBI, bool MASK, int DROP, int NW, int BN>
__global__ __launch_bounds__(NW * 64, 2) void attn_bwd_dq(const BwdParams p) {
  DropKey dkey{};
  if constexpr (DROP) dkey = drop_key(p);
  constexpr int BM = NW * 32;
  constexpr int DS = D / 16, DB = D / 32, NB = BN / 32, UPR = D / 8;
  constexpr int LPW = BN * UPR / (64 * NW);

  __shared__ __attribute__((aligned(1024))) uint16_t lds_k0[BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_k1[BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_v0[BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_v1[BN * D];
  // keep words of the tile's rows (slot, wavefront, 32-key block, row): DROP == 2
  __shared__ __attribute__((aligned(256))) uint32_t lds_kq[DROP == 2 ? 2 * NW * NB * 32 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, g = lane >> 5;

  // (index_map.h; causal: longest rows first)
  const DqItem wi = bwd_dq_item((int)blockIdx.x, p.B, p.Hq, p.Hkv, p.G, p.num_mblk, p.causal != 0, BM);
  const int gq = wi.gq, hkv = wi.hkv, b = wi.b, m0 = wi.m0;
  const int hq = hkv * p.G + gq;
  const int iw0 = m0 + wave * 32;
  const int i = iw0 + r;
  const int ic = min(i, p.Sq - 1);
  const Band band(p);
  // keys this lane's row may see: i + dlo <= j <= i + dhi, 0 <= j < Sk (none if i >= Sq)
  const Span kspan = i < p.Sq ? Span(max((int64_t)0, (int64_t)i + band.dlo), min((int64_t)p.Sk - 1, (int64_t)i + band.dhi))
                              : Span(1, 0);
  const float c = p.scale_log2;

  u32x4_t qr[DS], dor[DS];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + hq * p.q_sh + (int64_t)ic * p.q_ss;
    const uint16_t* orow = p.dout + b * p.do_sb + hq * p.do_sh + (int64_t)ic * p.do_ss;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qr[ds] = *(const u32x4_t*)(qrow + ds * 16 + g * 8);
      dor[ds] = *(const u32x4_t*)(orow + ds * 16 + g * 8);
    }
  }
  const int64_t vo = ((int64_t)b * p.Hq + hq) * p.Sq + ic;
  // a row with no allowed key has lse -inf and every score -inf: a finite
  // floor keeps exp2(score - lse2) at 0 instead of exp2(-inf + inf) = NaN
  const float lse2 = fmaxf(p.lse[vo] * kLog2e, -FLT_MAX);
  const float dlt = p.delta[vo];
  float slope_l2 = 0.f;
  if constexpr (ALIBI) slope_l2 = -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e;
  const char* mrow = nullptr;
  if constexpr (MASK) {
    const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
    mrow = (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)ic * p.mk_si) * esz;
  }
  f32x16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = (f32x16_t){};

  // key tiles of the band of rows [m0, m0 + BM): j - i in [dlo, dhi]
  int t_lo, t_hi;
  bwd_key_tiles(m0, BM, p.Sq, p.Sk, band.dlo, band.dhi, BN, t_lo, t_hi);

  const uint16_t* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  auto ld_row = [&](int l) __attribute__((always_inline)) { return tile_copy_row(wave, LPW, l, lane, UPR); };
  auto ld_unit = [&](int l) __attribute__((always_inline)) { return (lane % UPR) ^ swz_kt<D>(ld_row(l)); };
  const uint32_t wave_lds = __builtin_amdgcn_readfirstlane((uint32_t)(wave * LPW * 1024));
  auto load_rows = [&](const uint16_t* base, int64_t ss, uint16_t* lds_tile, int tile) __attribute__((always_inline)) {
    const int n0 = tile * BN;
    const uint64_t gb = uniform_ptr((const char*)base + (int64_t)n0 * ss * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds_tile + wave_lds;
    const int last = p.Sk - 1 - n0;
#pragma unroll
    for (int l = 0; l < LPW; ++l) {
      const uint32_t row = (uint32_t)min(ld_row(l), last);
      dma_16b_s(tile_copy_offset(row, ss, (uint32_t)ld_unit(l)), gb,
                __builtin_amdgcn_readfirstlane(lds0 + l * 1024));
    }
  };
  const TileReader<D> rd(lane);

  // `edge` is a runtime flag and only the masking of the scores branches on
  // it (two instantiated copies of the dQ MFMAs cost 64 accumulator moves at
  // every join).
  // Keep words of this wavefront's 32 rows for tile t: the tile's NB blocks
  // of 128 bytes are consecutive in the map, 256 bytes per copy.
  auto load_keep = [&](uint32_t* slot_words, int t) __attribute__((always_inline)) {
    if constexpr (DROP == 2) {
      if (iw0 < p.Sq) {
#pragma unroll
        for (int c = 0; c < NB / 2; ++c) {
          const uint64_t gb = uniform_ptr(p.keep_map + keep_map_block((int64_t)b * p.Hq + hq, iw0 >> 5, (int64_t)t * NB,
                                                                      p.km_nbi, p.km_nbj) + c * 64);
          dma_4b_s((uint32_t)lane * 4u, gb,
                   __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(slot_words + wave * NB * 32 + c * 64)));
        }
      }
    }
  };

  auto tile_body = [&](bool edge, const uint16_t* kt, const uint16_t* vt, const uint32_t* kq, int t)
                       __attribute__((always_inline)) {
    const int n0 = t * BN;
    int mcode = 1;
    if constexpr (MASK) {
      if (p.bmap) {
        const uint8_t code = p.bmap[b * p.bm_sb + hq * p.bm_sh + (int64_t)(iw0 / 32) * p.bm_cols + n0 / 64];
        if (code == 2) return;
        mcode = code == 0 ? 0 : 1;
      }
    }
    // One 32-key half at a time (S, dP, dZ, then its dQ products): only one
    // pair of 32x32 score tiles is live, and with the operand reads pinned
    // PF MFMAs ahead (sched_group_barrier: 0x100 LDS read, 0x008 MFMA) the
    // kernel fits the 256 registers of two wavefronts per SIMD.
    constexpr int PF = ALIBI ? 2 : 4;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x16_t s = (f32x16_t){}, dp = (f32x16_t){};
      {
        auto kvread = [&](int k) __attribute__((always_inline)) {
          return k < DS ? rd.row(kt, nb, k) : rd.row(vt, nb, k - DS);
        };
        u32x4_t f[2 * DS];
#pragma unroll
        for (int k = 0; k < PF; ++k) f[k] = kvread(k);
#pragma unroll
        for (int k = 0; k < 2 * DS; ++k) {
          if (k + PF < 2 * DS) f[k + PF] = kvread(k + PF);
          if (k < DS) s = E::mfma(f[k], qr[k], s);
          else dp = E::mfma(f[k], dor[k - DS], dp);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
        for (int k = 0; k < 2 * DS; ++k) {
          if (k + PF < 2 * DS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      }
      float x[16];
      // |i - j| = |fi - (key offset in the block)| with fi = i - n0 - nb*32 - 4g
      // per tile: the per-element offsets are immediates, so no per-element
      // value is kept live across tiles
      const float fi = (float)(i - n0 - nb * 32 - 4 * g);
      // scale * log2 e * S^T - lse * log2 e in one FMA per element
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        x[v] = __builtin_fmaf(s[v], c, -lse2);
        if constexpr (ALIBI) x[v] += slope_l2 * fabsf(fi - (float)((v >> 2) * 8 + (v & 3)));
      }
      if constexpr (MASK) {
        // keys vq*8 + 4g + 0..3 of the 32-key block: one dtype switch per 4
        // consecutive keys (keys past Sk read key Sk-1; they are masked below)
        if (mcode > 0) {
#pragma unroll
          for (int vq = 0; vq < 4; ++vq) {
            float mv[4];
            load_mask4(mrow, p.mask_dtype, n0 + nb * 32 + vq * 8 + g * 4, p.mk_sj, p.Sk - 1, mv);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[vq * 4 + e] += mv[e] * kLog2e;
          }
        }
      }
      if (edge) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int jj = n0 + nb * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          x[v] = kspan.ok(jj) ? x[v] : -INFINITY;
        }
      }
      u32x4_t zb[2];
      {
        float z[16];
        if constexpr (DROP == 2) {
          // keep bits of the row's 16 elements of the block (bit v: element v,
          // key (v/4)*8 + 4g + v%4): half g of row i's word of the forward's
          // keep map
          const uint32_t km = kq[wave * NB * 32 + nb * 32 + r] >> (16 * g);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float dpk = __uint_as_float(__float_as_uint(dp[v]) & keep_word(km, v));
            z[v] = __builtin_amdgcn_exp2f(x[v]) * (dpk - dlt);
          }
        } else if constexpr (DROP && ALIBI && MASK && D == 128) {
          // every register in use: each lane makes the call of its own 8-key
          // group and keeps its 4 fields (4g..4g+3), one group at a time
#pragma unroll
          for (int vq = 0; vq < 4; ++vq) {
            const u32x4_t c = {(uint32_t)((n0 + nb * 32 + vq * 8) >> 3), (uint32_t)i, (uint32_t)(b * p.Hq + hq),
                               dkey.off_lo};
            const u32x4_t w = Philox::run(c, dkey.k0, dkey.k1);
            const uint32_t w0 = g ? w[2] : w[0], w1 = g ? w[3] : w[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float dpk = keep_field(e < 2 ? w0 : w1, e & 1, dkey.thresh) ? dp[vq * 4 + e] : 0.f;
              z[vq * 4 + e] = __builtin_amdgcn_exp2f(x[vq * 4 + e]) * (dpk - dlt);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        } else if constexpr (DROP) {
#pragma unroll
          for (int vp = 0; vp < 2; ++vp) {  // 8-key groups vq = 2vp, 2vp + 1: one call per lane pair
            uint32_t wq[2][2];
            philox_pair_words((uint32_t)((n0 + nb * 32 + vp * 16) >> 3), (uint32_t)i, (uint32_t)(b * p.Hq + hq),
                              dkey.off_lo, dkey.k0, dkey.k1, g, wq[0], wq[1]);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int v = (vp * 2 + h) * 4 + e;
                const float dpk = keep_field(wq[h][e >> 1], e & 1, dkey.thresh) ? dp[v] : 0.f;
                z[v] = __builtin_amdgcn_exp2f(x[v]) * (dpk - dlt);
              }
          }
        } else {
#pragma unroll
          for (int v = 0; v < 16; ++v) z[v] = __builtin_amdgcn_exp2f(x[v]) * (dp[v] - dlt);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          zb[kk] = (u32x4_t){E::pack(z[kk * 8 + 0], z[kk * 8 + 1]), E::pack(z[kk * 8 + 2], z[kk * 8 + 3]),
                             E::pack(z[kk * 8 + 4], z[kk * 8 + 5]), E::pack(z[kk * 8 + 6], z[kk * 8 + 7])};
      }
      {
        constexpr int NM = DB * 2;
        u32x4_t f[NM];
#pragma unroll
        for (int m = 0; m < PF; ++m) f[m] = rd.tr(kt, nb, m / 2, m % 2);
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          if (m + PF < NM) f[m + PF] = rd.tr(kt, nb, (m + PF) / 2, (m + PF) % 2);
          acc[m / 2] = E::mfma(f[m], zb[m % 2], acc[m / 2]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          if (m + PF < NM) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      }
    }
  };

  if (t_lo < t_hi) {
    load_rows(kbase, p.k_ss, lds_k0, t_lo);
    load_rows(vbase, p.v_ss, lds_v0, t_lo);
    load_keep(lds_kq, t_lo);
  }
  const bool wave_live = iw0 < p.Sq;
  auto step = [&](auto slot_c, int t) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot_c)::value;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 1 < t_hi) {
      load_rows(kbase, p.k_ss, SL ? lds_k0 : lds_k1, t + 1);
      load_rows(vbase, p.v_ss, SL ? lds_v0 : lds_v1, t + 1);
      load_keep(lds_kq + (1 - SL) * NW * NB * 32, t + 1);
    }
    const uint16_t* kt = SL ? lds_k1 : lds_k0;
    const uint16_t* vt = SL ? lds_v1 : lds_v0;
    const int n0 = t * BN;
    const int iwl = min(iw0 + 31, p.Sq - 1);
    const int nl = min(n0 + BN, p.Sk) - 1;
    if (!wave_live || n0 - iwl > band.dhi || nl - iw0 < band.dlo) return;  // no allowed pair
    const bool full = iw0 + 31 < p.Sq && n0 + BN <= p.Sk && nl - iw0 <= band.dhi && n0 - iwl >= band.dlo;
    tile_body(!full, kt, vt, lds_kq + SL * NW * NB * 32, t);
  };
  int t = t_lo;
  for (; t + 1 < t_hi; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    step(std::integral_constant<int, 1>{}, t + 1);
  }
  if (t < t_hi) step(std::integral_constant<int, 0>{}, t);

  if (i < p.Sq) {
    uint16_t* qrow = p.dq + b * p.dq_sb + hq * p.dq_sh + (int64_t)i * p.dq_ss;
    // with dropout the 1/(1-p) of keep*dP (delta comes scaled by 1-p) is
    // applied here, once per output element
    const float f = DROP ? p.scale * p.drop_scale : p.scale;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq) {
        const int d0 = db * 32 + vq * 8 + g * 4;
        *(u32x2_t*)(qrow + d0) = (u32x2_t){E::pack(acc[db][vq * 4 + 0] * f, acc[db][vq * 4 + 1] * f),
                                           E::pack(acc[db][vq * 4 + 2] * f, acc[db][vq * 4 + 3] * f)};
      }
  }
}

// Launch of both gradient kernels for one (dtype, D); feat = kFeatAlibi |
// kFeatMask | kFeatDropout.
// Launch of both gradient kernels of one feature set; DROP as in the
// kernels (0 none, 1 regenerated keep mask, 2 the forward's keep map).
template <class E, int D, bool A, bool M, int DROP>
hipError_t launch_bwd_pair(const BwdParams& p, hipStream_t st) {
  const dim3 g_kv((unsigned)(p.B * p.Hkv * p.num_kblk)), g_q((unsigned)(p.B * p.Hq * p.num_mblk)), blk(256),
      blk_kv(512);
  const hipError_t e = launch_kernel(&attn_bwd_dkdv<E, D, A, M, DROP>, g_kv, blk_kv, 0, st, p);
  if (e != hipSuccess) return e;
  if constexpr (D == 128 && !M)
    if (p.dq_wide) return launch_kernel(&attn_bwd_dq<E, D, A, M, DROP, 8, 128>, g_q, blk_kv, 0, st, p);
  return launch_kernel(&attn_bwd_dq<E, D, A, M, DROP, 4, 64>, g_q, blk, 0, st, p);
}

// Launch of both gradient kernels for one (dtype, D); feat = kFeatAlibi |
// kFeatMask | kFeatDropout (with p.keep_map: the map-reading variants).
template <class E, int D>
hipError_t launch_bwd(const BwdParams& p, int feat, hipStream_t st) {
  switch (feat & 7) {
#define TRINIX_BWD_CASE(F)                                                                                \
  case F:                                                                                                 \
  {                                                                                                       \
    constexpr bool A = (F & kFeatAlibi) != 0, M = (F & kFeatMask) != 0, DR = (F & kFeatDropout) != 0;     \
    if constexpr (DR) {                                                                                   \
      if (p.keep_map) return launch_bwd_pair<E, D, A, M, 2>(p, st);                                       \
      return launch_bwd_pair<E, D, A, M, 1>(p, st);                                                       \
    }                                                                                                     \
    return launch_bwd_pair<E, D, A, M, 0>(p, st);                                                         \
  }
    TRINIX_BWD_CASE(0)
    TRINIX_BWD_CASE(1)
    TRINIX_BWD_CASE(2)
    TRINIX_BWD_CASE(3)
    TRINIX_BWD_CASE(4)
    TRINIX_BWD_CASE(5)
    TRINIX_BWD_CASE(6)
    TRINIX_BWD_CASE(7)
#undef TRINIX_BWD_CASE
  }
  return hipErrorNotSupported;
}

#define TRINIX_ATTN_BWD16_LAUNCHER(NAME, E, D) \
  hipError_t NAME(const BwdParams& p, int feat, hipStream_t st) { return launch_bwd<E, D>(p, feat, st); }

hipError_t launch_bwd16_bf16_d64(const BwdParams& p, int feat, hipStream_t st);
hipError_t launch_bwd16_bf16_d128(const BwdParams& p, int feat, hipStream_t st);
hipError_t launch_bwd16_f16_d64(const BwdParams& p, int feat, hipStream_t st);
hipError_t launch_bwd16_f16_d128(const BwdParams& p, int feat, hipStream_t st);

// The generic backward (attn_bwd_generic.hip): fp32 products, any dtype
// (TRINIX_F32 / F16 / BF16), head_dim 64, 128 or 256, dropout, ALiBi and
// mask read per element.  Launches its own delta pre-pass.
hipError_t launch_bwd_generic(const BwdParams& p, int dtype, int D, hipStream_t st);
// Whether the generic kernels' grids fit 2^31 workgroups.
bool bwd_generic_fits(const BwdParams& p);

}  // namespace trinix
