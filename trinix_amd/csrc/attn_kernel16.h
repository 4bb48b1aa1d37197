// bf16 / fp16 attention-forward kernel for gfx950 (MFMA 32x32x16).
//
// Semantics: reference trinix/kernels/attention_kernel.py:123-216 and
// :341-416 -- s = q.k*scale (+ -slope*|i-j|) (+ mask), -inf where j >= Sk,
// j > i (causal, top-left), or outside -wl <= j-i <= wr (window); online
// softmax in fp32; P rounded to the input dtype before the PV product;
// out = acc / l.  Dropout follows the eager path (trinix/layers/attention/
// base.py:394-397): softmax first, then dropout, then PV.
//
// Decomposition: a workgroup of NW wavefronts owns one (batch, q-head,
// 32*NW query rows); each wavefront owns 32 rows.  Per K/V tile of BN keys a
// wavefront computes S^T = K Q^T with keys on the MFMA rows and its queries
// on the columns, so each lane owns one query row (row max / sum: one
// lane^32 exchange).  O^T = V^T P^T takes P^T straight from the S^T
// registers as the B operand; the V^T A operand is read from the row-major V
// tile with the LDS transpose read ds_read_b64_tr_b16.
//
// Memory pipeline: K and V tiles go global -> LDS directly
// (global_load_lds_dwordx4, no staging registers) into two LDS buffers
// each; the loads of tile t+1 are in flight while tile t is computed, with
// one barrier per tile.  Within a tile the LDS operand reads run ahead of
// their MFMAs (explicit prefetch, pinned with sched_group_barrier).  LDS
// tiles are row-major with 16-byte units XOR-swizzled per row so the MFMA
// operand reads are bank-conflict free.
//
// Tiles split into "full" tiles (every (i, j) of the workgroup allowed: no
// per-element predicate) and "edge" tiles (causal diagonal, window borders,
// the Sk tail); each kind runs its own straight-line loop body.  Tiles a
// wavefront's rows cannot see at all are skipped by that wavefront.
//
// Softmax: scores stay in log2 units (scale * log2 e folded into one FMA
// before v_exp_f32); the running max is raised only when a tile's max
// exceeds it by more than TAU = 8 (then O and l are rescaled), so most tiles
// skip the O rescale; p <= 2^TAU is exact enough in fp32 and in the 16-bit P
// operand.  The row sum adds the rounded P that the PV product uses.
#pragma once
#include <climits>
#include <type_traits>

#include "attn_params.h"
#include "lds_tile.h"

namespace trinix {

// DROP: 0 no dropout, 1 dropout, 2 dropout that also writes the keep map
// (p.keep_map, index_map.h) for the backward.
template <class E, int D, int BN, int NW, int OCC, int KS, bool ALIBI, bool MASK, int DROP, bool QN>
// The head_dim 64 mask kernels are held to three wavefronts per SIMD (168
// VGPRs), except the one writing a keep map (it does not fit); the other
// shapes to OCC.
__global__ __launch_bounds__(NW * 64, (MASK && D == 64 && DROP != 2) ? 3 : OCC) void attn_fwd_mfma16(const FwdParams p) {
  // KS = 2 splits each 32-row group's keys between two wavefronts: wavefront
  // 2r + kp owns rows 32r..32r+31 and the tiles t_lo + KS*s + kp; the halves
  // merge through LDS at the end.  It halves the longest dependency chain of
  // small problems (few row blocks, long causal rows).  KS = 0 decides per
  // work item (p.row_items): the long causal row blocks run split, as two
  // items of NW*16 rows, the short ones whole (NW*32 rows), so that no item's
  // chain of tiles is much longer than the others'.
  static_assert(KS == 0 || KS == 1 || KS == 2, "key split");
  constexpr int KSL = KS ? KS : 2;  // tiles per LDS buffer
  constexpr int DS = D / 16;   // MFMA k-steps over head_dim (QK^T)
  constexpr int NB = BN / 32;  // 32-key blocks per tile
  constexpr int DB = D / 32;   // 32-wide head_dim blocks of O^T
  constexpr int UPR = D / 8;   // 16-byte units per row
  constexpr int TILE_UNITS = BN * UPR;
  constexpr int LPW = TILE_UNITS / (64 * NW);  // direct loads per wavefront per tile (K or V)
  constexpr float TAU = 8.f;
  static_assert(D % 64 == 0 && BN % 64 == 0 && TILE_UNITS % (64 * NW) == 0, "tile shape");

  // Four separate LDS objects (not one array indexed by parity) so that the
  // compiler can tell the buffer being read from the one an asynchronous
  // global->LDS load is filling, and does not wait for that load.
  // With a key split each buffer holds the step's two tiles (tile kp at
  // kp*BN*D).
  __shared__ __attribute__((aligned(1024))) uint16_t lds_k0[KSL * BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_k1[KSL * BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_v0[KSL * BN * D];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_v1[KSL * BN * D];
  // Tile t lives in buffer slot (t - t_lo) & 1 of K and of V.  `slot` is a
  // std::integral_constant in the full-tile loop (static buffer choice) and
  // an int in the edge loops.
  auto kbuf = [&](auto slot) __attribute__((always_inline)) -> uint16_t* {
    if constexpr (std::is_integral_v<decltype(slot)>) return slot ? lds_k1 : lds_k0;
    else return decltype(slot)::value ? lds_k1 : lds_k0;
  };
  auto vbuf = [&](auto slot) __attribute__((always_inline)) -> uint16_t* {
    if constexpr (std::is_integral_v<decltype(slot)>) return slot ? lds_v1 : lds_v0;
    else return decltype(slot)::value ? lds_v1 : lds_v0;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r = lane & 31, g = lane >> 5;

  // work item: (b, kv-head, m-block, q-head within the group).  Each XCD owns
  // whole KV-head groups, so the q-heads sharing a KV head run on one XCD and
  // share its L2.  Causal row blocks are dispatched longest first across all
  // the head groups of an XCD (when the groups split evenly over the 8 XCDs):
  // the long chains then start first and run alone on their CUs, and the
  // short blocks fill in behind them.
  // (index_map.h: fwd_item, fwd_row_block)
  const FwdItem wi =
      fwd_item((int)blockIdx.x, p.B, p.Hkv, p.G, p.num_mblk, p.total_work, p.causal != 0, p.has_window != 0);
  const int gq = wi.gq, mi = wi.mi, hkv = wi.hkv, b = wi.b;
  const int hq = hkv * p.G + gq;
  // ks: wavefronts per 32-row group (1 or 2); bm: rows of the work item
  const RowBlock rb = fwd_row_block(KS, NW, mi, p.causal != 0, p.num_mblk, KS == 0 ? (uint32_t)p.row_items[mi] : 0u);
  const int ks = rb.ks, m0 = rb.m0;
  const int bm = NW * 32 / ks;
  const int kp = wave % ks;  // key parity of this wavefront (key split)
  const int iw0 = m0 + (wave / ks) * 32;
  const int iwl = min(iw0 + 31, p.Sq - 1);
  const int i = iw0 + r;
  const int ic = min(i, p.Sq - 1);
  const bool wave_live = iw0 < p.Sq;

  // Key tiles the workgroup visits, and the sub-range of full tiles.
  const TileRange trange = fwd_tile_range(m0, bm, p.Sq, p.Sk, p.causal != 0, p.has_window != 0, p.wl, p.wr, BN);
  const int t_lo = trange.t_lo, t_hi = trange.t_hi, t_flo = trange.t_flo, t_fhi = trange.t_fhi;
  // Scores stay in the raw domain, s = q.k (+ bias / c), and the scale
  // c = scale * log2 e > 0 is applied in the FMA before the exp, so the max of
  // the raw scores is the max of the scaled ones.  A negative scale negates
  // the q operand instead (exact: the sign bits); a zero scale zeroes it and
  // uses c = 1 (the q.k term is dropped, the biases remain).
  const bool q_neg = p.scale_log2 < 0.f, q_zero = p.scale_log2 == 0.f;
  const float c = q_neg ? -p.scale_log2 : (q_zero ? 1.f : p.scale_log2);

  // Q row in registers: qr[ds] = q[i][ds*16 + g*8 .. +8].
  u32x4_t qr[DS];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + hq * p.q_sh + (int64_t)ic * p.q_ss;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qr[ds] = *(const u32x4_t*)(qrow + ds * 16 + g * 8);
    if (p.rope_cos) {
#pragma clang fp contract(off)
      // Fused RoPE (reference trinix/layers/embeddings/rope.py:111-118):
      // x*cos + rotate_half(x)*sin, each product and the sum rounded to the
      // input dtype as eager PyTorch evaluates it.  d and d + D/2 share
      // cos/sin and sit in the same lane (chunks ds and ds + DS/2).
      const uint16_t* crow = p.rope_cos + (int64_t)ic * p.rope_stride;
      const uint16_t* srow = p.rope_sin + (int64_t)ic * p.rope_stride;
#pragma unroll
      for (int ds = 0; ds < DS / 2; ++ds) {
        const u32x4_t cw = *(const u32x4_t*)(crow + ds * 16 + g * 8);
        const u32x4_t sw = *(const u32x4_t*)(srow + ds * 16 + g * 8);
        u32x4_t x1 = qr[ds], x2 = qr[ds + DS / 2];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float c0 = E::lo(cw[e]), c1 = E::hi(cw[e]);
          const float s0 = E::lo(sw[e]), s1 = E::hi(sw[e]);
          const float a0 = E::lo(x1[e]), a1 = E::hi(x1[e]);
          const float b0 = E::lo(x2[e]), b1 = E::hi(x2[e]);
          const float lo0 = round_to<E>(round_to<E>(a0 * c0) - round_to<E>(b0 * s0));
          const float lo1 = round_to<E>(round_to<E>(a1 * c1) - round_to<E>(b1 * s1));
          const float hi0 = round_to<E>(round_to<E>(b0 * c0) + round_to<E>(a0 * s0));
          const float hi1 = round_to<E>(round_to<E>(b1 * c1) + round_to<E>(a1 * s1));
          x1[e] = E::pack(lo0, lo1);
          x2[e] = E::pack(hi0, hi1);
        }
        qr[ds] = x1;
        qr[ds + DS / 2] = x2;
      }
    }
    if constexpr (QN) {
#pragma clang fp contract(off)
      // Fused qk-norm (RMSNorm over head_dim after RoPE, reference
      // trinix/layers/attention/grouped_query_attention.py:167-177) with
      // trinix_qk_norm's arithmetic, so q is bitwise the q it writes.  There,
      // lane c of a row sums chunks c and c + DS (8 elements each) and a
      // shuffle tree adds c^1, c^2, c^4, ...  Here chunk k of this lane is
      // chunk c = 2k + g: c^1 is the same k in the other half-wave, c^2m is
      // chunk k^m of this lane.  IEEE addition is commutative, so every
      // pairing adds the same two values and all lanes end with one sum.
      constexpr int NH = DS / 2;
      float part[NH];
#pragma unroll
      for (int k = 0; k < NH; ++k) {
        float ssq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float y1 = (e & 1) ? E::hi(qr[k][e / 2]) : E::lo(qr[k][e / 2]);
          const float y2 = (e & 1) ? E::hi(qr[k + NH][e / 2]) : E::lo(qr[k + NH][e / 2]);
          ssq += y1 * y1 + y2 * y2;
        }
        part[k] = ssq;
      }
#pragma unroll
      for (int k = 0; k < NH; ++k) part[k] += __shfl_xor(part[k], 32);
#pragma unroll
      for (int m = 1; m < NH; m <<= 1) {
        float nxt[NH];
#pragma unroll
        for (int k = 0; k < NH; ++k) nxt[k] = part[k] + part[k ^ m];
#pragma unroll
        for (int k = 0; k < NH; ++k) part[k] = nxt[k];
      }
      // mean(h^2): D is a power of two, so sum / D is exact scaling
      const float rn = rsqrtf(part[0] / (float)D + p.qn_eps);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const u32x4_t ww = *(const u32x4_t*)(p.qn_w + ds * 16 + g * 8);
        u32x4_t x = qr[ds];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float n0 = round_to<E>(E::lo(x[e]) * rn), n1 = round_to<E>(E::hi(x[e]) * rn);
          x[e] = E::pack(E::lo(ww[e]) * n0, E::hi(ww[e]) * n1);
        }
        qr[ds] = x;
      }
      // the q attended with, for a backward (one writer per row: the
      // fused norm runs without the key split)
      if (p.qn_out && i < p.Sq) {
        uint16_t* qo = p.qn_out + (((int64_t)b * p.Sq + i) * p.Hq + hq) * D;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) *(u32x4_t*)(qo + ds * 16 + g * 8) = qr[ds];
      }
    }
    if (q_neg)
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) qr[ds] ^= (u32x4_t){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    if (q_zero)
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) qr[ds] = (u32x4_t){};
  }

  f32x16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = (f32x16_t){};
  float m_run = -INFINITY, l_run = 0.f;
  // Allowed keys of this row: jlo <= j <= jhi (empty if jlo > jhi), from
  // j < Sk, causal j <= i and window -wl <= j - i <= wr (clamped to int32).
  int jlo = 0, jhi = p.Sk - 1;
  if (p.causal) jhi = min(jhi, i);
  if (p.has_window) {
    jlo = (int)max((int64_t)jlo, (int64_t)i - p.wl);
    jhi = (int)min((int64_t)jhi, (int64_t)i + p.wr);
  }
  const uint32_t jspan = jhi >= jlo ? (uint32_t)(jhi - jlo) : 0u;
  if (jhi < jlo) jlo = INT_MAX;  // no allowed key: (j - jlo) wraps past jspan for every j
  float slope_l2 = 0.f;
  if constexpr (ALIBI) slope_l2 = -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e;
  DropKey dkey{};
  if constexpr (DROP) dkey = drop_key(p);
  // ALiBi is folded into the score accumulator: S^T starts at bias / c
  // instead of 0, so s * c = q.k * c + bias and the softmax of a full tile is
  // the plain one (raw max, one FMA before the exp).
  const float alibi_seed_mul = ALIBI ? slope_l2 / c : 0.f;
  const char* mrow = nullptr;
  if constexpr (MASK) {
    const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
    mrow = (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)ic * p.mk_si) * esz;
  }

  // ---- direct global -> LDS tile loads --------------------------------
  // Load l of this wavefront fills LDS units [64*(wave*LPW + l), +64) of the
  // tile (one per lane); unit u holds key row u / UPR, physical unit u % UPR,
  // i.e. logical 16-byte unit (u % UPR) ^ swz(row) of that row.  A tile is
  // addressed as a wave-uniform base in SGPRs (the tile's first row) plus a
  // per-lane 32-bit byte offset (the host guarantees BN rows of K/V span
  // less than 2^31 bytes), so issuing a tile costs no vector arithmetic.
  // In a tile reaching past Sk (the last one when Sk % BN != 0) rows past
  // Sk are loaded from row Sk-1 (finite data): their scores are masked to
  // -inf and their P is 0, so they never contribute.
  const uint16_t* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  auto ld_row = [&](int l) __attribute__((always_inline)) { return tile_copy_row(wave, LPW, l, lane, UPR); };
  auto ld_unit_k = [&](int l) __attribute__((always_inline)) { return (lane % UPR) ^ swz_k<D>(ld_row(l)); };
  auto ld_unit_v = [&](int l) __attribute__((always_inline)) { return (lane % UPR) ^ swz_v<D>(ld_row(l)); };
  uint32_t ld_koff[LPW], ld_voff[LPW];
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    ld_koff[l] = tile_copy_offset((uint32_t)ld_row(l), p.k_ss, (uint32_t)ld_unit_k(l));
    ld_voff[l] = tile_copy_offset((uint32_t)ld_row(l), p.v_ss, (uint32_t)ld_unit_v(l));
  }
  const uint64_t kbase_s = uniform_ptr(kbase), vbase_s = uniform_ptr(vbase);
  const uint32_t wave_lds = __builtin_amdgcn_readfirstlane((uint32_t)(wave * LPW * 1024));
  auto load_tile = [&](bool is_k, uint64_t base_s, int64_t ss, const uint32_t* offs, uint16_t* lds_tile, int tile)
                       __attribute__((always_inline)) {
    const int n0 = tile * BN;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds_tile + wave_lds;
    const uint64_t gb = base_s + (uint64_t)n0 * (uint64_t)(ss * 2);
    if (n0 + BN <= p.Sk) {
#pragma unroll
      for (int l = 0; l < LPW; ++l) dma_16b_s(offs[l], gb, __builtin_amdgcn_readfirstlane(lds0 + l * 1024));
    } else {
      const int last = p.Sk - 1 - n0;  // >= 0: tiles start below Sk
#pragma unroll
      for (int l = 0; l < LPW; ++l) {
        const uint32_t row = (uint32_t)min(ld_row(l), last);
        const uint32_t unit = (uint32_t)(is_k ? ld_unit_k(l) : ld_unit_v(l));
        dma_16b_s(tile_copy_offset(row, ss, unit), gb, __builtin_amdgcn_readfirstlane(lds0 + l * 1024));
      }
    }
  };
  auto load_k = [&](uint16_t* lds_tile, int tile) __attribute__((always_inline)) {
    load_tile(true, kbase_s, p.k_ss, ld_koff, lds_tile, tile);
  };
  auto load_v = [&](uint16_t* lds_tile, int tile) __attribute__((always_inline)) {
    load_tile(false, vbase_s, p.v_ss, ld_voff, lds_tile, tile);
  };

  // ---- per-tile pieces ---------------------------------------------------
  // Block-map codes of this wavefront's 32-row block (one per 64-key column)
  // are fetched 64 columns at a time into one register, lane l holding column
  // bm_c0 + l, ahead of the tile wait that covers their latency; a tile reads
  // its codes with readlane.  (A load at the tile's use would wait for the
  // next tile's K/V loads as well: both count on the same vmcnt.)  At D = 256
  // (one wavefront per SIMD, every register in use) the codes and their
  // fetch would push the mask kernels into spilling, so there every tile
  // reads the mask per element instead.
  constexpr int NCB = BN / 64;  // block-map columns per tile
  const uint8_t* bm_row = nullptr;
  if constexpr (MASK && D <= 128)
    if (p.bmap && wave_live) bm_row = p.bmap + b * p.bm_sb + hq * p.bm_sh + (int64_t)(iw0 / 32) * p.bm_cols;
  uint32_t bm_codes = 0;
  int bm_c0 = 0;
  auto bm_fetch = [&](int col0) __attribute__((always_inline)) {
    bm_c0 = col0;
    const int col = col0 + lane;
    bm_codes = col < p.bm_cols ? bm_row[col] : 0u;
  };
  // -1: every block of the tile is -inf (skip); 0: all zero (no mask term);
  // 1: read the mask per element.
  auto mask_code = [&](int t) __attribute__((always_inline)) -> int {
    if (!bm_row) return 1;
    bool all_skip = true, any_other = false;
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int col = t * NCB + cb;
      if (col >= p.bm_cols) break;  // past the last block-map column
      const uint32_t code = (uint32_t)__builtin_amdgcn_readlane((int)bm_codes, col - bm_c0);
      all_skip = all_skip && code == 2;
      any_other = any_other || code != 0;
    }
    return all_skip ? -1 : (any_other ? 1 : 0);
  };
  // Seed of the S^T accumulators: bias / c of ALiBi (element (nb, vq*4 + e)
  // is key n0 + nb*32 + vq*8 + 4g + e of row i), else 0.
  // At D = 256 with a mask the seeds are added after the QK products instead
  // (add_alibi): a seeded accumulator keeps the seeds and the products in
  // separate registers for a moment, which that variant cannot afford.
  constexpr bool ALIBI_SEED = ALIBI && !(D == 256 && MASK);
  auto seed_scores = [&](int n0, f32x16_t(&s)[NB]) __attribute__((always_inline)) {
    if constexpr (ALIBI_SEED) {
      const float fi = (float)(i - n0 - 4 * g);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq)
#pragma unroll
          for (int e = 0; e < 4; ++e) s[nb][vq * 4 + e] = fabsf(fi - (float)(nb * 32 + vq * 8 + e)) * alibi_seed_mul;
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[nb] = (f32x16_t){};
    }
  };  auto add_alibi = [&](int n0, f32x16_t(&s)[NB]) __attribute__((always_inline)) {
    if constexpr (ALIBI && !ALIBI_SEED) {
      const float fi = (float)(i - n0 - 4 * g);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s[nb][vq * 4 + e] = __builtin_fmaf(fabsf(fi - (float)(nb * 32 + vq * 8 + e)), alibi_seed_mul, s[nb][vq * 4 + e]);
    }
  };


  // S^T = K Q^T for one tile (keys nb*32 + MFMA row, queries on columns).
  // K fragments are read KPF MFMAs ahead; the sched_group_barriers keep the
  // reads ahead of their MFMAs instead of letting each MFMA wait on its read.
  constexpr int NQK = NB * DS;
  // mask kernels (and D = 256, with 192 registers of Q and O) hold more live
  // values: shorter read-ahead
  constexpr int KPF = D == 256 ? (MASK ? 1 : 2) : (MASK ? (DROP ? 2 : 3) : 6);
  // Byte offset of K fragment (nb, ds) of this lane in a K tile: row
  // nb*32 + r, unit (2ds + g) ^ swz_k(r) (the swizzle depends only on r).  As
  // 16*((2ds) ^ (g ^ swz)) = 32*ds ^ 16*(g ^ swz) and the row offset has no
  // bits below bit 8, it is nb*32*D*2 + (k_lane ^ 32*ds).  The DS XOR values
  // are loop-invariant and live in registers; each read uses one directly,
  // with nb's row offset in the instruction's immediate.
  const uint32_t k_lane = (uint32_t)(r * D * 2 + 16 * (g ^ swz_k<D>(r)));
  auto qk = [&](const uint16_t* kt, int n0, f32x16_t(&s)[NB]) __attribute__((always_inline)) {
    auto kread = [&](int k) __attribute__((always_inline)) {
      const int nb = k / DS, ds = k % DS;
      const uint32_t off = k_lane ^ (uint32_t)(ds << 5);
      return *(const u32x4_t*)((const char*)kt + nb * 32 * D * 2 + off);
    };
    u32x4_t kf[NQK];
#pragma unroll
    for (int k = 0; k < KPF; ++k) kf[k] = kread(k);
    seed_scores(n0, s);
#pragma unroll
    for (int k = 0; k < NQK; ++k) {
      if (k + KPF < NQK) kf[k + KPF] = kread(k + KPF);
      s[k / DS] = E::mfma(kf[k], qr[k % DS], s[k / DS]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, KPF, 0);
#pragma unroll
    for (int k = 0; k < NQK; ++k) {
      if (k + KPF < NQK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    add_alibi(n0, s);
  };

  // O^T += V^T P^T: the A operand (8 keys of one head_dim row per lane) comes
  // from two transpose reads of the row-major V tile.  16-lane group G of the
  // wavefront covers head_dim d0 + 0..15 (d0 = db*32 + 16*(G&1)) for k-group
  // g = G>>1; lane s of the group addresses 4 consecutive d (d0 + 4*(s&3))
  // at key row kb + 4g + s/4 (+8 for the second read) and receives the 4
  // keys kb + 4g + 0..3 of head_dim d0 + s.
  const int tr_G = lane >> 4, tr_s = lane & 15;
  const int tr_g = tr_G >> 1, tr_dh = tr_G & 1;
  // Byte offset of this lane's first transpose read in a V tile, per 32-wide
  // head_dim block; the other reads add constants (key rows nb*32 + kk*16
  // and +8 keep the row swizzle).  The empty asm keeps each offset one opaque
  // value, so every read's address is (LDS buffer + offset + constant): the
  // compiler then attributes the read to its buffer and does not wait for
  // global->LDS loads in flight into the other buffer.
  int tr_off[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int row0 = tr_g * 4 + (tr_s >> 2);
    const int u = db * 4 + tr_dh * 2 + ((tr_s & 3) >> 1);
    tr_off[db] = (row0 * D + (u ^ swz_v<D>(row0)) * 8 + (tr_s & 1) * 4) * 2;
    asm volatile("" : "+v"(tr_off[db]));
  }
  auto vread = [&](const uint16_t* vt, int m) __attribute__((always_inline)) {
    const int db = m / (NB * 2), nb = (m / 2) % NB, kk = m % 2;
    const char* base = (const char*)vt + tr_off[db] + (nb * 32 + kk * 16) * D * 2;
    const s16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)base);
    const s16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(base + 8 * D * 2));
    const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo4), h2 = __builtin_bit_cast(u32x2_t, hi4);
    return (u32x4_t){l2[0], l2[1], h2[0], h2[1]};
  };
  constexpr int NPV = DB * NB * 2;
  constexpr int VPF = D == 256 ? (MASK ? 1 : 2) : (MASK ? (DROP ? 1 : 2) : 4);
  // vpre: the first VPF fragments, read ahead (before the softmax) by the caller.
  auto pv = [&](const uint16_t* vt, const u32x4_t(&pb)[NB][2], const u32x4_t(&vpre)[VPF]) __attribute__((always_inline)) {
    u32x4_t vf[NPV];
#pragma unroll
    for (int m = 0; m < VPF; ++m) vf[m] = vpre[m];
#pragma unroll
    for (int m = 0; m < NPV; ++m) {
      if (m + VPF < NPV) vf[m + VPF] = vread(vt, m + VPF);
      acc[m / (NB * 2)] = E::mfma(vf[m], pb[(m / 2) % NB][m % 2], acc[m / (NB * 2)]);
    }
#pragma unroll
    for (int m = 0; m < NPV; ++m) {
      if (m + VPF < NPV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  };
  auto vprefetch = [&](const uint16_t* vt, u32x4_t(&vpre)[VPF]) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < VPF; ++m) vpre[m] = vread(vt, m);
  };

  // Keep map (DROP == 2): a tile's keep bits (half g of row i's word of each
  // 32-key block, index_map.h) are stored at the start of the wavefront's
  // next tile, after its loads are issued, or after the last tile.  Stored at
  // once, the step's s_waitcnt at the next tile would wait for the stores to
  // complete as well (stores count on vmcnt too).
  [[maybe_unused]] uint32_t km_pend[NB];
  [[maybe_unused]] int km_n0 = -1;  // first key of the pending tile, or -1
  auto flush_keep = [&]() __attribute__((always_inline)) {
    if constexpr (DROP == 2) {
      if (km_n0 >= 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          ((uint16_t*)p.keep_map)[2 * (keep_map_block((int64_t)b * p.Hq + hq, iw0 >> 5, (km_n0 >> 5) + nb, p.km_nbi,
                                                      p.km_nbj) + r) + g] = (uint16_t)km_pend[nb];
        km_n0 = -1;
      }
    }
  };

  // Softmax update of one tile; writes P^T packed as the PV B operand.  All
  // in the raw-score domain: a tile that reads the mask adds mask * log2e / c
  // to its raw scores, an edge tile sets the scores it may not see to -inf;
  // the row max is taken on the raw scores and the scale folds into one FMA
  // before the exp.  ALiBi is in the scores already (seed_scores).
  auto softmax = [&](auto pred_c, auto mask_c, f32x16_t(&s)[NB], int n0, int mcode, u32x4_t(&pb)[NB][2])
                     __attribute__((always_inline)) {
    constexpr bool PRED = decltype(pred_c)::value;
    constexpr bool MASKC = decltype(mask_c)::value;
    if constexpr (MASKC) {
      if (mcode > 0) {
        const float mscale = kLog2e / c;  // mask in the raw-score domain
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int vq = 0; vq < 4; ++vq) {
            float mv[4];
            load_mask4(mrow, p.mask_dtype, n0 + nb * 32 + vq * 8 + g * 4, p.mk_sj, p.Sk - 1, mv);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[nb][vq * 4 + e] = __builtin_fmaf(mv[e], mscale, s[nb][vq * 4 + e]);
            // D = 256 (every register in use), D = 64 (held to 168 VGPRs)
            // or with dropout: one group of mask values in flight at a time,
            // or their loads are hoisted together and the kernel spills
            if constexpr (D == 256 || D == 64 || DROP) __builtin_amdgcn_sched_barrier(0);
          }
      }
    }
    if constexpr (PRED) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int j = n0 + nb * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          s[nb][v] = (uint32_t)(j - jlo) <= jspan ? s[nb][v] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[nb][v]);
    mx = xlane_max(mx) * c;  // raw max scaled (c > 0)
    // Lazy rescale: keep the running max unless this tile exceeds it by TAU.
    if (__builtin_expect(wave_any(mx > m_run + TAU), 0)) {
      const float m_new = fmaxf(m_run, mx);
      // a row that has seen no allowed key yet (m_new = -inf; its acc and l
      // are 0) keeps alpha finite instead of exp2(-inf - -inf) = NaN
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
      m_run = m_new;
    }
    {
      // a row that has seen no allowed key keeps -inf scores: exp2(-inf) = 0
      const float mneg = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[nb][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[nb][v], c, mneg));
    }
    if constexpr (DROP) {
      // l sums the probabilities before dropout (eager: softmax, then dropout)
      float rs = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) rs += s[nb][v];
      l_run += rs;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        uint32_t kw = 0;  // keep bits of this lane's 16 elements of the block (bit v: element v)
#pragma unroll
        for (int vp = 0; vp < 2; ++vp) {
          // 8-key groups vq = 2vp, 2vp + 1: one Philox call per lane pair
          float xa[4], xb[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xa[e] = s[nb][vp * 8 + e];
            xb[e] = s[nb][vp * 8 + 4 + e];
          }
          kw |= dropout_pair(xa, xb, dkey, b * p.Hq + hq, i, n0 + nb * 32 + vp * 16, g) << (vp * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[nb][vp * 8 + e] = xa[e];
            s[nb][vp * 8 + 4 + e] = xb[e];
          }
          // with a mask too, one Philox call at a time (interleaved calls
          // need more registers than the kernel has)
          if constexpr (MASK) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (DROP == 2) km_pend[nb] = kw;
      }
      if constexpr (DROP == 2) km_n0 = n0;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        pb[nb][kk] = (u32x4_t){E::pack(s[nb][kk * 8 + 0], s[nb][kk * 8 + 1]), E::pack(s[nb][kk * 8 + 2], s[nb][kk * 8 + 3]),
                               E::pack(s[nb][kk * 8 + 4], s[nb][kk * 8 + 5]), E::pack(s[nb][kk * 8 + 6], s[nb][kk * 8 + 7])};
    if constexpr (!DROP) {
      // Row sum of the rounded P the PV product uses, two elements per
      // v_dot2 (x.lo*1 + x.hi*1 + acc), two independent accumulators, the
      // first one seeded with the running sum.
      float r2[2] = {l_run, 0.f};
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int e = 0; e < 4; ++e) r2[e & 1] = E::dot2_ones(pb[nb][kk][e], r2[e & 1]);
      l_run = r2[0] + r2[1];
    }
  };

  // Whether tile `tile` has any allowed (i, j) for this wavefront's rows.
  auto tile_live = [&](int tile) __attribute__((always_inline)) -> bool {
    if (!wave_live) return false;
    const int n0 = tile * BN;
    if (p.causal && n0 > iwl) return false;
    if (p.has_window && ((int64_t)n0 - iwl > p.wr || (int64_t)n0 + BN - 1 - iw0 < -p.wl)) return false;
    return true;
  };

  // ---- main loop -----------------------------------------------------------
  // Step s covers tiles T = t_lo + ks*s .. T + ks - 1 (this wavefront's tile
  // is T + kp), held in buffer slot s & 1 of K and V.  Step s: wait for the
  // step's tiles; barrier (every wavefront done with step s-1, whose buffers
  // now take the loads of step s+1); S = K Q^T; softmax; O += V^T P.
  auto step = [&](auto pred_c, auto slot, int T) __attribute__((always_inline)) {
    auto other = [&]() {
      if constexpr (std::is_integral_v<decltype(slot)>) return 1 - slot;
      else return std::integral_constant<int, 1 - decltype(slot)::value>{};
    }();
    const int t = T + kp;
    if constexpr (MASK && D <= 128)
      if (bm_row && (t + 1) * NCB - bm_c0 > 64) bm_fetch(t * NCB);  // next 64 columns, before the wait
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's loads of the step's tiles landed
    __syncthreads();                // ... and every wavefront's; buffers of step s-1 are free
#pragma unroll
    for (int u = 0; u < ks; ++u)
      if (T + ks + u < t_hi) {
        load_k(kbuf(other) + u * BN * D, T + ks + u);
        load_v(vbuf(other) + u * BN * D, T + ks + u);
      }
    flush_keep();
    if (t < t_hi && tile_live(t)) {
      const int n0 = t * BN;
      uint16_t* kt = kbuf(slot) + kp * BN * D;
      uint16_t* vt = vbuf(slot) + kp * BN * D;
      // MFMA sections at raised priority: the other wavefront on this SIMD
      // fills the MFMA pipe gaps with its softmax VALU work.
      const int mcode = MASK ? mask_code(t) : 0;
      if (mcode >= 0) {
        f32x16_t sc[NB];
        u32x4_t vpre[VPF];
        __builtin_amdgcn_s_setprio(1);
        qk(kt, n0, sc);
        vprefetch(vt, vpre);  // V operand reads in flight during the softmax
        __builtin_amdgcn_s_setprio(0);
        u32x4_t pb[NB][2];
        softmax(pred_c, std::bool_constant<MASK>{}, sc, n0, mcode, pb);
        __builtin_amdgcn_s_setprio(1);
        pv(vt, pb, vpre);
        __builtin_amdgcn_s_setprio(0);
      }
    }
  };
  if constexpr (MASK && D <= 128)
    if (bm_row) bm_fetch((t_lo + kp) * NCB);
#pragma unroll
  for (int u = 0; u < ks; ++u)
    if (t_lo + u < t_hi) {
      load_k(kbuf(std::integral_constant<int, 0>{}) + u * BN * D, t_lo + u);
      load_v(vbuf(std::integral_constant<int, 0>{}) + u * BN * D, t_lo + u);
    }
  // Steps whose tiles are all full run the straight-line body, in pairs
  // starting at an even step so that their buffer slots are static (the full
  // range is trimmed to start at an even step and to an even length; trimmed
  // steps run the edge body, which is always exact).
  const int s_hi = (t_hi - t_lo + ks - 1) / ks;
  int s_flo = (t_flo - t_lo + ks - 1) / ks;
  int s_fhi = max(s_flo, (t_fhi - t_lo) / ks);
  if ((s_flo & 1) && s_flo < s_fhi) ++s_flo;
  s_fhi -= (s_fhi - s_flo) & 1;
  int si = 0;
  for (; si < s_flo; ++si) step(std::true_type{}, si & 1, t_lo + ks * si);
  for (; si < s_fhi; si += 2) {
    step(std::false_type{}, std::integral_constant<int, 0>{}, t_lo + ks * si);
    step(std::false_type{}, std::integral_constant<int, 1>{}, t_lo + ks * (si + 1));
  }
  for (; si < s_hi; ++si) step(std::true_type{}, si & 1, t_lo + ks * si);
  flush_keep();

  if (KS != 1 && ks == 2) {
    // Merge the two key halves of each row group: wavefront 2r+1 hands its
    // (m, l, O) to wavefront 2r through LDS (the K buffers are free once every
    // wavefront has passed the barrier).  Lane-for-lane: both hold the same
    // rows and head_dim columns.
    float* mo = (float*)lds_k0;  // [row group][DB*16][64 lanes]
    float* ml = (float*)lds_v0;  // [row group][2][64 lanes]
    const int rg = wave / 2;
    __syncthreads();
    if (kp == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) mo[((rg * DB + db) * 16 + v) * 64 + lane] = acc[db][v];
      ml[(rg * 2 + 0) * 64 + lane] = m_run;
      ml[(rg * 2 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (kp == 0) {
      const float m1 = ml[(rg * 2 + 0) * 64 + lane], l1 = ml[(rg * 2 + 1) * 64 + lane];
      const float m = fmaxf(m_run, m1);
      // a half that saw no allowed key has m = -inf and contributes 0
      const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m);
      const float a1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
      l_run = l_run * a0 + l1 * a1;
      m_run = m;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[db][v] = acc[db][v] * a0 + mo[((rg * DB + db) * 16 + v) * 64 + lane] * a1;
    }
  }

  // Epilogue: O = acc / l (NaN for rows with no allowed key, like the eager
  // softmax over an all -inf row), optional log-sum-exp.  The row and lane
  // indices are passed through empty asm so that the compiler forms the
  // output addresses here rather than keeping prologue values (64-bit row
  // offsets) live across the loop, where the mask / dropout / ALiBi
  // variants have no registers to spare.
  int ie = i, ge = g;
  asm volatile("" : "+v"(ie), "+v"(ge));
  const float l = xlane_sum(l_run);
  if (ie < p.Sq && kp == 0) {
    // with dropout, the 1/(1-p) of the kept weights (dropout_pair)
    const float inv = (DROP ? p.drop_scale : 1.f) / l;
    uint16_t* orow = p.o + b * p.o_sb + hq * p.o_sh + (int64_t)ie * p.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq) {
        const int d0 = db * 32 + vq * 8 + ge * 4;
        const u32x2_t w2 = {E::pack(acc[db][vq * 4 + 0] * inv, acc[db][vq * 4 + 1] * inv),
                            E::pack(acc[db][vq * 4 + 2] * inv, acc[db][vq * 4 + 3] * inv)};
        *(u32x2_t*)(orow + d0) = w2;
      }
    if (p.lse && ge == 0) p.lse[((int64_t)b * p.Hq + hq) * p.Sq + ie] = (m_run + __log2f(l)) * kLn2;
  }
}

// Launcher of one tile shape: every feature combination.
template <class E, int D, int BN, int NW, int OCC, int KS>
hipError_t launch_feat(const FwdParams& p, int feat, hipStream_t st) {
  const dim3 grid((unsigned)p.total_work), block(NW * 64);
  switch (feat) {
#define TRINIX_CASE(F)                                                                                          \
  case F:                                                                                                       \
    return launch_kernel(&attn_fwd_mfma16<E, D, BN, NW, OCC, KS, (F & kFeatAlibi) != 0, (F & kFeatMask) != 0,  \
                                          (F & kFeatKeepMap) ? 2 : ((F & kFeatDropout) ? 1 : 0),               \
                                          (F & kFeatQNorm) != 0>,                                              \
                         grid, block, 0, st, p);
    TRINIX_CASE(0)
    TRINIX_CASE(1)
    TRINIX_CASE(2)
    TRINIX_CASE(3)
    TRINIX_CASE(4)
    TRINIX_CASE(5)
    TRINIX_CASE(6)
    TRINIX_CASE(7)
    default:
      break;
  }
  // Dropout writing the keep map: head_dim 64 and 128 (the backward that
  // reads it)
  if constexpr (D <= 128) {
    switch (feat) {
      TRINIX_CASE((kFeatDropout | kFeatKeepMap))
      TRINIX_CASE((kFeatDropout | kFeatKeepMap | kFeatAlibi))
      TRINIX_CASE((kFeatDropout | kFeatKeepMap | kFeatMask))
      TRINIX_CASE((kFeatDropout | kFeatKeepMap | kFeatAlibi | kFeatMask))
      default:
        break;
    }
  }
  // The fused q RMSNorm is its own instantiation (the other kernels keep
  // their code unchanged): without and with ALiBi, one wavefront per row
  // group; the host rejects it with a mask or dropout.
  if constexpr (KS == 1) {
    switch (feat) {
      TRINIX_CASE((kFeatQNorm))
      TRINIX_CASE((kFeatQNorm | kFeatAlibi))
      default:
        break;
    }
  }
#undef TRINIX_CASE
  return hipErrorNotSupported;
}

// Launcher of a tile shape built only for calls without a mask or dropout
// (ALiBi and the fused q RMSNorm included): the 128-key tiles at D = 128,
// whose mask and dropout variants would spill.
template <class E, int D, int BN, int NW, int OCC, int KS>
hipError_t launch_feat_plain(const FwdParams& p, int feat, hipStream_t st) {
  const dim3 grid((unsigned)p.total_work), block(NW * 64);
  switch (feat) {
#define TRINIX_CASE(F)                                                                                          \
  case F:                                                                                                       \
    return launch_kernel(&attn_fwd_mfma16<E, D, BN, NW, OCC, KS, (F & kFeatAlibi) != 0, false, 0,             \
                                          (F & kFeatQNorm) != 0>,                                              \
                         grid, block, 0, st, p);
    TRINIX_CASE(0)
    TRINIX_CASE((kFeatAlibi))
    TRINIX_CASE((kFeatQNorm))
    TRINIX_CASE((kFeatQNorm | kFeatAlibi))
    default:
      break;
#undef TRINIX_CASE
  }
  return hipErrorNotSupported;
}

// Launcher of the per-item key split (KS = 0, D = 64): causal calls without
// a mask, dropout or the fused q norm, with or without ALiBi.
template <class E, int D>
hipError_t launch_feat_split(const FwdParams& p, int feat, hipStream_t st) {
  const dim3 grid((unsigned)p.total_work), block(4 * 64);
  if (feat == 0) return launch_kernel(&attn_fwd_mfma16<E, D, 64, 4, 2, 0, false, false, 0, false>, grid, block, 0, st, p);
  if (feat == kFeatAlibi)
    return launch_kernel(&attn_fwd_mfma16<E, D, 64, 4, 2, 0, true, false, 0, false>, grid, block, 0, st, p);
  return hipErrorNotSupported;
}

// Tile configs built per (dtype, D), every feature combination:
// (nw, occ, bn, ks) = (4, 2, 64, 1) for D <= 128; (4, 1, 64, 1) for D = 256,
// whose Q fragment (64 VGPRs) and O accumulator (128) need one wavefront per
// SIMD, and whose double-buffered K/V tiles take 128 KiB of LDS; and for D = 64
// also (4, 2, 64, 2), the key split for small grids (64 KiB of LDS: two
// tiles per buffer), and (4, 2, 64, 0), the key split per work item.  For D = 128 without a mask or dropout also (8, 2, 128,
// 1): 256 rows and 128-key tiles per workgroup (128 KiB of LDS, one
// workgroup per CU).
#define TRINIX_ATTN16_LAUNCHER(NAME, E, D)                                                                   \
  hipError_t NAME(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st) {                                \
    constexpr int kOcc = (D) == 256 ? 1 : 2;                                                               \
    if constexpr ((D) == 128)                                                                              \
      if (cfg.nw == 8 && cfg.bn == 128 && cfg.occ == 2 && cfg.ks == 1)                                     \
        return launch_feat_plain<E, D, 128, 8, 2, 1>(p, feat, st);                                         \
    if (cfg.bn != 64 || cfg.nw != 4 || cfg.occ != kOcc) return hipErrorNotSupported;                       \
    if (cfg.ks == 1) return launch_feat<E, D, 64, 4, kOcc, 1>(p, feat, st);                                \
    if constexpr ((D) == 64) {                                                                             \
      if (cfg.ks == 2) return launch_feat<E, D, 64, 4, kOcc, 2>(p, feat, st);                              \
      if (cfg.ks == 0) return launch_feat_split<E, D>(p, feat, st);                                        \
    }                                                                                                      \
    return hipErrorNotSupported;                                                                             \
  }

}  // namespace trinix
