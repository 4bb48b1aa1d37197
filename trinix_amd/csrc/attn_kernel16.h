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
// NW*32*QB query rows); each wavefront owns QB blocks of 32 rows.  Per K/V
// tile of BN keys a wavefront computes S^T = K Q^T with keys on the MFMA rows
// and its queries on the columns, so each lane owns one query row of a block
// (row max / sum: one lane^32 exchange).  O^T = V^T P^T takes P^T straight
// from the S^T registers as the B operand; V sits transposed in LDS for the
// A operand.  K/V fragments read from LDS are reused for all QB blocks.
// K/V tiles are double-buffered in LDS: the global loads of tile t+1 are in
// flight while tile t is computed, with one barrier per tile.
//
// Tiles split into "full" tiles (every (i, j) of the workgroup allowed: no
// per-element predicate) and "edge" tiles (causal diagonal, window borders,
// the Sk tail); each kind runs its own straight-line loop body.  Edge tiles
// that a wavefront's rows cannot see at all are skipped by that wavefront.
//
// Softmax details: scores stay in log2 units (scale * log2 e folded into one
// FMA before v_exp_f32); the running max is only raised when the new tile
// max exceeds it by more than TAU = 8 (then O and l are rescaled), so most
// tiles skip the O rescale; p <= 2^TAU is exact enough in fp32 and in the
// 16-bit P operand.
#pragma once
#include <type_traits>

#include "attn_params.h"

namespace trinix {

template <class E, int D, int BN, int NW, int QB, bool ALIBI, bool MASK, bool DROP>
__global__ __launch_bounds__(NW * 64, QB == 1 ? 2 : 1) void attn_fwd_mfma16(const FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr int WR = 32 * QB;  // query rows per wavefront
  constexpr int BM = NW * WR;  // query rows per workgroup
  constexpr int DS = D / 16;   // MFMA k-steps over head_dim (QK^T)
  constexpr int NB = BN / 32;  // 32-key blocks per tile
  constexpr int DB = D / 32;   // 32-wide head_dim blocks of O^T
  constexpr int KCH = BN * D / 8;
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int VBLK = BN * D / 32;
  constexpr int VPT = (VBLK + NT - 1) / NT;
  constexpr float TAU = 8.f;
  static_assert(D % 64 == 0 && BN % 64 == 0, "tile shape");

  // K tile: row-major [key][D], 16-byte units XOR-swizzled by (key & 7).
  // V tile: transposed [d][BN]; in each 16-key chunk key 8a+4g+e is stored
  // at position 8g+4a+e, so one 16-byte read returns the 8 keys a lane of
  // k-group g feeds to the PV MFMA; units XOR-swizzled by (d & 7).
  __shared__ __attribute__((aligned(16))) uint16_t lds_k[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t lds_v[2][D * BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, g = lane >> 5;

  // work item: (b, kv-head, m-block, q-head within the group), the q-heads
  // sharing a KV head adjacent so they run on one XCD and share its L2.
  int w = xcd_remap(blockIdx.x, p.total_work);
  const int gq = w % p.G;
  w /= p.G;
  const int mi = w % p.num_mblk;
  w /= p.num_mblk;
  const int hkv = w % p.Hkv;
  const int b = w / p.Hkv;
  const int hq = hkv * p.G + gq;
  const int mblk = p.causal ? (p.num_mblk - 1 - mi) : mi;  // longest rows first
  const int m0 = mblk * BM;
  const int iw0 = m0 + wave * WR;
  const int iwl = min(iw0 + WR - 1, p.Sq - 1);
  const bool wave_live = iw0 < p.Sq;

  // Key tiles the workgroup visits, and the sub-range of full tiles.
  const int mlast = min(m0 + BM, p.Sq) - 1;
  int64_t lo = 0, hi = p.Sk, flo = 0, fhi = p.Sk;
  if (p.causal) {
    hi = min(hi, (int64_t)mlast + 1);
    fhi = min(fhi, (int64_t)m0 + 1);
  }
  if (p.has_window) {
    lo = max(lo, (int64_t)m0 - p.wl);
    hi = min(hi, (int64_t)mlast + p.wr + 1);
    flo = max(flo, (int64_t)mlast - p.wl);
    fhi = min(fhi, (int64_t)m0 + p.wr + 1);
  }
  const int t_lo = (int)(lo / BN);
  const int t_hi = hi > lo ? (int)((hi + BN - 1) / BN) : t_lo;
  int t_flo = (int)((flo + BN - 1) / BN);
  int t_fhi = fhi > 0 ? (int)(fhi / BN) : 0;
  t_flo = min(max(t_flo, t_lo), t_hi);
  t_fhi = min(max(t_fhi, t_flo), t_hi);
  if (!(p.scale_log2 > 0.f)) t_flo = t_fhi = t_hi;  // raw-max trick needs scale > 0

  // Q rows in registers: qr[qb][ds] = q[i][ds*16 + g*8 .. +8], i = iw0+32qb+r.
  u32x4_t qr[QB][DS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int ic = min(iw0 + qb * 32 + r, p.Sq - 1);
    const uint16_t* qrow = p.q + b * p.q_sb + hq * p.q_sh + (int64_t)ic * p.q_ss;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qr[qb][ds] = *(const u32x4_t*)(qrow + ds * 16 + g * 8);
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
        u32x4_t x1 = qr[qb][ds], x2 = qr[qb][ds + DS / 2];
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
        qr[qb][ds] = x1;
        qr[qb][ds + DS / 2] = x2;
      }
    }
  }

  f32x16_t acc[QB][DB];
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[qb][db] = (f32x16_t){};
  }
  const float c = p.scale_log2;
  float slope_l2 = 0.f;
  if constexpr (ALIBI) slope_l2 = -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e;
  const char* mrow[QB];
  if constexpr (MASK) {
    const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int ic = min(iw0 + qb * 32 + r, p.Sq - 1);
      mrow[qb] = (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)ic * p.mk_si) * esz;
    }
  }

  const uint16_t* kbase = p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hkv * p.v_sh;
  u32x4_t kst[KPT];
  u32x4_t vst[VPT][4];

  auto gload = [&](int tile) {
    const int n0 = tile * BN;
#pragma unroll
    for (int t = 0; t < KPT; ++t) {
      const int cidx = tid + t * NT;
      if (cidx < KCH) {
        const int key = cidx / (D / 8), unit = cidx % (D / 8);
        const int j = n0 + key;
        kst[t] = j < p.Sk ? *(const u32x4_t*)(kbase + (int64_t)j * p.k_ss + unit * 8) : (u32x4_t){};
      }
    }
#pragma unroll
    for (int t = 0; t < VPT; ++t) {
      const int blk = tid + t * NT;
      if (blk < VBLK) {
        const int kg = blk % (BN / 4), dch = blk / (BN / 4);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int j = n0 + kg * 4 + rr;
          vst[t][rr] = j < p.Sk ? *(const u32x4_t*)(vbase + (int64_t)j * p.v_ss + dch * 8) : (u32x4_t){};
        }
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int t = 0; t < KPT; ++t) {
      const int cidx = tid + t * NT;
      if (cidx < KCH) {
        const int key = cidx / (D / 8), unit = cidx % (D / 8);
        *(u32x4_t*)(&lds_k[buf][key * D + ((unit ^ (key & 7)) * 8)]) = kst[t];
      }
    }
#pragma unroll
    for (int t = 0; t < VPT; ++t) {
      const int blk = tid + t * NT;
      if (blk < VBLK) {
        const int kg = blk % (BN / 4), dch = blk / (BN / 4);
        const int c16 = kg >> 2, a = (kg >> 1) & 1, gg = kg & 1;
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
          const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
          const uint32_t w0 = __builtin_amdgcn_perm(vst[t][1][dd >> 1], vst[t][0][dd >> 1], sel);
          const uint32_t w1 = __builtin_amdgcn_perm(vst[t][3][dd >> 1], vst[t][2][dd >> 1], sel);
          const int d = dch * 8 + dd;
          const int unit = (2 * c16 + gg) ^ (d & 7);
          *(u32x2_t*)(&lds_v[buf][d * BN + unit * 8 + a * 4]) = (u32x2_t){w0, w1};
        }
      }
    }
  };

  // One tile: S = QK^T, softmax update, O += PV.  PRED: per-element
  // causal/window/bounds predicate needed; MCODE (MASK only): 0 = mask
  // block all zero (not read), 1 = read the mask.
  auto compute = [&](auto pred_c, int buf, int n0, int mcode) {
    constexpr bool PRED = decltype(pred_c)::value;
    constexpr bool GENERIC = PRED || ALIBI || MASK;
    f32x16_t s[QB][NB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[qb][nb] = (f32x16_t){};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = nb * 32 + r;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const int unit = (ds * 2 + g) ^ (row & 7);
        const u32x4_t a = *(const u32x4_t*)(&lds_k[buf][row * D + unit * 8]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[qb][nb] = E::mfma(a, qr[qb][ds], s[qb][nb]);
      }
    }
    u32x4_t pb[QB][NB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int i = iw0 + qb * 32 + r;
      float mx = -INFINITY;
      if constexpr (GENERIC) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int vq = 0; vq < 4; ++vq) {
            const int j0 = n0 + nb * 32 + vq * 8 + g * 4;
            float mv[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (MASK) {
              if (mcode) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  if (j0 + e < p.Sk) mv[e] = load_mask_elem(mrow[qb], p.mask_dtype, (int64_t)(j0 + e) * p.mk_sj);
              }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int j = j0 + e;
              float x = s[qb][nb][vq * 4 + e] * c;
              if constexpr (ALIBI) x += slope_l2 * (float)abs(i - j);
              if constexpr (MASK) x += mv[e] * kLog2e;
              if constexpr (PRED) {
                bool ok = j < p.Sk;
                if (p.causal) ok = ok && (j <= i);
                if (p.has_window) {
                  const int64_t dj = (int64_t)j - i;
                  ok = ok && (dj >= -p.wl) && (dj <= p.wr);
                }
                x = ok ? x : -INFINITY;
              }
              s[qb][nb][vq * 4 + e] = x;
              mx = fmaxf(mx, x);
            }
          }
        mx = xlane_max(mx);
      } else {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[qb][nb][v]);
        mx = xlane_max(mx) * c;  // raw max scaled: c > 0 on this path
      }
      // Lazy rescale: keep the running max unless this tile exceeds it by TAU.
      if (__builtin_expect(wave_any(mx > m_run[qb] + TAU), 0)) {
        const float m_new = fmaxf(m_run[qb], mx);
        // a row that has seen no allowed key yet (m_new = -inf; its acc and l
        // are 0) keeps alpha finite instead of exp2(-inf - -inf) = NaN
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[qb][db] *= alpha;
        m_run[qb] = m_new;
      }
      if constexpr (GENERIC) {
        const float m_use = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) s[qb][nb][v] = __builtin_amdgcn_exp2f(s[qb][nb][v] - m_use);
      } else {
        const float mneg = -m_run[qb];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) s[qb][nb][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][nb][v], c, mneg));
      }
      if constexpr (DROP) {
        // l sums the probabilities before dropout (eager: softmax, then dropout)
        float rs = 0.f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) rs += s[qb][nb][v];
        l_run[qb] += rs;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int vq = 0; vq < 4; ++vq) {
            float x[4] = {s[qb][nb][vq * 4 + 0], s[qb][nb][vq * 4 + 1], s[qb][nb][vq * 4 + 2],
                          s[qb][nb][vq * 4 + 3]};
            dropout_group(x, p, b * p.Hq + hq, i, n0 + nb * 32 + vq * 8 + g * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[qb][nb][vq * 4 + e] = x[e];
          }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          pb[qb][nb][kk] = (u32x4_t){E::pack(s[qb][nb][kk * 8 + 0], s[qb][nb][kk * 8 + 1]),
                                     E::pack(s[qb][nb][kk * 8 + 2], s[qb][nb][kk * 8 + 3]),
                                     E::pack(s[qb][nb][kk * 8 + 4], s[qb][nb][kk * 8 + 5]),
                                     E::pack(s[qb][nb][kk * 8 + 6], s[qb][nb][kk * 8 + 7])};
      if constexpr (!DROP) {
        // Row sum of the rounded P the PV product uses, two elements per
        // v_dot2 (x.lo*1 + x.hi*1 + acc), four independent accumulators.
        float r4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = E::dot2_ones(pb[qb][nb][kk][e], r4[e]);
        l_run[qb] += (r4[0] + r4[1]) + (r4[2] + r4[3]);
      }
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d = db * 32 + r;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int unit = (2 * (2 * nb + kk) + g) ^ (d & 7);
          const u32x4_t a = *(const u32x4_t*)(&lds_v[buf][d * BN + unit * 8]);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) acc[qb][db] = E::mfma(a, pb[qb][nb][kk], acc[qb][db]);
        }
    }
  };

  // Mask block-map code of this wavefront for the tile at n0 (MASK only):
  // -1 = every block of the wavefront's rows is all -inf (skip), 0 = all
  // zero (no load), 1 = load the mask.
  auto mask_code = [&](int n0) -> int {
    if (!p.bmap) return 1;
    bool all_skip = true, any_other = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int rb = (iw0 + qb * 32) / 32;
      if (iw0 + qb * 32 >= p.Sq) continue;
      const uint8_t* bm = p.bmap + b * p.bm_sb + hq * p.bm_sh + (int64_t)rb * p.bm_cols;
#pragma unroll
      for (int cb = 0; cb < BN / 64; ++cb) {
        if (n0 + cb * 64 >= p.Sk) break;  // past the last block-map column
        const uint8_t code = bm[n0 / 64 + cb];
        all_skip = all_skip && code == 2;
        any_other = any_other || code != 0;
      }
    }
    return all_skip ? -1 : (any_other ? 1 : 0);
  };

  auto step = [&](auto pred_c, int t, int buf) {
    constexpr bool PRED = decltype(pred_c)::value;
    lstore(buf);
    __syncthreads();
    if (t + 1 < t_hi) gload(t + 1);
    const int n0 = t * BN;
    bool live = wave_live;
    if constexpr (PRED) {
      if (p.causal && n0 > iwl) live = false;
      if (p.has_window && ((int64_t)n0 - iwl > p.wr || (int64_t)n0 + BN - 1 - iw0 < -p.wl)) live = false;
    }
    int mcode = 0;
    if constexpr (MASK) {
      if (live) {
        mcode = mask_code(n0);
        if (mcode < 0) live = false;
      }
    }
    if (live) compute(pred_c, buf, n0, mcode);
  };

  if (t_lo < t_hi) gload(t_lo);
  int t = t_lo, buf = 0;
  for (; t < t_flo; ++t, buf ^= 1) step(std::true_type{}, t, buf);
  for (; t < t_fhi; ++t, buf ^= 1) step(std::false_type{}, t, buf);
  for (; t < t_hi; ++t, buf ^= 1) step(std::true_type{}, t, buf);

  // Epilogue: O = acc / l (NaN for rows with no allowed key, like the eager
  // softmax over an all -inf row), optional log-sum-exp.
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = iw0 + qb * 32 + r;
    const float l = xlane_sum(l_run[qb]);
    if (i < p.Sq) {
      const float inv = 1.f / l;
      uint16_t* orow = p.o + b * p.o_sb + hq * p.o_sh + (int64_t)i * p.o_ss;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int d0 = db * 32 + vq * 8 + g * 4;
          const u32x2_t w2 = {E::pack(acc[qb][db][vq * 4 + 0] * inv, acc[qb][db][vq * 4 + 1] * inv),
                              E::pack(acc[qb][db][vq * 4 + 2] * inv, acc[qb][db][vq * 4 + 3] * inv)};
          *(u32x2_t*)(orow + d0) = w2;
        }
      if (p.lse && g == 0) p.lse[((int64_t)b * p.Hq + hq) * p.Sq + i] = (m_run[qb] + __log2f(l)) * kLn2;
    }
  }
}

// Instantiates the launcher of one (dtype, D): the given tile configs for
// every feature combination.
template <class E, int D, int BN, int NW, int QB>
hipError_t launch_feat(const FwdParams& p, int feat, hipStream_t st) {
  const dim3 grid((unsigned)p.total_work), block(NW * 64);
  switch (feat) {
#define TRINIX_CASE(F)                                                                                         \
  case F:                                                                                                      \
    hipLaunchKernelGGL((attn_fwd_mfma16<E, D, BN, NW, QB, (F & kFeatAlibi) != 0, (F & kFeatMask) != 0,       \
                                        (F & kFeatDropout) != 0>),                                             \
                       grid, block, 0, st, p);                                                                 \
    return hipGetLastError();
    TRINIX_CASE(0)
    TRINIX_CASE(1)
    TRINIX_CASE(2)
    TRINIX_CASE(3)
    TRINIX_CASE(4)
    TRINIX_CASE(5)
    TRINIX_CASE(6)
    TRINIX_CASE(7)
#undef TRINIX_CASE
    default: return hipErrorInvalidValue;
  }
}

// A tile config without ALiBi / mask / dropout.
template <class E, int D, int BN, int NW, int QB>
hipError_t launch_plain(const FwdParams& p, hipStream_t st) {
  hipLaunchKernelGGL((attn_fwd_mfma16<E, D, BN, NW, QB, false, false, false>), dim3((unsigned)p.total_work),
                     dim3(NW * 64), 0, st, p);
  return hipGetLastError();
}

// Tile configs built for every (dtype, D): (nw, qb, bn) = (4, 1, 64) with
// all feature combinations; (4, 2, 64) and (4, 1, 128) without features
// (kept for tuning sweeps).
#define TRINIX_ATTN16_LAUNCHER(NAME, E, D)                                                  \
  hipError_t NAME(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st) {               \
    if (cfg.bn == 64 && cfg.nw == 4 && cfg.qb == 1) return launch_feat<E, D, 64, 4, 1>(p, feat, st); \
    if (feat == 0 && cfg.bn == 64 && cfg.nw == 4 && cfg.qb == 2)                            \
      return launch_plain<E, D, 64, 4, 2>(p, st);                                           \
    if (feat == 0 && cfg.bn == 128 && cfg.nw == 4 && cfg.qb == 1)                           \
      return launch_plain<E, D, 128, 4, 1>(p, st);                                          \
    return hipErrorInvalidValue;                                                            \
  }

}  // namespace trinix
