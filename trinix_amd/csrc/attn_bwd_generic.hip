// Generic attention backward: every dtype the forward takes (fp32, and
// bf16/fp16 widened to fp32), head_dim 64, 128 or 256, with dropout, ALiBi,
// an additive mask, causal and window masking.  No counterpart in the
// reference (its Triton attention returns a detached output,
// trinix/kernels/attention_kernel.py:497-517); the gradients are those of
// the eager path dropout(softmax(z)) v, z = scale*q k^T + bias + mask
// (trinix/layers/attention/base.py:347-400, dropout at :395):
//   P = exp(z - lse), Pd = P * keep / (1 - p),
//   dV = Pd^T dO,  dZ = P * (keep * (dO V^T) / (1 - p) - delta),
//   dK = scale * dZ^T Q,  dQ = scale * dZ K,  delta = rowsum(dO * O),
// keep being the forward's dropout mask, regenerated from the same Philox
// counters (common.h keep_field).
//
// All products run on v_mfma_f32_32x32x2f32 (exact fp32 products, fp32
// sums), so fp32 gradients keep fp32 accuracy.  The kernels work on 32x32
// (query, key) tiles with D/64 wavefronts per workgroup; wavefront w owns
// head_dim columns [64w, 64w + 64):
//   bwd_dkdv_generic  one workgroup per (batch, KV head, 32 keys): the K/V
//                     columns of the lane's key stay in registers; per
//                     query tile of every q-head of the group, each
//                     wavefront forms its partial S and dP over its columns,
//                     the partials are summed through LDS, each thread turns
//                     4 consecutive keys of one row into Pd and dZ (one
//                     Philox call, the 8-key group's), and each wavefront accumulates its
//                     columns of dV += Pd^T dO and dK += dZ^T Q;
//   bwd_dq_generic    one workgroup per (batch, q-head, 32 query rows), the
//                     same with the Q/dO rows in registers and K/V tiles in
//                     LDS: dQ += dZ K.
// Two launches plus the delta pre-pass, no atomics (deterministic).  Q, dO,
// K and V tiles live in LDS as fp32 rows of pitch D + 1, so the 32 rows a
// half-wavefront reads for one MFMA operand fall on 32 distinct banks.
#include <cmath>

#include "attn_bwd16.h"

namespace trinix {
namespace {

// Storage type T <-> fp32.
template <class T>
struct Elem;
template <>
struct Elem<float> {
  __device__ static inline float ld(const void* b, int64_t i) { return ((const float*)b)[i]; }
  __device__ static inline void st(void* b, int64_t i, float x) { ((float*)b)[i] = x; }
};
template <>
struct Elem<BF16> {
  __device__ static inline float ld(const void* b, int64_t i) {
    return __uint_as_float((uint32_t)((const uint16_t*)b)[i] << 16);
  }
  __device__ static inline void st(void* b, int64_t i, float x) { ((uint16_t*)b)[i] = (uint16_t)BF16::pack(x, 0.f); }
};
template <>
struct Elem<F16> {
  __device__ static inline float ld(const void* b, int64_t i) { return (float)((const _Float16*)b)[i]; }
  __device__ static inline void st(void* b, int64_t i, float x) { ((uint16_t*)b)[i] = (uint16_t)F16::pack(x, 0.f); }
};

__device__ inline f32x16_t mfma_f32(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

constexpr int kBT = 32;  // query rows and keys per tile
constexpr int kSP = 33;  // pitch of the 32x32 score tiles in LDS

// Keys j .. j+3 (j % 4 == 0) of query row i: from the summed scores s and
// dO.V products dp, P = exp2(s*c + bias - lse2) where (i, j) is allowed;
// s becomes Pd = P * keep / (1 - p) and dp becomes dZ.  A row whose lse is
// -inf (no allowed key: the forward wrote NaN) gets zero gradients.
__device__ inline void grad_group(const BwdParams& p, const DropKey& dkey, const Band& band, int bh, int i, int j,
                                  float lse2, float delta, float slope_l2, const char* mrow, float (&s)[4],
                                  float (&dp)[4]) {
  // keys j..j+3 are fields (j % 8) + e of the call of their 8-key group
  u32x4_t rr = {0u, 0u, 0u, 0u};
  if (p.use_dropout) rr = Philox::run((u32x4_t){(uint32_t)(j >> 3), (uint32_t)i, (uint32_t)bh, dkey.off_lo}, dkey.k0, dkey.k1);
  const bool row_ok = i < p.Sq && lse2 != -INFINITY;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int jj = j + e;
    const bool ok = row_ok && jj < p.Sk && band.ok(i, jj);
    float z = s[e] * p.scale_log2 - lse2;
    if (p.alibi) z += slope_l2 * fabsf((float)(i - jj));
    if (p.mask && ok) z += load_mask_elem(mrow, p.mask_dtype, (int64_t)jj * p.mk_sj) * kLog2e;
    const float pr = ok ? exp2f(z) : 0.f;
    const int kf = (j & 7) + e;
    const float keep = p.use_dropout ? (keep_field(rr[kf >> 1], kf & 1, dkey.thresh) ? p.drop_scale : 0.f) : 1.f;
    s[e] = pr * keep;
    dp[e] = pr * (dp[e] * keep - delta);
  }
}

__device__ inline const char* mask_row(const BwdParams& p, int b, int hq, int i) {
  if (!p.mask || i >= p.Sq) return nullptr;
  const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
  return (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)i * p.mk_si) * esz;
}

// delta[(b*Hq + h)*Sq + i] = sum_d dO * O, one wavefront per row.
template <class T, int D>
__global__ __launch_bounds__(256) void bwd_delta_generic(const BwdParams p, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int i = (int)(row % p.Sq);
  const int64_t bh = row / p.Sq;
  const int h = (int)(bh % p.Hq);
  const int64_t b = bh / p.Hq;
  const int64_t oo = b * p.o_sb + (int64_t)i * p.o_ss + h * p.o_sh;
  const int64_t od = b * p.do_sb + (int64_t)i * p.do_ss + h * p.do_sh;
  float acc = 0.f;
#pragma unroll
  for (int d = lane; d < D; d += 64) acc += Elem<T>::ld(p.o, oo + d) * Elem<T>::ld(p.dout, od + d);
#pragma unroll
  for (int m = 32; m >= 1; m /= 2) acc += __shfl_xor(acc, m);
  // a row with no allowed key (lse -inf, NaN output): delta 0, so that its
  // gradients are 0 rather than 0 * NaN
  if (lane == 0) p.delta[row] = p.lse[row] == -INFINITY ? 0.f : acc;
}

template <class T, int D>
__global__ __launch_bounds__(D, 1) void bwd_dkdv_generic(const BwdParams p) {
  const DropKey dkey = p.use_dropout ? drop_key(p) : DropKey{};
  constexpr int NW = D / 64, P1 = D + 1, NGRP = kBT * kBT / 4 / D;
  __shared__ float lq[kBT * P1];
  __shared__ float ldo[kBT * P1];
  __shared__ float lsp[NW * kBT * kSP];
  __shared__ float ldp[NW * kBT * kSP];
  __shared__ float lpd[kBT * kSP];
  __shared__ float ldz[kBT * kSP];
  __shared__ float llse[kBT], ldel[kBT];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d0 = wave * 64;
  const int nkb = (p.Sk + kBT - 1) / kBT;
  int w = blockIdx.x;
  const int kb = w % nkb;
  w /= nkb;
  const int hkv = w % p.Hkv;
  const int b = w / p.Hkv;
  const int j0 = kb * kBT;
  const Band band(p);

  // B operands: K and V of the lane's key j0 + l32 (keys past Sk read key
  // Sk-1; their scores are masked), element 2k + hi of the wave's columns.
  float kr[32], vr[32];
  {
    const int j = min(j0 + l32, p.Sk - 1);
    const int64_t ko = b * p.k_sb + (int64_t)j * p.k_ss + hkv * p.k_sh + d0 + hi;
    const int64_t vo = b * p.v_sb + (int64_t)j * p.v_ss + hkv * p.v_sh + d0 + hi;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      kr[k] = Elem<T>::ld(p.k, ko + 2 * k);
      vr[k] = Elem<T>::ld(p.v, vo + 2 * k);
    }
  }
  f32x16_t dk[2], dv[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) dk[t] = dv[t] = (f32x16_t){};

  // queries these keys may see: i - j in [-dhi, -dlo]
  const int jmax = min(j0 + kBT, p.Sk) - 1;
  const int64_t ilo = max((int64_t)0, (int64_t)j0 - band.dhi);
  const int64_t ihi = min((int64_t)p.Sq - 1, (int64_t)jmax - band.dlo);
  if (ihi >= ilo) {
    const int t0 = (int)(ilo / kBT), t1 = (int)(ihi / kBT);
    for (int gh = 0; gh < p.G; ++gh) {
      const int hq = hkv * p.G + gh;
      const float slope_l2 = p.alibi ? -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e : 0.f;
      const int64_t rb = ((int64_t)b * p.Hq + hq) * p.Sq;
      for (int t = t0; t <= t1; ++t) {
        const int i0 = t * kBT;
        for (int r = 0; r < kBT; ++r) {
          const int i = i0 + r;
          float qv = 0.f, ov = 0.f;
          if (i < p.Sq) {
            qv = Elem<T>::ld(p.q, b * p.q_sb + (int64_t)i * p.q_ss + hq * p.q_sh + tid);
            ov = Elem<T>::ld(p.dout, b * p.do_sb + (int64_t)i * p.do_ss + hq * p.do_sh + tid);
          }
          lq[r * P1 + tid] = qv;
          ldo[r * P1 + tid] = ov;
        }
        if (tid < kBT) {
          const int64_t ro = rb + min(i0 + tid, p.Sq - 1);
          llse[tid] = p.lse[ro] * kLog2e;
          ldel[tid] = p.delta[ro];
        }
        __syncthreads();
        // partial S = Q K^T and dO V^T over the wave's columns
        f32x16_t s = {}, dpp = {};
#pragma unroll
        for (int k = 0; k < 32; ++k) {
          const int dd = d0 + 2 * k + hi;
          s = mfma_f32(lq[l32 * P1 + dd], kr[k], s);
          dpp = mfma_f32(ldo[l32 * P1 + dd], vr[k], dpp);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int q = (v >> 2) * 8 + hi * 4 + (v & 3);
          lsp[(wave * kBT + q) * kSP + l32] = s[v];
          ldp[(wave * kBT + q) * kSP + l32] = dpp[v];
        }
        __syncthreads();
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
          const int grp = tid + gi * D;
          const int q = grp >> 3, kq = (grp & 7) * 4;
          float sv[4], pv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float a = 0.f, c = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
              a += lsp[(ww * kBT + q) * kSP + kq + e];
              c += ldp[(ww * kBT + q) * kSP + kq + e];
            }
            sv[e] = a;
            pv[e] = c;
          }
          const int i = i0 + q;
          grad_group(p, dkey, band, b * p.Hq + hq, i, j0 + kq, llse[q], ldel[q], slope_l2, mask_row(p, b, hq, i), sv, pv);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            lpd[q * kSP + kq + e] = sv[e];
            ldz[q * kSP + kq + e] = pv[e];
          }
        }
        __syncthreads();
        // dV += Pd^T dO, dK += dZ^T Q: rows = keys, k = queries
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int q = 2 * k + hi;
          const float a1 = lpd[q * kSP + l32], a2 = ldz[q * kSP + l32];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            dv[tt] = mfma_f32(a1, ldo[q * P1 + d0 + tt * 32 + l32], dv[tt]);
            dk[tt] = mfma_f32(a2, lq[q * P1 + d0 + tt * 32 + l32], dk[tt]);
          }
        }
        __syncthreads();
      }
    }
  }
  // element v of a lane: key j0 + (v/4)*8 + 4*hi + v%4, column d0 + 32tt + l32
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int j = j0 + (v >> 2) * 8 + hi * 4 + (v & 3);
      if (j < p.Sk) {
        const int d = d0 + tt * 32 + l32;
        Elem<T>::st(p.dk, b * p.dk_sb + (int64_t)j * p.dk_ss + hkv * p.dk_sh + d, dk[tt][v] * p.scale);
        Elem<T>::st(p.dv, b * p.dv_sb + (int64_t)j * p.dv_ss + hkv * p.dv_sh + d, dv[tt][v]);
      }
    }
}

template <class T, int D>
__global__ __launch_bounds__(D, 1) void bwd_dq_generic(const BwdParams p) {
  const DropKey dkey = p.use_dropout ? drop_key(p) : DropKey{};
  constexpr int NW = D / 64, P1 = D + 1, NGRP = kBT * kBT / 4 / D;
  __shared__ float lk[kBT * P1];
  __shared__ float lv[kBT * P1];
  __shared__ float lsp[NW * kBT * kSP];
  __shared__ float ldp[NW * kBT * kSP];
  __shared__ float ldz[kBT * kSP];
  __shared__ float llse[kBT], ldel[kBT];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d0 = wave * 64;
  const int nqb = (p.Sq + kBT - 1) / kBT;
  int w = blockIdx.x;
  const int qb = w % nqb;
  w /= nqb;
  const int hq = w % p.Hq;
  const int b = w / p.Hq;
  const int hkv = hq / p.G;
  const int i0 = qb * kBT;
  const Band band(p);
  const float slope_l2 = p.alibi ? -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e : 0.f;

  // A operands: Q and dO of the lane's row i0 + l32, element 2k + hi of the wave's columns
  float qr[32], orr[32];
  {
    const int i = min(i0 + l32, p.Sq - 1);
    const int64_t qo = b * p.q_sb + (int64_t)i * p.q_ss + hq * p.q_sh + d0 + hi;
    const int64_t oo = b * p.do_sb + (int64_t)i * p.do_ss + hq * p.do_sh + d0 + hi;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      qr[k] = Elem<T>::ld(p.q, qo + 2 * k);
      orr[k] = Elem<T>::ld(p.dout, oo + 2 * k);
    }
  }
  if (tid < kBT) {
    const int64_t ro = ((int64_t)b * p.Hq + hq) * p.Sq + min(i0 + tid, p.Sq - 1);
    llse[tid] = p.lse[ro] * kLog2e;
    ldel[tid] = p.delta[ro];
  }
  f32x16_t acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) acc[t] = (f32x16_t){};

  // keys these rows may see: j - i in [dlo, dhi]
  const int ilast = min(i0 + kBT, p.Sq) - 1;
  const int64_t jlo = max((int64_t)0, (int64_t)i0 + band.dlo);
  const int64_t jhi = min((int64_t)p.Sk - 1, (int64_t)ilast + band.dhi);
  if (jhi >= jlo) {
    const int t0 = (int)(jlo / kBT), t1 = (int)(jhi / kBT);
    for (int t = t0; t <= t1; ++t) {
      const int jt = t * kBT;
      for (int r = 0; r < kBT; ++r) {
        const int j = jt + r;
        float kv = 0.f, vv = 0.f;
        if (j < p.Sk) {
          kv = Elem<T>::ld(p.k, b * p.k_sb + (int64_t)j * p.k_ss + hkv * p.k_sh + tid);
          vv = Elem<T>::ld(p.v, b * p.v_sb + (int64_t)j * p.v_ss + hkv * p.v_sh + tid);
        }
        lk[r * P1 + tid] = kv;
        lv[r * P1 + tid] = vv;
      }
      __syncthreads();
      f32x16_t s = {}, dpp = {};
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const int dd = d0 + 2 * k + hi;
        s = mfma_f32(qr[k], lk[l32 * P1 + dd], s);
        dpp = mfma_f32(orr[k], lv[l32 * P1 + dd], dpp);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int q = (v >> 2) * 8 + hi * 4 + (v & 3);
        lsp[(wave * kBT + q) * kSP + l32] = s[v];
        ldp[(wave * kBT + q) * kSP + l32] = dpp[v];
      }
      __syncthreads();
#pragma unroll
      for (int gi = 0; gi < NGRP; ++gi) {
        const int grp = tid + gi * D;
        const int q = grp >> 3, kq = (grp & 7) * 4;
        float sv[4], pv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = 0.f, c = 0.f;
#pragma unroll
          for (int ww = 0; ww < NW; ++ww) {
            a += lsp[(ww * kBT + q) * kSP + kq + e];
            c += ldp[(ww * kBT + q) * kSP + kq + e];
          }
          sv[e] = a;
          pv[e] = c;
        }
        const int i = i0 + q;
        grad_group(p, dkey, band, b * p.Hq + hq, i, jt + kq, llse[q], ldel[q], slope_l2, mask_row(p, b, hq, i), sv, pv);
#pragma unroll
        for (int e = 0; e < 4; ++e) ldz[q * kSP + kq + e] = pv[e];
      }
      __syncthreads();
      // dQ += dZ K: rows = queries, k = keys
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int kk = 2 * k + hi;
        const float a = ldz[l32 * kSP + kk];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[tt] = mfma_f32(a, lk[kk * P1 + d0 + tt * 32 + l32], acc[tt]);
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int i = i0 + (v >> 2) * 8 + hi * 4 + (v & 3);
      if (i < p.Sq)
        Elem<T>::st(p.dq, b * p.dq_sb + (int64_t)i * p.dq_ss + hq * p.dq_sh + d0 + tt * 32 + l32, acc[tt][v] * p.scale);
    }
}

template <class T, int D>
hipError_t launch_generic(const BwdParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  hipError_t err = launch_kernel(&bwd_delta_generic<T, D>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, p,
                                 rows);
  const int64_t nkv = (int64_t)p.B * p.Hkv * ((p.Sk + kBT - 1) / kBT);
  const int64_t nq = (int64_t)p.B * p.Hq * ((p.Sq + kBT - 1) / kBT);
  if (err == hipSuccess) err = launch_kernel(&bwd_dkdv_generic<T, D>, dim3((unsigned)nkv), dim3(D), 0, st, p);
  if (err == hipSuccess) err = launch_kernel(&bwd_dq_generic<T, D>, dim3((unsigned)nq), dim3(D), 0, st, p);
  return err;
}

template <class T>
hipError_t launch_generic_d(const BwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 64: return launch_generic<T, 64>(p, st);
    case 128: return launch_generic<T, 128>(p, st);
    case 256: return launch_generic<T, 256>(p, st);
  }
  return hipErrorNotSupported;
}

}  // namespace

bool bwd_generic_fits(const BwdParams& p) {
  const int64_t nkv = (int64_t)p.B * p.Hkv * ((p.Sk + kBT - 1) / kBT);
  const int64_t nq = (int64_t)p.B * p.Hq * ((p.Sq + kBT - 1) / kBT);
  return nkv < (1ll << 31) && nq < (1ll << 31) && ((int64_t)p.B * p.Hq * p.Sq + 3) / 4 < (1ll << 31);
}

hipError_t launch_bwd_generic(const BwdParams& p, int dtype, int D, hipStream_t st) {
  switch (dtype) {
    case TRINIX_F32: return launch_generic_d<float>(p, D, st);
    case TRINIX_BF16: return launch_generic_d<BF16>(p, D, st);
    case TRINIX_F16: return launch_generic_d<F16>(p, D, st);
  }
  return hipErrorNotSupported;
}

}  // namespace trinix
