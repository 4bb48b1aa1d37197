// Launch parameters of the attention kernels and the small device helpers
// they share (mask element loads, dropout, cross-lane reductions).
#pragma once
#include "common.h"
#include "host_plan.h"
#include "trinix_attn.h"

namespace trinix {

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int B, Sq, Sk, Hq, Hkv, G;
  int num_mblk, total_work;
  float scale_log2;  // softmax_scale * log2(e)
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
  int use_dropout;
  uint32_t drop_thresh;  // drop when the 16-bit Philox field < drop_thresh
  float drop_scale;      // 1 / (1 - p)
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
  const uint64_t* drop_state;  // {seed, offset} in device memory, read in place of the four above; or null
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  int64_t rope_stride;
  const uint16_t* qn_w;  // fused q RMSNorm weight (head_dim), or null
  float qn_eps;
  uint16_t* qn_out;  // the normalised q, contiguous (B, Sq, Hq, D), or null
  uint32_t* keep_map;    // dropout keep bits written for the backward (index_map.h), or null
  int64_t km_nbi, km_nbj;  // its row / key blocks per (batch, q-head)
  // work items of the per-item key split (Cfg16 ks = 0), longest chain
  // first: row block << 2 | split << 1 | half (plan_split_rows)
  uint8_t row_items[kMaxRowItems];
};


__device__ inline float load_mask_elem(const void* base, int dtype, int64_t idx) {
  switch (dtype) {
    case TRINIX_F32: return ((const float*)base)[idx];
    case TRINIX_F16: return (float)((const _Float16*)base)[idx];
    case TRINIX_BF16: return __uint_as_float(((uint32_t)((const uint16_t*)base)[idx]) << 16);
    default: return (float)((const uint8_t*)base)[idx];
  }
}

// Mask values of keys j0..j0+3 (element stride sj) of one row: one
// wave-uniform dtype switch for the four loads, keys past jmax read key jmax
// (their scores are masked anyway), so the loads carry no branches.  The
// element offsets are 32-bit: the host requires 0 <= (Sk - 1) * sj < 2^31
// for a key stride, and 0 <= min(Sq - 1, 31) * si < 2^31 for a row stride
// read within a 32-row sub-tile (mask_strides_ok, host_plan.cpp).
__device__ inline void load_mask4(const void* base, int dtype, int j0, int64_t sj, int jmax, float (&mv)[4]) {
  uint32_t idx[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) idx[e] = (uint32_t)min(j0 + e, jmax) * (uint32_t)sj;
  switch (dtype) {
    case TRINIX_F32:
#pragma unroll
      for (int e = 0; e < 4; ++e) mv[e] = ((const float*)base)[idx[e]];
      break;
    case TRINIX_F16:
#pragma unroll
      for (int e = 0; e < 4; ++e) mv[e] = (float)((const _Float16*)base)[idx[e]];
      break;
    case TRINIX_BF16:
#pragma unroll
      for (int e = 0; e < 4; ++e) mv[e] = __uint_as_float(((uint32_t)((const uint16_t*)base)[idx[e]]) << 16);
      break;
    default:
#pragma unroll
      for (int e = 0; e < 4; ++e) mv[e] = (float)((const uint8_t*)base)[idx[e]];
      break;
  }
}

// The dropout stream of one launch (common.h keep_field): Philox key
// (seed_lo ^ offset_hi, seed_hi), counter word 3 = offset_lo, and the keep
// threshold.  The seed and offset are the launch arguments, or, when the
// caller passes dropout_state, the two uint64 there, read once at the start
// of the kernel (a HIP graph replay then runs with the values a preceding
// trinix_dropout_state_advance wrote).
struct DropKey {
  uint32_t k0, k1, off_lo, thresh;
};
template <class P>
__device__ inline DropKey drop_key(const P& p) {
  uint32_t slo = p.seed_lo, shi = p.seed_hi, olo = p.off_lo, ohi = p.off_hi;
  if (p.drop_state) {
    const uint64_t s = p.drop_state[0], o = p.drop_state[1];
    slo = (uint32_t)s;
    shi = (uint32_t)(s >> 32);
    olo = (uint32_t)o;
    ohi = (uint32_t)(o >> 32);
  }
  return DropKey{slo ^ ohi, shi, olo, p.drop_thresh};
}

// Dropout (common.h keep_field) on keys ga + 4g + e (xa) and ga + 8 + 4g + e
// (xb), e = 0..3, of row i, ga % 8 == 0, g the lane half (the lane pair
// l, l + 32 holds row i): p <- keep ? p : 0.  The 1/(1-p) of the kept
// weights is applied to the output once, in the kernels' epilogues.
// Returns the keep bits: bit e for xa's key e, bit 4 + e for xb's (the
// lane's elements 4q + e of a 32x32 MFMA result block hold keys
// 8q + 4g + e of the block, so bits of the two calls of a block, shifted
// left by 8 * (ga % 32) / 16, give bit v for element v).
__device__ inline uint32_t dropout_pair(float (&xa)[4], float (&xb)[4], const DropKey& dkey, int bh, int i, int ga,
                                        int g) {
  uint32_t wa[2], wb[2];
  philox_pair_words((uint32_t)(ga >> 3), (uint32_t)i, (uint32_t)bh, dkey.off_lo, dkey.k0, dkey.k1, g, wa, wb);
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bool ka = keep_field(wa[e >> 1], e & 1, dkey.thresh), kb = keep_field(wb[e >> 1], e & 1, dkey.thresh);
    xa[e] = ka ? xa[e] : 0.f;
    xb[e] = kb ? xb[e] : 0.f;
    bits |= (ka ? 1u : 0u) << e;
    bits |= (kb ? 1u : 0u) << (4 + e);
  }
  return bits;
}

// All ones when bit v of keep bits m is set, else 0: one v_bfe_i32.  The
// empty asm hides the value from the backend, which would otherwise turn
// x & keep_word(m, v) into an and, a compare and a select (three
// instructions per element where v_bfe_i32 and v_and_b32 take two).
__device__ inline uint32_t keep_word(uint32_t m, int v) {
  int w = __builtin_amdgcn_sbfe((int)m, v, 1);
  asm("" : "+v"(w));
  return (uint32_t)w;
}

// Combine a value with the one held by lane l ^ 32 (v_permlane32_swap).
__device__ inline float xlane_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xlane_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave-uniform "any lane" vote.
__device__ inline bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

// Launchers of the 16-bit kernels, one translation unit per (dtype, D).
// Return hipErrorNotSupported for a (cfg, features) pair not instantiated.
hipError_t launch_attn16_bf16_d64(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);
hipError_t launch_attn16_bf16_d128(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);
hipError_t launch_attn16_f16_d64(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);
hipError_t launch_attn16_f16_d128(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);
hipError_t launch_attn16_bf16_d256(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);
hipError_t launch_attn16_f16_d256(const FwdParams& p, Cfg16 cfg, int feat, hipStream_t st);


// Feature bits of a launch (compile-time flags of the 16-bit kernels).
enum : int { kFeatAlibi = 1, kFeatMask = 2, kFeatDropout = 4, kFeatQNorm = 8, kFeatKeepMap = 16 };

}  // namespace trinix
