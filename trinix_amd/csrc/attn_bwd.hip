// Host entry point of the attention backward (C ABI) and the delta pre-pass.
//
// trinix_attn_bwd validates the arguments, computes delta = rowsum(dO * O)
// into the caller's workspace and launches the dK/dV and dQ kernels: the
// bf16/fp16 MFMA pipeline (attn_bwd16.h, instantiated per (dtype, head_dim)
// in attn_bwd16_*.hip) for head_dim 64/128, dropout included, the generic
// fp32-product kernels (attn_bwd_generic.hip) for fp32 and head_dim 256.
#include <cstdint>

#include "attn_bwd16.h"
#include "host_plan.h"

namespace trinix {
namespace {

// delta[(b*Hq + h)*Sq + i] = sum_d dO[b,i,h,d] * O[b,i,h,d] in fp32; D/8 lanes
// per row, one 16-byte chunk each, reduced across the lanes of the row.
template <class E, int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const uint16_t* __restrict__ o, int64_t o_sb, int64_t o_ss,
                                                        int64_t o_sh, const uint16_t* __restrict__ dout, int64_t do_sb,
                                                        int64_t do_ss, int64_t do_sh, const float* __restrict__ lse,
                                                        float* __restrict__ delta, float dmul, int Hq, int Sq,
                                                        int64_t rows) {
  constexpr int LPR = D / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int t = threadIdx.x % LPR;
  float acc = 0.f;
  if (row < rows) {
    const int i = (int)(row % Sq);
    const int64_t bh = row / Sq;
    const int h = (int)(bh % Hq);
    const int64_t b = bh / Hq;
    const u32x4_t ov = *(const u32x4_t*)(o + b * o_sb + i * o_ss + h * o_sh + t * 8);
    const u32x4_t dv = *(const u32x4_t*)(dout + b * do_sb + i * do_ss + h * do_sh + t * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc += E::lo(ov[e]) * E::lo(dv[e]) + E::hi(ov[e]) * E::hi(dv[e]);
  }
#pragma unroll
  for (int m = LPR / 2; m >= 1; m /= 2) acc += __shfl_xor(acc, m);
  // a row with no allowed key (lse -inf) has a NaN output and P = 0: its
  // delta is 0, so that its dZ = P (dP - delta) is 0 rather than 0 * NaN
  // dmul = 1 - p with dropout: the kernels then use keep*dP - delta*(1-p)
  // and apply 1/(1-p) to dq and dk in their epilogues
  if (t == 0 && row < rows) delta[row] = lse[row] == -INFINITY ? 0.f : acc * dmul;
}

template <class E, int D>
hipError_t launch_delta(const BwdParams& p, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  return launch_kernel(&bwd_delta_kernel<E, D>, dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, st, p.o,
                       p.o_sb, p.o_ss, p.o_sh, p.dout, p.do_sb, p.do_ss, p.do_sh, p.lse, p.delta,
                       p.use_dropout ? 1.f / p.drop_scale : 1.f, p.Hq, p.Sq, rows);
}

}  // namespace
}  // namespace trinix

using namespace trinix;

extern "C" int trinix_attn_bwd(const trinix_attn_bwd_args* a, void* stream) {
  const int vrc = validate_bwd_args(a);
  if (vrc != TRINIX_OK) return vrc;

  BwdParams p{};
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k;
  p.v = (const uint16_t*)a->v;
  p.o = (const uint16_t*)a->out;
  p.dout = (const uint16_t*)a->dout;
  p.lse = a->lse;
  p.delta = a->delta;
  p.dq = (uint16_t*)a->dq;
  p.dk = (uint16_t*)a->dk;
  p.dv = (uint16_t*)a->dv;
  p.q_sb = a->q_stride[0]; p.q_ss = a->q_stride[1]; p.q_sh = a->q_stride[2];
  p.k_sb = a->k_stride[0]; p.k_ss = a->k_stride[1]; p.k_sh = a->k_stride[2];
  p.v_sb = a->v_stride[0]; p.v_ss = a->v_stride[1]; p.v_sh = a->v_stride[2];
  p.o_sb = a->out_stride[0]; p.o_ss = a->out_stride[1]; p.o_sh = a->out_stride[2];
  p.do_sb = a->dout_stride[0]; p.do_ss = a->dout_stride[1]; p.do_sh = a->dout_stride[2];
  p.dq_sb = a->dq_stride[0]; p.dq_ss = a->dq_stride[1]; p.dq_sh = a->dq_stride[2];
  p.dk_sb = a->dk_stride[0]; p.dk_ss = a->dk_stride[1]; p.dk_sh = a->dk_stride[2];
  p.dv_sb = a->dv_stride[0]; p.dv_ss = a->dv_stride[1]; p.dv_sh = a->dv_stride[2];
  p.B = (int)a->batch;
  p.Sq = (int)a->seqlen_q;
  p.Sk = (int)a->seqlen_k;
  p.Hq = (int)a->nheads_q;
  p.Hkv = (int)a->nheads_kv;
  p.G = p.Hq / p.Hkv;
  p.scale = a->softmax_scale;
  p.scale_log2 = a->softmax_scale * kLog2e;
  p.causal = a->causal ? 1 : 0;
  p.has_window = a->has_window ? 1 : 0;
  p.wl = clamp_window(a->window_left);
  p.wr = clamp_window(a->window_right);
  p.alibi = a->alibi_slopes;
  p.al_sb = a->alibi_stride[0];
  p.al_sh = a->alibi_stride[1];
  p.mask = a->mask;
  p.mask_dtype = a->mask_dtype;
  p.mk_sb = a->mask_stride[0]; p.mk_sh = a->mask_stride[1]; p.mk_si = a->mask_stride[2]; p.mk_sj = a->mask_stride[3];
  p.bmap = a->mask_blockmap;
  p.bm_sb = a->blockmap_stride[0];
  p.bm_sh = a->blockmap_stride[1];
  p.bm_cols = (int)((a->seqlen_k + 63) / 64);
  BwdPlan plan;
  const int prc = plan_bwd(a, &plan);
  if (prc != TRINIX_OK) return prc;
  p.num_kblk = plan.num_kblk;
  p.num_mblk = plan.num_mblk;
  p.dq_wide = plan.dq_wide ? 1 : 0;
  p.use_dropout = a->dropout_p > 0.f ? 1 : 0;
  {
    // dropped when the key's 16-bit Philox field < floor(p * 2^16)
    const double th = (double)a->dropout_p * 65536.0;
    p.drop_thresh = th >= 65535.0 ? 65535u : (uint32_t)th;
    p.drop_scale = a->dropout_p > 0.f ? 1.f / (1.f - a->dropout_p) : 1.f;
  }
  p.seed_lo = (uint32_t)a->dropout_seed;
  p.seed_hi = (uint32_t)(a->dropout_seed >> 32);
  p.off_lo = (uint32_t)a->dropout_offset;
  p.off_hi = (uint32_t)(a->dropout_offset >> 32);
  p.drop_state = a->dropout_state;
  p.keep_map = (const uint32_t*)a->dropout_keep_map;
  p.km_nbi = keep_map_nbi(a->seqlen_q);
  p.km_nbj = keep_map_nbj(a->seqlen_k);
  const int feat = (a->alibi_slopes ? kFeatAlibi : 0) | (a->mask ? kFeatMask : 0) | (p.use_dropout ? kFeatDropout : 0);

  hipStream_t st = (hipStream_t)stream;
  hipError_t err;
  if (a->dtype == TRINIX_F32 || a->head_dim == 256) {
    if (!bwd_generic_fits(p)) return TRINIX_ERR_BAD_SHAPE;
    err = launch_bwd_generic(p, a->dtype, (int)a->head_dim, st);
    return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
  }
  const bool bf = a->dtype == TRINIX_BF16;
  if (a->head_dim == 128) {
    err = bf ? launch_delta<BF16, 128>(p, st) : launch_delta<F16, 128>(p, st);
    if (err == hipSuccess) err = bf ? launch_bwd16_bf16_d128(p, feat, st) : launch_bwd16_f16_d128(p, feat, st);
  } else {
    err = bf ? launch_delta<BF16, 64>(p, st) : launch_delta<F16, 64>(p, st);
    if (err == hipSuccess) err = bf ? launch_bwd16_bf16_d64(p, feat, st) : launch_bwd16_f16_d64(p, feat, st);
  }
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}
