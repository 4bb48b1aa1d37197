// Host entry points of the attention library (C ABI) and the fp32 kernel.
//
// trinix_attn_fwd validates the arguments, picks a tile configuration for
// (dtype, head_dim, problem size), the feature flags (ALiBi, mask, dropout)
// and launches the bf16/fp16 MFMA kernel (attn_kernel16.h, instantiated per
// (dtype, head_dim) in attn16_*.hip) or the fp32 kernel below.
//
// The fp32 kernel uses v_mfma_f32_32x32x2f32 (exact fp32 products, fp32
// sums) with one 32-key tile at a time and K/V row-major in LDS; it follows
// the same semantics and work decomposition as the 16-bit kernel
// (reference trinix/kernels/attention_kernel.py:123-216, :341-416).
#include <atomic>
#include <cstring>

#include <cstdio>
#include <cstdlib>

#include "attn_params.h"
#include "host_plan.h"

namespace trinix {

// Applies scale, ALiBi, the additive mask and the allowed-pair predicate to a
// group of 4 consecutive keys j0..j0+3 of query row i, in the log2 domain.
template <bool PRED>
__device__ inline void score_group(float* x, const FwdParams& p, int i, int ic, int j0,
                                   float slope_l2, const char* mrow, bool use_mask) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = j0 + e;
    float y = x[e] * p.scale_log2;
    if (p.alibi) y += slope_l2 * fabsf((float)(i - j));
    if (use_mask && j < p.Sk) y += load_mask_elem(mrow, p.mask_dtype, (int64_t)j * p.mk_sj) * kLog2e;
    if (PRED) {
      bool ok = j < p.Sk;
      if (p.causal) ok = ok && (j <= i);
      if (p.has_window) {
        const int64_t dj = (int64_t)j - i;
        ok = ok && (dj >= -p.wl) && (dj <= p.wr);
      }
      y = ok ? y : -INFINITY;
    }
    x[e] = y;
  }
  (void)ic;
}

// Per-wavefront decision for one K/V tile [n0, n0+BN) against rows
// [iw0, iwl]: 0 = skip (no allowed pair), else bit 1 = per-element predicate
// needed, bit 2 = mask must be loaded.
template <int BN>
__device__ inline int classify_tile(const FwdParams& p, int b, int hq, int iw0, int iwl, int n0) {
  const int n1 = n0 + BN - 1;
  if (p.causal && n0 > iwl) return 0;
  if (p.has_window && ((int64_t)n0 - iwl > p.wr || (int64_t)n1 - iw0 < -p.wl)) return 0;
  int flags = 1;
  bool pred = n1 >= p.Sk;
  if (p.causal && n1 > iw0) pred = true;
  if (p.has_window && ((int64_t)n0 - iwl < -p.wl || (int64_t)n1 - iw0 > p.wr)) pred = true;
  if (pred) flags |= 2;
  if (p.mask) {
    if (p.bmap) {
      const uint8_t* bm = p.bmap + b * p.bm_sb + hq * p.bm_sh + (int64_t)(iw0 / 32) * p.bm_cols;
      bool all_skip = true, any_load = false;
#pragma unroll
      for (int c = 0; c < BN / 64; ++c) {
        const uint8_t code = bm[n0 / 64 + c];
        all_skip = all_skip && code == 2;
        any_load = any_load || code == 1;
        if (code == 2) pred = true;
      }
      if (all_skip) return 0;
      if (any_load) flags |= 4;
      // A block of -inf is applied by loading it: simplest exact handling of
      // tiles that mix -inf blocks with others.
      if (pred && !any_load) {
        for (int c = 0; c < BN / 64; ++c)
          if (bm[n0 / 64 + c] == 2) flags |= 4;
      }
    } else {
      flags |= 4;
    }
  }
  return flags;
}

template <int D, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd_f32(const FwdParams p) {
  const DropKey dkey = p.use_dropout ? drop_key(p) : DropKey{};
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  constexpr int BN = 32;
  constexpr int DB = D / 32;
  constexpr int KP = D + 1;  // padded pitch: lanes reading one column of 32 rows hit 32 banks
  __shared__ float lds_k[BN * KP];
  __shared__ float lds_v[BN * D];
  const float* q = (const float*)p.q;
  const float* kp = (const float*)p.k;
  const float* vp = (const float*)p.v;
  float* o = (float*)p.o;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, g = lane >> 5;
  int w = xcd_remap(blockIdx.x, p.total_work);
  const int gq = w % p.G;
  w /= p.G;
  const int mi = w % p.num_mblk;
  w /= p.num_mblk;
  const int hkv = w % p.Hkv;
  const int b = w / p.Hkv;
  const int hq = hkv * p.G + gq;
  const int mblk = p.causal ? (p.num_mblk - 1 - mi) : mi;
  const int m0 = mblk * BM;
  const int iw0 = m0 + wave * 32;
  const int iwl = min(iw0 + 31, p.Sq - 1);
  const int i = iw0 + r;
  const int ic = min(i, p.Sq - 1);
  const int mlast = min(m0 + BM, p.Sq) - 1;
  int64_t lo = 0, hi = p.Sk;
  if (p.causal) hi = min(hi, (int64_t)mlast + 1);
  if (p.has_window) {
    lo = max(lo, (int64_t)m0 - p.wl);
    hi = min(hi, (int64_t)mlast + p.wr + 1);
  }
  // The block map is built on 64-column blocks; fp32 tiles are 32 wide, so
  // align the loop to 64 and classify per 64 columns.
  const int t_lo = (int)(lo / 64) * 2;
  const int t_hi = hi > lo ? (int)((hi + BN - 1) / BN) : t_lo;

  float qf[D / 2];
  {
    const float* qrow = q + b * p.q_sb + hq * p.q_sh + (int64_t)ic * p.q_ss;
#pragma unroll
    for (int ds = 0; ds < D / 2; ++ds) qf[ds] = qrow[2 * ds + g];
    if (p.rope_cos) {
#pragma clang fp contract(off)
      const float* crow = (const float*)p.rope_cos + (int64_t)ic * p.rope_stride;
      const float* srow = (const float*)p.rope_sin + (int64_t)ic * p.rope_stride;
#pragma unroll
      for (int ds = 0; ds < D / 4; ++ds) {
        const int d = 2 * ds + g;
        const float c = crow[d], s = srow[d];
        const float x1 = qf[ds], x2 = qf[ds + D / 4];
        // separate roundings, as eager PyTorch's mul / add kernels
        qf[ds] = x1 * c - x2 * s;
        qf[ds + D / 4] = x2 * c + x1 * s;
      }
    }
  }
  f32x16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = (f32x16_t){};
  float m_run = -INFINITY, l_run = 0.f;
  const float slope_l2 = p.alibi ? -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e : 0.f;
  const char* mrow = nullptr;
  if (p.mask) {
    const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
    mrow = (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)ic * p.mk_si) * esz;
  }
  const float* kbase = kp + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = vp + b * p.v_sb + hkv * p.v_sh;

  for (int t = t_lo; t < t_hi; ++t) {
    const int n0 = t * BN;
    __syncthreads();
    for (int e = tid; e < BN * D; e += NT) {
      const int key = e / D, d = e % D;
      const int j = n0 + key;
      const float kv = j < p.Sk ? kbase[(int64_t)j * p.k_ss + d] : 0.f;
      const float vv = j < p.Sk ? vbase[(int64_t)j * p.v_ss + d] : 0.f;
      lds_k[key * KP + d] = kv;
      lds_v[key * D + d] = vv;
    }
    __syncthreads();
    // classify against the 64-wide block-map column containing this tile
    int cls = 0;
    if (iw0 < p.Sq) {
      cls = classify_tile<64>(p, b, hq, iw0, iwl, (n0 / 64) * 64);
      if (cls) {
        // refine the pair predicate to this 32-wide tile
        const int n1 = n0 + BN - 1;
        if (p.causal && n0 > iwl) cls = 0;
        if (p.has_window && ((int64_t)n0 - iwl > p.wr || (int64_t)n1 - iw0 < -p.wl)) cls = 0;
      }
    }
    if (!cls) continue;
    f32x16_t s = (f32x16_t){};
#pragma unroll
    for (int ds = 0; ds < D / 2; ++ds)
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(lds_k[r * KP + 2 * ds + g], qf[ds], s, 0, 0, 0);
    const bool pred = cls & 2, use_mask = cls & 4;
    float mx = -INFINITY;
#pragma unroll
    for (int vq = 0; vq < 4; ++vq) {
      float x[4] = {s[vq * 4 + 0], s[vq * 4 + 1], s[vq * 4 + 2], s[vq * 4 + 3]};
      const int j0 = n0 + vq * 8 + g * 4;
      if (pred) score_group<true>(x, p, i, ic, j0, slope_l2, mrow, use_mask);
      else score_group<false>(x, p, i, ic, j0, slope_l2, mrow, use_mask);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[vq * 4 + e] = x[e];
        mx = fmaxf(mx, x[e]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float e = exp2f(s[v] - m_use);
      s[v] = e;
      rs += e;
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
    if (p.use_dropout) {
#pragma unroll
      for (int vp = 0; vp < 2; ++vp) {  // 8-key groups vq = 2vp, 2vp + 1
        float xa[4], xb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xa[e] = s[vp * 8 + e];
          xb[e] = s[vp * 8 + 4 + e];
        }
        dropout_pair(xa, xb, dkey, b * p.Hq + hq, i, n0 + vp * 16, g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[vp * 8 + e] = xa[e];
          s[vp * 8 + 4 + e] = xb[e];
        }
      }
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      acc[db] *= alpha;
#pragma unroll
      for (int tt = 0; tt < 16; ++tt) {
        const int key = (tt >> 2) * 8 + g * 4 + (tt & 3);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(lds_v[key * D + db * 32 + r], s[tt], acc[db], 0, 0, 0);
      }
    }
  }
  const float l = l_run + __shfl_xor(l_run, 32);
  if (i < p.Sq) {
    float* orow = o + b * p.o_sb + hq * p.o_sh + (int64_t)i * p.o_ss;
    // with dropout, the 1/(1-p) of the kept weights (dropout_pair)
    const float os = p.use_dropout ? p.drop_scale : 1.f;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int d = db * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
        orow[d] = acc[db][v] * os / l;
      }
    if (p.lse && g == 0) p.lse[((int64_t)b * p.Hq + hq) * p.Sq + i] = (m_run + log2f(l)) * kLn2;
  }
}

}  // namespace trinix

// ---------------------------------------------------------------------------
// Host side: validation, tile table, launch.
// ---------------------------------------------------------------------------
using namespace trinix;

namespace {


}  // namespace

extern "C" {

int trinix_abi_version(void) { return TRINIX_ATTN_ABI_VERSION; }

const char* trinix_status_string(int status) {
  switch (status) {
    case TRINIX_OK: return "ok";
    case TRINIX_ERR_NULL_POINTER: return "a required pointer is NULL";
    case TRINIX_ERR_BAD_DTYPE: return "unsupported dtype";
    case TRINIX_ERR_BAD_HEAD_DIM: return "unsupported head_dim (forward and backward kernels are built for 64, 128 and 256; split-KV for 64 and 128)";
    case TRINIX_ERR_BAD_SHAPE: return "invalid or inconsistent sizes";
    case TRINIX_ERR_BAD_STRIDE: return "unsupported strides or alignment (head_dim stride must be 1, 16-byte aligned rows, 16-bit K/V key-row stride below 2^22 elements)";
    case TRINIX_ERR_BAD_ARGUMENT: return "invalid argument";
    case TRINIX_ERR_NO_DEVICE: return "no gfx950 device available";
    case TRINIX_ERR_LAUNCH: return "kernel launch failed";
    case TRINIX_ERR_SCRATCH_TOO_SMALL: return "the call needs more scratch than the library's static buffer holds (TRINIX_SPLITKV_SCRATCH_BYTES); use the entry point that takes a workspace";
    default: return "unknown status";
  }
}

int trinix_attn_is_available(void) {
  // The architecture of each device is read once and kept (0 = not read yet,
  // 1 = not gfx950, 2 = gfx950); later calls cost one hipGetDevice.
  static std::atomic<int> arch_ok[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int known = arch_ok[dev].load(std::memory_order_relaxed);
    if (known) return known == 2 ? 1 : 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  const int ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  if (dev < 64) arch_ok[dev].store(ok ? 2 : 1, std::memory_order_relaxed);
  return ok;
}

int trinix_attn_tile_config(int64_t head_dim, int32_t dtype, trinix_tile_cfg* out) {
  if (!out) return TRINIX_ERR_NULL_POINTER;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return TRINIX_ERR_BAD_HEAD_DIM;
  if (dtype == TRINIX_BF16 || dtype == TRINIX_F16) {
    const Cfg16 c = pick_cfg16(head_dim, 1 << 20, 1, 1 << 20, true, true);  // large-problem choice
    out->block_m = 32 * c.nw / c.ks;
    out->block_n = c.bn;
    out->block_d = (int32_t)head_dim;
    out->waves = c.nw;
    out->lds_bytes = (int32_t)(2 * 2 * c.ks * c.bn * head_dim * 2);
  } else if (dtype == TRINIX_F32) {
    out->block_m = 32 * kWavesF32;
    out->block_n = 32;
    out->block_d = (int32_t)head_dim;
    out->waves = kWavesF32;
    out->lds_bytes = (int32_t)(32 * (head_dim + 1) * 4 + 32 * head_dim * 4);
  } else {
    return TRINIX_ERR_BAD_DTYPE;
  }
  return TRINIX_OK;
}

int trinix_attn_fwd(const trinix_attn_fwd_args* a, void* stream) {
  const int vrc = validate_fwd_args(a);
  if (vrc != TRINIX_OK) return vrc;

  FwdParams p{};  // value-initialised: fields a configuration does not use are zero
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k;
  p.v = (const uint16_t*)a->v;
  p.o = (uint16_t*)a->out;
  p.lse = a->lse;
  p.q_sb = a->q_stride[0]; p.q_ss = a->q_stride[1]; p.q_sh = a->q_stride[2];
  p.k_sb = a->k_stride[0]; p.k_ss = a->k_stride[1]; p.k_sh = a->k_stride[2];
  p.v_sb = a->v_stride[0]; p.v_ss = a->v_stride[1]; p.v_sh = a->v_stride[2];
  p.o_sb = a->out_stride[0]; p.o_ss = a->out_stride[1]; p.o_sh = a->out_stride[2];
  p.B = (int)a->batch;
  p.Sq = (int)a->seqlen_q;
  p.Sk = (int)a->seqlen_k;
  p.Hq = (int)a->nheads_q;
  p.Hkv = (int)a->nheads_kv;
  p.G = p.Hq / p.Hkv;
  const bool f32 = a->dtype == TRINIX_F32;
  FwdPlan plan;
  const int prc = plan_fwd(a, &plan);
  if (prc != TRINIX_OK) return prc;
  const Cfg16 cfg = plan.cfg;
  p.num_mblk = plan.num_mblk;
  for (int k = 0; k < plan.n_items; ++k) p.row_items[k] = plan.row_items[k];
  p.total_work = (int)plan.total_work;
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
  p.rope_cos = (const uint16_t*)a->rope_cos;
  p.rope_sin = (const uint16_t*)a->rope_sin;
  p.rope_stride = a->rope_stride;
  p.qn_w = (const uint16_t*)a->q_norm_weight;
  p.qn_eps = a->q_norm_eps;
  p.qn_out = (uint16_t*)a->q_norm_out;
  p.keep_map = (uint32_t*)a->dropout_keep_map;
  p.km_nbi = keep_map_nbi(a->seqlen_q);
  p.km_nbj = keep_map_nbj(a->seqlen_k);

  hipStream_t st = (hipStream_t)stream;
  hipError_t err;
  if (f32) {
    const dim3 grid((unsigned)p.total_work), block(kWavesF32 * 64);
    if (a->head_dim == 64) err = launch_kernel(&attn_fwd_f32<64, kWavesF32>, grid, block, 0, st, p);
    else if (a->head_dim == 128) err = launch_kernel(&attn_fwd_f32<128, kWavesF32>, grid, block, 0, st, p);
    else err = launch_kernel(&attn_fwd_f32<256, kWavesF32>, grid, block, 0, st, p);
  } else {
    const int feat = (p.alibi ? kFeatAlibi : 0) | (p.mask ? kFeatMask : 0) | (p.use_dropout ? kFeatDropout : 0) |
                     (p.qn_w ? kFeatQNorm : 0) | (p.use_dropout && p.keep_map ? kFeatKeepMap : 0);
    const bool bf = a->dtype == TRINIX_BF16;
    if (a->head_dim == 64)
      err = bf ? launch_attn16_bf16_d64(p, cfg, feat, st) : launch_attn16_f16_d64(p, cfg, feat, st);
    else if (a->head_dim == 128)
      err = bf ? launch_attn16_bf16_d128(p, cfg, feat, st) : launch_attn16_f16_d128(p, cfg, feat, st);
    else
      err = bf ? launch_attn16_bf16_d256(p, cfg, feat, st) : launch_attn16_f16_d256(p, cfg, feat, st);
    if (err == hipErrorNotSupported) return TRINIX_ERR_BAD_ARGUMENT;  // tile config not built
  }
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

}  // extern "C"
