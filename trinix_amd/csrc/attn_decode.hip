// Split-KV attention forward for decode-shaped problems: few query rows
// (seqlen_q <= 16) against a long KV cache.  Same semantics as
// trinix_attn_fwd (reference trinix/kernels/attention_kernel.py:123-216 and
// the eager path trinix/layers/attention/base.py:347-400, top-left causal).
//
// The 128-row tiles of the prefill kernel leave a decode step with one
// workgroup per (batch, q-head) walking every key serially.  Here a
// workgroup owns (batch, KV head, 16 packed rows, one chunk of keys):
//   * the 16 rows are (query position, q-head) pairs of one GQA group, row
//     r = i*G + g, so the KV head's tiles are read once for all its q-heads;
//   * the key range any row may see is cut into chunks ("splits") so that a
//     small batch still spreads over all CUs; a second kernel merges the
//     chunks' partial results (log-sum-exp weighted), or, with one chunk,
//     the workgroup writes the output itself.
//
// Per wavefront and 16-key step (4 wavefronts take interleaved steps):
//   S^T (16 keys x 16 rows) = K Q^T with v_mfma_f32_16x16x32 (K rows loaded
//     straight into the A-operand registers, 8 consecutive d per lane);
//   online softmax in fp32 (row max over the 4 lanes holding a row);
//   O^T += V^T P^T with v_mfma_f32_16x16x4_f32: lane l holds one V row
//     segment of D/16 consecutive d, so the fp32 A operand of d-block db is
//     element db of that segment and P (fp32, never rounded to 16 bits) is
//     the B operand as the score MFMA left it.  No transpose, no LDS.
// The 4 wavefronts' (max, sum, O) are merged through LDS at the end.
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "attn_params.h"
#include "host_plan.h"

namespace trinix {

struct DecParams {
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
  int M;                // packed rows per (batch, KV head): G * Sq
  int RG;               // 16-row groups: ceil(M / 16)
  int n_splits, chunk;  // key chunks and keys per chunk (multiple of 64)
  int klo, khi;         // keys any row may see: [klo, khi)
  float scale_log2;
  int causal, has_window;
  int64_t wl, wr;       // clamped to +-2^40
  const float* alibi;
  int64_t al_sb, al_sh;
  const void* mask;
  int mask_dtype;
  int64_t mk_sb, mk_sh, mk_si, mk_sj;
  float* part_o;        // (B*Hkv*M, n_splits, D) fp32, normalised partial O
  float* part_lse;      // (B*Hkv*M, n_splits) log2-domain partial lse
};


template <class E, int D, bool ALIBI, bool MASK>
__global__ __launch_bounds__(256) void attn_decode16(DecParams p) {
  constexpr int KK = D / 32;  // score MFMAs per 16-key step
  constexpr int VC = D / 16;  // consecutive d of one V row held by a lane
  using VT = typename std::conditional<D == 128, u32x4_t, u32x2_t>::type;
  constexpr int LDO = D + 4;
  __shared__ float lds_o[4][16][LDO];
  __shared__ float lds_m[4][16];
  __shared__ float lds_l[4][16];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;

  const DecItem wi = dec_item((int)blockIdx.x, p.RG, p.n_splits);  // (index_map.h)
  const int rg = wi.rg, split = wi.split, bh = wi.bh;
  const int b = bh / p.Hkv, kvh = bh % p.Hkv;

  // This lane's row (column lr of every score tile).
  const int r = rg * 16 + lr;
  const bool row_ok = r < p.M;
  const int i = row_ok ? r / p.G : 0;
  const int hq = kvh * p.G + (row_ok ? r % p.G : 0);

  int c0, c1;
  dec_chunk(p.klo, p.khi, p.chunk, split, c0, c1);

  // Allowed keys of row i within this chunk: [jlo, jhi].
  int jlo, jhi;
  {
    int64_t lo = c0, hi = (int64_t)c1 - 1;
    if (p.causal) hi = hi < i ? hi : i;
    if (p.has_window) {
      lo = lo > i - p.wl ? lo : i - p.wl;
      hi = hi < i + p.wr ? hi : i + p.wr;
    }
    if (!row_ok || hi < lo) {
      lo = 1;
      hi = 0;
    }
    jlo = (int)lo;
    jhi = (int)hi;
  }

  // Q and the slope are loaded on every lane (a padding row reads row 0 of
  // the group's first head, then zeroes it) so that no branch separates these
  // loads from the first K/V loads: they share one memory round trip.
  u32x4_t qv[KK];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + (int64_t)i * p.q_ss + hq * p.q_sh + lg * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u32x4_t w = *(const u32x4_t*)(qrow + kk * 32);
      qv[kk] = row_ok ? w : (u32x4_t){0u, 0u, 0u, 0u};
    }
  }
  float slope_l2 = 0.f;
  if (ALIBI) slope_l2 = -p.alibi[b * p.al_sb + hq * p.al_sh] * kLog2e;
  const char* mrow = nullptr;
  if (MASK && row_ok) {
    const int esz = p.mask_dtype == TRINIX_F32 ? 4 : (p.mask_dtype == TRINIX_U8 ? 1 : 2);
    mrow = (const char*)p.mask + (b * p.mk_sb + hq * p.mk_sh + (int64_t)i * p.mk_si) * esz;
  }

  const uint16_t* kbase = p.k + b * p.k_sb + kvh * p.k_sh + lg * 8;
  const uint16_t* vbase = p.v + b * p.v_sb + kvh * p.v_sh + lr * VC;
  const int klast = p.Sk - 1;

  // K: lane holds key j0 + lr, d = kk*32 + lg*8 .. +8 (A operand of kk).
  auto load_k = [&](int j0, u32x4_t (&kv)[KK]) {
    const int j = min(j0 + lr, klast);
    const uint16_t* krow = kbase + (int64_t)j * p.k_ss;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) kv[kk] = *(const u32x4_t*)(krow + kk * 32);
  };
  // V: lane holds keys j0 + lg*4 + v (v = 0..3), d = lr*VC .. +VC.
  auto load_v = [&](int j0, VT (&vv)[4]) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = min(j0 + lg * 4 + v, klast);
      vv[v] = *(const VT*)(vbase + (int64_t)j * p.v_ss);
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t acc[VC];  // acc[db][u]: row lr, d = (lg*4 + u)*VC + db
#pragma unroll
  for (int db = 0; db < VC; ++db) acc[db] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

  auto step = [&](int j0, const u32x4_t (&kv)[KK], const VT (&vv)[4]) {
    f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s = E::mfma16(kv[kk], qv[kk], s);
    // s[v]: key j0 + lg*4 + v, row lr
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = j0 + lg * 4 + v;
      const bool ok = j >= jlo && j <= jhi;
      float y = s[v] * p.scale_log2;
      if (ALIBI) y += slope_l2 * fabsf((float)(i - j));
      if (MASK && ok) y += load_mask_elem(mrow, p.mask_dtype, (int64_t)j * p.mk_sj) * kLog2e;
      x[v] = ok ? y : -INFINITY;
      mx = fmaxf(mx, x[v]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = xlane_max(mx);
    const float m_new = fmaxf(m_run, mx);
    // all keys so far masked: keep exp2 arguments finite (-inf - -inf = NaN)
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      x[v] = __builtin_amdgcn_exp2f(x[v] - m_use);
      rs += x[v];
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < VC; ++db) acc[db] *= alpha;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
#pragma unroll
      for (int db = 0; db < VC; ++db) {
        const uint32_t w = vv[v][db >> 1];
        const float vf = (db & 1) ? E::hi(w) : E::lo(w);
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf, x[v], acc[db], 0, 0, 0);
      }
    }
  };

  // Wavefront w takes the 16-key steps c0 + 16w + 64t, two per iteration;
  // each step's K/V are loaded one step ahead.  Loads and steps are
  // unconditional inside an iteration: a load under a condition, or an exit
  // test between a prefetch and its use, lets the compiler wait for (or sink)
  // the prefetch at the join, serialising load and compute.  A step past the
  // last one gets key positions beyond every row's range (scores -inf, no
  // effect) and re-reads the last step's rows (cache hits).  A scheduling
  // barrier after each prefetch stops the scheduler from moving the loads
  // down next to their use to save registers.
  {
    const int jw = c0 + 16 * wave;
    const int nsteps = jw < c1 ? (c1 - jw + 63) / 64 : 0;
    if (nsteps > 0) {
      constexpr int kDead = 1 << 30;  // > any jhi
      u32x4_t ka[KK], kb[KK];
      VT va[4], vb[4];
      load_k(jw, ka);
      load_v(jw, va);
      for (int t = 0; t < nsteps; t += 2) {
        const int ja = jw + 64 * t;
        const bool b_live = t + 1 < nsteps;
        const int jb = b_live ? ja + 64 : ja;
        load_k(jb, kb);
        load_v(jb, vb);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the step
        step(ja, ka, va);
        const int jc = t + 2 < nsteps ? ja + 128 : jb;
        load_k(jc, ka);
        load_v(jc, va);
        __builtin_amdgcn_sched_barrier(0);
        step(b_live ? jb : kDead, kb, vb);
      }
    }
  }

  // Row sums over the 4 lanes of a row, then merge the 4 wavefronts.
  float l_row = l_run + __shfl_xor(l_run, 16);
  l_row = xlane_sum(l_row);
  if (lg == 0) {
    lds_m[wave][lr] = m_run;
    lds_l[wave][lr] = l_row;
  }
#pragma unroll
  for (int db = 0; db < VC; ++db)
#pragma unroll
    for (int u = 0; u < 4; ++u) lds_o[wave][lr][(lg * 4 + u) * VC + db] = acc[db][u];
  __syncthreads();

  const int rr = tid >> 4, dc = (tid & 15) * VC;
  float mw[4], mmax = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = lds_m[w][rr];
    mmax = fmaxf(mmax, mw[w]);
  }
  const float m_use = mmax == -INFINITY ? 0.f : mmax;
  float L = 0.f, o[VC];
#pragma unroll
  for (int e = 0; e < VC; ++e) o[e] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f = __builtin_amdgcn_exp2f(mw[w] - m_use);
    L += lds_l[w][rr] * f;
#pragma unroll
    for (int e = 0; e < VC; ++e) o[e] += lds_o[w][rr][dc + e] * f;
  }
  const int r2 = rg * 16 + rr;
  if (r2 >= p.M) return;
  const int i2 = r2 / p.G, hq2 = kvh * p.G + r2 % p.G;
  if (p.n_splits == 1) {
    // O / L: NaN for a row with no allowed key, as the eager softmax gives
    const float inv = 1.f / L;
    uint16_t* orow = p.o + b * p.o_sb + (int64_t)i2 * p.o_ss + hq2 * p.o_sh + dc;
    if constexpr (VC == 8) {
      *(u32x4_t*)orow = (u32x4_t){E::pack(o[0] * inv, o[1] * inv), E::pack(o[2] * inv, o[3] * inv),
                                  E::pack(o[4] * inv, o[5] * inv), E::pack(o[6] * inv, o[7] * inv)};
    } else {
      *(u32x2_t*)orow = (u32x2_t){E::pack(o[0] * inv, o[1] * inv), E::pack(o[2] * inv, o[3] * inv)};
    }
    if (p.lse && (tid & 15) == 0) p.lse[((int64_t)b * p.Hq + hq2) * p.Sq + i2] = (mmax + __log2f(L)) * kLn2;
  } else {
    const int64_t idx = dec_partial_index(bh, p.M, r2, p.n_splits, split);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float* dst = p.part_o + idx * D + dc;
#pragma unroll
    for (int e = 0; e < VC; e += 4) *(f32x4_t*)(dst + e) = (f32x4_t){o[e] * inv, o[e + 1] * inv, o[e + 2] * inv, o[e + 3] * inv};
    if ((tid & 15) == 0) p.part_lse[idx] = L > 0.f ? mmax + __log2f(L) : -INFINITY;
  }
}

// Merge of the chunks of one packed row, one workgroup per row.  Thread t
// reads 4 consecutive d (slice c = t % (D/4)) of chunks s = t / (D/4) + k*NG
// (NG chunk groups), all its loads issued at once; each thread merges its
// chunks online (m = max lse, L = sum 2^(lse - m), O = sum 2^(lse - m) O_s),
// then one thread per slice merges the NG groups from LDS:
// out = O / L, lse = m + log2(L).  A row whose chunks are all empty gets NaN
// (and lse -inf), like the eager softmax over an all -inf row.
template <class E, int D>
__global__ __launch_bounds__(256) void attn_decode_combine(DecParams p) {
  constexpr int TPS = D / 4;      // threads per chunk row
  constexpr int NG = 256 / TPS;   // chunk groups
  constexpr int UNR = 8;          // chunks per thread per batch of loads
  __shared__ f32x4_t s_o[NG][TPS];
  __shared__ float s_m[NG], s_l[NG];
  const int row = blockIdx.x;
  const int t = threadIdx.x, g = t / TPS, c = t % TPS;
  const int bh = row / p.M, r = row % p.M;
  const int b = bh / p.Hkv, kvh = bh % p.Hkv;
  const int i = r / p.G, hq = kvh * p.G + r % p.G;
  const int n = p.n_splits;
  const float* pl = p.part_lse + (int64_t)row * n;
  const float* po = p.part_o + (int64_t)row * n * D + c * 4;
  float m = -INFINITY, L = 0.f;
  f32x4_t o = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = g; s0 < n; s0 += NG * UNR) {
    float ls[UNR];
    f32x4_t ov[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int s = s0 + u * NG;
      const int sc = min(s, n - 1);
      ls[u] = s < n ? pl[sc] : -INFINITY;
      ov[u] = *(const f32x4_t*)(po + (int64_t)sc * D);
    }
    float mn = m;
#pragma unroll
    for (int u = 0; u < UNR; ++u) mn = fmaxf(mn, ls[u]);
    const float m_use = mn == -INFINITY ? 0.f : mn;
    const float a = __builtin_amdgcn_exp2f(m - m_use);
    L *= a;
    o *= a;
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const float w = __builtin_amdgcn_exp2f(ls[u] - m_use);
      L += w;
      o += w * ov[u];
    }
    m = mn;
  }
  s_o[g][c] = o;
  if (c == 0) {
    s_m[g] = m;
    s_l[g] = L;
  }
  __syncthreads();
  if (t >= TPS) return;
  float mm = -INFINITY;
#pragma unroll
  for (int k = 0; k < NG; ++k) mm = fmaxf(mm, s_m[k]);
  const float m_use = mm == -INFINITY ? 0.f : mm;
  float LL = 0.f;
  f32x4_t oo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    const float w = __builtin_amdgcn_exp2f(s_m[k] - m_use);
    LL += w * s_l[k];
    oo += w * s_o[k][t];
  }
  const float inv = 1.f / LL;
  uint16_t* orow = p.o + b * p.o_sb + (int64_t)i * p.o_ss + hq * p.o_sh + t * 4;
  *(u32x2_t*)orow = (u32x2_t){E::pack(oo[0] * inv, oo[1] * inv), E::pack(oo[2] * inv, oo[3] * inv)};
  if (p.lse && t == 0) p.lse[((int64_t)b * p.Hq + hq) * p.Sq + i] = (mm + __log2f(LL)) * kLn2;
}

template <class E, int D>
hipError_t launch_decode(const DecParams& p, int feat, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)p.B * p.Hkv * p.RG * p.n_splits)), block(256);
  hipError_t err;
  switch (feat) {
    case 0: err = launch_kernel(&attn_decode16<E, D, false, false>, grid, block, 0, st, p); break;
    case kFeatAlibi: err = launch_kernel(&attn_decode16<E, D, true, false>, grid, block, 0, st, p); break;
    case kFeatMask: err = launch_kernel(&attn_decode16<E, D, false, true>, grid, block, 0, st, p); break;
    case kFeatAlibi | kFeatMask: err = launch_kernel(&attn_decode16<E, D, true, true>, grid, block, 0, st, p); break;
    default: return hipErrorNotSupported;
  }
  if (err != hipSuccess || p.n_splits == 1) return err;
  const int64_t rows = (int64_t)p.B * p.Hkv * p.M;
  return launch_kernel(&attn_decode_combine<E, D>, dim3((unsigned)rows), dim3(256), 0, st, p);
}

}  // namespace trinix

using namespace trinix;

extern "C" int trinix_attn_fwd_splitkv_plan(const trinix_attn_fwd_args* a, int32_t* num_splits,
                                            int64_t* workspace_bytes) {
  if (!num_splits || !workspace_bytes) return TRINIX_ERR_NULL_POINTER;
  const int rc = validate_fwd_args(a);
  if (rc != TRINIX_OK) return rc;
  SplitPlan pl;
  if (!make_split_plan(a, &pl)) {
    *num_splits = 0;
    *workspace_bytes = 0;
    return TRINIX_OK;
  }
  *num_splits = pl.n_splits;
  *workspace_bytes = pl.ws_bytes;
  return TRINIX_OK;
}

namespace {

// Launches the split-KV forward of a validated call with plan `pl`; the
// partial results go to `workspace` (pl.ws_bytes bytes, 16-byte aligned).
int launch_splitkv(const trinix_attn_fwd_args* a, const SplitPlan& pl, void* workspace, hipStream_t st) {
  DecParams p;
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
  p.M = pl.M;
  p.RG = pl.RG;
  p.n_splits = pl.n_splits;
  p.chunk = pl.chunk;
  p.klo = pl.klo;
  p.khi = pl.khi;
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
  const int64_t nrows = (int64_t)p.B * p.Hkv * p.M * p.n_splits;
  p.part_o = pl.ws_bytes > 0 ? (float*)workspace : nullptr;
  p.part_lse = pl.ws_bytes > 0 ? (float*)workspace + nrows * a->head_dim : nullptr;
  const int feat = (p.alibi ? kFeatAlibi : 0) | (p.mask ? kFeatMask : 0);

  hipError_t err;
  if (a->dtype == TRINIX_BF16)
    err = a->head_dim == 128 ? launch_decode<BF16, 128>(p, feat, st) : launch_decode<BF16, 64>(p, feat, st);
  else
    err = a->head_dim == 128 ? launch_decode<F16, 128>(p, feat, st) : launch_decode<F16, 64>(p, feat, st);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

// Scratch of trinix_attn_fwd_splitkv_noalloc: the partial (O, lse) of every
// (row, chunk), in device memory that the code object holds on each GPU the
// library runs on, until the process ends.  In host code the name `scratch`
// only stands in for the symbol: its address on the current device comes
// from hipGetSymbolAddress, looked up once per device and kept.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[TRINIX_SPLITKV_SCRATCH_BYTES / sizeof(float)];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch of the current device, which must be the device of `stream`
// (the kernels run on the stream's device, and each device holds its own
// copy of the array at its own address).  The null stream belongs to the
// current device.
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TRINIX_ERR_NO_DEVICE;
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) return TRINIX_ERR_BAD_ARGUMENT;
  }
  std::lock_guard<std::mutex> guard(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return TRINIX_ERR_NO_DEVICE;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TRINIX_OK;
}

}  // namespace

extern "C" int trinix_attn_fwd_splitkv(const trinix_attn_fwd_args* a, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  const int rc = validate_fwd_args(a);
  if (rc != TRINIX_OK) return rc;
  SplitPlan pl;
  if (!make_split_plan(a, &pl)) return TRINIX_ERR_BAD_ARGUMENT;
  if (pl.ws_bytes > 0 && (!workspace || workspace_bytes < pl.ws_bytes || ((uintptr_t)workspace & 15) != 0))
    return TRINIX_ERR_BAD_ARGUMENT;
  return launch_splitkv(a, pl, workspace, (hipStream_t)stream);
}

extern "C" int trinix_attn_fwd_splitkv_noalloc(const trinix_attn_fwd_args* a, void* stream) {
  const int rc = validate_fwd_args(a);
  if (rc != TRINIX_OK) return rc;
  SplitPlan pl;
  if (!make_split_plan(a, &pl)) return TRINIX_ERR_BAD_ARGUMENT;
  if (pl.ws_bytes > (int64_t)TRINIX_SPLITKV_SCRATCH_BYTES) return TRINIX_ERR_SCRATCH_TOO_SMALL;
  void* ws = nullptr;
  if (pl.ws_bytes > 0) {
    const int src = scratch_for_stream((hipStream_t)stream, &ws);
    if (src != TRINIX_OK) return src;
  }
  return launch_splitkv(a, pl, ws, (hipStream_t)stream);
}
