// Fused RoPE + qk-norm over head_dim: the qk-norm step of the attention
// layers (reference trinix/layers/attention/base.py:163-176 builds
// FastRMSNorm(head_dim) or FastLayerNorm(head_dim); grouped_query_attention.py
// :171-177 applies it to q and k after RoPE), forward and backward.
//
// For head_dim <= 2048 FastRMSNorm always runs its PyTorch path
// (trinix/layers/norm/rmsnorm.py:62-75):
//   h = x.float(); h = h * rsqrt(mean(h^2) + eps); out = weight * h.to(dtype)
// and for head_dim <= 4096 FastLayerNorm runs F.layer_norm with the weight
// and bias cast to the input dtype (trinix/layers/norm/layernorm.py:83-88),
// which normalises and applies the affine in fp32.  In eager mode either is
// several elementwise passes over q and k.  Here it is one pass: each row of
// head_dim elements is read once (rotated first when cos/sin are given, with
// the RoPE kernel's rounding), normalised in fp32 and written once.
//
// Rounding follows the eager order: the rotated value is rounded to the
// dtype (as the eager RoPE output is); RMSNorm rounds h*r to the dtype and
// weight * that again; LayerNorm rounds (y - mean) * rstd * w + b once.  The
// fp32 reductions are ordered differently from torch's, so an output
// element can differ from eager by one ulp of the dtype, rarely.
//
// The backward recomputes the rotated row and its statistics and follows
// eager autograd through the same steps:
//   RMSNorm: dn = to_dtype(dout * w); dh = dn*r - (r^3 / D) * sum(dn*y) * y
//   LayerNorm: g = dout * w (fp32); dh = rstd * (g - mean(g) - xhat * mean(g*xhat))
//   dy = to_dtype(dh); dx = RoPE^T(dy): dx1 = dy1*cos + dy2*sin,
//   dx2 = dy2*cos - dy1*sin, each product and the sum rounded to the dtype
//   (the gradients of x*cos and rotate_half(x)*sin, summed by autograd).
// dweight (RMSNorm: sum of to_dtype(dout * to_dtype(h*r)); LayerNorm: sum of
// dout * xhat) and dbias (sum of dout) are summed in fp32 per workgroup into
// caller-provided partial rows; the caller adds the rows (a fixed order:
// deterministic) and rounds to the weight's dtype.
#include "common.h"
#include "trinix_attn.h"

namespace trinix {

namespace {

// A row of D elements is handled by NCH = D/16 consecutive lanes; lane c
// holds d in [8c, 8c+8) and the RoPE partners d + D/2.  NCH is a power of
// two <= 16, so a row's lanes never straddle a wavefront.

template <class E>
__device__ inline void unpack8(const u32x4_t v, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (e & 1) ? E::hi(v[e / 2]) : E::lo(v[e / 2]);
}

// (B, S, H) coordinates of flat row `row` (row = (b*S + s)*H + h).
struct RowPos {
  int b, s, h;
};
__device__ inline RowPos row_pos(int64_t row, int S, int H) {
  RowPos r;
  r.h = (int)(row % H);
  row /= H;
  r.s = (int)(row % S);
  r.b = (int)(row / S);
  return r;
}

// The row's elements after RoPE (rounded as the eager RoPE output is), or
// the raw elements without cos/sin.  Also returns the cos/sin of the lane's
// 8 columns (for the backward).
template <class E>
__device__ inline void load_rotated(const uint16_t* xr, int d, int half, const uint16_t* cosp, const uint16_t* sinp,
                                    int64_t cs, int64_t cs_rows, const int64_t* pos, const RowPos& rp, int S,
                                    float (&y1)[8], float (&y2)[8], float (&co)[8], float (&si)[8]) {
#pragma clang fp contract(off)
  const u32x4_t x1 = *(const u32x4_t*)(xr + d);
  const u32x4_t x2 = *(const u32x4_t*)(xr + d + half);
  if (cosp) {
    // position ids are clamped to the table (the host rejects out-of-range
    // ids except while a graph is being captured, when it cannot read them)
    const int64_t ps = pos ? min(max(pos[(int64_t)rp.b * S + rp.s], (int64_t)0), cs_rows - 1) : rp.s;
    unpack8<E>(*(const u32x4_t*)(cosp + ps * cs + d), co);
    unpack8<E>(*(const u32x4_t*)(sinp + ps * cs + d), si);
    float a[8], bb[8];
    unpack8<E>(x1, a);
    unpack8<E>(x2, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y1[e] = round_to<E>(round_to<E>(a[e] * co[e]) - round_to<E>(bb[e] * si[e]));
      y2[e] = round_to<E>(round_to<E>(bb[e] * co[e]) + round_to<E>(a[e] * si[e]));
    }
  } else {
    unpack8<E>(x1, y1);
    unpack8<E>(x2, y2);
  }
}

// Sum over the NCH lanes of a row.
__device__ inline float row_sum(float v, int nch) {
  for (int m = 1; m < nch; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

template <class E>
__device__ inline u32x4_t pack8(const float (&f)[8]) {
  u32x4_t v;
#pragma unroll
  for (int e = 0; e < 8; e += 2) v[e / 2] = E::pack(f[e], f[e + 1]);
  return v;
}

}  // namespace

template <class E, bool LN>
__global__ __launch_bounds__(256) void qk_norm_kernel(const uint16_t* x, int64_t xsb, int64_t xss, int64_t xsh,
                                                      uint16_t* out, int64_t osb, int64_t oss, int64_t osh, int S,
                                                      int H, int D, const uint16_t* w, const uint16_t* bias,
                                                      float eps, const uint16_t* cosp, const uint16_t* sinp,
                                                      int64_t cs, int64_t cs_rows, const int64_t* pos,
                                                      int64_t rows) {
#pragma clang fp contract(off)
  const int nch = D / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row_t = t / nch;
  const int c = (int)(t % nch);
  const bool live = row_t < rows;
  const RowPos rp = row_pos(live ? row_t : rows - 1, S, H);  // dead lanes still join the row reduction
  const int d = c * 8, half = D / 2;
  float y1[8], y2[8], co[8], si[8];
  load_rotated<E>(x + rp.b * xsb + rp.s * xss + rp.h * xsh, d, half, cosp, sinp, cs, cs_rows, pos, rp, S, y1, y2,
                  co, si);
  float w1[8], w2[8], o1[8], o2[8];
  if constexpr (LN) {
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += y1[e] + y2[e];
    // D is a power of two: sum / D is exact scaling
    const float mean = row_sum(sum, nch) / (float)D;
    float ssd = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ssd += (y1[e] - mean) * (y1[e] - mean) + (y2[e] - mean) * (y2[e] - mean);
    const float rstd = rsqrtf(row_sum(ssd, nch) / (float)D + eps);
    if (!live) return;
    float b1[8], b2[8];
    unpack8<E>(*(const u32x4_t*)(w + d), w1);
    unpack8<E>(*(const u32x4_t*)(w + d + half), w2);
    unpack8<E>(*(const u32x4_t*)(bias + d), b1);
    unpack8<E>(*(const u32x4_t*)(bias + d + half), b2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = __builtin_fmaf((y1[e] - mean) * rstd, w1[e], b1[e]);
      o2[e] = __builtin_fmaf((y2[e] - mean) * rstd, w2[e], b2[e]);
    }
  } else {
    float ssq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ssq += y1[e] * y1[e] + y2[e] * y2[e];
    // mean(h^2): D is a power of two, so sum * (1/D) == sum / D exactly
    const float r = rsqrtf(row_sum(ssq, nch) / (float)D + eps);
    if (!live) return;
    unpack8<E>(*(const u32x4_t*)(w + d), w1);
    unpack8<E>(*(const u32x4_t*)(w + d + half), w2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = w1[e] * round_to<E>(y1[e] * r);
      o2[e] = w2[e] * round_to<E>(y2[e] * r);
    }
  }
  uint16_t* orow = out + rp.b * osb + rp.s * oss + rp.h * osh;
  *(u32x4_t*)(orow + d) = pack8<E>(o1);
  *(u32x4_t*)(orow + d + half) = pack8<E>(o2);
}

// Backward.  Each workgroup walks rows blockIdx.x*RPB + k*gridDim.x*RPB
// (RPB = 256/NCH rows per pass) and writes its fp32 dweight (and, for
// LayerNorm, dbias) column sums to row blockIdx.x of the partial arrays.
// RMSNorm fits four wavefronts per SIMD (128 registers); LayerNorm, with
// its dbias sums, three.
template <class E, bool LN>
__global__ __launch_bounds__(256, LN ? 3 : 4) void qk_norm_bwd_kernel(
    const uint16_t* x, int64_t xsb, int64_t xss, int64_t xsh, const uint16_t* dout, int64_t gsb, int64_t gss,
    int64_t gsh, uint16_t* dx, int64_t osb, int64_t oss, int64_t osh, int S, int H, int D, const uint16_t* w,
    float eps, const uint16_t* cosp, const uint16_t* sinp, int64_t cs, int64_t cs_rows, const int64_t* pos,
    int64_t rows, float* dw_part, float* db_part) {
#pragma clang fp contract(off)
  __shared__ float red_w[256 * 16];
  __shared__ float red_b[LN ? 256 * 16 : 1];
  const int nch = D / 16;
  const int rpb = 256 / nch;
  const int lrow = threadIdx.x / nch, c = threadIdx.x % nch;
  const int d = c * 8, half = D / 2;
  float aw[16] = {}, ab[16] = {};
  for (int64_t row0 = (int64_t)blockIdx.x * rpb; row0 < rows; row0 += (int64_t)gridDim.x * rpb) {
    // the weight is read per row (cache-resident) rather than held across
    // the loop: registers for four wavefronts per SIMD
    float w1[8], w2[8];
    unpack8<E>(*(const u32x4_t*)(w + d), w1);
    unpack8<E>(*(const u32x4_t*)(w + d + half), w2);
    const int64_t row_t = row0 + lrow;
    const bool live = row_t < rows;
    const RowPos rp = row_pos(live ? row_t : rows - 1, S, H);
    float y1[8], y2[8], co[8], si[8];
    load_rotated<E>(x + rp.b * xsb + rp.s * xss + rp.h * xsh, d, half, cosp, sinp, cs, cs_rows, pos, rp, S, y1, y2,
                    co, si);
    const uint16_t* grow = dout + rp.b * gsb + rp.s * gss + rp.h * gsh;
    float g1[8], g2[8];
    unpack8<E>(*(const u32x4_t*)(grow + d), g1);
    unpack8<E>(*(const u32x4_t*)(grow + d + half), g2);
    float dh1[8], dh2[8];
    if constexpr (LN) {
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += y1[e] + y2[e];
      const float mean = row_sum(sum, nch) / (float)D;
      float ssd = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ssd += (y1[e] - mean) * (y1[e] - mean) + (y2[e] - mean) * (y2[e] - mean);
      const float rstd = rsqrtf(row_sum(ssd, nch) / (float)D + eps);
      float xh1[8], xh2[8], gw1[8], gw2[8], s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xh1[e] = (y1[e] - mean) * rstd;
        xh2[e] = (y2[e] - mean) * rstd;
        gw1[e] = g1[e] * w1[e];
        gw2[e] = g2[e] * w2[e];
        s1 += gw1[e] + gw2[e];
        s2 += gw1[e] * xh1[e] + gw2[e] * xh2[e];
      }
      const float m1 = row_sum(s1, nch) / (float)D, m2 = row_sum(s2, nch) / (float)D;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dh1[e] = rstd * (gw1[e] - m1 - xh1[e] * m2);
        dh2[e] = rstd * (gw2[e] - m1 - xh2[e] * m2);
      }
      if (live)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aw[e] += g1[e] * xh1[e];
          aw[8 + e] += g2[e] * xh2[e];
          ab[e] += g1[e];
          ab[8 + e] += g2[e];
        }
    } else {
      float ssq = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ssq += y1[e] * y1[e] + y2[e] * y2[e];
      const float r = rsqrtf(row_sum(ssq, nch) / (float)D + eps);
      // out = w * to_dtype(y*r): the gradient of the rounded product is
      // to_dtype(dout * w), of w it is to_dtype(dout * to_dtype(y*r))
      float dn1[8], dn2[8], sd = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dn1[e] = round_to<E>(g1[e] * w1[e]);
        dn2[e] = round_to<E>(g2[e] * w2[e]);
        sd += dn1[e] * y1[e] + dn2[e] * y2[e];
      }
      // d rsqrt(v) = -r^3/2 dv, d mean(y^2) = 2y/D
      const float gv = row_sum(sd, nch) * -0.5f * (r * r * r);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dh1[e] = dn1[e] * r + (gv / (float)D) * 2.f * y1[e];
        dh2[e] = dn2[e] * r + (gv / (float)D) * 2.f * y2[e];
      }
      if (live)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aw[e] += round_to<E>(g1[e] * round_to<E>(y1[e] * r));
          aw[8 + e] += round_to<E>(g2[e] * round_to<E>(y2[e] * r));
        }
    }
    float o1[8], o2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d1 = round_to<E>(dh1[e]), d2 = round_to<E>(dh2[e]);
      if (cosp) {
        o1[e] = round_to<E>(round_to<E>(d1 * co[e]) + round_to<E>(d2 * si[e]));
        o2[e] = round_to<E>(round_to<E>(d2 * co[e]) - round_to<E>(d1 * si[e]));
      } else {
        o1[e] = d1;
        o2[e] = d2;
      }
    }
    if (live) {
      uint16_t* orow = dx + rp.b * osb + rp.s * oss + rp.h * osh;
      *(u32x4_t*)(orow + d) = pack8<E>(o1);
      *(u32x4_t*)(orow + d + half) = pack8<E>(o2);
    }
  }
  // Column sums over the block's rows: lane c of every row holds columns
  // 8c..8c+7 (aw[0..7]) and D/2 + 8c.. (aw[8..15]).
#pragma unroll
  for (int k = 0; k < 16; ++k) red_w[threadIdx.x * 16 + k] = aw[k];
  if constexpr (LN)
#pragma unroll
    for (int k = 0; k < 16; ++k) red_b[threadIdx.x * 16 + k] = ab[k];
  __syncthreads();
  for (int col = threadIdx.x; col < D; col += blockDim.x) {
    const int cc = col < half ? col / 8 : (col - half) / 8;
    const int k = col < half ? col % 8 : 8 + (col - half) % 8;
    float sw = 0.f, sb = 0.f;
    for (int r2 = 0; r2 < rpb; ++r2) {
      sw += red_w[(r2 * nch + cc) * 16 + k];
      if constexpr (LN) sb += red_b[(r2 * nch + cc) * 16 + k];
    }
    dw_part[(int64_t)blockIdx.x * D + col] = sw;
    if constexpr (LN) db_part[(int64_t)blockIdx.x * D + col] = sb;
  }
}

namespace {

bool aligned16_ptr(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Shape / stride checks shared by the three entry points.
int check_rows(const void* x, const int64_t* x_stride, int64_t batch, int64_t seqlen, int64_t nheads,
               int64_t head_dim, int32_t dtype, const void* cos, const void* sin, int64_t cs_stride, int64_t cs_rows,
               const int64_t* position_ids) {
  if (!x || !x_stride) return TRINIX_ERR_NULL_POINTER;
  if (dtype != TRINIX_BF16 && dtype != TRINIX_F16) return TRINIX_ERR_BAD_DTYPE;
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return TRINIX_ERR_BAD_HEAD_DIM;
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || seqlen >= (1ll << 30) || nheads >= (1ll << 30) ||
      batch >= (1ll << 30))
    return TRINIX_ERR_BAD_SHAPE;
  if ((cos == nullptr) != (sin == nullptr)) return TRINIX_ERR_NULL_POINTER;
  if (cos && (!aligned16_ptr(cos) || !aligned16_ptr(sin) || cs_stride % 8 != 0 || cs_stride < head_dim / 2))
    return TRINIX_ERR_BAD_STRIDE;
  if (cos && cs_rows < (position_ids ? 1 : seqlen)) return TRINIX_ERR_BAD_SHAPE;
  return TRINIX_OK;
}

int check_tensor16(const void* p, const int64_t* stride) {
  if (!p || !stride) return TRINIX_ERR_NULL_POINTER;
  if (stride[3] != 1 || !aligned16_ptr(p)) return TRINIX_ERR_BAD_STRIDE;
  for (int a = 0; a < 3; ++a)
    if (stride[a] % 8 != 0) return TRINIX_ERR_BAD_STRIDE;
  return TRINIX_OK;
}

template <bool LN>
int qk_norm_forward(const void* x, const int64_t x_stride[4], void* out, const int64_t out_stride[4], int64_t batch,
                    int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype, const void* weight,
                    const void* bias, float eps, const void* cos, const void* sin, int64_t cs_stride,
                    int64_t cs_rows, const int64_t* position_ids, void* stream) {
  int rc = check_rows(x, x_stride, batch, seqlen, nheads, head_dim, dtype, cos, sin, cs_stride, cs_rows,
                      position_ids);
  if (rc) return rc;
  if (!weight || (LN && !bias)) return TRINIX_ERR_NULL_POINTER;
  if ((rc = check_tensor16(x, x_stride)) || (rc = check_tensor16(out, out_stride))) return rc;
  if (!aligned16_ptr(weight) || (LN && !aligned16_ptr(bias))) return TRINIX_ERR_BAD_STRIDE;
  const int64_t rows = batch * seqlen * nheads;
  const int64_t threads = rows * (head_dim / 16);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(256);
  auto go = [&](auto kernel) {
    return launch_kernel(kernel, grid, block, 0, st, (const uint16_t*)x, x_stride[0], x_stride[1], x_stride[2],
                         (uint16_t*)out, out_stride[0], out_stride[1], out_stride[2], (int)seqlen, (int)nheads,
                         (int)head_dim, (const uint16_t*)weight, (const uint16_t*)bias, eps, (const uint16_t*)cos,
                         (const uint16_t*)sin, cs_stride, cs_rows, position_ids, rows);
  };
  const hipError_t err = dtype == TRINIX_BF16 ? go(&qk_norm_kernel<BF16, LN>) : go(&qk_norm_kernel<F16, LN>);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

}  // namespace

}  // namespace trinix

using namespace trinix;

extern "C" int trinix_qk_norm(const void* x, const int64_t x_stride[4], void* out, const int64_t out_stride[4],
                              int64_t batch, int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype,
                              const void* weight, float eps, const void* cos, const void* sin, int64_t cs_stride,
                              int64_t cs_rows, const int64_t* position_ids, void* stream) {
  return qk_norm_forward<false>(x, x_stride, out, out_stride, batch, seqlen, nheads, head_dim, dtype, weight,
                                nullptr, eps, cos, sin, cs_stride, cs_rows, position_ids, stream);
}

extern "C" int trinix_qk_layernorm(const void* x, const int64_t x_stride[4], void* out, const int64_t out_stride[4],
                                   int64_t batch, int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype,
                                   const void* weight, const void* bias, float eps, const void* cos, const void* sin,
                                   int64_t cs_stride, int64_t cs_rows, const int64_t* position_ids, void* stream) {
  return qk_norm_forward<true>(x, x_stride, out, out_stride, batch, seqlen, nheads, head_dim, dtype, weight, bias,
                               eps, cos, sin, cs_stride, cs_rows, position_ids, stream);
}

extern "C" int trinix_qk_norm_bwd(const void* x, const int64_t x_stride[4], const void* dout,
                                  const int64_t dout_stride[4], void* dx, const int64_t dx_stride[4], int64_t batch,
                                  int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype, int32_t norm_type,
                                  const void* weight, float eps, const void* cos, const void* sin, int64_t cs_stride,
                                  int64_t cs_rows, const int64_t* position_ids, float* dweight_partial,
                                  float* dbias_partial, int64_t partial_rows, void* stream) {
  int rc = check_rows(x, x_stride, batch, seqlen, nheads, head_dim, dtype, cos, sin, cs_stride, cs_rows,
                      position_ids);
  if (rc) return rc;
  if (norm_type != TRINIX_NORM_RMS && norm_type != TRINIX_NORM_LAYER) return TRINIX_ERR_BAD_ARGUMENT;
  const bool ln = norm_type == TRINIX_NORM_LAYER;
  if (!weight || !dweight_partial || (ln && !dbias_partial)) return TRINIX_ERR_NULL_POINTER;
  if ((rc = check_tensor16(x, x_stride)) || (rc = check_tensor16(dout, dout_stride)) ||
      (rc = check_tensor16(dx, dx_stride)))
    return rc;
  if (!aligned16_ptr(weight)) return TRINIX_ERR_BAD_STRIDE;
  if (partial_rows <= 0 || partial_rows >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  const int64_t rows = batch * seqlen * nheads;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)partial_rows), block(256);
  auto go = [&](auto kernel) {
    return launch_kernel(kernel, grid, block, 0, st, (const uint16_t*)x, x_stride[0], x_stride[1], x_stride[2],
                         (const uint16_t*)dout, dout_stride[0], dout_stride[1], dout_stride[2], (uint16_t*)dx,
                         dx_stride[0], dx_stride[1], dx_stride[2], (int)seqlen, (int)nheads, (int)head_dim,
                         (const uint16_t*)weight, eps, (const uint16_t*)cos, (const uint16_t*)sin, cs_stride,
                         cs_rows, position_ids, rows, dweight_partial, dbias_partial);
  };
  hipError_t err;
  if (dtype == TRINIX_BF16)
    err = ln ? go(&qk_norm_bwd_kernel<BF16, true>) : go(&qk_norm_bwd_kernel<BF16, false>);
  else
    err = ln ? go(&qk_norm_bwd_kernel<F16, true>) : go(&qk_norm_bwd_kernel<F16, false>);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}
