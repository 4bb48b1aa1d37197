// Fused RoPE + RMSNorm over head_dim: the qk-norm step of the attention
// layers (reference trinix/layers/attention/base.py:163-176 builds
// FastRMSNorm(head_dim); grouped_query_attention.py:171-177 applies it to q
// and k after RoPE).  For head_dim <= 2048 FastRMSNorm always runs its
// PyTorch path (trinix/layers/norm/rmsnorm.py:62-75):
//   h = x.float(); h = h * rsqrt(mean(h^2) + eps); out = weight * h.to(dtype)
// which in eager mode is about seven elementwise passes over q and k.  Here
// it is one pass: each row of head_dim elements is read once (rotated first
// when cos/sin are given, with the RoPE kernel's rounding), normalised in
// fp32 and written once.
//
// Rounding follows the eager order: the rotated value is rounded to the
// dtype (as the eager RoPE output is), the normalised value h*r is rounded to
// the dtype, and weight * that is rounded again.  The sum of squares is fp32
// in a different order from torch's reduction, so r can differ by an ulp of
// fp32, and an output element by one ulp of the dtype, rarely.
#include "common.h"
#include "trinix_attn.h"

namespace trinix {

// A row of D elements is handled by NCH = D/16 consecutive lanes; lane c
// holds d in [8c, 8c+8) and the RoPE partners d + D/2.  NCH is a power of
// two <= 16, so a row's lanes never straddle a wavefront.
template <class E>
__global__ __launch_bounds__(256) void qk_norm_kernel(const uint16_t* x, int64_t xsb, int64_t xss, int64_t xsh,
                                                      uint16_t* out, int64_t osb, int64_t oss, int64_t osh, int S,
                                                      int H, int D, const uint16_t* w, float eps,
                                                      const uint16_t* cosp, const uint16_t* sinp, int64_t cs,
                                                      int64_t cs_rows, const int64_t* pos, int64_t rows) {
#pragma clang fp contract(off)
  const int nch = D / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row_t = t / nch;
  const int c = (int)(t % nch);
  const bool live = row_t < rows;
  int64_t row = live ? row_t : rows - 1;  // dead lanes still join the row reduction
  const int h = (int)(row % H);
  row /= H;
  const int s = (int)(row % S);
  const int b = (int)(row / S);
  const uint16_t* xr = x + b * xsb + s * xss + h * xsh;
  const int d = c * 8, half = D / 2;
  const u32x4_t x1 = *(const u32x4_t*)(xr + d);
  const u32x4_t x2 = *(const u32x4_t*)(xr + d + half);
  float y1[8], y2[8];
  if (cosp) {
    // position ids are clamped to the table (the host rejects out-of-range
    // ids except while a graph is being captured, when it cannot read them)
    const int64_t ps = pos ? min(max(pos[(int64_t)b * S + s], (int64_t)0), cs_rows - 1) : s;
    const u32x4_t cw = *(const u32x4_t*)(cosp + ps * cs + d);
    const u32x4_t sw = *(const u32x4_t*)(sinp + ps * cs + d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t xa = x1[e / 2], xb = x2[e / 2], cc = cw[e / 2], ss = sw[e / 2];
      const float a = (e & 1) ? E::hi(xa) : E::lo(xa);
      const float bb = (e & 1) ? E::hi(xb) : E::lo(xb);
      const float co = (e & 1) ? E::hi(cc) : E::lo(cc);
      const float si = (e & 1) ? E::hi(ss) : E::lo(ss);
      y1[e] = round_to<E>(round_to<E>(a * co) - round_to<E>(bb * si));
      y2[e] = round_to<E>(round_to<E>(bb * co) + round_to<E>(a * si));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y1[e] = (e & 1) ? E::hi(x1[e / 2]) : E::lo(x1[e / 2]);
      y2[e] = (e & 1) ? E::hi(x2[e / 2]) : E::lo(x2[e / 2]);
    }
  }
  float ssq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ssq += y1[e] * y1[e] + y2[e] * y2[e];
  for (int m = 1; m < nch; m <<= 1) ssq += __shfl_xor(ssq, m);
  // mean(h^2): D is a power of two, so sum * (1/D) == sum / D exactly
  const float r = rsqrtf(ssq / (float)D + eps);
  if (!live) return;
  const u32x4_t w1 = *(const u32x4_t*)(w + d);
  const u32x4_t w2 = *(const u32x4_t*)(w + d + half);
  u32x4_t o1, o2;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const float n10 = round_to<E>(y1[e] * r), n11 = round_to<E>(y1[e + 1] * r);
    const float n20 = round_to<E>(y2[e] * r), n21 = round_to<E>(y2[e + 1] * r);
    o1[e / 2] = E::pack(E::lo(w1[e / 2]) * n10, E::hi(w1[e / 2]) * n11);
    o2[e / 2] = E::pack(E::lo(w2[e / 2]) * n20, E::hi(w2[e / 2]) * n21);
  }
  uint16_t* orow = out + b * osb + s * oss + h * osh;
  *(u32x4_t*)(orow + d) = o1;
  *(u32x4_t*)(orow + d + half) = o2;
}

bool aligned16_ptr(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace trinix

using namespace trinix;

extern "C" int trinix_qk_norm(const void* x, const int64_t x_stride[4], void* out, const int64_t out_stride[4],
                              int64_t batch, int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype,
                              const void* weight, float eps, const void* cos, const void* sin, int64_t cs_stride,
                              int64_t cs_rows, const int64_t* position_ids, void* stream) {
  if (!x || !out || !x_stride || !out_stride || !weight) return TRINIX_ERR_NULL_POINTER;
  if (dtype != TRINIX_BF16 && dtype != TRINIX_F16) return TRINIX_ERR_BAD_DTYPE;
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return TRINIX_ERR_BAD_HEAD_DIM;
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || seqlen >= (1ll << 30) || nheads >= (1ll << 30) ||
      batch >= (1ll << 30))
    return TRINIX_ERR_BAD_SHAPE;
  if ((cos == nullptr) != (sin == nullptr)) return TRINIX_ERR_NULL_POINTER;
  if (x_stride[3] != 1 || out_stride[3] != 1 || !aligned16_ptr(x) || !aligned16_ptr(out) || !aligned16_ptr(weight))
    return TRINIX_ERR_BAD_STRIDE;
  for (int a = 0; a < 3; ++a)
    if (x_stride[a] % 8 != 0 || out_stride[a] % 8 != 0) return TRINIX_ERR_BAD_STRIDE;
  if (cos && (!aligned16_ptr(cos) || !aligned16_ptr(sin) || cs_stride % 8 != 0 || cs_stride < head_dim / 2))
    return TRINIX_ERR_BAD_STRIDE;
  if (cos && cs_rows < (position_ids ? 1 : seqlen)) return TRINIX_ERR_BAD_SHAPE;
  const int64_t rows = batch * seqlen * nheads;
  const int64_t threads = rows * (head_dim / 16);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(256);
  hipError_t err;
  if (dtype == TRINIX_BF16)
    err = launch_kernel(&qk_norm_kernel<BF16>, grid, block, 0, st, (const uint16_t*)x, x_stride[0], x_stride[1],
                       x_stride[2], (uint16_t*)out, out_stride[0], out_stride[1], out_stride[2], (int)seqlen,
                       (int)nheads, (int)head_dim, (const uint16_t*)weight, eps, (const uint16_t*)cos,
                       (const uint16_t*)sin, cs_stride, cs_rows, position_ids, rows);
  else
    err = launch_kernel(&qk_norm_kernel<F16>, grid, block, 0, st, (const uint16_t*)x, x_stride[0], x_stride[1],
                       x_stride[2], (uint16_t*)out, out_stride[0], out_stride[1], out_stride[2], (int)seqlen,
                       (int)nheads, (int)head_dim, (const uint16_t*)weight, eps, (const uint16_t*)cos,
                       (const uint16_t*)sin, cs_stride, cs_rows, position_ids, rows);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}
