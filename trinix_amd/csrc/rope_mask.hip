// Producers either side of the attention kernel:
//  * trinix_rope_apply: rotary embedding with eager-PyTorch rounding
//    (reference trinix/layers/embeddings/rope.py:111-134 and the Triton
//    kernel trinix/kernels/rope_kernel.py:10-88), used for K before the
//    fused-RoPE attention launch and as the standalone RoPE op.
//  * trinix_attn_mask_blockmap: classifies an additive mask into 32x64
//    blocks (all zero / all -inf / mixed) so the attention kernel skips
//    -inf blocks and never reads all-zero blocks.  Replaces the (B,H,S,S)
//    materialisation of trinix/kernels/attention_kernel.py:479-495.
#include <cstring>
#include "common.h"
#include "trinix_attn.h"

namespace trinix {

// One thread: 8 consecutive pairs (d, d + D/2), d in [8c, 8c+8).
template <class E>
__global__ __launch_bounds__(256) void rope16_kernel(const uint16_t* x, int64_t xsb, int64_t xss, int64_t xsh,
                                                     uint16_t* out, int64_t osb, int64_t oss, int64_t osh,
                                                     int S, int H, int D, const uint16_t* cosp,
                                                     const uint16_t* sinp, int64_t cs, int64_t cs_rows,
                                                     const int64_t* pos, int64_t total) {
  // One rounding per product and per sum, as eager PyTorch: no contraction
  // of x*c - y*s into an fma (which would drop the rounding of one product).
#pragma clang fp contract(off)
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int nch = D / 16;  // chunks of 8 in the first half
  const int c = (int)(t % nch);
  int64_t row = t / nch;
  const int h = (int)(row % H);
  row /= H;
  const int s = (int)(row % S);
  const int b = (int)(row / S);
  // position ids are clamped to the table (the host rejects out-of-range
  // ids except while a graph is being captured, when it cannot read them)
  const int64_t ps = pos ? min(max(pos[(int64_t)b * S + s], (int64_t)0), cs_rows - 1) : s;
  const uint16_t* xr = x + b * xsb + s * xss + h * xsh;
  uint16_t* orow = out + b * osb + s * oss + h * osh;
  const int d = c * 8, half = D / 2;
  const u32x4_t x1 = *(const u32x4_t*)(xr + d);
  const u32x4_t x2 = *(const u32x4_t*)(xr + d + half);
  const u32x4_t cw = *(const u32x4_t*)(cosp + ps * cs + d);
  const u32x4_t sw = *(const u32x4_t*)(sinp + ps * cs + d);
  u32x4_t o1, o2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float c0 = E::lo(cw[e]), c1 = E::hi(cw[e]);
    const float s0 = E::lo(sw[e]), s1 = E::hi(sw[e]);
    const float a0 = E::lo(x1[e]), a1 = E::hi(x1[e]);
    const float b0 = E::lo(x2[e]), b1 = E::hi(x2[e]);
    o1[e] = E::pack(round_to<E>(round_to<E>(a0 * c0) - round_to<E>(b0 * s0)),
                    round_to<E>(round_to<E>(a1 * c1) - round_to<E>(b1 * s1)));
    o2[e] = E::pack(round_to<E>(round_to<E>(b0 * c0) + round_to<E>(a0 * s0)),
                    round_to<E>(round_to<E>(b1 * c1) + round_to<E>(a1 * s1)));
  }
  *(u32x4_t*)(orow + d) = o1;
  *(u32x4_t*)(orow + d + half) = o2;
}

// Generic element-wise variant (any even D, any dtype incl. fp32): one pair
// per thread.
struct BF16Scalar {
  __device__ static float ld(const uint16_t* p, int64_t i) { return __uint_as_float(((uint32_t)p[i]) << 16); }
  __device__ static void st(uint16_t* p, int64_t i, float v) { p[i] = (uint16_t)(BF16::pack(v, 0.f) & 0xffffu); }
  __device__ static float rnd(float v) { return round_to<BF16>(v); }
};
struct F16Scalar {
  __device__ static float ld(const uint16_t* p, int64_t i) { return (float)((const _Float16*)p)[i]; }
  __device__ static void st(uint16_t* p, int64_t i, float v) { p[i] = (uint16_t)(F16::pack(v, 0.f) & 0xffffu); }
  __device__ static float rnd(float v) { return round_to<F16>(v); }
};
struct F32Scalar {
  __device__ static float ld(const float* p, int64_t i) { return p[i]; }
  __device__ static void st(float* p, int64_t i, float v) { p[i] = v; }
  __device__ static float rnd(float v) { return v; }
};

// Products and sums are separate roundings (no FMA contraction), matching
// eager PyTorch's separate mul / add kernels.
template <class S>
__device__ inline float rope_lo(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return S::rnd(S::rnd(a * c) - S::rnd(b * s));
}
template <class S>
__device__ inline float rope_hi(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return S::rnd(S::rnd(b * c) + S::rnd(a * s));
}

template <class S, class T>
__global__ __launch_bounds__(256) void rope_scalar_kernel(const T* x, int64_t xsb, int64_t xss, int64_t xsh, T* out,
                                                          int64_t osb, int64_t oss, int64_t osh, int Sn, int H,
                                                          int D, const T* cosp, const T* sinp, int64_t cs,
                                                          int64_t cs_rows, const int64_t* pos, int64_t total) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int half = D / 2;
  const int d = (int)(t % half);
  int64_t row = t / half;
  const int h = (int)(row % H);
  row /= H;
  const int s = (int)(row % Sn);
  const int b = (int)(row / Sn);
  const int64_t ps = pos ? min(max(pos[(int64_t)b * Sn + s], (int64_t)0), cs_rows - 1) : s;
  const T* xr = x + b * xsb + s * xss + h * xsh;
  T* orow = out + b * osb + s * oss + h * osh;
  const float a = S::ld(xr, d), bb = S::ld(xr, d + half);
  const float c = S::ld(cosp, ps * cs + d), sn = S::ld(sinp, ps * cs + d);
  S::st(orow, d, rope_lo<S>(a, bb, c, sn));
  S::st(orow, d + half, rope_hi<S>(a, bb, c, sn));
}

// One workgroup per 32x64 block; 8 consecutive elements per thread.  `vec`
// (host-checked: key stride 1, every row start 16-byte aligned) loads them
// with one or two 16-byte loads (fewer for 8-bit masks); rows that reach
// past Sk, or strided masks, load element by element.
__device__ inline void classify(float v, int& all_zero, int& all_ninf) {
  all_zero &= (v == 0.f);
  all_ninf &= (v == -INFINITY);
}
__global__ __launch_bounds__(256) void blockmap_kernel(const char* mask, int dtype, int64_t sb, int64_t sh,
                                                       int64_t si, int64_t sj, int mh, int Sq, int Sk,
                                                       int rows, int cols, int vec, uint8_t* out) {
  const int cb = blockIdx.x, rb = blockIdx.y, bh = blockIdx.z;
  const int b = bh / mh, h = bh % mh;
  const int tid = threadIdx.x;
  const int i = rb * TRINIX_BLOCKMAP_ROWS + tid / 8;
  const int jb = cb * TRINIX_BLOCKMAP_COLS + (tid % 8) * 8;
  const int esz = dtype == TRINIX_F32 ? 4 : (dtype == TRINIX_U8 ? 1 : 2);
  int all_zero = 1, all_ninf = 1;
  if (i < Sq) {
    const char* rowp = mask + (b * sb + h * sh + (int64_t)i * si) * esz;
    if (vec && jb + 8 <= Sk) {
      const char* p8 = rowp + (int64_t)jb * esz;
      switch (dtype) {
        case TRINIX_F32: {
          const float4 a = *(const float4*)p8, c = *(const float4*)(p8 + 16);
          classify(a.x, all_zero, all_ninf); classify(a.y, all_zero, all_ninf);
          classify(a.z, all_zero, all_ninf); classify(a.w, all_zero, all_ninf);
          classify(c.x, all_zero, all_ninf); classify(c.y, all_zero, all_ninf);
          classify(c.z, all_zero, all_ninf); classify(c.w, all_zero, all_ninf);
          break;
        }
        case TRINIX_F16:
        case TRINIX_BF16: {
          const uint4 w = *(const uint4*)p8;
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = dtype == TRINIX_F16 ? F16::lo(ws[e]) : BF16::lo(ws[e]);
            const float hi = dtype == TRINIX_F16 ? F16::hi(ws[e]) : BF16::hi(ws[e]);
            classify(lo, all_zero, all_ninf);
            classify(hi, all_zero, all_ninf);
          }
          break;
        }
        default: {
          const uint2 w = *(const uint2*)p8;
          // bytes: all zero <=> both words zero; an 8-bit mask is never -inf
          all_zero &= (w.x == 0u && w.y == 0u);
          all_ninf = 0;
          break;
        }
      }
    } else {
      for (int e = 0; e < 8; ++e) {
        const int j = jb + e;
        if (j >= Sk) break;
        float v;
        const int64_t idx = (int64_t)j * sj;
        switch (dtype) {
          case TRINIX_F32: v = ((const float*)rowp)[idx]; break;
          case TRINIX_F16: v = (float)((const _Float16*)rowp)[idx]; break;
          case TRINIX_BF16: v = __uint_as_float(((uint32_t)((const uint16_t*)rowp)[idx]) << 16); break;
          default: v = (float)((const uint8_t*)rowp)[idx]; break;
        }
        classify(v, all_zero, all_ninf);
      }
    }
  }
  all_zero = __syncthreads_and(all_zero);
  all_ninf = __syncthreads_and(all_ninf);
  if (tid == 0) {
    const uint8_t code = all_zero ? 0 : (all_ninf ? 2 : 1);
    out[((int64_t)bh * rows + rb) * cols + cb] = code;
  }
}

}  // namespace trinix

using namespace trinix;

extern "C" {

int trinix_rope_apply(const void* x, const int64_t xs[4], void* out, const int64_t os[4], int64_t batch,
                      int64_t seqlen, int64_t nheads, int64_t head_dim, int32_t dtype, const void* cosp,
                      const void* sinp, int64_t cs, int64_t cs_rows, const int64_t* position_ids,
                      void* stream) {
  if (!x || !out || !cosp || !sinp || !xs || !os) return TRINIX_ERR_NULL_POINTER;
  if (cs_rows < (position_ids ? 1 : seqlen)) return TRINIX_ERR_BAD_SHAPE;
  if (batch <= 0 || seqlen <= 0 || nheads <= 0 || head_dim <= 0 || head_dim % 2) return TRINIX_ERR_BAD_SHAPE;
  if (xs[3] != 1 || os[3] != 1) return TRINIX_ERR_BAD_STRIDE;
  if (seqlen >= (1ll << 31) || batch >= (1ll << 31) || nheads >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  hipError_t err;
  const int S = (int)seqlen, H = (int)nheads, D = (int)head_dim;
  const bool vec = dtype != TRINIX_F32 && D % 16 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                   ((uintptr_t)cosp & 15) == 0 && ((uintptr_t)sinp & 15) == 0 && cs % 8 == 0 &&
                   xs[0] % 8 == 0 && xs[1] % 8 == 0 && xs[2] % 8 == 0 && os[0] % 8 == 0 && os[1] % 8 == 0 &&
                   os[2] % 8 == 0;
  if (vec) {
    const int64_t total = batch * seqlen * nheads * (D / 16);
    const dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == TRINIX_BF16)
      err = launch_kernel(&rope16_kernel<BF16>, grid, dim3(256), 0, st, (const uint16_t*)x, xs[0], xs[1], xs[2],
                         (uint16_t*)out, os[0], os[1], os[2], S, H, D, (const uint16_t*)cosp,
                         (const uint16_t*)sinp, cs, cs_rows, position_ids, total);
    else if (dtype == TRINIX_F16)
      err = launch_kernel(&rope16_kernel<F16>, grid, dim3(256), 0, st, (const uint16_t*)x, xs[0], xs[1], xs[2],
                         (uint16_t*)out, os[0], os[1], os[2], S, H, D, (const uint16_t*)cosp,
                         (const uint16_t*)sinp, cs, cs_rows, position_ids, total);
    else
      return TRINIX_ERR_BAD_DTYPE;
  } else {
    const int64_t total = batch * seqlen * nheads * (D / 2);
    const dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == TRINIX_BF16)
      err = launch_kernel(&rope_scalar_kernel<BF16Scalar, uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)x,
                         xs[0], xs[1], xs[2], (uint16_t*)out, os[0], os[1], os[2], S, H, D,
                         (const uint16_t*)cosp, (const uint16_t*)sinp, cs, cs_rows, position_ids, total);
    else if (dtype == TRINIX_F16)
      err = launch_kernel(&rope_scalar_kernel<F16Scalar, uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)x,
                         xs[0], xs[1], xs[2], (uint16_t*)out, os[0], os[1], os[2], S, H, D,
                         (const uint16_t*)cosp, (const uint16_t*)sinp, cs, cs_rows, position_ids, total);
    else if (dtype == TRINIX_F32)
      err = launch_kernel(&rope_scalar_kernel<F32Scalar, float>, grid, dim3(256), 0, st, (const float*)x, xs[0],
                         xs[1], xs[2], (float*)out, os[0], os[1], os[2], S, H, D, (const float*)cosp,
                         (const float*)sinp, cs, cs_rows, position_ids, total);
    else
      return TRINIX_ERR_BAD_DTYPE;
  }
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

int trinix_attn_mask_blockmap(const void* mask, int32_t mask_dtype, int64_t mb, int64_t mh, int64_t seqlen_q,
                              int64_t seqlen_k, const int64_t stride[4], uint8_t* out, void* stream) {
  if (!mask || !out || !stride) return TRINIX_ERR_NULL_POINTER;
  if (mask_dtype != TRINIX_F32 && mask_dtype != TRINIX_F16 && mask_dtype != TRINIX_BF16 && mask_dtype != TRINIX_U8)
    return TRINIX_ERR_BAD_DTYPE;
  if (mb <= 0 || mh <= 0 || seqlen_q <= 0 || seqlen_k <= 0) return TRINIX_ERR_BAD_SHAPE;
  if (seqlen_q >= (1ll << 30) || seqlen_k >= (1ll << 30) || mb * mh >= 65536) return TRINIX_ERR_BAD_SHAPE;
  const int rows = (int)((seqlen_q + TRINIX_BLOCKMAP_ROWS - 1) / TRINIX_BLOCKMAP_ROWS);
  const int cols = (int)((seqlen_k + TRINIX_BLOCKMAP_COLS - 1) / TRINIX_BLOCKMAP_COLS);
  if (rows >= 65536) return TRINIX_ERR_BAD_SHAPE;
  // 16-byte loads of 8 elements when every row start is 16-byte aligned and
  // the key stride is 1 (element strides of the batch / head / row axes are
  // multiples of 16 bytes, or those axes have one entry)
  const int64_t esz = mask_dtype == TRINIX_F32 ? 4 : (mask_dtype == TRINIX_U8 ? 1 : 2);
  const int64_t align = mask_dtype == TRINIX_U8 ? 8 : 16;
  auto aligned = [&](int64_t s, int64_t n) { return n <= 1 || (s * esz) % align == 0; };
  const int vec = stride[3] == 1 && ((uintptr_t)mask % align) == 0 && aligned(stride[0], mb) &&
                  aligned(stride[1], mh) && aligned(stride[2], seqlen_q);
  hipStream_t st = (hipStream_t)stream;
  const hipError_t err = launch_kernel(&blockmap_kernel, dim3(cols, rows, (unsigned)(mb * mh)), dim3(256), 0, st,
                                       (const char*)mask, (int)mask_dtype, stride[0], stride[1], stride[2], stride[3],
                                       (int)mh, (int)seqlen_q, (int)seqlen_k, rows, cols, vec, out);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}

}  // extern "C"
