// ALiBi bias producer (reference trinix/kernels/alibi_kernel.py:8-54):
// out[h][i][j] = -slope[h] * |i - j| in fp32.  HBM-bound: one 4-byte store
// per element, 16-byte stores when a row is 16-byte aligned.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "trinix_attn.h"

namespace {

using trinix::f32x4_t;

// One workgroup per (head, query row); each thread writes runs of 4 keys.
__global__ __launch_bounds__(256) void alibi_bias_kernel(const float* __restrict__ slopes, int64_t sl_stride,
                                                         int64_t seqlen, float* __restrict__ out, int64_t os_h,
                                                         int64_t os_i, int vec4) {
  const int64_t row = blockIdx.x;
  const int64_t h = row / seqlen, i = row % seqlen;
  const float slope = slopes[h * sl_stride];
  float* orow = out + h * os_h + i * os_i;
  // |i - j| < 2^24 is exact in fp32; the product is rounded once, as in
  // the reference's -slope * distance.
  if (vec4) {
    for (int64_t j = (int64_t)threadIdx.x * 4; j < seqlen; j += 1024) {
      f32x4_t v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = -(slope * (float)(i > j + e ? i - (j + e) : (j + e) - i));
      *(f32x4_t*)(orow + j) = v;
    }
  } else {
    for (int64_t j = threadIdx.x; j < seqlen; j += 256) orow[j] = -(slope * (float)(i > j ? i - j : j - i));
  }
}

}  // namespace

extern "C" int trinix_alibi_bias(const float* slopes, int64_t slope_stride, int64_t nheads, int64_t seqlen,
                                 float* out, int64_t out_stride_h, int64_t out_stride_i, void* stream) {
  if (!slopes || !out) return TRINIX_ERR_NULL_POINTER;
  if (nheads <= 0 || seqlen <= 0 || seqlen >= (1ll << 24) || nheads * seqlen >= (1ll << 31)) return TRINIX_ERR_BAD_SHAPE;
  const int vec4 = seqlen % 4 == 0 && out_stride_i % 4 == 0 && out_stride_h % 4 == 0 && ((uintptr_t)out & 15) == 0;
  const hipError_t err = trinix::launch_kernel(alibi_bias_kernel, dim3((unsigned)(nheads * seqlen)), dim3(256), 0,
                                       (hipStream_t)stream, slopes, slope_stride, seqlen, out, out_stride_h,
                                       out_stride_i, vec4);
  return err == hipSuccess ? TRINIX_OK : TRINIX_ERR_LAUNCH;
}
