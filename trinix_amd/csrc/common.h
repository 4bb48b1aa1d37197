// Shared device helpers for the gfx950 attention library: element traits
// (bf16 / fp16 storage, fp32 math), MFMA wrappers and the workgroup->work
// mapping across the 8 XCDs of an MI355X.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <type_traits>
#include <utility>

#include "index_map.h"

namespace trinix {

// Launches `kernel` on `st` through hipLaunchKernel and returns the status of
// this launch alone.  hipGetLastError is never called, so an error an
// earlier call left for the caller stays there for the caller to read.
// Arguments are converted to the kernel's parameter types first.
template <typename... KArgs, typename... Args>
inline hipError_t launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem, hipStream_t st,
                                Args&&... args) {
  static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
  std::tuple<std::decay_t<KArgs>...> vals(static_cast<std::decay_t<KArgs>>(std::forward<Args>(args))...);
  return std::apply(
      [&](auto&... v) {
        void* ptrs[] = {static_cast<void*>(&v)...};
        return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, shmem, st);
      },
      vals);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 16-bit storage types.  A 32-bit word holds two elements, element 0 in the
// low half.  pack() rounds to nearest-even (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32).  mfma() is D = A*B + C for a 32x32x16 tile: lane l
// supplies row (l%32) of A and column (l%32) of B, 8 consecutive k each for
// k-group l/32; D element v of lane l is row (v/4)*8 + (l/32)*4 + v%4,
// column l%32.  mfma16() is the 16x16x32 tile: lane l supplies row (l%16)
// of A and column (l%16) of B, 8 consecutive k each for k-group l/16; D
// element v of lane l is row (l/16)*4 + v, column l%16.
struct BF16 {
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
  }
  // acc + lo(w) + hi(w) (v_dot2_f32_bf16 against (1, 1))
  __device__ static inline float dot2_ones(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, 0x3f803f80u),
                                           acc, false);
  }
  __device__ static inline f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};

struct F16 {
  __device__ static inline float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[0]; }
  __device__ static inline float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[1]; }
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
  }
  // acc + lo(w) + hi(w) (v_dot2_f32_f16 against (1, 1))
  __device__ static inline float dot2_ones(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
  }
  __device__ static inline f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

// Round an fp32 value to the storage precision of E and back.
template <class E>
__device__ inline float round_to(float x) { return E::lo(E::pack(x, 0.f)); }

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC'11), the counter-based generator used for dropout.
// A round is two v_mad_u64_u32 (each 32x32 -> 64-bit product gives hi and
// lo at once, where __umulhi and a 32-bit multiply are two instructions) and
// two v_bitop3_b32 (gfx950; truth table 0x96 = a ^ b ^ c in one
// instruction).  Same values as the textbook round; a causal dropout forward
// at B=1, S=8192, 32 heads, D=128 took 0.92 ms with the four-multiply form
// and 0.80 ms with this one.
struct Philox {
  __device__ static inline u32x4_t run(u32x4_t c, uint32_t k0, uint32_t k1) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
      const uint64_t p0 = (uint64_t)M0 * c[0], p1 = (uint64_t)M1 * c[2];
      const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0, hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
      c = (u32x4_t){(uint32_t)__builtin_amdgcn_bitop3_b32(hi1, c[1], k0, 0x96), lo1,
                    (uint32_t)__builtin_amdgcn_bitop3_b32(hi0, c[3], k1, 0x96), lo0};
      k0 += W0;
      k1 += W1;
    }
    return c;
  }
};

// Dropout keep decisions.  One Philox call, counter (j/8, i, b*H+h,
// offset_lo) and key (seed_lo ^ offset_hi, seed_hi), decides keys
// 8*(j/8) .. +7 of row i: key 8m + k takes 16-bit field k of the four words
// (word k/2, the low half for even k) and is kept when that field is at
// least drop_thresh = floor(p * 2^16).
__device__ inline bool keep_field(uint32_t w, int half, uint32_t th) { return (half ? (w >> 16) : (w & 0xffffu)) >= th; }

// Keep words of two consecutive 8-key groups (c8, c8 + 1 in units of 8 keys)
// of one row, for a lane pair (l, l + 32) that holds keys 4g .. 4g+3 of each
// group (g = l / 32): lane half g makes the call of group c8 + g, and two
// v_permlane32_swap hand each lane the two words of its own keys of both
// groups (wa: group c8, wb: group c8 + 1; key 4g + e of a group is field e,
// word e / 2).  One call per 8 elements; both lanes of every pair execute it.
__device__ inline void philox_pair_words(uint32_t c8, uint32_t i, uint32_t bh, uint32_t off_lo, uint32_t k0,
                                         uint32_t k1, int g, uint32_t (&wa)[2], uint32_t (&wb)[2]) {
  const u32x4_t w = Philox::run((u32x4_t){c8 + (uint32_t)g, i, bh, off_lo}, k0, k1);
  // swap(x, y): lanes 32..63 of x trade with lanes 0..31 of y, so the first
  // result holds group c8's words in both halves and the second group c8+1's
  const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  wa[0] = s0[0];
  wa[1] = s1[0];
  wb[0] = s0[1];
  wb[1] = s1[1];
}

}  // namespace trinix
