// Shared device-side definitions of the angle-domain compressed-KV kernels
// (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace sphkv {

constexpr int kHeaderBytes = 8;     // paging.py:2 HEADER_BYTES (config.py:3)
constexpr int kDenseTier = 0xFF;    // header tier id of a dense fp16 K page
constexpr int kTile = 16;           // tokens per page handled as one MFMA tile
constexpr int kWave = 64;

// Tier geometry of tiers.py:35-41 (tier id -> group size, bits per code).
__host__ __device__ constexpr int tier_g(int tid) { return tid == 3 ? 32 : 16; }
__host__ __device__ constexpr int tier_b(int tid) { return tid == 1 ? 6 : (tid == 2 ? 4 : 3); }
__host__ __device__ constexpr int tier_C(int tid) { return 1 << tier_b(tid); }

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Orders this wave's LDS traffic: every LDS access issued before the call is
// complete before any issued after it.  Waves do not wait for each other.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Every per-page load is a buffer load against a resource that covers exactly
// the bytes that page may need; a resource of 0 bytes makes the load return
// zeros without touching memory.  So each loop iteration issues the same
// loads in the same order whatever the page holds, and the vmcnt waits the
// compiler derives are exact (a branch around a load makes them conservative,
// down to waiting for every prefetch in flight).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kOOB = 0x7FFFFF00;       // offset beyond any resource

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// xor-shuffle within a wave (ds_bpermute / DPP chosen by the compiler).
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }

// Reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with the gfx950 row-swap instructions (VALU, no LDS round trip).
// v_permlane32_swap a, b: a's upper 32 lanes <-> b's lower 32 lanes;
// v_permlane16_swap a, b: a's odd rows <-> b's even rows.  With a = b = x the
// sum a + b pairs every lane with its partner row.  Issued as inline asm: the
// clang builtin of this toolchain reads the first result twice when both
// inputs are the same value, and the instructions need the s_nop guard
// (measured: results are wrong without it, right with it).
__device__ __forceinline__ void swap32(float& a, float& b) {
  asm volatile("s_nop 4\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(float& a, float& b) {
  asm volatile("s_nop 4\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float rows_max(float x) {
  float a = x, b = x;
  swap32(a, b);
  float c = fmaxf(a, b), d = c;
  swap16(c, d);
  return fmaxf(c, d);
}
__device__ __forceinline__ float rows_sum(float x) {
  float a = x, b = x;
  swap32(a, b);
  float c = a + b, d = c;
  swap16(c, d);
  return c + d;
}
__device__ __forceinline__ uint32_t rows_or(uint32_t x) {
  float a = __builtin_bit_cast(float, x), b = a;
  swap32(a, b);
  float c = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, a) | __builtin_bit_cast(uint32_t, b)), d = c;
  swap16(c, d);
  return __builtin_bit_cast(uint32_t, c) | __builtin_bit_cast(uint32_t, d);
}

// ---- bit-exact torch CPU arithmetic of _encode_keys_with_codebooks
// (spherical_kv_pipeline.py:1136-1144), shared by the fused encode and the
// decode-time tail.  Every operation is an explicit IEEE fp32 operation
// (fmaf or *_rn), so the result does not depend on the translation unit's
// contraction setting.

// torch CPU fp32 L2 norm of a contiguous group (ATen vectorised last-dim
// reduction, 8 lanes, fused multiply-add accumulation, lanes summed in order).
__device__ __forceinline__ float torch_norm(const float* x, int g) {
  float acc[8];
  for (int l = 0; l < 8; ++l) acc[l] = 0.f;
  for (int d = 0; d < g; d += 8)
    for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(x[d + l], x[d + l], acc[l]);
  float b = acc[0];
  for (int l = 1; l < 8; ++l) b = __fadd_rn(b, acc[l]);
  return __builtin_sqrtf(b);  // correctly rounded expansion (v_sqrt_f32 alone is not)
}

// dir[i] = x[i] / den, correctly rounded, for the GG values of one group
// (den = the group's norm + 1e-8 > 0).  The division's own sequence is a
// reciprocal of den refined once, then the quotient refined twice, framed by
// operand scaling and a special-value fixup; with fp16 inputs (x = 0 or
// 2^-24 <= |x| <= den) and a finite den, neither the scaling nor the fixup
// changes anything (no operand or quotient is denormal or near overflow), so
// the same steps run with the reciprocal shared by the group and give the
// same bits.  (The fixup gives a zero quotient the sign of x; copysign does
// here.)  Other inputs divide each value on its own.
template <int GG>
__device__ __forceinline__ void group_directions(const float* x, float den, bool fp16_in, float* dir) {
  if (fp16_in && den < 1e30f) {
    const float r0 = __builtin_amdgcn_rcpf(den);
    const float r = __builtin_fmaf(__builtin_fmaf(-den, r0, 1.0f), r0, r0);
#pragma unroll
    for (int i = 0; i < GG; ++i) {
      const float q = __fmul_rn(x[i], r);
      const float q1 = __builtin_fmaf(__builtin_fmaf(-den, q, x[i]), r, q);
      const float q2 = __builtin_fmaf(__builtin_fmaf(-den, q1, x[i]), r, q1);
      dir[i] = __builtin_copysignf(q2, x[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < GG; ++i) dir[i] = __fdiv_rn(x[i], den);
  }
}

}  // namespace sphkv
