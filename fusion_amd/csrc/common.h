// Shared device helpers for the GLM-5.2 MoE block kernels (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this library:
//   * bf16 tensors are passed as `const uint16_t*` and converted with the helpers
//     below; fp32 -> bf16 is round-to-nearest-even with NaN mapped to 0x7fc0, which is
//     the rounding torch's `.to(torch.bfloat16)` applies.
//   * 16-byte (8 x bf16) vector accesses use `uint4`; callers guarantee 16-byte
//     alignment of the base pointers and of every row stride they pass.
//   * Every launch goes on the caller's stream and nothing here allocates memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GLM52_DEV __device__ __forceinline__

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

namespace glm52 {

constexpr int kWave = 64;

GLM52_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

GLM52_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Low / high bf16 of a packed 32-bit word, as fp32.
GLM52_DEV float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
GLM52_DEV float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

GLM52_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// Unpack 8 bf16 held in a uint4 into 8 floats.
GLM52_DEV void unpack8(const uint4& v, float* f) {
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x);
  f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z);
  f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}

GLM52_DEV uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

GLM52_DEV bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// Wave-wide fp32 sum (result valid in every lane); fixed butterfly order.
GLM52_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Wave-wide fp64 sum (result valid in every lane); fixed butterfly order.
GLM52_DEV double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// silu(g) * u in fp32, the SwiGLU of `glm52/reference.py:36-40`, with the hardware
// reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE divide, whose ten-instruction expansion
// dominated the prefill GEMM's gated epilogue; every caller rounds the result to bf16.
// g -> -inf: exp overflows and the reciprocal is 0, as the quotient was.
GLM52_DEV float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

}  // namespace glm52

// Error codes returned by every C-ABI entry point (0 = success; positive values are
// hipError_t codes from the launch; negative values are argument errors).
#define GLM52_OK 0
#define GLM52_EINVAL (-1)      // a size / stride / pointer argument is invalid
#define GLM52_EUNSUPPORTED (-2)  // a valid argument combination this build does not implement

#define GLM52_RETURN_LAUNCH()                 \
  do {                                        \
    hipError_t _e = hipGetLastError();        \
    return _e == hipSuccess ? GLM52_OK : (int)_e; \
  } while (0)
