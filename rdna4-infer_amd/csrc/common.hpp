// Shared device helpers for the gfx950 full-attention library.
//
// KV storage layouts are the reference's (include/rdna4/kv.h:71-98 and
// quants.h:88-101, themselves llama.cpp's ggml-common.h blocks) because the
// cache bytes are the drop-in contract:
//   q8_0 {f16 d; i8 qs[32]}              34 B / 32 elements
//   q4_0 {f16 d; u8 qs[16]}              18 B   element j low nibble, j+16 high
//   q5_0 {f16 d; u8 qh[4]; u8 qs[16]}    22 B   bit 4 of element e = bit e of qh
//   q4_1 {f16 d; f16 m; u8 qs[16]}       20 B
// Every multi-byte field is read and written as 16-bit halves: blocks are only
// 2-byte aligned inside a row.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#pragma clang fp contract(off)

namespace rd4 {

// f32 multiply / add / subtract, each rounded on its own. They are written
// here, under this file's `fp contract(off)`, so no caller can have them fused
// into an FMA: HIP's __fmul_rn / __fadd_rn are defined before that pragma with
// contraction allowed, and a product of one feeding the other does get fused.
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }
__device__ __forceinline__ float sub_rn(float a, float b) { return a - b; }

enum KvType : int { F32 = 0, F16 = 1, Q8_0 = 2, Q4_0 = 3, Q5_0 = 4, Q4_1 = 5 };
constexpr int kNumTypes = 6;

__host__ __device__ constexpr int block_bytes(int t) {
  return t == Q8_0 ? 34 : t == Q4_0 ? 18 : t == Q5_0 ? 22 : t == Q4_1 ? 20 : 0;
}

__host__ __device__ inline int64_t row_bytes(int t, int head_dim) {
  const int64_t blocks = ((int64_t)head_dim + 31) / 32;
  switch (t) {
    case F32: return (int64_t)head_dim * 4;
    case F16: return (int64_t)head_dim * 2;
    case Q8_0:
    case Q4_0:
    case Q5_0:
    case Q4_1: return blocks * block_bytes(t);
    default: return -1;
  }
}

// IEEE f16 bits -> f32 (hardware conversion, exact for every f16 value).
__device__ __forceinline__ float h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// f32 -> f16 bits, round to nearest even, with the reference's special cases
// (include/rdna4/fp16.h:36-57): overflow, inf and NaN give a signed infinity,
// magnitudes below half the smallest subnormal a signed zero. Integer-only, so
// the result cannot depend on the FP mode.
__host__ __device__ __forceinline__ uint16_t f2h(float f) {
  const uint32_t x = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  const int e = (int)(a >> 23) - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const int sh = 14 - e;
    uint32_t r = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)e << 10) | ((a >> 13) & 0x3ffu);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) {
  return *(const uint16_t *)p;
}
__device__ __forceinline__ void st_u16(uint8_t *p, uint16_t v) { *(uint16_t *)p = v; }

// Dequantize 4 consecutive elements [e, e+4) of a stored row (e % 4 == 0), as
// kv_load<> (kv.h:177-229) would return them one by one. Every product here is
// exact in f32; q4_1's d*q + m keeps its two roundings (no FMA).
template <int T>
__device__ __forceinline__ void load4(const uint8_t *row, int64_t e, float out[4]) {
  if constexpr (T == F32) {
    const float *p = (const float *)row + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = p[i];
  } else if constexpr (T == F16) {
    const uint16_t *p = (const uint16_t *)row + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = h2f(p[i]);
  } else {
    const uint8_t *b = row + (e >> 5) * block_bytes(T);
    const int j = (int)(e & 31);
    const float d = h2f(ld_u16(b));
    if constexpr (T == Q8_0) {
      const uint32_t lo = ld_u16(b + 2 + j), hi = ld_u16(b + 4 + j);
      const uint32_t w = lo | (hi << 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = __fmul_rn(d, (float)(int8_t)(w >> (8 * i)));
    } else {
      const int qs_off = (T == Q4_0) ? 2 : (T == Q5_0) ? 6 : 4;
      const int i0 = j & 15;
      const uint32_t lo = ld_u16(b + qs_off + i0), hi = ld_u16(b + qs_off + i0 + 2);
      const uint32_t w = (lo | (hi << 16)) >> ((j & 16) ? 4 : 0);
      if constexpr (T == Q4_0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __fmul_rn(d, (float)((int)((w >> (8 * i)) & 15u) - 8));
      } else if constexpr (T == Q5_0) {
        const uint32_t qh = b[2 + (j >> 3)] >> (j & 7);  // j % 4 == 0: 4 bits stay in one byte
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = (int)((w >> (8 * i)) & 15u) | (int)(((qh >> i) & 1u) << 4);
          out[i] = __fmul_rn(d, (float)(n - 16));
        }
      } else {
        const float m = h2f(ld_u16(b + 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __fadd_rn(__fmul_rn(d, (float)((w >> (8 * i)) & 15u)), m);
      }
    }
  }
}

// Split-half RoPE of one pair (attn.cuh:36-46): the angle pos * base^(-2p/n_rot)
// is formed in f32, and every product and sum rounds on its own (no FMA
// contraction), so the standalone rope kernel and the fused epilogue give the
// same bits.
__device__ __forceinline__ void rope_cs(int pos, int p, int n_rot, float freq_base, float *c,
                                        float *s) {
  const float theta = (float)pos * powf(freq_base, -2.0f * (float)p / (float)n_rot);
  *c = cosf(theta);
  *s = sinf(theta);
}
__device__ __forceinline__ float rope_lo(float x0, float x1, float c, float s) {
  return __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
}
__device__ __forceinline__ float rope_hi(float x0, float x1, float c, float s) {
  return __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

// Wave64 butterfly helpers (lane masks stay inside the 64-lane wavefront).
__device__ __forceinline__ float xor_f(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ uint32_t xor_u(uint32_t v, int m) {
  return (uint32_t)__shfl_xor((int)v, m, 64);
}

}  // namespace rd4
