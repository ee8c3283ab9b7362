// Block quantizers shared by the KV store kernel and the fused decode append.
//
// Reference semantics: kv_store_row_kernel (include/rdna4/kv.h:386-501), i.e.
// llama.cpp's quantize_row_{q8_0,q4_0,q5_0,q4_1}_ref. One 32-element block per
// 8-lane group, 4 elements per lane; statistics are reduced with xor shuffles
// (order independent, or carrying the element index for the first-occurrence
// tie-break), and every f32 step is rounded on its own (mul_rn / add_rn /
// sub_rn, never fused into an FMA), as in the reference's host mirror and
// llama.cpp's reference quantizers. The bytes equal the serial loop's.
#pragma once
#include "common.hpp"

namespace rd4 {

__device__ __forceinline__ int trunc_i8_clamp(float v, int hi) {
  int q = (int)(int8_t)(int)v;  // C's (int8_t) conversion: truncation toward zero
  return q > hi ? hi : (q < 0 ? 0 : q);
}

// Signed value of largest magnitude over the 32-element block held by this
// 8-lane group (4 elements per lane, element index 4*sub+i); ties go to the
// lowest index, and an all-zero block gives +0 (kv.h:478-485).
__device__ __forceinline__ float group_signed_absmax(const float x[4], int sub) {
  float am = 0.0f, vm = 0.0f;
  int ix = 1 << 30;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (am < fabsf(x[i])) {
      am = fabsf(x[i]);
      vm = x[i];
      ix = 4 * sub + i;
    }
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) {
    const float am2 = xor_f(am, m), vm2 = xor_f(vm, m);
    const int ix2 = __shfl_xor(ix, m, 64);
    if (am2 > am || (am2 == am && ix2 < ix)) {
      am = am2;
      vm = vm2;
      ix = ix2;
    }
  }
  return vm;
}

// Quantize the block whose 32 source values sit 4 per lane in the 8-lane group
// (lane `sub` holds elements 4*sub..4*sub+3) into `blk`.
template <int T>
__device__ __forceinline__ void quant_block8(const float x[4], int sub, uint8_t *blk) {
  if constexpr (T == Q8_0) {
    float am = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) am = fmaxf(am, xor_f(am, m));
    const float d = __fdiv_rn(am, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) w |= ((uint32_t)(uint8_t)(int8_t)(int)roundf(mul_rn(x[i], id))) << (8 * i);
    if (sub == 0) st_u16(blk, f2h(d));
    st_u16(blk + 2 + 4 * sub, (uint16_t)w);
    st_u16(blk + 4 + 4 * sub, (uint16_t)(w >> 16));
  } else if constexpr (T == Q4_0 || T == Q5_0) {
    constexpr float kDiv = (T == Q4_0) ? -8.0f : -16.0f;
    constexpr float kOff = (T == Q4_0) ? 8.5f : 16.5f;
    constexpr int kMax = (T == Q4_0) ? 15 : 31;
    constexpr int kQs = (T == Q4_0) ? 2 : 6;
    const float d = __fdiv_rn(group_signed_absmax(x, sub), kDiv);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t nib = 0, bits = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = trunc_i8_clamp(add_rn(mul_rn(x[i], id), kOff), kMax);
      nib |= (uint32_t)(q & 15) << (8 * i);
      bits |= (uint32_t)(q >> 4) << (4 * sub + i);
    }
    const uint32_t hi_nib = xor_u(nib, 4);  // lanes 4..7 hold elements 16..31
    if constexpr (T == Q5_0) {
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) bits |= xor_u(bits, m);
    }
    if (sub == 0) {
      st_u16(blk, f2h(d));
      if constexpr (T == Q5_0) {
        st_u16(blk + 2, (uint16_t)bits);
        st_u16(blk + 4, (uint16_t)(bits >> 16));
      }
    }
    if (sub < 4) {
      const uint32_t w = nib | (hi_nib << 4);
      st_u16(blk + kQs + 4 * sub, (uint16_t)w);
      st_u16(blk + kQs + 2 + 4 * sub, (uint16_t)(w >> 16));
    }
  } else if constexpr (T == Q4_1) {
    float lo = fminf(fminf(x[0], x[1]), fminf(x[2], x[3]));
    float hi = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      lo = fminf(lo, xor_f(lo, m));
      hi = fmaxf(hi, xor_f(hi, m));
    }
    const float d = __fdiv_rn(sub_rn(hi, lo), 15.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t nib = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = trunc_i8_clamp(add_rn(mul_rn(sub_rn(x[i], lo), id), 0.5f), 15);
      nib |= (uint32_t)q << (8 * i);
    }
    const uint32_t hi_nib = xor_u(nib, 4);
    if (sub == 0) {
      st_u16(blk, f2h(d));
      st_u16(blk + 2, f2h(lo));
    }
    if (sub < 4) {
      const uint32_t w = nib | (hi_nib << 4);
      st_u16(blk + 4 + 4 * sub, (uint16_t)w);
      st_u16(blk + 6 + 4 * sub, (uint16_t)(w >> 16));
    }
  }
}

// Store the 4 values of this lane (elements 4*sub..+3 of block `blk`) as type T.
// F32/F16: element-wise at element offset e of dst.
template <int T>
__device__ __forceinline__ void store_group4(const float x[4], int sub, uint8_t *row, int blk) {
  if constexpr (T == F32) {
    float *p = (float *)row + blk * 32 + 4 * sub;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = x[i];
  } else if constexpr (T == F16) {
    uint16_t *p = (uint16_t *)row + blk * 32 + 4 * sub;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = f2h(x[i]);
  } else {
    quant_block8<T>(x, sub, row + blk * block_bytes(T));
  }
}

}  // namespace rd4
