// KV append/quantize, seeded fill and dequantize-to-f32 kernels (gfx950).
//
// Reference semantics: kv_store_row_kernel (include/rdna4/kv.h:386-501),
// kv_fill_kernel (kv.h:508-671), kv_load (kv.h:174-229).
//
// Layout of the work: one 32-element block per 8-lane group, 4 elements per
// lane, so a wave quantizes 8 blocks and its 64 lanes read 1 KiB of f32 source
// with 16-byte loads. The block statistics (amax, signed max with its
// first-occurrence tie-break, min/max, the q5_0 bit plane) are reduced across
// the 8 lanes with xor shuffles; every statistic is order independent or
// carries its element index, so the bytes equal the serial loop's.
// All arithmetic that the reference performs as separate f32 statements is
// written with explicit round-to-nearest intrinsics so the compiler cannot
// contract it into an FMA.
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
    for (int i = 0; i < 4; ++i) w |= ((uint32_t)(uint8_t)(int8_t)(int)roundf(__fmul_rn(x[i], id))) << (8 * i);
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
      const int q = trunc_i8_clamp(__fadd_rn(__fmul_rn(x[i], id), kOff), kMax);
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
    const float d = __fdiv_rn(__fsub_rn(hi, lo), 15.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t nib = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = trunc_i8_clamp(__fadd_rn(__fmul_rn(__fsub_rn(x[i], lo), id), 0.5f), 15);
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

// Source of the values to store: a f32 array, or the seeded fill hash.
struct SrcArray {
  const float *p;
  __device__ __forceinline__ void get4(int64_t e, float x[4]) const {
    const float4 v = *(const float4 *)(p + e);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  }
  __device__ __forceinline__ float get1(int64_t e) const { return p[e]; }
};

// kv_rand (kv.h:508-513): element e of the flattened cache gets hash(e, seed).
struct SrcHash {
  uint32_t seed;
  __device__ __forceinline__ float get1(int64_t e) const {
    uint32_t h = ((uint32_t)e * 2654435761u) ^ (seed * 2246822519u);
    h ^= h >> 13;
    h *= 1274126177u;
    return __fsub_rn((float)(h >> 8) * (1.0f / 8388608.0f), 1.0f);
  }
  __device__ __forceinline__ void get4(int64_t e, float x[4]) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = get1(e + i);
  }
};

// Quantized types: one block per 8-lane group.
template <int T, class Src>
__global__ __launch_bounds__(256) void kv_store_blocks(Src src, uint8_t *__restrict__ dst,
                                                       int64_t n_blocks) {
  const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int sub = threadIdx.x & 7;
  if (g >= n_blocks) return;  // whole 8-lane groups exit together
  float x[4];
  src.get4(g * 32 + 4 * sub, x);
  quant_block8<T>(x, sub, dst + g * block_bytes(T));
}

// F32/F16: element-wise, 4 per thread with an exact tail.
template <int T, class Src>
__global__ __launch_bounds__(256) void kv_store_elems(Src src, uint8_t *__restrict__ dst,
                                                      int64_t n) {
  const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (e >= n) return;
  if (e + 4 <= n) {
    float x[4];
    src.get4(e, x);
    if constexpr (T == F32) {
      *(float4 *)((float *)dst + e) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
      const uint32_t lo = f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16);
      const uint32_t hi = f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16);
      *(uint2 *)((uint16_t *)dst + e) = make_uint2(lo, hi);
    }
  } else {
    for (int64_t i = e; i < n; ++i) {
      if constexpr (T == F32)
        ((float *)dst)[i] = src.get1(i);
      else
        ((uint16_t *)dst)[i] = f2h(src.get1(i));
    }
  }
}

template <int T>
__global__ __launch_bounds__(256) void kv_load_kernel(const uint8_t *__restrict__ src,
                                                      float *__restrict__ dst, int64_t n) {
  const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (e >= n) return;
  if (e + 4 <= n) {
    float x[4];
    load4<T>(src, e, x);
    *(float4 *)(dst + e) = make_float4(x[0], x[1], x[2], x[3]);
  } else {  // F32/F16 tail (quantized widths are multiples of 32)
    for (int64_t i = e; i < n; ++i)
      dst[i] = (T == F32) ? ((const float *)src)[i] : h2f(((const uint16_t *)src)[i]);
  }
}

}  // namespace rd4

namespace rd4 {

template <int T>
static hipError_t store_typed(const float *src, uint8_t *dst, int64_t width, hipStream_t st) {
  if (width == 0) return hipSuccess;
  if constexpr (T == F32 || T == F16) {
    const int64_t threads = (width + 3) / 4;
    hipLaunchKernelGGL((kv_store_elems<T, SrcArray>), dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, st, SrcArray{src}, dst, width);
  } else {
    const int64_t nb = width / 32;
    hipLaunchKernelGGL((kv_store_blocks<T, SrcArray>), dim3((unsigned)((nb * 8 + 255) / 256)),
                       dim3(256), 0, st, SrcArray{src}, dst, nb);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t fill_typed(uint8_t *dst, int64_t n, uint32_t seed, hipStream_t st) {
  if (n == 0) return hipSuccess;
  if constexpr (T == F32 || T == F16) {
    const int64_t threads = (n + 3) / 4;
    hipLaunchKernelGGL((kv_store_elems<T, SrcHash>), dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, st, SrcHash{seed}, dst, n);
  } else {
    const int64_t nb = n / 32;
    hipLaunchKernelGGL((kv_store_blocks<T, SrcHash>), dim3((unsigned)((nb * 8 + 255) / 256)),
                       dim3(256), 0, st, SrcHash{seed}, dst, nb);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t load_typed(const uint8_t *src, float *dst, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL((kv_load_kernel<T>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, src, dst, n);
  return hipGetLastError();
}

#define RD4_TYPE_SWITCH(t, FN, ...)                  \
  switch (t) {                                       \
    case F32: return FN<F32>(__VA_ARGS__);           \
    case F16: return FN<F16>(__VA_ARGS__);           \
    case Q8_0: return FN<Q8_0>(__VA_ARGS__);         \
    case Q4_0: return FN<Q4_0>(__VA_ARGS__);         \
    case Q5_0: return FN<Q5_0>(__VA_ARGS__);         \
    case Q4_1: return FN<Q4_1>(__VA_ARGS__);         \
    default: return hipErrorInvalidValue;            \
  }

hipError_t kv_store_launch(int t, const float *src, uint8_t *dst, int64_t width, hipStream_t st) {
  RD4_TYPE_SWITCH(t, store_typed, src, dst, width, st)
}
hipError_t kv_fill_launch(int t, uint8_t *dst, int64_t n, uint32_t seed, hipStream_t st) {
  RD4_TYPE_SWITCH(t, fill_typed, dst, n, seed, st)
}
hipError_t kv_load_launch(int t, const uint8_t *src, float *dst, int64_t n, hipStream_t st) {
  RD4_TYPE_SWITCH(t, load_typed, src, dst, n, st)
}

}  // namespace rd4
