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
#include "kv_quant.hpp"

namespace rd4 {

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
