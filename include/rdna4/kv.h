// Drop-in replacement of rdna4-infer's include/rdna4/kv.h (host side).
//
// Keeps the reference's names, values and semantics -- KvType (kv.h:89-98),
// the q5_0 / q4_1 block layouts (kv.h:70-87),
// kv_type_name/parse (kv.h:100-137), kv_bytes_per_elem (kv.h:139),
// kv_row_bytes (kv.h:155), kv_fill_launch (kv.h:632), kv_store_row_launch
// (kv.h:673-694) and the abort-on-unknown-type contract of kv_unreachable
// (kv.h:58-69) -- and forwards every launch to librdna4attn (gfx950). The
// device-side readers kv_load<> / kv_load8<> (kv.h:174-368) are defined here
// for HIP translation units (tests and benches call them); they return the
// same f32 bits as the reference's.
#pragma once
#include <hip/hip_runtime_api.h>
#if defined(__HIPCC__)
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#define RD4_SHIM_HD __host__ __device__
#else
#define RD4_SHIM_HD
#endif

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "../rdna4attn.h"

namespace rdna4 {

enum class KvType : std::uint32_t { F32 = 0, F16 = 1, Q8_0 = 2, Q4_0 = 3, Q5_0 = 4, Q4_1 = 5 };

// 32-element blocks of the two types the KV cache adds to the weight formats
// (same bytes as llama.cpp's ggml-common.h): d and m are IEEE f16 bits.
struct block_q5_0 {
  std::uint16_t d;
  std::uint8_t qh[4];  // 5th bit of element e: bit (e & 7) of qh[e >> 3]
  std::uint8_t qs[16]; // element j low nibble, j + 16 high nibble
};
struct block_q4_1 {
  std::uint16_t d;
  std::uint16_t m;
  std::uint8_t qs[16];
};
static_assert(sizeof(block_q5_0) == 22, "block_q5_0 is 22 bytes");
static_assert(sizeof(block_q4_1) == 20, "block_q4_1 is 20 bytes");

// A value outside the enum is a programming error: abort on the host (trap on
// the device) instead of guessing.
[[noreturn]] RD4_SHIM_HD inline void kv_unreachable(const char *what) {
#if defined(__HIP_DEVICE_COMPILE__)
  (void)what;
  __builtin_trap();
#else
  std::fprintf(stderr, "rdna4: %s: unknown KvType -- the value is outside the enum\n", what);
  std::abort();
#endif
}

inline const char *kv_type_name(KvType t) { return rd4_kv_type_name((int)t); }

struct KvTypeName {
  const char *name;
  KvType t;
};
inline constexpr KvTypeName kKvTypeNames[] = {
    {"f32", KvType::F32},   {"f16", KvType::F16},   {"q8_0", KvType::Q8_0},
    {"q4_0", KvType::Q4_0}, {"q5_0", KvType::Q5_0}, {"q4_1", KvType::Q4_1}};

// nullptr and *out set on success, otherwise the error message.
inline const char *kv_type_parse(const char *name, KvType *out) {
  int v = -1;
  const char *err = rd4_kv_type_parse(name, &v);
  if (err == nullptr) *out = (KvType)v;
  return err;
}

inline double kv_bytes_per_elem(KvType t) {
  const double b = rd4_kv_bytes_per_elem((int)t);
  if (!(b > 0.0)) kv_unreachable("kv_bytes_per_elem");
  return b;
}

// Bytes of one head_dim row; the same table as the library, usable in device code.
RD4_SHIM_HD inline std::uint64_t kv_row_bytes(KvType t, int head_dim) {
  const std::uint64_t blocks = (std::uint64_t)(head_dim + 31) / 32;
  switch (t) {
    case KvType::F32: return (std::uint64_t)head_dim * 4;
    case KvType::F16: return (std::uint64_t)head_dim * 2;
    case KvType::Q8_0: return blocks * 34;
    case KvType::Q4_0: return blocks * 18;
    case KvType::Q5_0: return blocks * 22;
    case KvType::Q4_1: return blocks * 20;
  }
  kv_unreachable("kv_row_bytes");
}

inline bool kv_fill_launch(KvType t, void *d_cache, std::int64_t n_rows, int head_dim,
                           unsigned seed, hipStream_t stream = nullptr) {
  return rd4_kv_fill_launch((int)t, d_cache, n_rows, head_dim, seed, (void *)stream) == RD4_OK;
}

// `head_dim` is the element count: one row, or n_tok*n_head_kv*head_dim rows.
inline bool kv_store_row_launch(KvType t, const float *d_src, void *d_dst, int head_dim,
                                hipStream_t stream = nullptr) {
  return rd4_kv_store_row_launch((int)t, d_src, d_dst, head_dim, (void *)stream) == RD4_OK;
}

template <KvType CT>
inline bool kv_store_row_launch(const float *d_src, void *d_dst, int head_dim,
                                hipStream_t stream = nullptr) {
  return kv_store_row_launch(CT, d_src, d_dst, head_dim, stream);
}

#if defined(__HIPCC__)
// ---- device readers (kv.h:174-368) ------------------------------------------
// Element e of a stored row as f32. Every product below is exact in f32 (an
// 11-bit f16 significand times an integer of at most 8 bits), except q4_1's
// d*q + m, which keeps the reference's two roundings (no fused multiply-add).
namespace kv_detail {
__device__ __forceinline__ float h2f(const void *p) {
  return __half2float(__ushort_as_half(*(const std::uint16_t *)p));
}
template <KvType CT>
__device__ __forceinline__ float elem(const std::uint8_t *row, int e) {
  if constexpr (CT == KvType::F32) {
    return ((const float *)row)[e];
  } else if constexpr (CT == KvType::F16) {
    return h2f(row + 2 * e);
  } else {
    const int j = e & 31;
    if constexpr (CT == KvType::Q8_0) {
      const std::uint8_t *b = row + 34 * (e >> 5);
      return h2f(b) * (float)(std::int8_t)b[2 + j];
    } else if constexpr (CT == KvType::Q4_0) {
      const std::uint8_t *b = row + 18 * (e >> 5);
      const int q = (b[2 + (j & 15)] >> (j < 16 ? 0 : 4)) & 15;
      return h2f(b) * (float)(q - 8);
    } else if constexpr (CT == KvType::Q5_0) {
      const std::uint8_t *b = row + 22 * (e >> 5);
      const int q = ((b[6 + (j & 15)] >> (j < 16 ? 0 : 4)) & 15) | (((b[2 + (j >> 3)] >> (j & 7)) & 1) << 4);
      return h2f(b) * (float)(q - 16);
    } else {
      const std::uint8_t *b = row + 20 * (e >> 5);
      const int q = (b[4 + (j & 15)] >> (j < 16 ? 0 : 4)) & 15;
      return __fadd_rn(__fmul_rn(h2f(b), (float)q), h2f(b + 2));
    }
  }
}
}  // namespace kv_detail

template <KvType CT>
__device__ __forceinline__ float kv_load(const void *row, int d) {
  return kv_detail::elem<CT>((const std::uint8_t *)row, d);
}

// Dims lane*8 .. lane*8+7 of a row, the same values as 8 kv_load calls.
template <KvType CT>
__device__ __forceinline__ void kv_load8(const void *row, int lane, float out[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = kv_detail::elem<CT>((const std::uint8_t *)row, lane * 8 + i);
}
#endif  // __HIPCC__

}  // namespace rdna4
