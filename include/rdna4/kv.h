// Drop-in replacement of rdna4-infer's include/rdna4/kv.h (host side).
//
// Keeps the reference's names, values and semantics -- KvType (kv.h:89-98),
// kv_type_name/parse (kv.h:100-137), kv_bytes_per_elem (kv.h:139),
// kv_row_bytes (kv.h:155), kv_fill_launch (kv.h:632), kv_store_row_launch
// (kv.h:673-694) and the abort-on-unknown-type contract of kv_unreachable
// (kv.h:58-69) -- and forwards every launch to librdna4attn (gfx950).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "../rdna4attn.h"

namespace rdna4 {

enum class KvType : std::uint32_t { F32 = 0, F16 = 1, Q8_0 = 2, Q4_0 = 3, Q5_0 = 4, Q4_1 = 5 };

// A value outside the enum is a programming error: abort instead of guessing.
[[noreturn]] inline void kv_unreachable(const char *what) {
  std::fprintf(stderr, "rdna4: %s: unknown KvType -- the value is outside the enum\n", what);
  std::abort();
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
#if defined(__HIPCC__)
__host__ __device__
#endif
inline std::uint64_t kv_row_bytes(KvType t, int head_dim) {
  const std::uint64_t blocks = (std::uint64_t)(head_dim + 31) / 32;
  switch (t) {
    case KvType::F32: return (std::uint64_t)head_dim * 4;
    case KvType::F16: return (std::uint64_t)head_dim * 2;
    case KvType::Q8_0: return blocks * 34;
    case KvType::Q4_0: return blocks * 18;
    case KvType::Q5_0: return blocks * 22;
    case KvType::Q4_1: return blocks * 20;
  }
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_trap();
#else
  kv_unreachable("kv_row_bytes");
#endif
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

}  // namespace rdna4
