// Drop-in replacement of the KV budget helpers of rdna4-infer's
// include/rdna4/device.h (kQwen35KvElemsPerToken :43, kAllocatorMarginBytes /
// kRuntimeReserveBytes / kOverheadBytes :157-162, kMaxCtxSize :168,
// kv_cache_bytes :176-185, required_bytes :191-194), forwarding to librdna4attn.
// The rest of device.h (device query, gfx1201 checks, graph buffer mirror) is
// engine code outside this library.
#pragma once
#include <cstdint>

#include "rdna4/kv.h"

namespace rdna4 {

inline constexpr std::uint64_t kQwen35KvElemsPerToken = 16u * 4u * (256u + 256u);
inline constexpr std::uint64_t kAllocatorMarginBytes = 384u << 20;
inline constexpr std::uint64_t kRuntimeReserveBytes = 64u << 20;
inline constexpr std::uint64_t kOverheadBytes = kAllocatorMarginBytes + kRuntimeReserveBytes;
inline constexpr std::uint64_t kMaxCtxSize = 1u << 24;

inline std::uint64_t kv_cache_bytes(std::uint64_t ctx_size, KvType kv_k, KvType kv_v) {
  return rd4_kv_cache_bytes(ctx_size, (int)kv_k, (int)kv_v);
}
inline std::uint64_t kv_cache_bytes(std::uint64_t ctx_size, const char *kv_k, const char *kv_v) {
  KvType k = KvType::F16, v = KvType::F16;
  if (kv_type_parse(kv_k, &k) != nullptr || kv_type_parse(kv_v, &v) != nullptr) return 0;
  return kv_cache_bytes(ctx_size, k, v);
}
inline std::uint64_t required_bytes(std::uint64_t weights_bytes, std::uint64_t ctx_size,
                                    KvType kv_k, KvType kv_v, std::uint64_t buffers_bytes) {
  return weights_bytes + buffers_bytes + kv_cache_bytes(ctx_size, kv_k, kv_v) + kOverheadBytes;
}
// Largest --ctx-size whose caches fit in budget after the weights, buffers and
// overhead (no counterpart in the reference; the MI355X budget is 288 GB).
inline std::uint64_t max_ctx_size(std::uint64_t budget_bytes, std::uint64_t weights_bytes,
                                  std::uint64_t buffers_bytes, KvType kv_k, KvType kv_v) {
  return rd4_kv_max_ctx(budget_bytes, weights_bytes + buffers_bytes + kOverheadBytes, 16, 4, 256,
                        (int)kv_k, (int)kv_v);
}

}  // namespace rdna4
