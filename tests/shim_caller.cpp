// A caller written against the reference's rdna4:: API (kv.h, attn.cuh,
// attn_fa2.cuh, nn.cuh's gate) that builds against the include/rdna4 shims and
// links librdna4attn. Host-only checks: tables, parse, admission and argument
// rejection (no kernel runs). Prints "OK" on success.
#include <cstdio>
#include <cstring>
#include <type_traits>

#include "rdna4/attn.cuh"
#include "rdna4/attn_fa2.cuh"
#include "rdna4/attn_gate.h"
#include "rdna4/kv_budget.h"

using namespace rdna4;

// The launchers keep the reference's exact parameter lists.
static_assert(std::is_same_v<decltype(&attn_launch_split),
                             bool (*)(const float *, const void *, const void *, float *, float *,
                                      int, int, int, int, float, KvType, KvType, int,
                                      hipStream_t)>);
static_assert(std::is_same_v<decltype(&fa2_prefill_launch),
                             bool (*)(const float *, const void *, const void *, float *,
                                      const int *, int, int, int, int, int, int, float,
                                      hipStream_t)>);
static_assert(std::is_same_v<decltype(&sigmoid_gate_launch),
                             bool (*)(float *, float *, std::int64_t, hipStream_t)>);
static_assert(std::is_same_v<decltype(&rms_norm_launch),
                             bool (*)(const float *, const float *, float *, std::int64_t,
                                      std::int64_t, float, hipStream_t)>);

// The reference's templated bench overload (attn.cuh:613-628) keeps its form.
static_assert(std::is_same_v<decltype(&attn_launch_split_wpb<KvType::Q8_0, KvType::Q8_0>),
                             bool (*)(const float *, const void *, const void *, float *, float *,
                                      int, int, int, int, float, int, int, hipStream_t)>);

static int fails = 0;
#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
      ++fails;                                                \
    }                                                         \
  } while (0)

int main(int argc, char **argv) {
  if (argc > 1 && std::strcmp(argv[1], "abort") == 0) {
    // kv_unreachable (kv.h:58-69): a KvType outside the enum aborts the process
    const auto n = kv_row_bytes((KvType)99, 256);
    std::printf("no abort: %llu\n", (unsigned long long)n);
    return 0;
  }
  const KvType all[] = {KvType::F32, KvType::F16, KvType::Q8_0,
                        KvType::Q4_0, KvType::Q5_0, KvType::Q4_1};
  const unsigned long long rows[] = {1024, 512, 272, 144, 176, 160};
  for (int i = 0; i < 6; ++i) {
    CHECK(kv_row_bytes(all[i], 256) == rows[i]);
    CHECK((long long)kv_row_bytes(all[i], 256) == rd4_kv_row_bytes((int)all[i], 256));
    CHECK(kv_bytes_per_elem(all[i]) * 256 == (double)rows[i]);
    KvType t = KvType::F32;
    CHECK(kv_type_parse(kKvTypeNames[i].name, &t) == nullptr && t == kKvTypeNames[i].t);
    CHECK(std::strcmp(kv_type_name(all[i]), kKvTypeNames[i].name) == 0);
  }
  KvType t = KvType::Q8_0;
  CHECK(kv_type_parse("q9_9", &t) != nullptr && t == KvType::Q8_0);
  CHECK(attn_partial_bytes(24, 256, 32) == (size_t)24 * 32 * (256 + 2) * sizeof(float));
  CHECK(attn_split_wpb(64) == 8 || attn_split_wpb(64) == 16);
  CHECK(fa2_prefill_usable(KvType::F16, KvType::F16, 512, 0, 24, 4, 256));
  CHECK(!fa2_prefill_usable(KvType::Q8_0, KvType::F16, 512, 0, 24, 4, 256));
  // Argument checks reject before any HIP call: bad head_dim, bad wpb.
  CHECK(!attn_launch_split(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 24, 4, 255, 1.f,
                           KvType::F16, KvType::F16, 1));
  CHECK(!attn_launch_split_wpb(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 24, 4, 256, 1.f,
                               KvType::F16, KvType::F16, 1, 12));
  {
    auto typed = &attn_launch_split_wpb<KvType::F16, KvType::F16>;
    CHECK(!typed(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 24, 4, 256, 1.f, 1, 12, nullptr));
  }
  // device.h budget helpers (check_kvtype.hip:150-152 values)
  CHECK(kv_cache_bytes(131072, KvType::F16, KvType::F16) == 8589934592ull);
  CHECK(kv_cache_bytes(131072, "q8_0", "q8_0") == 4563402752ull);
  CHECK(kv_cache_bytes(131072, "q9_9", "q8_0") == 0);
  CHECK(required_bytes(1000, 0, KvType::F16, KvType::F16, 24) == 1024 + kOverheadBytes);
  CHECK(max_ctx_size(288000000000ull, 20000000000ull, 0, KvType::Q4_0, KvType::Q4_0) > 0);
  std::printf(fails ? "FAILED %d\n" : "OK\n", fails);
  return fails ? 1 : 0;
}
