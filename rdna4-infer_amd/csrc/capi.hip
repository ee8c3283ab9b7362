// C ABI of the gfx950 full-attention library (declared in include/rdna4attn.h).
//
// Validation, split policy, per-device scratch and dispatch to the kernels. The
// reference's launchers (include/rdna4/attn.cuh, attn_fa2.cuh, kv.h, nn.cuh)
// return false for an unsupported shape or a launch error; these return a
// negative RD4_E* code in the same cases.
#include <cstdio>
#include <cstring>
#include <map>
#include <vector>
#include <mutex>

#include "../../include/rdna4attn.h"
#include "merge.hpp"
#include "prefill.hpp"

namespace rd4 {
hipError_t kv_store_launch(int t, const float *src, uint8_t *dst, int64_t width, hipStream_t st);
hipError_t kv_fill_launch(int t, uint8_t *dst, int64_t n, uint32_t seed, hipStream_t st);
hipError_t kv_load_launch(int t, const uint8_t *src, float *dst, int64_t n, hipStream_t st);
hipError_t sigmoid_gate_launch(float *g, float *y, int64_t n, hipStream_t st);
hipError_t fill_u32_launch(uint32_t *p, int64_t n, uint32_t v, hipStream_t st);
hipError_t read_probe_launch(const void *p, int64_t bytes, uint32_t *sink, hipStream_t st);
hipError_t rope_launch(float *x, int n_tokens, int n_heads, int head_dim, int n_rot,
                       float freq_base, const int *pos, hipStream_t st);
hipError_t rms_norm_launch(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                           float eps, hipStream_t st);
hipError_t qk_epilogue_launch(const float *qg, const float *k, const float *v, const float *qw,
                              const float *kw, float eps, int n_rot, float freq_base,
                              const int *pos, int n_tok, int n_head, int n_head_kv, int head_dim,
                              float *q_out, float *gate_out, float *k_out, uint8_t *kc,
                              uint8_t *vc, int kt, int vt, hipStream_t st);
}  // namespace rd4

using namespace rd4;

namespace {

thread_local char g_err[256] = "";

int fail(int code, const char *fmt, const char *detail = "") {
  std::snprintf(g_err, sizeof(g_err), fmt, detail);
  return code;
}

int launched(hipError_t e, const char *what) {
  if (e == hipSuccess) return RD4_OK;
  std::snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return RD4_ELAUNCH;
}

bool valid_type(int t) { return t >= 0 && t < kNumTypes; }

// Library scratch for split records and merge counters, one set per (device,
// stream): launches on different streams never share records or counters.
// rd4_init creates the null stream's set and one spare. A stream seen for the
// first time gets a new set made by hipMalloc plus a stream-ordered fill kernel
// (no synchronisation), or, while it is capturing a HIP graph (when nothing may
// be allocated), the spare. Sets are never freed. Caller-owned `partial` buffers are used instead when the
// records fit (see run_attn).
constexpr int64_t kPartialFloats = 16ll << 20;  // 64 MiB of records per stream
constexpr int64_t kCounterWords = 1 << 20;
struct Scratch {
  float *partial = nullptr;    // uncached: records exchanged between CTAs inside a launch
  float *partial_c = nullptr;  // cached: records handed to a later launch
  unsigned *counters = nullptr;
};
std::map<std::pair<int, uintptr_t>, Scratch> g_scratch;
std::map<int, std::vector<Scratch>> g_spare;  // per device, made by rd4_init, not yet assigned
std::mutex g_scratch_mu;

// A new set on the current device; its counters are zeroed by a fill kernel on
// `st` (waited for when `blocking`).
int new_scratch(hipStream_t st, bool blocking, Scratch *out) {
  Scratch n;
  // Uncached: the generic kernel's split records cross XCDs inside one launch
  // (see merge.hpp). Uncached memory is never freed once a kernel has read it.
  if (hipExtMallocWithFlags((void **)&n.partial, kPartialFloats * sizeof(float),
                            hipDeviceMallocUncached) != hipSuccess ||
      hipMalloc(&n.partial_c, kPartialFloats * sizeof(float)) != hipSuccess ||
      hipMalloc(&n.counters, kCounterWords * sizeof(unsigned)) != hipSuccess)
    return fail(RD4_ENOMEM, "scratch allocation failed%s");
  const bool ok = fill_u32_launch(n.counters, kCounterWords, 0u, st) == hipSuccess &&
                  (!blocking || hipStreamSynchronize(st) == hipSuccess);
  if (!ok) return fail(RD4_ELAUNCH, "scratch counter fill failed%s");
  *out = n;
  return RD4_OK;
}

int current_device(int *dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0) return fail(RD4_EINVAL, "no current HIP device%s");
  return RD4_OK;
}

int get_scratch(hipStream_t st, Scratch **out) {
  int dev = 0, rc;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find({dev, (uintptr_t)st});
  if (it == g_scratch.end()) {
    Scratch n;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = st && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    std::vector<Scratch> &sp = g_spare[dev];
    if (!capturing) {
      if ((rc = new_scratch(st, false, &n))) return rc;
    } else if (!sp.empty()) {  // nothing may be allocated while a graph is captured
      n = sp.back();
      sp.pop_back();
    } else {
      return fail(RD4_ENOMEM, "no library scratch for this stream: call rd4_init or rd4_stream_init(stream) before capturing%s");
    }
    it = g_scratch.emplace(std::make_pair(dev, (uintptr_t)st), n).first;
  }
  *out = &it->second;
  return RD4_OK;
}

int check_attn_shape(int n_head, int n_head_kv, int head_dim, int kt, int vt) {
  if (!valid_type(kt) || !valid_type(vt)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (head_dim <= 0 || head_dim % 32 != 0 || head_dim / 32 > 16)
    return fail(RD4_EINVAL, "head_dim must be a multiple of 32, at most 512%s");
  if (n_head_kv <= 0 || n_head <= 0 || n_head % n_head_kv != 0)
    return fail(RD4_EINVAL, "n_head must be a positive multiple of n_head_kv%s");
  return RD4_OK;
}

// Splits the GPU wants for `keys` keys of one token: `target` CTAs in total
// (the MFMA kernel's CTA fills a CU; the generic kernel's takes a quarter of
// one), and at least `min_keys` keys per split.
int auto_splits(int keys, int ctas_per_split, int target, int min_keys) {
  static const int env = [] {  // tuning override, read once
    const char *e = std::getenv("RD4_DECODE_SPLITS");
    return e ? std::atoi(e) : 0;
  }();
  if (env >= 1) return env > kMaxSplits ? kMaxSplits : env;
  int s = (target + ctas_per_split - 1) / ctas_per_split;
  const int by_keys = (keys + min_keys - 1) / min_keys;
  if (s > by_keys) s = by_keys;
  if (s > kMaxSplits) s = kMaxSplits;
  return s < 1 ? 1 : s;
}

// Fixed scratch of the allocation-free entry point: records go to `partial`
// (at most `floats` floats) and are merged by the merge launch.
struct FixedScratch {
  float *partial;
  unsigned *counters;
  int64_t floats;
};

// Common body of every decode-style launch.
int run_attn(const float *q, const void *k, const void *v, float *out, float *gate,
             const int *pos, int t, int n_tok, int n_head, int n_head_kv, int head_dim,
             float scale, int kt, int vt, int splits, hipStream_t st,
             const float *k_new = nullptr, const float *v_new = nullptr, int tok_pair = 0,
             float *caller_partial = nullptr, int caller_splits = 0,
             const FixedScratch *fixed = nullptr) {
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  if (n_tok < 1) return fail(RD4_EINVAL, "n_tok must be >= 1%s");
  if (!q || !k || !v || !out) return fail(RD4_EINVAL, "null buffer%s");
  const int n_chunks = (n_head / n_head_kv + 7) / 8;
  const int64_t rec = 2 + head_dim;
  const bool aligned16 = ((((uintptr_t)k) | ((uintptr_t)v) | ((uintptr_t)q)) & 15) == 0;
  const bool mfma = aligned16 && decode_mfma_supported(kt, vt, n_head, n_head_kv, head_dim);
  // RD_ATTN_SPLITS (graph.cuh:509-519): a forced split count for the automatic
  // and minimum-count launches, so the reference's split-vs-unsplit checks
  // (RD_ATTN_SPLITS=1 = one split) mean what they meant.
  static const int env_splits = [] {
    const char *e = std::getenv("RD_ATTN_SPLITS");
    return e ? std::atoi(e) : 0;
  }();
  if (splits <= 0 && env_splits > 0) splits = env_splits > kMaxSplits ? kMaxSplits : env_splits;
  const bool exact = splits > 0;
  const int min_s = exact ? splits : -splits;
  if (splits <= 0) {  // automatic, at least -splits
    // CTAs per split: every token's (kv head, head chunk) pairs; the keys of
    // the first token bound the split count
    // (token pairs share a CTA in the MFMA kernel's pair mode)
    const bool pairs = tok_pair && mfma && decode_mfma_pairs(kt, vt) && n_chunks == 1 && n_tok >= 2 &&
                       !pos && !k_new;
    const int per_split = n_head_kv * n_chunks * (pairs ? (n_tok + 1) / 2 : n_tok);
    splits = mfma ? auto_splits(t + 1, per_split, 256, 64) : auto_splits(t + 1, per_split, 1024, 64);
    if (splits < min_s) splits = min_s;
  }
  if (fixed && !mfma) {
    // the generic kernel merges splits through uncached library scratch: with a
    // fixed scratch it runs one split, which needs no records
    if (exact && splits > 1) return fail(RD4_EINVAL, "this shape takes the generic kernel: n_splits must be 0 or 1 here%s");
    splits = 1;
  }
  if (splits < 1) splits = 1;
  if (splits > kMaxSplits) {
    if (exact || min_s > kMaxSplits) return fail(RD4_EINVAL, "n_splits above the library's maximum (256)%s");
    splits = kMaxSplits;
  }
  AttnArgs a{};
  a.q = q;
  a.k = (const uint8_t *)k;
  a.v = (const uint8_t *)v;
  a.out = out;
  a.gate = gate;
  a.k_new = k_new;
  a.v_new = v_new;
  a.pos = pos;
  a.t = t;
  a.n_head = n_head;
  a.n_head_kv = n_head_kv;
  a.head_dim = head_dim;
  a.scale = scale;
  a.tok_pair = tok_pair;
  if (splits > 1) {
    const int64_t rows = (int64_t)n_tok * n_head;
    if (fixed) {
      // records [head][split][hd] + (m, l) must fit; an automatic count shrinks
      auto fits_fixed = [&](int S) { return rows * S * rec <= fixed->floats; };
      while (!fits_fixed(splits) && !exact && splits > 1) --splits;
      if (!fits_fixed(splits))
        return fail(RD4_EINVAL, "split records exceed the fixed scratch (4 MiB): use fewer splits%s");
      a.partial = fixed->partial;
      a.counters = fixed->counters;
      a.ml0_off = rows * splits * head_dim;
      a.ext_merge = 1;  // the merge launch: records stay in the fixed scratch, no in-kernel tree
      a.n_splits = splits;
      a.dbg = 0;
      return launched(decode_mfma_launch(kt, vt, a, n_tok, st), "decode kernel");
    }
    const bool ext = mfma;  // the MFMA decode merges its records in a second launch
    // (its records are stored as 16-byte vectors: a misaligned buffer is not used)
    const bool use_caller = ext && caller_partial && splits <= caller_splits &&
                            ((uintptr_t)caller_partial & 15) == 0;
    if (!use_caller) {
      // level-0 (+ level-1) records and the counters must fit the stream's scratch
      auto fits = [&](int S, int64_t ntok) {
        const int NG = (S + kMergeFan - 1) / kMergeFan;
        return ntok * n_head * (rec + 2) * (S + (NG > 1 ? NG : 0)) <= kPartialFloats &&
               ntok * n_head_kv * n_chunks * kCtrStride <= kCounterWords;
      };
      // an automatic count above the caller's minimum shrinks to fit first
      while (!fits(splits, n_tok) && splits > min_s && splits > 1) --splits;
      if (!fits(splits, n_tok)) {
        if (!fits(splits, 1)) return fail(RD4_EINVAL, "split records of one token exceed the library scratch (64 MiB)%s");
        // too many tokens at this split count: consecutive launches over token
        // chunks, on the same stream (results are the same as one launch)
        int per = 1;
        while (fits(splits, 2 * per) && 2 * per < n_tok) per *= 2;
        if (tok_pair && per > 1) per &= ~1;
        for (int t0 = 0; t0 < n_tok; t0 += per) {
          const int cnt = n_tok - t0 < per ? n_tok - t0 : per;
          const int64_t off = (int64_t)t0 * n_head * head_dim;
          rc = run_attn(q + off, k, v, out + off, gate ? gate + off : nullptr, pos ? pos + t0 : nullptr,
                        pos ? t : t + t0, cnt, n_head, n_head_kv, head_dim, scale, kt, vt, splits, st,
                        k_new, v_new, tok_pair, nullptr, 0);
          if (rc) return rc;
        }
        return RD4_OK;
      }
    }
    const int NG = (splits + kMergeFan - 1) / kMergeFan;
    a.ml0_off = rows * splits * head_dim;
    if (use_caller) {
      // The caller's partial (sized attn_partial_bytes(n_head, hd, caller_splits)
      // per token) holds the level-0 records [tok][head][split][hd] + (m, l), as
      // in attn.cuh:593-608; the merge launch reads them on the same stream.
      a.partial = caller_partial;
      a.counters = nullptr;
    } else {
      Scratch *s = nullptr;
      if ((rc = get_scratch(st, &s))) return rc;
      // The MFMA decode merges its records in a second launch (cached scratch
      // suffices); the in-kernel merge tree needs the uncached one.
      a.partial = ext ? s->partial_c : s->partial;
      a.counters = s->counters;
    }
    a.acc1_off = a.ml0_off + rows * splits * 2;
    a.acc1_off = (a.acc1_off + 3) / 4 * 4;  // 16-byte aligned level-1 records
    a.ml1_off = a.acc1_off + rows * NG * head_dim;
  }
  a.n_splits = splits;
  static const int dbg = [] { const char *e = std::getenv("RD4_DECODE_DBG"); return e ? std::atoi(e) : 0; }();
  a.dbg = dbg;
  if (mfma)
    return launched(decode_mfma_launch(kt, vt, a, n_tok, st), "decode kernel");
  return launched(attn_generic_launch(kt, vt, a, n_tok, st), "attention kernel");
}

// ---- fixed scratch of the allocation-free entry point ------------------------
// Split records of rd4_attn_decode_append_noalloc live in this file-scope
// device array (one copy per GPU, held until the process ends). In host code
// its name is only a stand-in: the device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
// Every record a call reads was written by that call's split kernel, so
// nothing in it must start at zero.
constexpr int64_t kFixedFloats = 1 << 20;  // 4 MiB: records of <= 1M floats
static __device__ __align__(256) float scratch[kFixedFloats];

std::map<int, float *> g_fixed;  // device -> address of `scratch` there
std::mutex g_fixed_mu;

// Looks up, once per device and with that device current, the address of
// `scratch` on that device.
int fixed_scratch(FixedScratch *out) {
  int dev = 0, rc;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lk(g_fixed_mu);
  auto it = g_fixed.find(dev);
  if (it == g_fixed.end()) {
    float *ptr = nullptr;
    if (hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return fail(RD4_ELAUNCH, "hipGetSymbolAddress of the fixed scratch failed%s");
    it = g_fixed.emplace(dev, ptr).first;
  }
  out->partial = it->second;
  out->counters = nullptr;  // the merge launch uses no counters
  out->floats = kFixedFloats;
  return RD4_OK;
}

}  // namespace

extern "C" {

const char *rd4_version(void) { return "rdna4attn-gfx950 0.1"; }

int rd4_init(void) {
  int dev = 0, rc;
  if ((rc = current_device(&dev))) return rc;
  // The null stream's set, and one spare for the next stream seen (a graph
  // capture stream included), zeroed with a blocking memset: this is the init
  // call, not a launch.
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch.count({dev, (uintptr_t)0})) {
    Scratch n;
    if ((rc = new_scratch(nullptr, true, &n))) return rc;
    g_scratch.emplace(std::make_pair(dev, (uintptr_t)0), n);
  }
  std::vector<Scratch> &sp = g_spare[dev];
  if (sp.empty()) {
    Scratch n;
    if ((rc = new_scratch(nullptr, true, &n))) return rc;
    sp.push_back(n);
  }
  FixedScratch f;
  if ((rc = fixed_scratch(&f))) return rc;
  return hipDeviceSynchronize() == hipSuccess ? RD4_OK : fail(RD4_ELAUNCH, "init sync failed%s");
}

int rd4_stream_init(void *stream) {
  Scratch *s = nullptr;
  return get_scratch((hipStream_t)stream, &s);
}

const char *rd4_last_error(void) { return g_err; }

uint64_t rd4_kv_cache_bytes_shape(uint64_t ctx_size, int n_layers, int n_head_kv, int head_dim,
                                  int kt, int vt) {
  if (!valid_type(kt) || !valid_type(vt) || n_layers <= 0 || n_head_kv <= 0 || head_dim <= 0)
    return 0;
  // per token: n_layers * n_head_kv * head_dim elements on each side; the
  // reference forms the product in double and truncates (device.h:176-179)
  const double half = (double)n_layers * (double)n_head_kv * (double)head_dim;
  return (uint64_t)((double)ctx_size * half * (rd4_kv_bytes_per_elem(kt) + rd4_kv_bytes_per_elem(vt)));
}

uint64_t rd4_kv_cache_bytes(uint64_t ctx_size, int kt, int vt) {
  return rd4_kv_cache_bytes_shape(ctx_size, 16, 4, 256, kt, vt);
}

uint64_t rd4_kv_max_ctx(uint64_t budget_bytes, uint64_t reserved_bytes, int n_layers, int n_head_kv,
                        int head_dim, int kt, int vt) {
  constexpr uint64_t kMaxCtx = 1ull << 24;  // the reference's kMaxCtxSize
  if (rd4_kv_cache_bytes_shape(1, n_layers, n_head_kv, head_dim, kt, vt) == 0 ||
      reserved_bytes >= budget_bytes)
    return 0;
  const uint64_t avail = budget_bytes - reserved_bytes;
  auto fits = [&](uint64_t c) {
    return rd4_kv_cache_bytes_shape(c, n_layers, n_head_kv, head_dim, kt, vt) <= avail;
  };
  if (fits(kMaxCtx)) return kMaxCtx;
  uint64_t lo = 0, hi = kMaxCtx;  // fits(lo), !fits(hi)
  while (hi - lo > 1) {
    const uint64_t mid = lo + (hi - lo) / 2;
    (fits(mid) ? lo : hi) = mid;
  }
  return lo;
}

const char *rd4_kv_type_name(int type) {
  static const char *names[] = {"f32", "f16", "q8_0", "q4_0", "q5_0", "q4_1"};
  return valid_type(type) ? names[type] : "<unknown-kv-type>";
}

const char *rd4_kv_type_parse(const char *name, int *out) {
  for (int t = 0; t < kNumTypes; ++t) {
    if (name && std::strcmp(name, rd4_kv_type_name(t)) == 0) {
      if (out) *out = t;
      return nullptr;
    }
  }
  return "kv type must be one of f32, f16, q8_0, q4_0, q5_0, q4_1";
}

double rd4_kv_bytes_per_elem(int type) {
  if (!valid_type(type)) return 0.0;
  if (type == RD4_KV_F32) return 4.0;
  if (type == RD4_KV_F16) return 2.0;
  return block_bytes(type) / 32.0;
}

int64_t rd4_kv_row_bytes(int type, int head_dim) { return row_bytes(type, head_dim); }

int rd4_kv_store_row_launch(int type, const float *src, void *dst, int64_t width, void *stream) {
  if (!valid_type(type)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (width < 0 || (type >= RD4_KV_Q8_0 && width % 32 != 0))
    return fail(RD4_EINVAL, "width must be a multiple of 32 for quantized types%s");
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & (type == RD4_KV_F32 ? 15 : type == RD4_KV_F16 ? 7 : 1)))
    return fail(RD4_EINVAL, "src must be 16-byte aligned, dst aligned to its element store%s");
  return launched(kv_store_launch(type, src, (uint8_t *)dst, width, (hipStream_t)stream),
                  "kv store");
}

int rd4_kv_fill_launch(int type, void *cache, int64_t n_rows, int head_dim, uint32_t seed,
                       void *stream) {
  if (!valid_type(type)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (n_rows < 0 || head_dim <= 0 || head_dim % 32 != 0)
    return fail(RD4_EINVAL, "head_dim must be a positive multiple of 32%s");
  if ((uintptr_t)cache & (type == RD4_KV_F32 ? 15 : type == RD4_KV_F16 ? 7 : 1))
    return fail(RD4_EINVAL, "cache pointer misaligned%s");
  return launched(kv_fill_launch(type, (uint8_t *)cache, n_rows * head_dim, seed,
                                 (hipStream_t)stream),
                  "kv fill");
}

int rd4_kv_load_rows_launch(int type, const void *src, float *dst, int64_t width, void *stream) {
  if (!valid_type(type)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (width < 0 || (type >= RD4_KV_Q8_0 && width % 32 != 0))
    return fail(RD4_EINVAL, "width must be a multiple of 32 for quantized types%s");
  if (((uintptr_t)dst & 15) || ((uintptr_t)src & 3))
    return fail(RD4_EINVAL, "dst must be 16-byte and src 4-byte aligned%s");
  return launched(kv_load_launch(type, (const uint8_t *)src, dst, width, (hipStream_t)stream),
                  "kv load");
}

int rd4_attn_decode(const float *q, const void *k, const void *v, float *out, float *gate, int t,
                    int n_head, int n_head_kv, int head_dim, float scale, int kt, int vt,
                    int n_splits, void *stream) {
  if (n_splits < 0) return fail(RD4_EINVAL, "n_splits must be >= 0%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  return run_attn(q, k, v, out, gate, nullptr, t, 1, n_head, n_head_kv, head_dim, scale, kt, vt,
                  n_splits, (hipStream_t)stream);
}

int rd4_attn_decode_append(const float *q, const float *k_new, const float *v_new, void *k,
                           void *v, float *out, float *gate, int t, int n_head, int n_head_kv,
                           int head_dim, float scale, int kt, int vt, int n_splits, void *stream) {
  if (n_splits < 0 || t < 0 || !k_new || !v_new)
    return fail(RD4_EINVAL, "append needs t >= 0, n_splits >= 0 and both new rows%s");
  if ((((uintptr_t)k_new) | ((uintptr_t)v_new)) & 15)
    return fail(RD4_EINVAL, "new rows must be 16-byte aligned%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  if ((kt >= RD4_KV_Q8_0 && ((uintptr_t)k & 1)) || (vt >= RD4_KV_Q8_0 && ((uintptr_t)v & 1)))
    return fail(RD4_EINVAL, "cache pointers misaligned%s");
  return run_attn(q, k, v, out, gate, nullptr, t, 1, n_head, n_head_kv, head_dim, scale, kt, vt,
                  n_splits, (hipStream_t)stream, k_new, v_new);
}

int rd4_attn_decode_append_noalloc(const float *q, const float *k_new, const float *v_new, void *k,
                                   void *v, float *out, float *gate, int t, int n_head, int n_head_kv,
                                   int head_dim, float scale, int kt, int vt, int n_splits, void *stream) {
  if (n_splits < 0 || t < 0 || !k_new || !v_new)
    return fail(RD4_EINVAL, "append needs t >= 0, n_splits >= 0 and both new rows%s");
  if ((((uintptr_t)k_new) | ((uintptr_t)v_new)) & 15)
    return fail(RD4_EINVAL, "new rows must be 16-byte aligned%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  if ((kt >= RD4_KV_Q8_0 && ((uintptr_t)k & 1)) || (vt >= RD4_KV_Q8_0 && ((uintptr_t)v & 1)))
    return fail(RD4_EINVAL, "cache pointers misaligned%s");
  FixedScratch f;
  if ((rc = fixed_scratch(&f))) return rc;
  return run_attn(q, k, v, out, gate, nullptr, t, 1, n_head, n_head_kv, head_dim, scale, kt, vt,
                  n_splits, (hipStream_t)stream, k_new, v_new, 0, nullptr, 0, &f);
}

int rd4_attn_decode_tokens(const float *q, const void *k, const void *v, float *out, float *gate,
                           int t0, int n_tok, int n_head, int n_head_kv, int head_dim, float scale,
                           int kt, int vt, int n_splits, void *stream) {
  if (n_splits < 0 || n_tok < 1 || t0 < 0)
    return fail(RD4_EINVAL, "need n_tok >= 1, t0 >= 0 and n_splits >= 0%s");
  return run_attn(q, k, v, out, gate, nullptr, t0, n_tok, n_head, n_head_kv, head_dim, scale, kt,
                  vt, n_splits, (hipStream_t)stream, nullptr, nullptr, /*tok_pair=*/1);
}

int rd4_attn_launch(const float *q, const void *k, const void *v, float *out, int t, int n_head,
                    int n_head_kv, int head_dim, float scale, int kt, int vt, void *stream) {
  return rd4_attn_decode(q, k, v, out, nullptr, t, n_head, n_head_kv, head_dim, scale, kt, vt, 0,
                         stream);
}

int rd4_attn_launch_split(const float *q, const void *k, const void *v, float *out,
                          float *partial, int t, int n_head, int n_head_kv, int head_dim,
                          float scale, int kt, int vt, int n_splits, void *stream) {
  if (n_splits < 1) return fail(RD4_EINVAL, "n_splits must be >= 1%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  return run_attn(q, k, v, out, nullptr, nullptr, t, 1, n_head, n_head_kv, head_dim, scale, kt,
                  vt, -n_splits, (hipStream_t)stream, nullptr, nullptr, 0, partial, n_splits);
}

int rd4_attn_launch_split_wpb(const float *q, const void *k, const void *v, float *out,
                              float *partial, int t, int n_head, int n_head_kv, int head_dim,
                              float scale, int kt, int vt, int n_splits, int wpb, void *stream) {
  if (wpb != 8 && wpb != 16 && wpb != 32) return fail(RD4_EINVAL, "wpb must be 8, 16 or 32%s");
  return rd4_attn_launch_split(q, k, v, out, partial, t, n_head, n_head_kv, head_dim, scale, kt,
                               vt, n_splits, stream);
}

size_t rd4_attn_partial_bytes(int n_head, int head_dim, int n_splits) {
  return (size_t)n_head * (size_t)n_splits * (2 + (size_t)head_dim) * sizeof(float);
}

int rd4_attn_split_wpb(int n_splits) { return (n_splits <= 4 || n_splits >= 16) ? 16 : 8; }

int rd4_attn_batch_launch(const float *q, const void *k, const void *v, float *out,
                          const int *pos, int n_tok, int n_head, int n_head_kv, int head_dim,
                          float scale, int kt, int vt, void *stream) {
  if (!pos) return fail(RD4_EINVAL, "pos must be a device array%s");
  return run_attn(q, k, v, out, nullptr, pos, 0, n_tok, n_head, n_head_kv, head_dim, scale, kt,
                  vt, 1, (hipStream_t)stream);
}

int rd4_attn_split_batch_launch(const float *q, const void *k, const void *v, float *out,
                                float *partial, const int *pos, int n_tok, int n_head,
                                int n_head_kv, int head_dim, float scale, int kt, int vt,
                                int n_splits, void *stream) {
  if (!pos) return fail(RD4_EINVAL, "pos must be a device array%s");
  if (n_splits < 1 || n_tok < 1) return fail(RD4_EINVAL, "n_splits and n_tok must be >= 1%s");
  return run_attn(q, k, v, out, nullptr, pos, 0, n_tok, n_head, n_head_kv, head_dim, scale, kt,
                  vt, n_splits, (hipStream_t)stream, nullptr, nullptr, 0, partial, n_splits);
}

// The MFMA prefill's key splits write records to the stream's library
// scratch; a call that would split gets it here (without it, no split).
void prefill_part(PrefillArgs &p, int kt, int vt, hipStream_t st) {
  const uintptr_t al = (uintptr_t)p.q | (uintptr_t)p.k | (uintptr_t)p.v | (uintptr_t)p.out | (uintptr_t)p.gate;
  if ((al & 15) || !prefill_mfma_supported(kt, vt, p.n_head, p.n_head_kv, p.head_dim)) return;
  const int s = prefill_ksplits(p);
  if (s <= 1 || prefill_part_floats(p, s) > kPartialFloats) return;
  // a stream without a set under graph capture runs unsplit: the lookup's
  // failure is not the call's, so its message is not left behind
  char saved[sizeof(g_err)];
  std::memcpy(saved, g_err, sizeof(g_err));
  Scratch *sc = nullptr;
  if (get_scratch(st, &sc) == RD4_OK) {
    p.part = sc->partial_c;
    p.part_floats = kPartialFloats;
  } else {
    std::memcpy(g_err, saved, sizeof(g_err));
  }
}

int rd4_fa2_prefill_usable(int kt, int vt, int n_q, int pos0, int n_head, int n_head_kv,
                           int head_dim) {
  const char *e = std::getenv("RD_GFX12_FA2_PREFILL");
  if (e && std::atoi(e) == 0) return 0;
  if (kt != RD4_KV_F16 || vt != RD4_KV_F16) return 0;
  if (n_q < 1 || pos0 < 0) return 0;
  return prefill_supported(kt, vt, n_head, n_head_kv, head_dim) ? 1 : 0;
}

int rd4_fa2_prefill_launch(const float *q, const void *k, const void *v, float *o,
                           const int *pos, int n_q, int kmax, int keys_total, int n_head,
                           int n_head_kv, int head_dim, float scale, void *stream) {
  if (n_q < 1 || kmax < 0 || keys_total <= 0 || !pos)
    return fail(RD4_EINVAL, "bad prefill shape%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, RD4_KV_F16, RD4_KV_F16);
  if (rc) return rc;
  PrefillArgs p{};
  p.q = q;
  p.q_f16 = 0;
  p.k = (const uint8_t *)k;
  p.v = (const uint8_t *)v;
  p.out = o;
  p.gate = nullptr;
  p.pos = pos;
  p.pos0 = -1;
  p.kmax = kmax < keys_total - 1 ? kmax : keys_total - 1;
  p.n_q = n_q;
  p.n_head = n_head;
  p.n_head_kv = n_head_kv;
  p.head_dim = head_dim;
  p.scale = scale;
  prefill_part(p, RD4_KV_F16, RD4_KV_F16, (hipStream_t)stream);
  return launched(prefill_launch(RD4_KV_F16, RD4_KV_F16, p, (hipStream_t)stream), "prefill");
}

int rd4_prefill(const void *q, int q_f16, const void *k, const void *v, float *out, float *gate,
                int pos0, int n_q, int n_head, int n_head_kv, int head_dim, float scale, int kt,
                int vt, void *stream) {
  if (n_q < 1 || pos0 < 0 || !q || !k || !v || !out) return fail(RD4_EINVAL, "bad prefill shape%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  PrefillArgs p{};
  p.q = q;
  p.q_f16 = q_f16 ? 1 : 0;
  p.k = (const uint8_t *)k;
  p.v = (const uint8_t *)v;
  p.out = out;
  p.gate = gate;
  p.pos = nullptr;
  p.pos0 = pos0;
  p.kmax = pos0 + n_q - 1;
  p.n_q = n_q;
  p.n_head = n_head;
  p.n_head_kv = n_head_kv;
  p.head_dim = head_dim;
  p.scale = scale;
  prefill_part(p, kt, vt, (hipStream_t)stream);
  return launched(prefill_launch(kt, vt, p, (hipStream_t)stream), "prefill");
}

int rd4_prefill_append(const void *q, int q_f16, const void *k, const void *v, float *out,
                       float *gate, int pos0, int n_q, int n_head, int n_head_kv, int head_dim,
                       float scale, int kt, int vt, const float *k_new, const float *v_new,
                       void *k_dst, void *v_dst, int dst_type, void *stream) {
  if (n_q < 1 || pos0 < 0 || !q || !k || !v || !out) return fail(RD4_EINVAL, "bad prefill shape%s");
  int rc = check_attn_shape(n_head, n_head_kv, head_dim, kt, vt);
  if (rc) return rc;
  if (!valid_type(dst_type)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (!k_new || !v_new || !k_dst || !v_dst) return fail(RD4_EINVAL, "null append buffer%s");
  // The fused append writes while the attention reads: the destination rows must
  // lie outside the attended rows 0 .. pos0 + n_q - 1 of either cache.
  const int64_t app = (int64_t)n_q * n_head_kv * row_bytes(dst_type, head_dim);
  const int64_t att_k = (int64_t)(pos0 + n_q) * n_head_kv * row_bytes(kt, head_dim);
  const int64_t att_v = (int64_t)(pos0 + n_q) * n_head_kv * row_bytes(vt, head_dim);
  auto overlap = [](const void *a, int64_t na, const void *b, int64_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
  };
  if (overlap(k_dst, app, k, att_k) || overlap(k_dst, app, v, att_v) || overlap(v_dst, app, k, att_k) ||
      overlap(v_dst, app, v, att_v) || overlap(k_dst, app, v_dst, app))
    return fail(RD4_EINVAL, "append destination overlaps the attended cache rows%s");
  // The store launch's alignment rules hold on both paths (checked before
  // anything is enqueued, so a refused call writes nothing).
  const uintptr_t dst_al = dst_type == RD4_KV_F32 ? 15 : dst_type == RD4_KV_F16 ? 7 : 1;
  if ((((uintptr_t)k_new) | (uintptr_t)v_new) & 15 || (((uintptr_t)k_dst) | (uintptr_t)v_dst) & dst_al)
    return fail(RD4_EINVAL, "new rows must be 16-byte aligned, destinations aligned to their element store%s");
  if (dst_type >= RD4_KV_Q8_0 && head_dim % 32 != 0)
    return fail(RD4_EINVAL, "quantized append needs a head_dim that is a multiple of 32%s");
  const bool mfma = ((((uintptr_t)q) | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)gate |
                      (uintptr_t)k_new | (uintptr_t)v_new) & 15) == 0 &&
                    prefill_mfma_supported(kt, vt, n_head, n_head_kv, head_dim);
  if (!mfma) {  // other shapes: the store launch, then the prefill launch, on the same stream
    if ((rc = rd4_kv_store_row_launch(dst_type, k_new, k_dst, (int64_t)n_q * n_head_kv * head_dim, stream)))
      return rc;
    if ((rc = rd4_kv_store_row_launch(dst_type, v_new, v_dst, (int64_t)n_q * n_head_kv * head_dim, stream)))
      return rc;
    return rd4_prefill(q, q_f16, k, v, out, gate, pos0, n_q, n_head, n_head_kv, head_dim, scale, kt, vt,
                       stream);
  }
  PrefillArgs p{};
  p.q = q;
  p.q_f16 = q_f16 ? 1 : 0;
  p.k = (const uint8_t *)k;
  p.v = (const uint8_t *)v;
  p.out = out;
  p.gate = gate;
  p.pos0 = pos0;
  p.kmax = pos0 + n_q - 1;
  p.n_q = n_q;
  p.n_head = n_head;
  p.n_head_kv = n_head_kv;
  p.head_dim = head_dim;
  p.scale = scale;
  p.app_k_src = k_new;
  p.app_v_src = v_new;
  p.app_k = (uint8_t *)k_dst;
  p.app_v = (uint8_t *)v_dst;
  p.app_type = dst_type;
  prefill_part(p, kt, vt, (hipStream_t)stream);
  return launched(prefill_launch(kt, vt, p, (hipStream_t)stream), "prefill");
}

int rd4_read_probe(const void *buf, int64_t bytes, void *sink, void *stream) {
  if (bytes < 0 || (bytes > 0 && (!buf || !sink)) || ((uintptr_t)buf & 15) || (bytes & 15) ||
      ((uintptr_t)sink & 3))
    return fail(RD4_EINVAL, "read probe needs a 16-byte aligned buffer, a multiple of 16 bytes and a sink%s");
  return launched(read_probe_launch(buf, bytes, (uint32_t *)sink, (hipStream_t)stream), "read probe");
}

int rd4_sigmoid_gate_launch(float *g_io, float *y_io, int64_t n, void *stream) {
  if (n < 0 || (n > 0 && (!g_io || !y_io))) return fail(RD4_EINVAL, "bad gate buffers%s");
  return launched(sigmoid_gate_launch(g_io, y_io, n, (hipStream_t)stream), "sigmoid gate");
}

int rd4_rope_launch(float *x, int n_tokens, int n_heads, int head_dim, int n_rot,
                    float freq_base, const int *pos, void *stream) {
  if (n_tokens < 0 || n_heads < 0 || n_rot < 0 || n_rot > head_dim || (n_rot & 1))
    return fail(RD4_EINVAL, "bad rope shape%s");
  return launched(
      rope_launch(x, n_tokens, n_heads, head_dim, n_rot, freq_base, pos, (hipStream_t)stream),
      "rope");
}

int rd4_rms_norm_launch(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                        float eps, void *stream) {
  if (nrows < 0 || ncols < 0 || nrows > 0x7fffffff || (nrows > 0 && ncols > 0 && (!x || !y)))
    return fail(RD4_EINVAL, "bad rms_norm shape%s");
  return launched(rms_norm_launch(x, w, y, nrows, ncols, eps, (hipStream_t)stream), "rms_norm");
}

int rd4_qk_norm_rope_append(const float *qg, const float *k_new, const float *v_new,
                            const float *q_norm, const float *k_norm, float eps, int n_rot,
                            float freq_base, const int *pos, int n_tok, int n_head, int n_head_kv,
                            int head_dim, float *q_out, float *gate_out, float *k_out, void *k,
                            void *v, int kt, int vt, void *stream) {
  if (!valid_type(kt) || !valid_type(vt)) return fail(RD4_ETYPE, "KvType outside the enum%s");
  if (n_tok < 0 || n_head < 1 || n_head_kv < 1 || n_head % n_head_kv != 0 ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256 && head_dim != 512) || n_rot < 0 ||
      n_rot > head_dim || (n_rot & 1))
    return fail(RD4_EINVAL, "bad epilogue shape%s");
  if (n_tok == 0) return RD4_OK;
  if (!qg || !k_new || !v_new || !pos || !q_out || !k || !v)
    return fail(RD4_EINVAL, "epilogue buffer is NULL%s");
  const void *f32s[] = {qg, k_new, v_new, q_out, gate_out, k_out};
  for (const void *p : f32s)
    if (((uintptr_t)p & 15) != 0) return fail(RD4_EINVAL, "epilogue f32 buffer not 16-byte aligned%s");
  if (((uintptr_t)k & 3) || ((uintptr_t)v & 3))
    return fail(RD4_EINVAL, "KV cache not 4-byte aligned%s");
  return launched(qk_epilogue_launch(qg, k_new, v_new, q_norm, k_norm, eps, n_rot, freq_base, pos,
                                     n_tok, n_head, n_head_kv, head_dim, q_out, gate_out, k_out,
                                     (uint8_t *)k, (uint8_t *)v, kt, vt, (hipStream_t)stream),
                  "qk epilogue");
}

}  // extern "C"
