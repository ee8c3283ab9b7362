// Internal interface of the attention kernels (not part of the C ABI).
#pragma once
#include "common.hpp"

namespace rd4 {

// Split count ceiling of the library's partial scratch per (token, head).
constexpr int kMaxSplits = 256;

struct AttnArgs {
  const float *q;         // [n_tok][n_head][hd] f32 (or f16 when q_f16)
  int q_f16;
  const uint8_t *k;       // cache rows [pos][n_head_kv][row]
  const uint8_t *v;
  float *out;             // [n_tok][n_head][hd] f32 (may alias q)
  float *gate;            // optional [n_tok][n_head][hd]: in logits, out sigmoid
  const float *k_new;     // optional fused append (single token): f32 [n_head_kv][hd] rows
  const float *v_new;     //   written to cache row t before it is attended
  const int *pos;         // device positions per token, or nullptr -> t
  int t;                  // last key index for the single-token launch
  int kcap;               // > 0: keys from kcap on are never attended (prefill kmax + 1)
  int n_head, n_head_kv, head_dim;
  float scale;
  int n_splits;           // key splits per (token, kv head)
  float *partial;         // split records (uncached scratch), layout below
  // acc [n_tok][n_head][n_splits][hd] at partial; (m, l) [n_tok][n_head][n_splits][2]
  // at partial + ml0_off; level-1 merge records likewise at acc1_off / ml1_off.
  int64_t ml0_off, acc1_off, ml1_off;
  unsigned *counters;     // [n_tok][n_head_kv][n_chunks][kCtrStride], zero between launches
  // filled by the launcher
  int n_chunks;
  int k_lds_stride, v_lds_stride;
  int ext_merge;  // 1: the kernel only writes level-0 records; merge_splits_launch merges
  // MFMA decode only: 1 = each CTA carries two consecutive tokens (query rows
  // 0-7 the first token's heads, 8-15 the second's, f16 queries), positions
  // t + token; n_tok is the token count of the launch
  int tok_pair, n_tok;
  // Profiling knob (env RD4_DECODE_DBG, 0 in production), MFMA decode kernel:
  // 1 skip the split merge, 2 skip the QK product, 4 skip the PV product,
  // 32 no key tiles, 2048 no tile loads (compute on stale LDS).
  int dbg;
};

// Merge the level-0 split records of n_tok tokens into out (and apply the gate):
// one short kernel after the split kernel on the same stream.
hipError_t merge_splits_launch(const AttnArgs &a, int n_tok, hipStream_t st);

hipError_t attn_generic_launch(int kt, int vt, AttnArgs a, int n_tok, hipStream_t st);
size_t generic_lds_bytes(int kt, int vt, int hd, int n_splits);

}  // namespace rd4
