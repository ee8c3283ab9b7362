// Internal interface of the prefill and MFMA decode kernels.
#pragma once
#include "attn_generic.hpp"

namespace rd4 {

struct PrefillArgs {
  const void *q;      // [n_q][n_head][hd], f32 or f16 (q_f16)
  int q_f16;
  const uint8_t *k, *v;
  float *out;         // [n_q][n_head][hd] f32 (may alias q when q is f32)
  float *gate;        // optional, same shape: logits in, sigmoid out
  const int *pos;     // device positions, or nullptr -> pos0 + i
  int pos0;
  int kmax;           // last key index any query may attend
  int n_q, n_head, n_head_kv, head_dim;
  float scale;
  int dbg;  // profiling knob bits (0 in production)
  // Optional append fused into the same launch: the chunk's new K/V rows, f32
  // [n_q][n_head_kv][hd] each, quantized to app_type into app_k / app_v (rows
  // contiguous, the chunk's first row at the pointer), as kv_store_row_launch.
  const float *app_k_src, *app_v_src;
  uint8_t *app_k, *app_v;
  int app_type;
  // Key splits (filled by prefill_mfma_launch): with n_ksplit > 1 CTA split s
  // takes the key blocks [s * ksplit_blocks, (s + 1) * ksplit_blocks) of its
  // rows and writes unnormalized records to part (O: [split][q * n_head +
  // head][hd], then (m, l): [split][q * n_head + head][2]); a merge launch
  // folds them. part (part_floats floats, library scratch) may be null: then
  // the kernel never splits.
  int n_ksplit, ksplit_blocks;
  float *part;
  int64_t part_floats;
};

bool prefill_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim);
hipError_t prefill_launch(int kt, int vt, const PrefillArgs &p, hipStream_t st);

bool prefill_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim);
hipError_t prefill_mfma_launch(const PrefillArgs &p, hipStream_t st);
// Key splits the MFMA kernel would run for p (1: none) and the scratch floats
// their records take; the caller passes the scratch in p.part.
int prefill_ksplits(const PrefillArgs &p);
int64_t prefill_part_floats(const PrefillArgs &p, int splits);

bool decode_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim);
hipError_t decode_mfma_launch(int kt, int vt, const AttnArgs &a, int n_tok, hipStream_t st);
// True when multi-token decode of this cache pair can put two tokens in a CTA.
bool decode_mfma_pairs(int kt, int vt);
// True when split records are merged by a second launch (not the in-kernel tree).

}  // namespace rd4
