// Drop-in replacement of rdna4-infer's include/rdna4/attn.cuh (launchers).
//
// Same names and signatures as the reference (attn.cuh:56, 200, 373, 630, 665,
// 895, 903, 958); every call forwards to librdna4attn's gfx950 kernels. The
// `partial` buffer the caller passes receives the split records whenever the
// split count the library runs fits it (attn_partial_bytes for the caller's
// n_splits); otherwise the records go to the stream's own library scratch, so
// launches on different streams never share records. n_splits is the minimum
// split count the caller asks for (RD_ATTN_SPLITS keeps its meaning of forcing
// a split path; the library may split further to fill the GPU).
#pragma once
#include <cstddef>

#include "rdna4/kv.h"

namespace rdna4 {

inline bool rope_launch(float *d_x, int n_tokens, int n_heads, int head_dim, int n_rot,
                        float freq_base, const int *d_pos, hipStream_t stream = nullptr) {
  return rd4_rope_launch(d_x, n_tokens, n_heads, head_dim, n_rot, freq_base, d_pos,
                         (void *)stream) == RD4_OK;
}

inline bool attn_launch(const float *d_q, const void *d_k, const void *d_v, float *d_out, int t,
                        int n_head, int n_head_kv, int head_dim, float scale, KvType kt,
                        KvType vt, hipStream_t stream = nullptr) {
  return rd4_attn_launch(d_q, d_k, d_v, d_out, t, n_head, n_head_kv, head_dim, scale, (int)kt,
                         (int)vt, (void *)stream) == RD4_OK;
}

inline bool attn_batch_launch(const float *d_q, const void *d_k, const void *d_v, float *d_out,
                              const int *d_pos, int n_tok, int n_head, int n_head_kv, int head_dim,
                              float scale, KvType kt, KvType vt, hipStream_t stream = nullptr) {
  return rd4_attn_batch_launch(d_q, d_k, d_v, d_out, d_pos, n_tok, n_head, n_head_kv, head_dim,
                               scale, (int)kt, (int)vt, (void *)stream) == RD4_OK;
}

inline std::size_t attn_partial_bytes(int n_head, int head_dim, int n_splits) {
  return rd4_attn_partial_bytes(n_head, head_dim, n_splits);
}

inline int attn_split_wpb(int n_splits) { return rd4_attn_split_wpb(n_splits); }

inline bool attn_launch_split(const float *d_q, const void *d_k, const void *d_v, float *d_out,
                              float *d_partial, int t, int n_head, int n_head_kv, int head_dim,
                              float scale, KvType kt, KvType vt, int n_splits,
                              hipStream_t stream = nullptr) {
  return rd4_attn_launch_split(d_q, d_k, d_v, d_out, d_partial, t, n_head, n_head_kv, head_dim,
                               scale, (int)kt, (int)vt, n_splits, (void *)stream) == RD4_OK;
}

inline bool attn_launch_split_wpb(const float *d_q, const void *d_k, const void *d_v,
                                  float *d_out, float *d_partial, int t, int n_head,
                                  int n_head_kv, int head_dim, float scale, KvType kt, KvType vt,
                                  int n_splits, int wpb, hipStream_t stream = nullptr) {
  return rd4_attn_launch_split_wpb(d_q, d_k, d_v, d_out, d_partial, t, n_head, n_head_kv,
                                   head_dim, scale, (int)kt, (int)vt, n_splits, wpb,
                                   (void *)stream) == RD4_OK;
}

// Templated form of the bench overload (attn.cuh:613-628): the types are
// template arguments, wpb is 8, 16 or 32.
template <KvType KT, KvType VT>
inline bool attn_launch_split_wpb(const float *d_q, const void *d_k, const void *d_v, float *d_out,
                                  float *d_partial, int t, int n_head, int n_head_kv, int head_dim,
                                  float scale, int n_splits, int wpb, hipStream_t stream) {
  return rd4_attn_launch_split_wpb(d_q, d_k, d_v, d_out, d_partial, t, n_head, n_head_kv,
                                   head_dim, scale, (int)KT, (int)VT, n_splits, wpb,
                                   (void *)stream) == RD4_OK;
}

inline bool attn_split_batch_launch(const float *d_q, const void *d_k, const void *d_v,
                                    float *d_out, float *d_partial, const int *d_pos, int n_tok,
                                    int n_head, int n_head_kv, int head_dim, float scale,
                                    KvType kt, KvType vt, int n_splits,
                                    hipStream_t stream = nullptr) {
  return rd4_attn_split_batch_launch(d_q, d_k, d_v, d_out, d_partial, d_pos, n_tok, n_head,
                                     n_head_kv, head_dim, scale, (int)kt, (int)vt, n_splits,
                                     (void *)stream) == RD4_OK;
}

}  // namespace rdna4
