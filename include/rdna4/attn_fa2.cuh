// Drop-in replacement of rdna4-infer's include/rdna4/attn_fa2.cuh.
//
// fa2_prefill_launch (attn_fa2.cuh:173) and fa2_prefill_usable (:192) with the
// reference's signatures, forwarding to librdna4attn's f16-MFMA prefill. The
// gfx950 kernel admits every chunk size and key count for f16/f16 K/V with
// head_dim 256 (the reference's admission required n_q == 512 and 2048..8192
// keys); RD_GFX12_FA2_PREFILL=0 still disables it.
#pragma once
#include "rdna4/kv.h"

namespace rdna4 {

inline bool fa2_prefill_launch(const float *d_q, const void *d_k, const void *d_v, float *d_o,
                               const int *d_pos, int n_q, int kmax, int keys_total, int n_head,
                               int n_head_kv, int head_dim, float scale,
                               hipStream_t stream = nullptr) {
  return rd4_fa2_prefill_launch(d_q, d_k, d_v, d_o, d_pos, n_q, kmax, keys_total, n_head,
                                n_head_kv, head_dim, scale, (void *)stream) == RD4_OK;
}

inline bool fa2_prefill_usable(KvType kt, KvType vt, int n_q, int pos0, int n_head, int n_head_kv,
                               int head_dim) {
  return rd4_fa2_prefill_usable((int)kt, (int)vt, n_q, pos0, n_head, n_head_kv, head_dim) != 0;
}

}  // namespace rdna4
