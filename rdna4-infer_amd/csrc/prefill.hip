// Prefill dispatch. First version: the generic split-KV kernel with one CTA per
// (token, kv head) (positions pos0 + i); f32 queries only.
#include "prefill.hpp"

namespace rd4 {

bool prefill_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  (void)kt; (void)vt; (void)n_head; (void)n_head_kv; (void)head_dim;
  return true;
}

hipError_t prefill_launch(int kt, int vt, const PrefillArgs &p, hipStream_t st) {
  AttnArgs a{};
  a.q = (const float *)p.q;
  a.q_f16 = p.q_f16;
  a.k = p.k;
  a.v = p.v;
  a.out = p.out;
  a.gate = p.gate;
  a.pos = p.pos;
  a.t = p.pos0;
  a.n_head = p.n_head;
  a.n_head_kv = p.n_head_kv;
  a.head_dim = p.head_dim;
  a.scale = p.scale;
  a.n_splits = 1;
  return attn_generic_launch(kt, vt, a, p.n_q, st);
}

}  // namespace rd4
