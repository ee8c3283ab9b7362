// Prefill dispatch: the MFMA kernel (attn_prefill_mfma.hip) for f16 K/V with
// head_dim 256 and 16-byte aligned buffers; every other shape runs the generic
// kernel with one CTA per (token, kv head) over keys 0..position.
#include <cstdlib>

#include "prefill.hpp"

namespace rd4 {

bool prefill_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  (void)kt; (void)vt; (void)n_head; (void)n_head_kv; (void)head_dim;
  return true;
}

hipError_t prefill_launch(int kt, int vt, const PrefillArgs &p, hipStream_t st) {
  const uintptr_t al = (uintptr_t)p.q | (uintptr_t)p.k | (uintptr_t)p.v | (uintptr_t)p.out |
                       (uintptr_t)p.gate;
  if ((al & 15) == 0 && prefill_mfma_supported(kt, vt, p.n_head, p.n_head_kv, p.head_dim)) {
    static const int dbg = [] { const char *e = std::getenv("RD4_PREFILL_DBG"); return e ? std::atoi(e) : 0; }();
    PrefillArgs q = p;
    q.dbg = dbg;
    return prefill_mfma_launch(q, st);
  }
  AttnArgs a{};
  a.q = (const float *)p.q;
  a.q_f16 = p.q_f16;
  a.k = p.k;
  a.v = p.v;
  a.out = p.out;
  a.gate = p.gate;
  a.pos = p.pos;
  a.t = p.pos0;
  a.kcap = p.kmax + 1;  // keys 0..min(pos[i], kmax), as the reference's tiling bound
  a.n_head = p.n_head;
  a.n_head_kv = p.n_head_kv;
  a.head_dim = p.head_dim;
  a.scale = p.scale;
  a.n_splits = 1;
  return attn_generic_launch(kt, vt, a, p.n_q, st);
}

}  // namespace rd4
