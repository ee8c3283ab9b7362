// Split-KV merge tail shared by the decode kernels.
//
// Semantics: attn_merge_kernel (include/rdna4/attn.cuh:563-590): for records
// (m_s, l_s, acc_s[hd]) of one query head, mm = max_s m_s, w_s = exp(m_s - mm)
// (0 for an empty split, m_s = -inf), out = sum_s w_s acc_s / sum_s w_s l_s, and
// zeros when every split is empty.
//
// Structure (gfx950-specific): the merge runs inside the attention launch, as a
// two-level tree over groups of kMergeFan splits. The last CTA of each group to
// finish (device-scope counter, reset by that CTA) folds its group's records into
// one level-1 record; the last group-merger folds the level-1 records into the
// output. The records live in uncached device memory, so CTAs on different XCDs
// (whose L2s are not coherent with each other) exchange them with plain 16-byte
// loads and stores; a writer only waits for its stores to complete before the
// counter increment, and a merger issues all of its record loads at once.
#pragma once
#include "attn_generic.hpp"

namespace rd4 {

constexpr int kMergeFan = 16;
constexpr int kCtrStride = 1 + kMaxSplits / kMergeFan;  // level-2 + level-1 counters
constexpr int kGMaxMerge = 8;

// Wait until this thread's vector memory stores are acknowledged; also a
// compiler barrier for memory.
__device__ __forceinline__ void stores_done() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float sigmoid_dev(float x) { return 1.0f / (1.0f + expf(-x)); }

// Fold n (<= kMergeFan) records per head for G heads. acc: head 0's first
// record, heads acc_hs floats apart, records hd floats apart; ml likewise with
// (m, l) pairs. final: normalize, gate and write a.out/a.gate at qoff; else
// write one record per head to dacc/dml. w_s: LDS [kGMaxMerge][kMergeFan];
// ml_s: LDS [kGMaxMerge][2]. All NT threads of the CTA call it.
template <int NT>
__device__ __forceinline__ void merge_records(const float *acc, const float *ml, int64_t acc_hs,
                                              int64_t ml_hs, int n, int G, int hd, bool final,
                                              const AttnArgs &a, int64_t qoff, float *dacc,
                                              float *dml, int64_t dacc_hs, int64_t dml_hs,
                                              float *w_s, float *ml_s) {
  const int tid = threadIdx.x;
  // Record loads first (one item of 4 dims per thread when G*hd/4 <= NT), so the
  // (m, l) round trip and the record round trip overlap.
  const int nq = hd / 4;
  const int it0 = tid;
  const bool have0 = it0 < G * nq;
  const int g0 = have0 ? it0 / nq : 0, d0 = have0 ? 4 * (it0 - g0 * nq) : 0;
  float4 v0[kMergeFan];
  {
    const float *r = acc + g0 * acc_hs + d0;
#pragma unroll
    for (int si = 0; si < kMergeFan; ++si)
      v0[si] = (have0 && si < n) ? *(const float4 *)(r + (int64_t)si * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid < kGMaxMerge * kMergeFan) {
    const int g = tid / kMergeFan, si = tid % kMergeFan;
    const bool on = g < G && si < n;
    const float ms = on ? ml[g * ml_hs + 2 * si] : -INFINITY;
    const float ls = on ? ml[g * ml_hs + 2 * si + 1] : 0.0f;
    float mm = ms;
#pragma unroll
    for (int m = 1; m < kMergeFan; m <<= 1) mm = fmaxf(mm, xor_f(mm, m));
    const float w = (ms == -INFINITY) ? 0.0f : expf(ms - mm);
    float L = w * ls;
#pragma unroll
    for (int m = 1; m < kMergeFan; m <<= 1) L += xor_f(L, m);
    w_s[g * kMergeFan + si] = w;
    if (si == 0) {
      ml_s[2 * g] = mm;
      ml_s[2 * g + 1] = L;
    }
  }
  __syncthreads();
  if (!final && tid < G) {
    dml[tid * dml_hs] = ml_s[2 * tid];
    dml[tid * dml_hs + 1] = ml_s[2 * tid + 1];
  }
  for (int it = tid; it < G * nq; it += NT) {
    const int g = it / nq, d = 4 * (it - g * nq);
    float4 v[kMergeFan];
    if (it == it0) {
#pragma unroll
      for (int si = 0; si < kMergeFan; ++si) v[si] = v0[si];
    } else {
      const float *r = acc + g * acc_hs + d;
#pragma unroll
      for (int si = 0; si < kMergeFan; ++si)
        v[si] = si < n ? *(const float4 *)(r + (int64_t)si * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int si = 0; si < kMergeFan; ++si) {
      const float w = w_s[g * kMergeFan + si];
      o.x += v[si].x * w;
      o.y += v[si].y * w;
      o.z += v[si].z * w;
      o.w += v[si].w * w;
    }
    if (final) {
      const float mm = ml_s[2 * g], L = ml_s[2 * g + 1];
      const float inv = (mm == -INFINITY) ? 0.0f : ((L > 0.0f) ? 1.0f / L : 0.0f);
      float ov[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
      const int64_t oi = qoff + (int64_t)g * hd + d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (a.gate) {
          const float sg = sigmoid_dev(a.gate[oi + i]);
          a.gate[oi + i] = sg;
          ov[i] = ov[i] * sg;
        }
        a.out[oi + i] = ov[i];
      }
    } else {
      *(float4 *)(dacc + g * dacc_hs + d) = o;
    }
  }
}

// Called by every CTA after it has written its level-0 records for heads
// h0..h0+G-1 of token tok, split s. flag: LDS int. Returns after the merge (or
// at once for CTAs that are not the last of their group).
template <int NT>
__device__ __forceinline__ void split_tail(const AttnArgs &a, int tok, int kvh, int hc, int h0,
                                           int G, int s, int *flag, float *w_s, float *ml_s) {
  const int tid = threadIdx.x;
  const int hd = a.head_dim, S = a.n_splits;
  const int NG = (S + kMergeFan - 1) / kMergeFan;
  const int group = s / kMergeFan;
  const int n_in = min(kMergeFan, S - group * kMergeFan);
  unsigned *ctr = a.counters + (((int64_t)tok * a.n_head_kv + kvh) * a.n_chunks + hc) * kCtrStride;

  stores_done();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr + 1 + group, 1u);
    flag[0] = (done == (unsigned)(n_in - 1));
    if (flag[0]) atomicExch(ctr + 1 + group, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * hd;
  const int64_t hrow = (int64_t)tok * a.n_head + h0;  // first head row of this chunk
  const float *acc0 = a.partial + (hrow * S + group * kMergeFan) * hd;
  const float *ml0 = a.partial + a.ml0_off + (hrow * S + group * kMergeFan) * 2;
  if (NG == 1) {
    merge_records<NT>(acc0, ml0, (int64_t)S * hd, (int64_t)S * 2, n_in, G, hd, true, a, qoff,
                      nullptr, nullptr, 0, 0, w_s, ml_s);
    return;
  }
  float *acc1 = a.partial + a.acc1_off + hrow * NG * hd;
  float *ml1 = a.partial + a.ml1_off + hrow * NG * 2;
  merge_records<NT>(acc0, ml0, (int64_t)S * hd, (int64_t)S * 2, n_in, G, hd, false, a, qoff,
                    acc1 + group * hd, ml1 + group * 2, (int64_t)NG * hd, (int64_t)NG * 2, w_s,
                    ml_s);
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr, 1u);
    flag[0] = (done == (unsigned)(NG - 1));
    if (flag[0]) atomicExch(ctr, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;
  merge_records<NT>(acc1, ml1, (int64_t)NG * hd, (int64_t)NG * 2, NG, G, hd, true, a, qoff,
                    nullptr, nullptr, 0, 0, w_s, ml_s);
}

// Lane exchanges without LDS round trips: DPP within 16-lane rows (xor 1, xor 2,
// then the half-row and row mirrors, which pair the 4- and 8-lane groups), and
// the gfx950 row / half-wave swaps for lanes ^ 16 and ^ 32 (asm with tied
// operands; s_nop 1 covers the VALU-write -> swap-read hazard).
__device__ __forceinline__ float dpp_f(float x, int ctrl_sel) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  switch (ctrl_sel) {  // the DPP control must be a constant
    case 0: r = __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    case 1: r = __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
    case 2: r = __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: r = __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ void swap16(float &a, float &b) {
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float &a, float &b) {
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// max / sum over the 64 lanes of the wave, in every lane
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int c = 0; c < 4; ++c) x = fmaxf(x, dpp_f(x, c));
  float a = x, b = x;
  swap16(a, b);
  float c = fmaxf(a, b), d = c;
  swap32(c, d);
  return fmaxf(c, d);
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int c = 0; c < 4; ++c) x += dpp_f(x, c);
  float a = x, b = x;
  swap16(a, b);
  float c = a + b, d = c;
  swap32(c, d);
  return c + d;
}

// Level-0 record of head row `hrow` (= tok * n_head + head), split s.
__device__ __forceinline__ float *rec_acc(const AttnArgs &a, int64_t hrow, int s) {
  return a.partial + (hrow * a.n_splits + s) * a.head_dim;
}
__device__ __forceinline__ float *rec_ml(const AttnArgs &a, int64_t hrow, int s) {
  return a.partial + a.ml0_off + (hrow * a.n_splits + s) * 2;
}

}  // namespace rd4
