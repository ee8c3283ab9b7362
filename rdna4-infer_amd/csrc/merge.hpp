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
// output. Each merging CTA reads at most kMergeFan records per head, so the
// serial tail stays short even with 256 splits, and the partials never need a
// second kernel launch.
#pragma once
#include "attn_generic.hpp"

namespace rd4 {

constexpr int kMergeFan = 16;
constexpr int kCtrStride = 1 + kMaxSplits / kMergeFan;  // level-2 + level-1 counters

__device__ __forceinline__ float sigmoid_dev(float x) { return 1.0f / (1.0f + expf(-x)); }

// Fold n (<= kMergeFan) records per head for G heads. src points at head 0's
// first record; heads are src_hstride floats apart, records rec floats apart.
// final: normalize, gate and write a.out/a.gate at qoff; else write one record
// per head to dst (dst_hstride floats apart). w_s: LDS [kGMaxMerge][kMergeFan],
// ml_s: LDS [kGMaxMerge][2]. All NT threads must call.
constexpr int kGMaxMerge = 8;
template <int NT>
__device__ __forceinline__ void merge_records(const float *src, int64_t src_hstride, int n, int G,
                                              int hd, bool final, const AttnArgs &a, int64_t qoff,
                                              float *dst, int64_t dst_hstride, float *w_s,
                                              float *ml_s) {
  const int tid = threadIdx.x;
  const int rec = 2 + hd;
  if (tid < kGMaxMerge * kMergeFan) {
    const int g = tid / kMergeFan, si = tid % kMergeFan;
    const bool on = g < G && si < n;
    const float *r = src + g * src_hstride + (int64_t)si * rec;
    const float ms = on ? r[0] : -INFINITY;
    const float ls = on ? r[1] : 0.0f;
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
    dst[tid * dst_hstride] = ml_s[2 * tid];
    dst[tid * dst_hstride + 1] = ml_s[2 * tid + 1];
  }
  for (int i = tid; i < G * hd; i += NT) {
    const int g = i / hd, d = i - g * hd;
    const float *r = src + g * src_hstride + 2 + d;
    float o = 0.0f;
    for (int si = 0; si < n; ++si) o += r[(int64_t)si * rec] * w_s[g * kMergeFan + si];
    if (final) {
      const float mm = ml_s[2 * g], L = ml_s[2 * g + 1];
      o = (mm == -INFINITY) ? 0.0f : o * ((L > 0.0f) ? 1.0f / L : 0.0f);
      const int64_t oi = qoff + i;
      if (a.gate) {
        const float sg = sigmoid_dev(a.gate[oi]);
        a.gate[oi] = sg;
        o = o * sg;
      }
      a.out[oi] = o;
    } else {
      dst[g * dst_hstride + 2 + d] = o;
    }
  }
}

// Called by every CTA after it has written its level-0 record(s) for heads
// h0..h0+G-1 of token tok, split s. flag: LDS int. Returns after the merge (or
// immediately for CTAs that are not the last of their group).
template <int NT>
__device__ __forceinline__ void split_tail(const AttnArgs &a, int tok, int kvh, int hc, int h0,
                                           int G, int s, int *flag, float *w_s, float *ml_s) {
  const int tid = threadIdx.x;
  const int hd = a.head_dim, rec = 2 + hd, S = a.n_splits;
  const int NG = (S + kMergeFan - 1) / kMergeFan;
  const int group = s / kMergeFan;
  const int n_in = min(kMergeFan, S - group * kMergeFan);
  unsigned *ctr = a.counters + (((int64_t)tok * a.n_head_kv + kvh) * a.n_chunks + hc) * kCtrStride;

  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr + 1 + group, 1u);
    flag[0] = (done == (unsigned)(n_in - 1));
    if (flag[0]) atomicExch(ctr + 1 + group, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;
  __threadfence();

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * hd;
  const float *src = a.partial + (((int64_t)tok * a.n_head + h0) * S + group * kMergeFan) * rec;
  if (NG == 1) {
    merge_records<NT>(src, (int64_t)S * rec, n_in, G, hd, true, a, qoff, nullptr, 0, w_s, ml_s);
    return;
  }
  float *l1 = a.partial + (int64_t)a.l1_offset;
  float *dst = l1 + (((int64_t)tok * a.n_head + h0) * NG + group) * rec;
  merge_records<NT>(src, (int64_t)S * rec, n_in, G, hd, false, a, qoff, dst, (int64_t)NG * rec,
                    w_s, ml_s);
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr, 1u);
    flag[0] = (done == (unsigned)(NG - 1));
    if (flag[0]) atomicExch(ctr, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;
  __threadfence();
  const float *src1 = l1 + ((int64_t)tok * a.n_head + h0) * NG * rec;
  merge_records<NT>(src1, (int64_t)NG * rec, NG, G, hd, true, a, qoff, nullptr, 0, w_s, ml_s);
}

}  // namespace rd4
