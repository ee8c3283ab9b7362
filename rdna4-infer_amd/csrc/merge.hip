// Split merge as its own launch: the LSE merge of attn_merge_kernel
// (include/rdna4/attn.cuh:563-590) plus the output gate (nn.cuh:405-412).
//
// The split kernel's level-0 records (m_s in ln units, l_s, acc_s[hd]) are
// visible to this launch without any fence (kernel boundary). One 64-lane CTA
// per (token, head, 64-dim quarter): every lane folds the weights of all splits
// (m, l pairs read once per lane group), then lane (c, sub) sums the float4
// column c over splits sub, sub + 4, ...; the four partial sums meet through
// lane exchanges. All record loads of a lane are issued before they are used,
// so the merge costs about one memory round trip.
#include "merge.hpp"

namespace rd4 {

namespace {

constexpr int kQuarterDims = 64;

// x summed over lanes l, l ^ 16, l ^ 32, l ^ 48
__device__ __forceinline__ float sum_groups4(float x) {
  float a = x, b = x;
  swap16(a, b);
  float c = a + b, d = c;
  swap32(c, d);
  return c + d;
}

__global__ __launch_bounds__(64) void merge_splits_kernel(AttnArgs a) {
  __shared__ float w_s[kMaxSplits];
  const int lane = threadIdx.x;
  const int hd = a.head_dim, S = a.n_splits;
  const int nq = hd / kQuarterDims;
  const int head = blockIdx.x / nq, quarter = blockIdx.x - head * nq;
  const int tok = blockIdx.y;
  const int64_t hrow = (int64_t)tok * a.n_head + head;
  const float *ml = a.partial + a.ml0_off + hrow * S * 2;

  // record loads first (the first kBatch splits of this lane), then (m, l)
  const int c = lane & 15, sub = lane >> 4;
  const float *acc = a.partial + hrow * S * hd + quarter * kQuarterDims + 4 * c;
  constexpr int kBatch = 16;
  float4 v[kBatch];
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    const int s = sub + 4 * b;
    v[b] = s < S ? *(const float4 *)(acc + (int64_t)s * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int64_t oi = hrow * hd + quarter * kQuarterDims + 4 * c;
  const float4 gl = (a.gate && sub == 0) ? *(const float4 *)(a.gate + oi) : make_float4(0.f, 0.f, 0.f, 0.f);
  float mv[kMaxSplits / 64], lv[kMaxSplits / 64];
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) {
    const int s = lane + 64 * i;
    const float2 r = s < S ? *(const float2 *)(ml + 2 * s) : make_float2(-INFINITY, 0.0f);
    mv[i] = r.x;
    lv[i] = r.y;
  }
  float mm = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) mm = fmaxf(mm, mv[i]);
  mm = wave_max(mm);
  float L = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) {
    const int s = lane + 64 * i;
    const float w = (mv[i] == -INFINITY) ? 0.0f : expf(mv[i] - mm);
    if (s < S) w_s[s] = w;
    L += w * lv[i];
  }
  L = wave_sum(L);
  __syncthreads();
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = sub;; s0 += 4 * kBatch) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int s = s0 + 4 * b;
      const float w = s < S ? w_s[s] : 0.0f;
      sum.x += v[b].x * w;
      sum.y += v[b].y * w;
      sum.z += v[b].z * w;
      sum.w += v[b].w * w;
    }
    if (s0 + 4 * kBatch >= S) break;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int s = s0 + 4 * kBatch + 4 * b;
      v[b] = s < S ? *(const float4 *)(acc + (int64_t)s * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  sum.x = sum_groups4(sum.x);
  sum.y = sum_groups4(sum.y);
  sum.z = sum_groups4(sum.z);
  sum.w = sum_groups4(sum.w);
  if (sub != 0) return;
  const float inv = (mm == -INFINITY) ? 0.0f : ((L > 0.0f) ? 1.0f / L : 0.0f);
  float ov[4] = {sum.x * inv, sum.y * inv, sum.z * inv, sum.w * inv};
  if (a.gate) {
    const float gv[4] = {gl.x, gl.y, gl.z, gl.w};
    float sg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sg[i] = sigmoid_dev(gv[i]);
      ov[i] *= sg[i];
    }
    *(float4 *)(a.gate + oi) = make_float4(sg[0], sg[1], sg[2], sg[3]);
  }
  *(float4 *)(a.out + oi) = make_float4(ov[0], ov[1], ov[2], ov[3]);
}

}  // namespace

hipError_t merge_splits_launch(const AttnArgs &a, int n_tok, hipStream_t st) {
  if (a.head_dim % kQuarterDims != 0 || a.n_splits > kMaxSplits) return hipErrorInvalidValue;
  dim3 grid((unsigned)(a.n_head * (a.head_dim / kQuarterDims)), (unsigned)n_tok);
  hipLaunchKernelGGL(merge_splits_kernel, grid, dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace rd4
