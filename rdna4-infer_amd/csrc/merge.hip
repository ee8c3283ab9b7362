// Split merge as its own launch: the LSE merge of attn_merge_kernel
// (include/rdna4/attn.cuh:563-590) plus the output gate (nn.cuh:405-412).
//
// The split kernel's level-0 records (m_s in ln units, l_s, acc_s[hd]) are
// visible to this launch without any fence (kernel boundary). One 64-lane CTA
// per (token, head, 16-dim group): lane (c, sub) = (lane & 3, lane >> 2) owns
// float4 c of the group for splits sub, sub + 16, ..., and loads those records
// and their (m, l) pairs in one batch, with the gate logits, before using any
// of them. Every split's m is then in some lane, so the max, the weights and
// the sum l come from lane exchanges (DPP and the row / half-wave swaps)
// without LDS, and the 16 split classes of a float4 meet the same way. The
// merge costs one memory round trip plus a short dependent chain; the grid
// (n_head * hd / 16 CTAs per token, 384 at 24 heads) spreads the loads over
// the CUs.
#include "merge.hpp"

namespace rd4 {

namespace {

constexpr int kGroupDims = 16;
constexpr int kPerLane = kMaxSplits / 16;  // record slots per lane

// x + the value of lane (l + 4) % 16 and (l + 8) % 16 of its 16-lane row:
// the sum over the four lanes of the row with the same l % 4
__device__ __forceinline__ float sum_row_stride4(float x) {
  int v = __builtin_bit_cast(int, x);
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(v, v, 0x124, 0xF, 0xF, false));  // row_ror:4
  v = __builtin_bit_cast(int, x);
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false));  // row_ror:8
  return x;
}
// x summed over lanes l, l ^ 16, l ^ 32, l ^ 48
__device__ __forceinline__ float sum_rows(float x) {
  float a = x, b = x;
  swap16(a, b);
  float c = a + b, d = c;
  swap32(c, d);
  return c + d;
}

#ifndef RD4_MERGE_EXP
#define RD4_MERGE_EXP 0
#endif
__global__ __launch_bounds__(64) void merge_splits_kernel(AttnArgs a) {
  if (RD4_MERGE_EXP == 1) return;  // timing experiment: launch cost alone
  const int lane = threadIdx.x;
  const int hd = a.head_dim, S = a.n_splits;
  const int ng = hd / kGroupDims;
  const int head = blockIdx.x / ng, grp = blockIdx.x - head * ng;
  const int tok = blockIdx.y;
  const int64_t hrow = (int64_t)tok * a.n_head + head;
  const int c = lane & 3, sub = lane >> 2;
  const float *acc = a.partial + hrow * S * hd + kGroupDims * grp + 4 * c;
  const float *ml = a.partial + a.ml0_off + hrow * S * 2;
  const int64_t oi = hrow * hd + kGroupDims * grp + 4 * c;

  // every load first: records and (m, l) of splits sub + 16 b, the gate logits
  float4 v[kPerLane];
  float2 r[kPerLane];
#pragma unroll
  for (int b = 0; b < kPerLane; ++b) {
    const int s = sub + 16 * b;
    v[b] = make_float4(0.f, 0.f, 0.f, 0.f);
    r[b] = make_float2(-INFINITY, 0.0f);
    if (16 * b < S && s < S) {  // (16 b < S is uniform: slots past the count issue nothing)
      v[b] = *(const float4 *)(acc + (int64_t)s * hd);
      r[b] = *(const float2 *)(ml + 2 * s);
    }
  }
  const float4 gl = (a.gate && sub == 0) ? *(const float4 *)(a.gate + oi) : make_float4(0.f, 0.f, 0.f, 0.f);

  float mm = -INFINITY;
#pragma unroll
  for (int b = 0; b < kPerLane; ++b)
    if (16 * b < S) mm = fmaxf(mm, r[b].x);
  mm = wave_max(mm);
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  float L = 0.0f;
#pragma unroll
  for (int b = 0; b < kPerLane; ++b) {
    if (16 * b >= S) continue;
    // an empty split (m = -inf) weighs 0; so does every split when all are empty
    const float w = (r[b].x == -INFINITY) ? 0.0f : expf(r[b].x - mm);
    L = fmaf(w, r[b].y, L);
    sum.x = fmaf(v[b].x, w, sum.x);
    sum.y = fmaf(v[b].y, w, sum.y);
    sum.z = fmaf(v[b].z, w, sum.z);
    sum.w = fmaf(v[b].w, w, sum.w);
  }
  // the 16 split classes: lanes c + 4 sub of each row, then the four rows
  sum.x = sum_rows(sum_row_stride4(sum.x));
  sum.y = sum_rows(sum_row_stride4(sum.y));
  sum.z = sum_rows(sum_row_stride4(sum.z));
  sum.w = sum_rows(sum_row_stride4(sum.w));
  // the lanes with c = 0 hold each split's l once
  L = wave_sum(c == 0 ? L : 0.0f);
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
  if (a.head_dim % kGroupDims != 0 || a.n_splits > kMaxSplits) return hipErrorInvalidValue;
  dim3 grid((unsigned)(a.n_head * (a.head_dim / kGroupDims)), (unsigned)n_tok);
  if (RD4_MERGE_EXP == 2) return hipSuccess;  // timing experiment: no merge launch
  hipLaunchKernelGGL(merge_splits_kernel, grid, dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace rd4
