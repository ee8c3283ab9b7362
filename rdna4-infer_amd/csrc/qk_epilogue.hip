// Pre-attention epilogue of a full-attention layer, fused (gfx950).
//
// The reference runs six launches between the QKV projections and attention
// (graph.cuh:914-954 for one token, graph.cuh:1444-1462 for a chunk):
//   deinterleave_q_gate (gdn.cuh:367-384, 836-860)  [q|gate] per head -> q, gate
//   rms_norm(q, attn_q_norm), rms_norm(k, attn_k_norm)        (nn.cuh:24-63)
//   rope(q), rope(k)                                         (attn.cuh:30-63)
//   kv_write_batch: K and V rows quantized into the cache    (kv.h:386-501)
// Every step is row-local, so one wave owns one head row of one token from
// load to store: the row is read once from HBM, normalised and rotated in
// registers, and written once (q, optionally k) plus its cache bytes.
//
// Bit-identity with the unfused sequence:
//   - the sum of squares follows rms_norm_kernel's order exactly: "thread" t
//     (t < 256) chains fmaf over elements t, t+256, ..., and the 256 partials
//     meet in the tree p[t] += p[t + s], s = 128 .. 1. A lane holds elements
//     4*lane + i (+256), so strides 128..4 are xor shuffles 32..1 (IEEE
//     addition commutes, so lane t^s adds the same pair) and strides 2, 1 are
//     the in-lane (e0+e2)+(e1+e3);
//   - rsqrtf(sum / ncols + eps), then (x * scale) * w;
//   - RoPE through rope_cs / rope_lo / rope_hi, shared with rope_kernel;
//   - the quantizer is store_group4, shared with kv_store_row and the decode
//     append, with the same lane-to-block mapping.
#include "kv_quant.hpp"

namespace rd4 {

namespace {

constexpr int kRmsThreads = 256;  // rms_norm_kernel's block (nn.cuh:22)
constexpr int kEpiWaves = 4;
constexpr int kEpiMaxHd = 512;

// Standalone row RMSNorm with the reference's arithmetic, any ncols.
__global__ __launch_bounds__(kRmsThreads) void rms_norm_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               float *y, int64_t ncols, float eps) {
  __shared__ float part[kRmsThreads];
  const int tid = threadIdx.x;
  const float *xr = x + (int64_t)blockIdx.x * ncols;
  float *yr = y + (int64_t)blockIdx.x * ncols;
  float acc = 0.0f;
  int64_t i = tid;
  for (; i + 3 * kRmsThreads < ncols; i += 4 * kRmsThreads) {
    const float v0 = xr[i], v1 = xr[i + kRmsThreads], v2 = xr[i + 2 * kRmsThreads],
                v3 = xr[i + 3 * kRmsThreads];
    acc = fmaf(v0, v0, acc);
    acc = fmaf(v1, v1, acc);
    acc = fmaf(v2, v2, acc);
    acc = fmaf(v3, v3, acc);
  }
  for (; i < ncols; i += kRmsThreads) acc = fmaf(xr[i], xr[i], acc);
  part[tid] = acc;
  __syncthreads();
  if (tid < 128) part[tid] = __fadd_rn(part[tid], part[tid + 128]);
  __syncthreads();
  if (tid < 64) {
    float v = __fadd_rn(part[tid], part[tid + 64]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = __fadd_rn(v, xor_f(v, m));
    if (tid == 0) part[0] = v;
  }
  __syncthreads();
  const float scale = rsqrtf(__fadd_rn(__fdiv_rn(part[0], (float)ncols), eps));
  for (int64_t j = tid; j < ncols; j += kRmsThreads) {
    const float s = __fmul_rn(xr[j], scale);
    yr[j] = w ? __fmul_rn(s, w[j]) : s;
  }
}

struct EpiArgs {
  const float *qg, *k, *v, *qw, *kw;
  const int *pos;
  float *q_out, *gate_out, *k_out;
  uint8_t *kc, *vc;
  int64_t krb, vrb;
  float eps, freq_base;
  int n_rot, n_tok, n_head, n_head_kv, head_dim, kt, vt;
};

__device__ __forceinline__ void store_typed(int t, const float x[4], int sub, uint8_t *row, int blk) {
  switch (t) {
    case F32: store_group4<F32>(x, sub, row, blk); break;
    case F16: store_group4<F16>(x, sub, row, blk); break;
    case Q8_0: store_group4<Q8_0>(x, sub, row, blk); break;
    case Q4_0: store_group4<Q4_0>(x, sub, row, blk); break;
    case Q5_0: store_group4<Q5_0>(x, sub, row, blk); break;
    default: store_group4<Q4_1>(x, sub, row, blk); break;
  }
}

// One wave per (token, row); rows of a token: n_head q heads, then n_head_kv
// k heads, then n_head_kv v heads.
template <int G>  // 256-element groups per row: 1 (head_dim <= 256) or 2
__global__ __launch_bounds__(64 * kEpiWaves) void qk_epilogue_kernel(EpiArgs a) {
  __shared__ float rows[kEpiWaves][kEpiMaxHd];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per_tok = a.n_head + 2 * a.n_head_kv;
  const int64_t task = (int64_t)blockIdx.x * kEpiWaves + wave;
  if (task >= (int64_t)a.n_tok * per_tok) return;
  const int tok = (int)(task / per_tok), r = (int)(task - (int64_t)tok * per_tok);
  const int HD = a.head_dim;
  const bool on = 4 * lane < (HD < 256 ? HD : 256);
  const int kind = r < a.n_head ? 0 : (r < a.n_head + a.n_head_kv ? 1 : 2);
  const int h = kind == 0 ? r : (kind == 1 ? r - a.n_head : r - a.n_head - a.n_head_kv);
  const int64_t hrow = (int64_t)tok * (kind == 0 ? a.n_head : a.n_head_kv) + h;
  const float *src = kind == 0 ? a.qg + hrow * 2 * HD : (kind == 1 ? a.k : a.v) + hrow * HD;

  float x[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float4 v = on ? *(const float4 *)(src + 256 * g + 4 * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
    x[g][0] = v.x;
    x[g][1] = v.y;
    x[g][2] = v.z;
    x[g][3] = v.w;
  }
  if (kind == 0 && a.gate_out && on) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      *(float4 *)(a.gate_out + hrow * HD + 256 * g + 4 * lane) =
          *(const float4 *)(src + HD + 256 * g + 4 * lane);
  }
  const int pos = a.pos[tok];

  if (kind != 2) {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t[i] = fmaf(x[0][i], x[0][i], 0.0f);
      if constexpr (G == 2) t[i] = fmaf(x[1][i], x[1][i], t[i]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = __fadd_rn(t[i], xor_f(t[i], m));
    const float sum = __fadd_rn(__fadd_rn(t[0], t[2]), __fadd_rn(t[1], t[3]));
    const float scale = rsqrtf(__fadd_rn(__fdiv_rn(sum, (float)HD), a.eps));
    const float *w = kind == 0 ? a.qw : a.kw;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = __fmul_rn(x[g][i], scale);
        x[g][i] = (w && on) ? __fmul_rn(s, w[256 * g + 4 * lane + i]) : s;
      }

    if (a.n_rot > 0) {
      float *row = rows[wave];
      if (on) {
#pragma unroll
        for (int g = 0; g < G; ++g)
          *(float4 *)(row + 256 * g + 4 * lane) = make_float4(x[g][0], x[g][1], x[g][2], x[g][3]);
      }
      // the row is exchanged between the lanes of this wave only
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int half = a.n_rot >> 1;
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 256 * g + 4 * lane + i;
          if (on && d < a.n_rot) {
            const int p = d < half ? d : d - half;
            float c, s;
            rope_cs(pos, p, a.n_rot, a.freq_base, &c, &s);
            const float x0 = row[p], x1 = row[p + half];
            x[g][i] = d < half ? rope_lo(x0, x1, c, s) : rope_hi(x0, x1, c, s);
          }
        }
    }
  }

  if (!on) return;
  if (kind == 0 || (kind == 1 && a.k_out)) {
    float *dst = (kind == 0 ? a.q_out : a.k_out) + hrow * HD;
#pragma unroll
    for (int g = 0; g < G; ++g)
      *(float4 *)(dst + 256 * g + 4 * lane) = make_float4(x[g][0], x[g][1], x[g][2], x[g][3]);
  }
  if (kind != 0) {
    const int type = kind == 1 ? a.kt : a.vt;
    uint8_t *row = (kind == 1 ? a.kc : a.vc) +
                   ((int64_t)pos * a.n_head_kv + h) * (kind == 1 ? a.krb : a.vrb);
#pragma unroll
    for (int g = 0; g < G; ++g) store_typed(type, x[g], lane & 7, row, 8 * g + (lane >> 3));
  }
}

}  // namespace

hipError_t rms_norm_launch(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                           float eps, hipStream_t st) {
  if (nrows <= 0 || ncols <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)nrows), dim3(kRmsThreads), 0, st, x, w, y,
                     ncols, eps);
  return hipGetLastError();
}

hipError_t qk_epilogue_launch(const float *qg, const float *k, const float *v, const float *qw,
                              const float *kw, float eps, int n_rot, float freq_base,
                              const int *pos, int n_tok, int n_head, int n_head_kv, int head_dim,
                              float *q_out, float *gate_out, float *k_out, uint8_t *kc,
                              uint8_t *vc, int kt, int vt, hipStream_t st) {
  EpiArgs a;
  a.qg = qg;
  a.k = k;
  a.v = v;
  a.qw = qw;
  a.kw = kw;
  a.pos = pos;
  a.q_out = q_out;
  a.gate_out = gate_out;
  a.k_out = k_out;
  a.kc = kc;
  a.vc = vc;
  a.krb = row_bytes(kt, head_dim);
  a.vrb = row_bytes(vt, head_dim);
  a.eps = eps;
  a.freq_base = freq_base;
  a.n_rot = n_rot;
  a.n_tok = n_tok;
  a.n_head = n_head;
  a.n_head_kv = n_head_kv;
  a.head_dim = head_dim;
  a.kt = kt;
  a.vt = vt;
  const int64_t tasks = (int64_t)n_tok * (n_head + 2 * n_head_kv);
  if (tasks <= 0) return hipSuccess;
  const dim3 grid((unsigned)((tasks + kEpiWaves - 1) / kEpiWaves)), block(64 * kEpiWaves);
  if (head_dim > 256)
    hipLaunchKernelGGL(qk_epilogue_kernel<2>, grid, block, 0, st, a);
  else
    hipLaunchKernelGGL(qk_epilogue_kernel<1>, grid, block, 0, st, a);
  return hipGetLastError();
}

}  // namespace rd4
