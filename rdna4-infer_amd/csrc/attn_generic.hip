// Generic split-KV GQA attention for any (K, V) storage pair (gfx950, wave64).
//
// Reference semantics: attn_kernel / attn_split_kernel / attn_merge_kernel and
// their batched forms (include/rdna4/attn.cuh:95-185, 268-356, 445-590, 686-845):
// query head h of token i attends keys 0..t_i of kv head h / (n_head/n_head_kv),
// softmax(q.k * scale) weighted sum of V, f32 accumulation, no keys -> zeros.
//
// Design (not the reference's): one CTA per (token, kv head, head chunk, key
// split). The CTA stages a 32-key tile of K and V in LDS ONCE and all query
// heads of the GQA group (up to 8 per chunk) read it, so each KV byte leaves
// HBM once per token instead of once per query head. Splits cover contiguous
// key ranges. When a token has more than one split, every CTA writes an
// (m, l, acc[hd]) partial into library scratch and the last CTA of the
// (token, kv head, chunk) to finish -- found with a device-scope counter that
// it resets afterwards -- merges them with the max-subtracted LSE rule and
// applies the optional sigmoid gate. One launch, no host sync, no memset.
//
// This kernel is the all-types path; the MFMA kernels in attn_decode_mfma.hip
// take the hot (K, V) pairs.
#include "kv_quant.hpp"
#include "merge.hpp"

namespace rd4 {

namespace {

constexpr int kThreads = 256;
constexpr int kTK = 32;    // keys per LDS tile
constexpr int kGMax = 8;   // query heads per CTA (GQA chunk)

// Byte copy of `rows` rows of `rb` bytes (global stride gstride) into LDS rows
// of stride `ls`, in 4-byte units when both strides allow it, else 2-byte.
__device__ __forceinline__ void copy_rows(uint8_t *lds, int ls, const uint8_t *g, int64_t gstride,
                                          int rb, int rows) {
  if ((rb & 3) == 0 && (gstride & 3) == 0 && (((uintptr_t)g) & 3) == 0) {
    const int per = rb >> 2;
    for (int u = threadIdx.x; u < rows * per; u += kThreads) {
      const int r = u / per, c = u - r * per;
      *(uint32_t *)(lds + r * ls + 4 * c) = *(const uint32_t *)(g + r * gstride + 4 * c);
    }
  } else {
    const int per = rb >> 1;
    for (int u = threadIdx.x; u < rows * per; u += kThreads) {
      const int r = u / per, c = u - r * per;
      *(uint16_t *)(lds + r * ls + 2 * c) = *(const uint16_t *)(g + r * gstride + 2 * c);
    }
  }
}

}  // namespace

template <int KT, int VT>
__global__ __launch_bounds__(kThreads) void attn_generic_kernel(AttnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int s = blockIdx.x;               // key split
  const int kvh = blockIdx.y / a.n_chunks;  // kv head
  const int hc = blockIdx.y - kvh * a.n_chunks;
  const int tok = blockIdx.z;
  const int tid = threadIdx.x;
  const int hd = a.head_dim;
  const int grp = a.n_head / a.n_head_kv;
  const int h0 = kvh * grp + hc * kGMax;            // first query head of this chunk
  const int G = min(kGMax, grp - hc * kGMax);      // heads in this chunk
  int t = a.pos ? a.pos[tok] : a.t + tok;        // consecutive positions without pos[]
  if (a.kcap > 0) t = min(t, a.kcap - 1);        // prefill: no key past kmax
  const int n_keys = t + 1;                        // may be <= 0: no keys

  // Contiguous key range of this split, in whole tiles.
  int chunk = (max(n_keys, 0) + a.n_splits - 1) / a.n_splits;
  chunk = (chunk + kTK - 1) / kTK * kTK;
  const int j_begin = s * chunk;
  const int j_end = min(n_keys, j_begin + chunk);

  const int krb = (int)row_bytes(KT, hd), vrb = (int)row_bytes(VT, hd);
  const int kls = a.k_lds_stride, vls = a.v_lds_stride;

  // LDS carve-up (sizes fixed by the host launcher).
  float *q_s = (float *)smem;                                  // [kGMax][hd]
  float *red = q_s + kGMax * hd;                               // [8][kGMax][kTK] partial dots
  float *p_s = red + 8 * kGMax * kTK;                          // [kGMax][kTK]
  float *m_s = p_s + kGMax * kTK;                              // [kGMax]
  float *l_s = m_s + kGMax;                                    // [kGMax]
  float *c_s = l_s + kGMax;                                    // [kGMax] rescale
  int *flag = (int *)(c_s + kGMax);                            // [4]
  uint8_t *k_t = (uint8_t *)(flag + 4);                        // [kTK][kls]
  uint8_t *v_t = k_t + kTK * kls;                              // [kTK][vls]

  const int64_t kstride = (int64_t)a.n_head_kv * krb, vstride = (int64_t)a.n_head_kv * vrb;
  const uint8_t *kbase = a.k + (int64_t)kvh * krb;
  const uint8_t *vbase = a.v + (int64_t)kvh * vrb;

  // Fused append: the CTA owning key t first writes the new K/V row of its kv head.
  if (a.k_new && j_begin <= t && t < j_end) {
    const bool isv = tid >= 128;
    const int u = tid & 127;
    if (u < hd / 4) {
      const float *src = (isv ? a.v_new : a.k_new) + (int64_t)kvh * hd + 4 * u;
      float x[4] = {src[0], src[1], src[2], src[3]};
      uint8_t *row = (uint8_t *)(isv ? vbase : kbase) + (int64_t)t * (isv ? vstride : kstride);
      if (isv)
        store_group4<VT>(x, tid & 7, row, u >> 3);
      else
        store_group4<KT>(x, tid & 7, row, u >> 3);
    }
  }
  if (a.k_new) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __syncthreads();

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * hd;
  if (a.q_f16) {
    const uint16_t *qh = (const uint16_t *)a.q;
    for (int i = tid; i < G * hd; i += kThreads) q_s[i] = h2f(qh[qoff + i]);
  } else {
    for (int i = tid; i < G * hd; i += kThreads) q_s[i] = a.q[qoff + i];
  }
  if (tid < kGMax) {
    m_s[tid] = -INFINITY;
    l_s[tid] = 0.0f;
    c_s[tid] = 1.0f;
  }

  // PV ownership: quad qd of dims [4qd, 4qd+4), key group kg of keys j = kg mod KG.
  const int nq = hd >> 2;
  const int KG = kThreads / nq;                 // >= 2 for hd <= 512
  const int qd = tid % nq, kg = tid / nq;
  const bool pv_on = kg < KG;
  float acc[kGMax][4];
#pragma unroll
  for (int g = 0; g < kGMax; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[g][i] = 0.0f;

  // QK ownership: key lane kj, dim slice sl of hd/8 dims.
  const int kj = tid & (kTK - 1), sl = tid / kTK;
  const int sl_len = hd >> 3;

  for (int j0 = j_begin; j0 < j_end; j0 += kTK) {
    const int nk = min(kTK, j_end - j0);
    __syncthreads();  // previous tile fully consumed
    copy_rows(k_t, kls, kbase + (int64_t)j0 * kstride, kstride, krb, nk);
    copy_rows(v_t, vls, vbase + (int64_t)j0 * vstride, vstride, vrb, nk);
    __syncthreads();

    // QK partial dots over this thread's dim slice.
    {
      float part[kGMax];
#pragma unroll
      for (int g = 0; g < kGMax; ++g) part[g] = 0.0f;
      if (kj < nk) {
        const uint8_t *kr = k_t + kj * kls;
        for (int d = sl * sl_len; d < (sl + 1) * sl_len; d += 4) {
          float kk[4];
          load4<KT>(kr, d, kk);
#pragma unroll
          for (int g = 0; g < kGMax; ++g) {
            if (g < G) {
              const float4 qv = *(const float4 *)(q_s + g * hd + d);
              part[g] = fmaf(qv.x, kk[0], part[g]);
              part[g] = fmaf(qv.y, kk[1], part[g]);
              part[g] = fmaf(qv.z, kk[2], part[g]);
              part[g] = fmaf(qv.w, kk[3], part[g]);
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < kGMax; ++g) red[(sl * kGMax + g) * kTK + kj] = part[g];
    }
    __syncthreads();

    // Online softmax per head: one 32-lane half-wave per head.
    if (tid < G * kTK) {
      const int g = tid / kTK, j = tid & (kTK - 1);
      float sc = -INFINITY;
      if (j < nk) {
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) sum += red[(c * kGMax + g) * kTK + j];
        sc = sum * a.scale;
      }
      float mt = sc;
#pragma unroll
      for (int m = 1; m < kTK; m <<= 1) mt = fmaxf(mt, xor_f(mt, m));
      const float m_old = m_s[g];
      const float m_new = fmaxf(m_old, mt);
      const float p = (m_new == -INFINITY || sc == -INFINITY) ? 0.0f : expf(sc - m_new);
      p_s[g * kTK + j] = p;
      float ps = p;
#pragma unroll
      for (int m = 1; m < kTK; m <<= 1) ps += xor_f(ps, m);
      if (j == 0) {
        const float corr = (m_old == -INFINITY) ? 0.0f : expf(m_old - m_new);
        c_s[g] = corr;
        l_s[g] = l_s[g] * corr + ps;
        m_s[g] = m_new;
      }
    }
    __syncthreads();

    // PV: rescale and accumulate this thread's keys and dims.
    if (pv_on) {
#pragma unroll
      for (int g = 0; g < kGMax; ++g) {
        const float c = c_s[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] *= c;
      }
      for (int j = kg; j < nk; j += KG) {
        float vv[4];
        load4<VT>(v_t + j * vls, 4 * qd, vv);
#pragma unroll
        for (int g = 0; g < kGMax; ++g) {
          if (g < G) {
            const float p = p_s[g * kTK + j];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(p, vv[i], acc[g][i]);
          }
        }
      }
    }
  }

  // Sum the key groups' accumulators into q_s (free now) -> [G][hd].
  __syncthreads();
  for (int i = tid; i < G * hd; i += kThreads) q_s[i] = 0.0f;
  for (int r = 0; r < KG; ++r) {
    __syncthreads();
    if (pv_on && kg == r) {
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) q_s[g * hd + 4 * qd + i] += acc[g][i];
    }
  }
  __syncthreads();

  if (a.n_splits == 1) {
    // Whole key range in this CTA: normalize, gate, write.
    for (int i = tid; i < G * hd; i += kThreads) {
      const int g = i / hd;
      const float l = l_s[g];
      float o = (m_s[g] == -INFINITY) ? 0.0f : q_s[i] * ((l > 0.0f) ? 1.0f / l : 0.0f);
      const int64_t oi = qoff + i;
      if (a.gate) {
        const float sg = sigmoid_dev(a.gate[oi]);
        a.gate[oi] = sg;
        o = o * sg;
      }
      a.out[oi] = o;
    }
    return;
  }

  // Publish this split's records, then merge.
  for (int i = tid; i < G * hd; i += kThreads) {
    const int hh = i / hd, d = i - hh * hd;
    rec_acc(a, (int64_t)tok * a.n_head + h0 + hh, s)[d] = q_s[i];
  }
  if (tid < G) {
    float *ml = rec_ml(a, (int64_t)tok * a.n_head + h0 + tid, s);
    ml[0] = m_s[tid];
    ml[1] = l_s[tid];
  }
  split_tail<kThreads>(a, tok, kvh, hc, h0, G, s, flag, red, red + kGMaxMerge * kMergeFan);
}

int generic_lds_stride(int rb) {
  int words = (rb + 3) / 4;
  if ((words & 1) == 0) ++words;  // odd word stride: lanes reading one column of 32 rows hit distinct banks
  return words * 4;
}

size_t generic_lds_bytes(int kt, int vt, int hd, int n_splits) {
  const size_t fixed = (size_t)kGMax * hd * 4 + 8 * kGMax * kTK * 4 + kGMax * kTK * 4 +
                       3 * kGMax * 4 + 16;
  const size_t kls = generic_lds_stride((int)row_bytes(kt, hd));
  const size_t vls = generic_lds_stride((int)row_bytes(vt, hd));
  (void)n_splits;
  return fixed + kTK * (kls + vls);
}

template <int KT, int VT>
static hipError_t launch_typed(const AttnArgs &a, int n_tok, hipStream_t st) {
  const size_t lds = generic_lds_bytes(KT, VT, a.head_dim, a.n_splits);
  dim3 grid((unsigned)a.n_splits, (unsigned)(a.n_head_kv * a.n_chunks), (unsigned)n_tok);
  hipLaunchKernelGGL((attn_generic_kernel<KT, VT>), grid, dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

hipError_t attn_generic_launch(int kt, int vt, AttnArgs a, int n_tok, hipStream_t st) {
  a.k_lds_stride = generic_lds_stride((int)row_bytes(kt, a.head_dim));
  a.v_lds_stride = generic_lds_stride((int)row_bytes(vt, a.head_dim));
  a.n_chunks = (a.n_head / a.n_head_kv + kGMax - 1) / kGMax;
#define RD4_PAIR(K, V) \
  if (kt == K && vt == V) return launch_typed<K, V>(a, n_tok, st);
#define RD4_ROW(K) \
  RD4_PAIR(K, F32) RD4_PAIR(K, F16) RD4_PAIR(K, Q8_0) RD4_PAIR(K, Q4_0) RD4_PAIR(K, Q5_0) RD4_PAIR(K, Q4_1)
  RD4_ROW(F32) RD4_ROW(F16) RD4_ROW(Q8_0) RD4_ROW(Q4_0) RD4_ROW(Q5_0) RD4_ROW(Q4_1)
#undef RD4_ROW
#undef RD4_PAIR
  return hipErrorInvalidValue;
}

}  // namespace rd4
