// Split-KV GQA decode on f16 MFMA (gfx950), K/V in f16, q8_0 or q4_0.
//
// Reference semantics: attn_split_kernel + attn_merge_kernel and the batched
// forms (include/rdna4/attn.cuh:445-590, 686-845) with the output gate of
// nn.cuh:405-412 and the append of graph.cuh:1011-1031 optionally fused:
// out[h] = softmax_j(q_h . k_j * scale) . V over keys 0..t, f32 accumulation.
//
// Work decomposition: CTA = 4 waves = one (token, kv head, <=8-query-head
// chunk, key split). Each wave walks its own 32-key tiles of the split
// (tiles w, w+4, ...) with a private online-softmax state, so the main loop
// has no CTA barrier. Per tile:
//   1. the tile's raw K and V rows (exactly the cache bytes) arrive with
//      16-byte global loads issued one tile ahead into registers, and are
//      written to a wave-private LDS buffer;
//   2. S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K
//      converted to f16 on the fly (f16 as is; q8_0/q4_0 integers, exact in
//      f16), B = the query rows. The 16 MFMA rows carry the group's query heads
//      twice, as f16 hi and lo parts (q = hi + lo to 2^-22), so the f32 query
//      costs no precision. Quantized K is scaled by its per-(key, block) d after
//      each 32-dim block's MFMA;
//   3. online softmax in registers (exp2 domain); the C layout of S^T gives each
//      lane one query row x 8 keys, exactly the B operand layout PV needs;
//   4. O^T += V^T P^T on the same MFMA: A = 16 dims x 32 keys of V read from
//      LDS, B = p (hi/lo rows again), with the quantized V's d folded into p per
//      32-dim block.
// The 4 waves' states merge through LDS into one (m, l, acc) record per query
// head; splits merge through the two-level tree of merge.hpp in the same launch.
#include <cstdlib>

#include "kv_quant.hpp"
#include "merge.hpp"
#include "prefill.hpp"

namespace rd4 {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHD = 256;     // head_dim of this kernel
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 32;    // keys per wave tile
constexpr int kG = 8;        // query heads per CTA (MFMA rows 0-7 hi, 8-15 lo)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int T>
__host__ __device__ constexpr int rowb() {
  return T == F16 ? kHD * 2 : (kHD / 32) * block_bytes(T);
}
// LDS row stride: 16-byte multiple whose word count is not a multiple of 64,
// so 16 lanes reading one column of 16 rows do not share a bank.
template <int T>
__host__ __device__ constexpr int lds_stride() {
  return (rowb<T>() / 4) % 64 == 0 ? rowb<T>() + 16 : rowb<T>();
}
template <int T>
__host__ __device__ constexpr int chunks_per_row() {
  return rowb<T>() / 16;
}
template <int KT, int VT>
__host__ __device__ constexpr int tile_chunks() {
  return kTile * (chunks_per_row<KT>() + chunks_per_row<VT>());
}
template <int KT, int VT>
__host__ __device__ constexpr int regs_per_lane() {
  return (tile_chunks<KT, VT>() + 63) / 64;
}
template <int KT, int VT>
__host__ __device__ constexpr int wave_lds_bytes() {
  return kTile * (lds_stride<KT>() + lds_stride<VT>());
}

__device__ __forceinline__ uint32_t lds_u16(const uint8_t *p) { return *(const uint16_t *)p; }
__device__ __forceinline__ uint32_t lds_u8(const uint8_t *p) { return *p; }

// Two signed bytes (bits 0-7 and 8-15 of v) -> two f16 holding the same integers.
// 0x6400 | (b ^ 0x80) is the f16 1024 + b + 128; subtracting 1152 is exact.
__device__ __forceinline__ uint32_t i8x2_to_h2(uint32_t v) {
  const uint32_t w = __builtin_amdgcn_perm(0u, v, 0x0c010c00u) ^ 0x64806480u;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 x = __builtin_bit_cast(h2, w);
  const h2 c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  x = x + c;
  return __builtin_bit_cast(uint32_t, x);
}
// Two 4-bit values (bits 0-3 and 16-19 of v) -> two f16 of (n - 8).
__device__ __forceinline__ uint32_t nib2_to_h2(uint32_t v) {
  const uint32_t w = (v & 0x000f000fu) | 0x64006400u;  // 1024 + n
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 x = __builtin_bit_cast(h2, w);
  const h2 c = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  x = x + c;
  return __builtin_bit_cast(uint32_t, x);
}

// A operand of S^T = K Q^T for one 16-key half and one 32-dim block: lane
// (key = l%16, g = l/16) gets dims 32b + 8g .. +7 of its key, as f16.
template <int KT>
__device__ __forceinline__ half8 k_frag(const uint8_t *krow, int b, int g) {
  u32x4 r;
  if constexpr (KT == F16) {
    r = *(const u32x4 *)(krow + 2 * (32 * b + 8 * g));
  } else if constexpr (KT == Q8_0) {
    const uint8_t *p = krow + 34 * b + 2 + 8 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = i8x2_to_h2(lds_u16(p + 2 * i));
  } else {  // Q4_0: element j < 16 is the low nibble of qs[j], j >= 16 the high nibble of qs[j-16]
    const uint8_t *p = krow + 18 * b + 2 + 8 * (g & 1);
    const int sh = (g & 2) ? 4 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = lds_u16(p + 2 * i) >> sh;  // byte0 -> bits 0-3, byte1 -> bits 8-11
      r[i] = nib2_to_h2((v & 0xfu) | ((v & 0xf00u) << 8));
    }
  }
  return __builtin_bit_cast(half8, r);
}

// A operand of O^T = V^T P^T for dim d (this lane's) and the 8 keys of k-slots
// 8g..8g+7 (keys 4g..4g+3 and 16+4g..16+4g+3 of the tile), as f16.
template <int VT>
__device__ __forceinline__ half8 v_frag(const uint8_t *vt, int d, int g) {
  constexpr int vs = lds_stride<VT>();
  uint32_t e[8];
  if constexpr (VT == F16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = (i < 4) ? 4 * g + i : 16 + 4 * g + i - 4;
      e[i] = lds_u16(vt + key * vs + 2 * d);
    }
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = e[2 * i] | (e[2 * i + 1] << 16);
    return __builtin_bit_cast(half8, r);
  } else if constexpr (VT == Q8_0) {
    const int off = 34 * (d >> 5) + 2 + (d & 31);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = (i < 4) ? 4 * g + i : 16 + 4 * g + i - 4;
      e[i] = lds_u8(vt + key * vs + off);
    }
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = i8x2_to_h2(e[2 * i] | (e[2 * i + 1] << 8));
    return __builtin_bit_cast(half8, r);
  } else {
    const int j = d & 31;
    const int off = 18 * (d >> 5) + 2 + (j & 15);
    const int sh = (j & 16) ? 4 : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = (i < 4) ? 4 * g + i : 16 + 4 * g + i - 4;
      e[i] = (lds_u8(vt + key * vs + off) >> sh) & 0xfu;
    }
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = nib2_to_h2(e[2 * i] | (e[2 * i + 1] << 16));
    return __builtin_bit_cast(half8, r);
  }
}

template <int T>
__device__ __forceinline__ float scale_of(const uint8_t *row, int b) {
  return h2f((uint16_t)lds_u16(row + block_bytes(T) * b));
}

// hi/lo f16 pair of an f32 (x = hi + lo to ~2^-22 relative).
__device__ __forceinline__ _Float16 hi_part(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 lo_part(float x) { return (_Float16)(x - (float)(_Float16)x); }

}  // namespace

template <int KT, int VT>
__global__ __launch_bounds__(kThreads, (KT == F16 || VT == F16) ? 1 : 2) void decode_mfma_kernel(AttnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int WL = wave_lds_bytes<KT, VT>();
  constexpr int KS = lds_stride<KT>(), VS = lds_stride<VT>();
  constexpr int KC = chunks_per_row<KT>(), VC = chunks_per_row<VT>();
  constexpr int NR = regs_per_lane<KT, VT>();

  const int s = blockIdx.x;
  const int kvh = blockIdx.y / a.n_chunks;
  const int hc = blockIdx.y - kvh * a.n_chunks;
  const int tok = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int grp = a.n_head / a.n_head_kv;
  const int h0 = kvh * grp + hc * kG;
  const int G = min(kG, grp - hc * kG);
  const int t = a.pos ? a.pos[tok] : a.t + tok;
  const int n_keys = t + 1;

  int chunk = (max(n_keys, 0) + a.n_splits - 1) / a.n_splits;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  const int j_begin = s * chunk;
  const int j_end = min(n_keys, j_begin + chunk);

  const int64_t kstride = (int64_t)a.n_head_kv * rowb<KT>();
  const int64_t vstride = (int64_t)a.n_head_kv * rowb<VT>();
  const uint8_t *kbase = a.k + (int64_t)kvh * rowb<KT>();
  const uint8_t *vbase = a.v + (int64_t)kvh * rowb<VT>();

  // Fused append: the CTA owning key t writes the new K/V row of its kv head.
  if (a.k_new && j_begin <= t && t < j_end) {
    const int sub = tid & 7;
    const bool isv = tid >= 128;
    const int u = tid & 127;  // 8 blocks x 8 lanes per row side (hd 256 -> 64 lanes used)
    if (u < kHD / 4) {
      const float *src = (isv ? a.v_new : a.k_new) + (int64_t)kvh * kHD + 4 * u;
      float x[4] = {src[0], src[1], src[2], src[3]};
      uint8_t *row = (uint8_t *)(isv ? vbase : kbase) + (int64_t)t * (isv ? vstride : kstride);
      if (isv)
        store_group4<VT>(x, sub, row, u >> 3);
      else
        store_group4<KT>(x, sub, row, u >> 3);
    }
  }
  if (a.k_new) __threadfence();  // the new row is visible before any wave loads it
  __syncthreads();

  // Query fragment (B operand of S^T = K Q^T): row n is head n (hi) or n-8 (lo).
  half8 qf[8];
  {
    const int hh = n & 7;
    const bool on = hh < G;
    const int64_t qoff = (((int64_t)tok * a.n_head + h0 + hh) * kHD);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = 32 * b + 8 * g + i;
        float qv = 0.0f;
        if (on) qv = a.q_f16 ? h2f(((const uint16_t *)a.q)[qoff + d]) : a.q[qoff + d];
        qf[b][i] = (n < 8) ? hi_part(qv) : lo_part(qv);
      }
    }
  }
  const float sl2 = a.scale * kLog2e;

  uint8_t *wl = smem + w * WL;  // this wave's LDS: K rows then V rows
  uint8_t *kl = wl, *vl = wl + kTile * KS;

  floatx4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  const int n_tiles = (j_end - j_begin + kTile - 1) / kTile;
  u32x4 raw[NR];

  auto issue = [&](int tile) {
    const int j0 = j_begin + tile * kTile;
    const int nk = min(kTile, j_end - j0);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int c = lane + 64 * r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (c < kTile * KC) {
        const int row = c / KC, col = c - row * KC;
        if (row < nk) v = *(const u32x4 *)(kbase + (int64_t)(j0 + row) * kstride + 16 * col);
      } else if (c < tile_chunks<KT, VT>()) {
        const int cc = c - kTile * KC;
        const int row = cc / VC, col = cc - row * VC;
        if (row < nk) v = *(const u32x4 *)(vbase + (int64_t)(j0 + row) * vstride + 16 * col);
      }
      raw[r] = v;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int c = lane + 64 * r;
      if (c < kTile * KC) {
        const int row = c / KC, col = c - row * KC;
        *(u32x4 *)(kl + row * KS + 16 * col) = raw[r];
      } else if (c < tile_chunks<KT, VT>()) {
        const int cc = c - kTile * KC;
        const int row = cc / VC, col = cc - row * VC;
        *(u32x4 *)(vl + row * VS + 16 * col) = raw[r];
      }
    }
  };

  int tile = w;
  if (tile < n_tiles) issue(tile);
  for (; tile < n_tiles; tile += kWaves) {
    const int j0 = j_begin + tile * kTile;
    const int nk = min(kTile, j_end - j0);
    wave_sync();  // previous tile's LDS reads are done
    stash();
    wave_sync();
    if (tile + kWaves < n_tiles) issue(tile + kWaves);

    // ---- S^T = K Q^T for the two 16-key halves
    float sc[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint8_t *krow = kl + (16 * h + n) * KS;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KT == F16) {
#pragma unroll
        for (int b = 0; b < 8; ++b)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g), qf[b], acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const floatx4 z = {0.f, 0.f, 0.f, 0.f};
          const floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g), qf[b], z, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float d = scale_of<KT>(kl + (16 * h + 4 * g + i) * KS, b);
            acc[i] = fmaf(d, c[i], acc[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * h + i] = acc[i];
    }
    // rows n and n^8 are the hi and lo halves of the same head
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = (i < 4) ? 4 * g + i : 16 + 4 * g + i - 4;
      float v = (sc[i] + xor_f(sc[i], 8)) * sl2;
      if (key >= nk) v = -INFINITY;
      sc[i] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = fmaxf(tmax, xor_f(tmax, 16));
    tmax = fmaxf(tmax, xor_f(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sc[i] = exp2f(sc[i] - m_new);
      psum += sc[i];
    }
    l_run = l_run * corr + psum;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] *= corr;

    // ---- O^T += V^T P^T
    if constexpr (VT == F16) {
      half8 pf;
#pragma unroll
      for (int i = 0; i < 8; ++i) pf[i] = (n < 8) ? hi_part(sc[i]) : lo_part(sc[i]);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v_frag<VT>(vl, 16 * dt + n, g), pf, o[dt], 0, 0, 0);
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        half8 pf;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int key = (i < 4) ? 4 * g + i : 16 + 4 * g + i - 4;
          const float pd = sc[i] * scale_of<VT>(vl + key * VS, b);
          pf[i] = (n < 8) ? hi_part(pd) : lo_part(pd);
        }
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          const int dt = 2 * b + dd;
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v_frag<VT>(vl, 16 * dt + n, g), pf, o[dt], 0, 0, 0);
        }
      }
    }
  }

  // ---- wave state: head n&7; hi+lo rows summed, l summed over the 4 key groups
  l_run += xor_f(l_run, 16);
  l_run += xor_f(l_run, 32);
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[dt][i] += xor_f(o[dt][i], 8);

  // ---- merge the 4 waves through LDS (reuses the tile buffers)
  __syncthreads();
  float *wm = (float *)smem;                 // [kWaves][kG] m, then l
  float *wo = wm + 2 * kWaves * kG;          // [kWaves][kG][kHD]
  if (lane < kG) {
    wm[w * kG + lane] = m_run;
    wm[kWaves * kG + w * kG + lane] = l_run;
  }
  if (n < 8) {
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) wo[(w * kG + n) * kHD + 16 * dt + 4 * g + i] = o[dt][i];
  }
  __syncthreads();
  float *ms = wm + 2 * kWaves * kG + kWaves * kG * kHD;  // [kG] m (natural log units), l, and per-wave weights
  if (tid < kG) {
    float mm = -INFINITY;
    for (int ww = 0; ww < kWaves; ++ww) mm = fmaxf(mm, wm[ww * kG + tid]);
    float L = 0.0f;
    for (int ww = 0; ww < kWaves; ++ww) {
      const float wt = (mm == -INFINITY) ? 0.0f : exp2f(wm[ww * kG + tid] - mm);
      ms[3 * kG + ww * kG + tid] = wt;
      L += wt * wm[kWaves * kG + ww * kG + tid];
    }
    ms[tid] = (mm == -INFINITY) ? -INFINITY : mm * 0.6931471805599453f;  // log2 -> ln units
    ms[kG + tid] = L;
  }
  __syncthreads();

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * kHD;
  if (a.n_splits == 1) {
    for (int i = tid; i < G * kHD; i += kThreads) {
      const int hh = i / kHD, d = i - hh * kHD;
      float acc = 0.0f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) acc += ms[3 * kG + ww * kG + hh] * wo[(ww * kG + hh) * kHD + d];
      const float L = ms[kG + hh];
      float o1 = (ms[hh] == -INFINITY) ? 0.0f : acc * ((L > 0.0f) ? 1.0f / L : 0.0f);
      const int64_t oi = qoff + i;
      if (a.gate) {
        const float sg = sigmoid_dev(a.gate[oi]);
        a.gate[oi] = sg;
        o1 = o1 * sg;
      }
      a.out[oi] = o1;
    }
    return;
  }
  const int rec = 2 + kHD;
  for (int i = tid; i < G * rec; i += kThreads) {
    const int hh = i / rec, c = i - hh * rec;
    float val;
    if (c == 0) {
      val = ms[hh];
    } else if (c == 1) {
      val = ms[kG + hh];
    } else {
      val = 0.0f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) val += ms[3 * kG + ww * kG + hh] * wo[(ww * kG + hh) * kHD + c - 2];
    }
    a.partial[(((int64_t)tok * a.n_head + h0 + hh) * a.n_splits + s) * rec + c] = val;
  }
  int *flag = (int *)(ms + 8 * kG);
  split_tail<kThreads>(a, tok, kvh, hc, h0, G, s, flag, (float *)(flag + 4),
                       (float *)(flag + 4) + kGMaxMerge * kMergeFan);
}

namespace {

template <int KT, int VT>
size_t decode_lds() {
  const size_t tiles = (size_t)kWaves * wave_lds_bytes<KT, VT>();
  const size_t merge = (2 * kWaves * kG + kWaves * kG * kHD + 8 * kG + 4) * 4 +
                       (kGMaxMerge * kMergeFan + 2 * kGMaxMerge) * 4;
  return tiles > merge ? tiles : merge;
}

template <int KT, int VT>
hipError_t launch(const AttnArgs &a, int n_tok, hipStream_t st) {
  dim3 grid((unsigned)a.n_splits, (unsigned)(a.n_head_kv * a.n_chunks), (unsigned)n_tok);
  hipLaunchKernelGGL((decode_mfma_kernel<KT, VT>), grid, dim3(kThreads), (decode_lds<KT, VT>()), st, a);
  return hipGetLastError();
}

bool hot_type(int t) { return t == F16 || t == Q8_0 || t == Q4_0; }

}  // namespace

bool decode_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  const char *e = std::getenv("RD4_DECODE_GENERIC");
  if (e && std::atoi(e) != 0) return false;
  return hot_type(kt) && hot_type(vt) && head_dim == kHD && n_head_kv > 0 &&
         n_head % n_head_kv == 0;
}

hipError_t decode_mfma_launch(int kt, int vt, const AttnArgs &a0, int n_tok, hipStream_t st) {
  AttnArgs a = a0;
  a.n_chunks = (a.n_head / a.n_head_kv + kG - 1) / kG;
#define RD4_D(K, V) \
  if (kt == K && vt == V) return launch<K, V>(a, n_tok, st);
  RD4_D(F16, F16) RD4_D(F16, Q8_0) RD4_D(F16, Q4_0)
  RD4_D(Q8_0, F16) RD4_D(Q8_0, Q8_0) RD4_D(Q8_0, Q4_0)
  RD4_D(Q4_0, F16) RD4_D(Q4_0, Q8_0) RD4_D(Q4_0, Q4_0)
#undef RD4_D
  return hipErrorInvalidValue;
}

}  // namespace rd4
