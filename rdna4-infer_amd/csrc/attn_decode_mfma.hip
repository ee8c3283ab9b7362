// Split-KV GQA decode on f16 MFMA (gfx950), K/V in f16, q8_0 or q4_0.
//
// Reference semantics: attn_split_kernel + attn_merge_kernel and the batched
// forms (include/rdna4/attn.cuh:445-590, 686-845) with the output gate of
// nn.cuh:405-412 and the append of graph.cuh:1011-1031 optionally fused:
// out[h] = softmax_j(q_h . k_j * scale) . V over keys 0..t, f32 accumulation.
//
// Work decomposition: CTA = 8 waves = one (token, kv head, <=8-query-head
// chunk, key split). Each wave walks its own 16-key tiles of the split
// (tiles w, w+8, ...: the 8 waves stream adjacent memory) with a private
// online-softmax state, so the main loop has no CTA barrier. Per tile:
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
//      lane one query row x 4 keys, exactly the B operand layout PV needs; the
//      O rescale is skipped when no row's running max moved;
//   4. O^T += V^T P^T on v_mfma_f32_16x16x16_f16: A = 16 dims x 16 keys of V
//      read from LDS, B = p (hi/lo rows again), with the quantized V's d folded
//      into p per 32-dim block.
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
constexpr int kTile = 16;    // keys per wave tile
constexpr int kG = 8;        // query heads per CTA (MFMA rows 0-7 hi, 8-15 lo)
constexpr float kLog2e = 1.4426950408889634f;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Wait until at most N of this wave's vector memory loads are outstanding
// (loads complete in issue order); also a compiler memory barrier.
template <int N>
__device__ __forceinline__ void wait_vm() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int T>
__host__ __device__ constexpr int rowb() {
  return T == F16 ? kHD * 2 : (kHD / 32) * block_bytes(T);
}
template <int T>
__host__ __device__ constexpr int chunks_per_row() {
  return rowb<T>() / 16;
}
// f16 rows are 32 chunks (512 B, a multiple of the 64 banks): the chunk of
// global column c in row r sits at slot c ^ (r & 15) so 16 lanes reading one
// column of 16 rows hit 16 different banks. Block-quantized rows (17 or 9
// chunks) are conflict-free unswizzled.
template <int T>
__device__ __forceinline__ int swz(int row, int col) {
  return T == F16 ? (col ^ (row & 15)) : col;
}

// Tile image in LDS: the tile's K rows then V rows, contiguous 16-byte chunks,
// padded to whole 64-chunk load instructions.
template <int KT, int VT>
struct TileShape {
  static constexpr int KC = chunks_per_row<KT>(), VC = chunks_per_row<VT>();
  static constexpr int KCH = kTile * KC, VCH = kTile * VC;
  static constexpr int NI = (KCH + VCH + 63) / 64;  // load instructions per tile
  static constexpr int TB = NI * 1024;              // bytes per ring stage
  // per-wave f32 scale tables [block][key] for the quantized K and V of a tile
  static constexpr int DT = (KT != F16 ? 512 : 0) + (VT != F16 ? 512 : 0);
#ifndef RD4_DEC_WAVES_SMALL
#define RD4_DEC_WAVES_SMALL 8
#endif
#ifndef RD4_DEC_RMAX
#define RD4_DEC_RMAX 3
#endif
  static constexpr int WAVES = TB <= 10240 ? RD4_DEC_WAVES_SMALL : 4;
  static constexpr int R0 = (152 * 1024 / WAVES - DT) / TB;
  static constexpr int R = R0 < 2 ? 2 : (R0 > RD4_DEC_RMAX ? RD4_DEC_RMAX : R0);  // ring stages per wave
};

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
__device__ __forceinline__ half8 k_frag(const uint8_t *krow, int b, int g, int n_of_row) {
  u32x4 r;
  if constexpr (KT == F16) {
    r = *(const u32x4 *)(krow + 16 * ((4 * b + g) ^ n_of_row));
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

// A operand of O^T = V^T P^T (v_mfma_f32_16x16x16_f16) for dim d (this lane's)
// and keys 4g..4g+3 of the tile, as f16.
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
template <int VT>
__device__ __forceinline__ half4 v_frag(const uint8_t *vt, int d, int g) {
  constexpr int vs = rowb<VT>();
  const uint8_t *p0 = vt + 4 * g * vs;
  uint32_t e[4];
  uint32_t r0, r1;
  if constexpr (VT == F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      e[i] = lds_u16(p0 + i * vs + 16 * ((d >> 3) ^ ((4 * g + i) & 15)) + 2 * (d & 7));
    r0 = e[0] | (e[1] << 16);
    r1 = e[2] | (e[3] << 16);
  } else if constexpr (VT == Q8_0) {
    // bytes land in the low byte of 16-bit halves; 0x64 | b^0x80 per half is
    // the f16 1024 + b + 128, so one xor and one packed add give b exactly
    const int off = 34 * (d >> 5) + 2 + (d & 31);
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    u16x2 a0, a1;
    a0.x = p0[off];
    a0.y = p0[vs + off];
    a1.x = p0[2 * vs + off];
    a1.y = p0[3 * vs + off];
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    r0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_bit_cast(uint32_t, a0) ^ 0x64806480u) + c);
    r1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_bit_cast(uint32_t, a1) ^ 0x64806480u) + c);
    (void)e;
  } else {
    const int j = d & 31;
    const int off = 18 * (d >> 5) + 2 + (j & 15);
    const int sh = (j & 16) ? 4 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = (lds_u8(p0 + i * vs + off) >> sh) & 0xfu;
    r0 = nib2_to_h2(e[0] | (e[1] << 16));
    r1 = nib2_to_h2(e[2] | (e[3] << 16));
  }
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(half4, u32x2{r0, r1});
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
__global__ __launch_bounds__((64 * TileShape<KT, VT>::WAVES), 1) void decode_mfma_kernel(AttnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  using TS = TileShape<KT, VT>;
  constexpr int kWaves = TS::WAVES, kThreads = 64 * kWaves;
  constexpr int KS = rowb<KT>(), VS = rowb<VT>();
  constexpr int KC = TS::KC, VC = TS::VC, KCH = TS::KCH, VCH = TS::VCH, NI = TS::NI;
  constexpr int TB = TS::TB, R = TS::R, DT = TS::DT;

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

  // Fused append: the CTA owning key t writes the new K/V row of its kv head
  // (8-lane groups per 32-element block, the store kernel's quantizer).
  if (a.k_new && j_begin <= t && t < j_end && tid < 128) {
    const bool isv = tid >= 64;
    const int u = tid & 63;
    const float *src = (isv ? a.v_new : a.k_new) + (int64_t)kvh * kHD + 4 * u;
    float x[4] = {src[0], src[1], src[2], src[3]};
    uint8_t *row = (uint8_t *)(isv ? vbase : kbase) + (int64_t)t * (isv ? vstride : kstride);
    if (isv)
      store_group4<VT>(x, u & 7, row, u >> 3);
    else
      store_group4<KT>(x, u & 7, row, u >> 3);
  }
  // the new row reaches this CU's L1 before any wave loads it (workgroup scope only)
  if (a.k_new) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __syncthreads();

  // Query fragment (B operand of S^T = K Q^T): row n is head n (hi) or n-8 (lo).
  // All of this lane's query loads are issued before any is used.
  half8 qf[8];
  {
    const int hh = n & 7;
    const bool on = hh < G;
    const int64_t qoff = (((int64_t)tok * a.n_head + h0 + (on ? hh : 0)) * kHD) + 8 * g;
    float qv[8][8];
    if (a.q_f16) {
      u32x4 r[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) r[b] = *(const u32x4 *)((const uint16_t *)a.q + qoff + 32 * b);
#pragma unroll
      for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[b][2 * i] = h2f((uint16_t)r[b][i]);
          qv[b][2 * i + 1] = h2f((uint16_t)(r[b][i] >> 16));
        }
    } else {
      float4 r[16];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        r[2 * b] = *(const float4 *)(a.q + qoff + 32 * b);
        r[2 * b + 1] = *(const float4 *)(a.q + qoff + 32 * b + 4);
      }
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        qv[b][0] = r[2 * b].x; qv[b][1] = r[2 * b].y; qv[b][2] = r[2 * b].z; qv[b][3] = r[2 * b].w;
        qv[b][4] = r[2 * b + 1].x; qv[b][5] = r[2 * b + 1].y; qv[b][6] = r[2 * b + 1].z; qv[b][7] = r[2 * b + 1].w;
      }
    }
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qf[b][i] = on ? ((n < 8) ? hi_part(qv[b][i]) : lo_part(qv[b][i])) : (_Float16)0.0f;
  }
  const float sl2 = a.scale * kLog2e;

  floatx4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  // ---- async tile ring: stage i of this wave at ring + (i % R) * TB
  uint8_t *ring = smem + w * (R * TB + DT);
  float *dk_t = (float *)(ring + R * TB);                  // [8][16] K scales (quantized K)
  float *dv_t = dk_t + (KT != F16 ? 128 : 0);              // [8][16] V scales (quantized V)
  const int n_tiles_all = (j_end - j_begin + kTile - 1) / kTile;
  const int my_tiles = (a.dbg & 32) ? 0 : (n_tiles_all > w ? (n_tiles_all - w + kWaves - 1) / kWaves : 0);
  // Global source of this lane's chunk in load instruction r of a full tile:
  // byte offset from the tile's K (or V) base, with the f16 swizzle applied.
  auto src_of = [&](int r, int nk, const uint8_t *kt0, const uint8_t *vt0) -> const uint8_t * {
    const int c = lane + 64 * r;
    if (c < KCH) {
      const int row = c / KC, slot = c - row * KC;
      const int col = swz<KT>(row, slot);
      return kt0 + (row < nk ? row * (int)kstride + 16 * col : 16 * col);
    }
    const int cv = c < KCH + VCH ? c - KCH : 0;
    const int row = cv / VC, slot = cv - row * VC;
    const int col = swz<VT>(row, slot);
    return vt0 + (row < nk ? row * (int)vstride + 16 * col : 16 * col);
  };
  auto issue = [&](int i) {  // i-th tile of this wave
    const int j0 = j_begin + (w + i * kWaves) * kTile;
    const int nk = min(kTile, j_end - j0);
    const uint8_t *kt0 = kbase + (int64_t)j0 * kstride;
    const uint8_t *vt0 = vbase + (int64_t)j0 * vstride;
    uint8_t *st = ring + (i % R) * TB;
#pragma unroll
    for (int r = 0; r < NI; ++r)
      __builtin_amdgcn_global_load_lds((const void *)src_of(r, nk, kt0, vt0),
                                       (lds_void *)(st + 1024 * r), 16, 0, 0);
  };
#pragma unroll
  for (int i = 0; i < R - 1; ++i)
    if (i < my_tiles) issue(i);

  for (int i = 0; i < my_tiles; ++i) {
    const int nk = min(kTile, j_end - (j_begin + (w + i * kWaves) * kTile));
    if (i + R - 1 < my_tiles) {
      // the stage being refilled was read by the previous iteration: those reads are done
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(i + R - 1);
    }
    // tile i is complete once at most the loads of the tiles issued after it remain
    const int after = min(R - 1, my_tiles - 1 - i);
    if (after >= 3) wait_vm<3 * NI>();
    else if (after == 2) wait_vm<2 * NI>();
    else if (after == 1) wait_vm<NI>();
    else wait_vm<0>();
    wave_sync();
    const uint8_t *kl = ring + (i % R) * TB;
    const uint8_t *vl = kl + KCH * 16;
    if constexpr (DT > 0) {  // f16 scales of the tile -> f32 tables, once per tile
#pragma unroll
      for (int j = 0; j < DT / 256; ++j) {
        const int v = lane + 64 * j;
        const bool isv = (KT == F16) || (VT != F16 && v >= 128);
        const int vv = v & 127, key = vv & 15, b = vv >> 4;
        const float d = isv ? scale_of<VT>(vl + key * VS, b) : scale_of<KT>(kl + key * KS, b);
        (isv ? dv_t : dk_t)[b * 16 + key] = d;
      }
      wave_sync();
    }

    // ---- S^T = K Q^T: lane holds keys 4g..4g+3 of row n
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (a.dbg & 2) {
      acc = floatx4{(float)lane, 1.f, 2.f, 3.f};
    } else {
      const uint8_t *krow = kl + n * KS;
      if constexpr (KT == F16) {
#pragma unroll
        for (int b = 0; b < 8; ++b)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g, n), qf[b], acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const floatx4 z = {0.f, 0.f, 0.f, 0.f};
          const floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g, n), qf[b], z, 0, 0, 0);
          const float4 dk = *(const float4 *)(dk_t + b * 16 + 4 * g);
          acc[0] = fmaf(dk.x, c[0], acc[0]);
          acc[1] = fmaf(dk.y, c[1], acc[1]);
          acc[2] = fmaf(dk.z, c[2], acc[2]);
          acc[3] = fmaf(dk.w, c[3], acc[3]);
        }
      }
    }
    // rows n and n^8 are the hi and lo halves of the same head
    float sc[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = (acc[i] + xor_f(acc[i], 8)) * sl2;
      if (4 * g + i >= nk) v = -INFINITY;
      sc[i] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = fmaxf(tmax, xor_f(tmax, 16));
    tmax = fmaxf(tmax, xor_f(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = __builtin_amdgcn_exp2f(sc[i] - m_new);
      psum += sc[i];
    }
    if (__any(m_new != m_run)) {  // lazy rescale: skipped when no row's max moved
      const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < 16; ++i) o[i] *= corr;
    }
    m_run = m_new;
    l_run += psum;

    // ---- O^T += V^T P^T (16 keys)
    if (a.dbg & 4) {
      o[0][0] += sc[0] + sc[3];
      (void)vl;
    } else if constexpr (VT == F16) {
      half4 pf;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = (n < 8) ? hi_part(sc[i]) : lo_part(sc[i]);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_frag<VT>(vl, 16 * dt + n, g), pf, o[dt], 0, 0, 0);
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        half4 pf;
        const float4 dv = *(const float4 *)(dv_t + b * 16 + 4 * g);
        const float dvv[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pd = sc[i] * dvv[i];
          pf[i] = (n < 8) ? hi_part(pd) : lo_part(pd);
        }
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          const int dt = 2 * b + dd;
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_frag<VT>(vl, 16 * dt + n, g), pf, o[dt], 0, 0, 0);
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

  // ---- merge the waves through LDS (reuses the tile buffers)
  __syncthreads();
  float *wm = (float *)smem;                 // [kWaves][kG] m, then [kWaves][kG] l
  float *wo = wm + 2 * kWaves * kG;          // [kWaves][kG][kHD]
  if (lane < kG) {
    wm[w * kG + lane] = m_run;
    wm[kWaves * kG + w * kG + lane] = l_run;
  }
  if (n < 8) {
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
      *(floatx4 *)(wo + (w * kG + n) * kHD + 16 * dt + 4 * g) = o[dt];
  }
  __syncthreads();
  float *ms = wo + kWaves * kG * kHD;  // [kG] m (ln units), [kG] L, [kWaves][kG] weights
  if (tid < kG) {
    float mm = -INFINITY;
    for (int ww = 0; ww < kWaves; ++ww) mm = fmaxf(mm, wm[ww * kG + tid]);
    float L = 0.0f;
    for (int ww = 0; ww < kWaves; ++ww) {
      const float wt = (mm == -INFINITY) ? 0.0f : exp2f(wm[ww * kG + tid] - mm);
      ms[2 * kG + ww * kG + tid] = wt;
      L += wt * wm[kWaves * kG + ww * kG + tid];
    }
    ms[tid] = (mm == -INFINITY) ? -INFINITY : mm * 0.6931471805599453f;  // log2 -> ln units
    ms[kG + tid] = L;
  }
  __syncthreads();

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * kHD;
  const int64_t hrow = (int64_t)tok * a.n_head + h0;
  for (int i = tid; i < G * kHD / 4; i += kThreads) {
    const int hh = i / (kHD / 4), d = 4 * (i - hh * (kHD / 4));
    floatx4 acc4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww)
      acc4 += ms[2 * kG + ww * kG + hh] * *(const floatx4 *)(wo + (ww * kG + hh) * kHD + d);
    if (a.n_splits == 1) {
      const float L = ms[kG + hh];
      const float inv = (ms[hh] == -INFINITY) ? 0.0f : ((L > 0.0f) ? 1.0f / L : 0.0f);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float o1 = acc4[k] * inv;
        const int64_t oi = qoff + hh * kHD + d + k;
        if (a.gate) {
          const float sg = sigmoid_dev(a.gate[oi]);
          a.gate[oi] = sg;
          o1 = o1 * sg;
        }
        a.out[oi] = o1;
      }
    } else {
      *(floatx4 *)(rec_acc(a, hrow + hh, s) + d) = acc4;
    }
  }
  if (a.n_splits == 1) return;
  if (tid < G) {
    float *ml = rec_ml(a, hrow + tid, s);
    ml[0] = ms[tid];
    ml[1] = ms[kG + tid];
  }
  int *flag = (int *)(ms + 2 * kG + kWaves * kG);
  if (a.dbg & 1) return;
  split_tail<kThreads>(a, tok, kvh, hc, h0, G, s, flag, (float *)(flag + 4),
                       (float *)(flag + 4) + kGMaxMerge * kMergeFan);
}

namespace {

template <int KT, int VT>
size_t decode_lds() {
  using TS = TileShape<KT, VT>;
  const size_t tiles = (size_t)TS::WAVES * (TS::R * TS::TB + TS::DT);
  const size_t merge = (2 * TS::WAVES * kG + TS::WAVES * kG * kHD + 2 * kG + TS::WAVES * kG + 4) * 4 +
                       (kGMaxMerge * kMergeFan + 2 * kGMaxMerge) * 4;
  return tiles > merge ? tiles : merge;
}

template <int KT, int VT>
hipError_t launch(const AttnArgs &a, int n_tok, hipStream_t st) {
  dim3 grid((unsigned)a.n_splits, (unsigned)(a.n_head_kv * a.n_chunks), (unsigned)n_tok);
  hipLaunchKernelGGL((decode_mfma_kernel<KT, VT>), grid, dim3(64 * TileShape<KT, VT>::WAVES),
                     (decode_lds<KT, VT>()), st, a);
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
