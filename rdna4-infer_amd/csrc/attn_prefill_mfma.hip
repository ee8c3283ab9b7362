// Causal GQA prefill on f16 MFMA (gfx950), f16 K/V cache, head_dim 256.
//
// Reference semantics: attn_fa2_prefill_kernel / fa2_prefill_launch
// (include/rdna4/attn_fa2.cuh:30-187) and the batched path of
// graph.cuh:1473-1535: query token i at position p_i attends cache keys
// 0..min(p_i, kmax) of kv head h / (n_head / n_head_kv); softmax(q.k * scale)
// weighted sum of V, f32 accumulation; then out *= sigmoid(gate) when a gate
// is given (gate <- sigmoid(gate)).
//
// Work decomposition: the (query, head) pairs of one kv head form rows
// r = query * group + head_in_group, so every head of a GQA group shares the K/V
// tiles. CTA = 4 waves = 128 consecutive rows of one kv head; each wave owns 32
// rows (two 16-row MFMA slabs). The CTA walks 64-key blocks:
//   * K block (64 x 256 f16) arrives by global->LDS DMA, row-major with the
//     16-byte chunks of row r XOR-swizzled by r & 15 (conflict-free reads);
//   * V block is loaded into registers and written to LDS transposed
//     ([dim][key]) so the PV operand is key-contiguous;
//   both are double-buffered: block j+1 is in flight while block j computes.
//   * S^T = K Q^T on v_mfma_f32_16x16x32_f16 (A = 16 keys x 32 dims of K from
//     LDS, reused by both slabs; B = the wave's query rows in registers);
//   * online softmax in registers (exp2 domain, lazy O rescale); the C layout
//     of S^T is the B operand of O^T += V^T P^T, so p never leaves registers;
//   * causal masking is applied only in blocks that cross a row's limit.
// Row blocks are scheduled heaviest (latest queries) first.
#include <cstdlib>

#include "prefill.hpp"

namespace rd4 {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kHD = 256;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsW = 32;                 // rows per wave (2 slabs of 16)
constexpr int kBM = kWaves * kRowsW;       // rows per CTA
constexpr int kBN = 64;                    // keys per block
constexpr int kKBytes = kBN * kHD * 2;     // K block, 32 KiB
constexpr int kVTStride = (kBN + 8) * 2;   // V^T row (one dim) stride in bytes
constexpr int kVTBytes = kHD * kVTStride;  // 36 KiB
constexpr int kStage = kKBytes + kVTBytes;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ _Float16 h16(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

}  // namespace

__global__ __launch_bounds__(kThreads, 1) void prefill_mfma_kernel(PrefillArgs p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int grp = p.n_head / p.n_head_kv;
  const int n_rows = p.n_q * grp;
  const int n_rb = (n_rows + kBM - 1) / kBM;
  const int rb = n_rb - 1 - (int)blockIdx.x;  // heaviest first
  const int kvh = blockIdx.y;
  const int r0 = rb * kBM;

  // Causal limit of a row: last key it may attend.
  auto limit_of = [&](int row) -> int {
    if (row >= n_rows) return -1;
    const int q = row / grp;
    const int lp = p.pos ? p.pos[q] : p.pos0 + q;
    return min(lp, p.kmax);
  };
  // Key range of the CTA: 0 .. max limit over its rows.
  __shared__ int s_kend;
  if (tid == 0) s_kend = -1;
  __syncthreads();
  {
    int lim = -1;
    for (int r = tid; r < kBM; r += kThreads) lim = max(lim, limit_of(r0 + r));
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) lim = max(lim, __shfl_xor(lim, m, 64));
    if (lane == 0) atomicMax(&s_kend, lim);
  }
  __syncthreads();
  const int kend = s_kend;  // inclusive
  const int n_blocks = (kend + kBN) / kBN;

  const int64_t kvstride = (int64_t)p.n_head_kv * kHD * 2;  // bytes between consecutive keys
  const uint8_t *kbase = p.k + (int64_t)kvh * kHD * 2;
  const uint8_t *vbase = p.v + (int64_t)kvh * kHD * 2;

  // ---- this wave's query rows: B operand of S^T (row n of slab s is row
  // r0 + 32w + 16s + n), f16 (f32 queries are rounded to f16)
  half8 qf[2][8];
  int lim_row[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const int row = r0 + kRowsW * w + 16 * sl + n;
    lim_row[sl] = limit_of(row);
    const bool on = row < n_rows;
    const int q = on ? row / grp : 0;
    const int head = kvh * grp + (on ? row % grp : 0);
    const int64_t qoff = ((int64_t)q * p.n_head + head) * kHD + 8 * g;
    if (p.q_f16) {
      u32x4 r[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) r[b] = *(const u32x4 *)((const uint16_t *)p.q + qoff + 32 * b);
#pragma unroll
      for (int b = 0; b < 8; ++b) qf[sl][b] = on ? __builtin_bit_cast(half8, r[b]) : half8{};
    } else {
      float4 r[16];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        r[2 * b] = *(const float4 *)((const float *)p.q + qoff + 32 * b);
        r[2 * b + 1] = *(const float4 *)((const float *)p.q + qoff + 32 * b + 4);
      }
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const float v[8] = {r[2 * b].x, r[2 * b].y, r[2 * b].z, r[2 * b].w,
                            r[2 * b + 1].x, r[2 * b + 1].y, r[2 * b + 1].z, r[2 * b + 1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[sl][b][i] = on ? (_Float16)v[i] : (_Float16)0.0f;
      }
    }
  }
  const float sl2 = p.scale * kLog2e;
  // The wave's smallest row limit: blocks whose last key is <= it need no mask.
  int wave_min_lim = min(lim_row[0], lim_row[1]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) wave_min_lim = min(wave_min_lim, __shfl_xor(wave_min_lim, m, 64));

  floatx4 o[2][16];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[sl][i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  // ---- block loads. K: 2048 chunks of 16 B per block = 8 DMA instructions per
  // lane; chunk c -> key c/32, LDS slot c%32 holds global column slot^(key&15).
  auto issue_k = [&](int blk, int stage) {
    uint8_t *kd = smem + stage * kStage;
    const int j0 = blk * kBN;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = (w * 8 + r) * 64 + lane;
      const int key = c >> 5, slot = c & 31;
      const int col = slot ^ (key & 15);
      const int jk = min(j0 + key, kend);  // rows past the range re-read a valid row (masked later)
      __builtin_amdgcn_global_load_lds((const void *)(kbase + (int64_t)jk * kvstride + 16 * col),
                                       (lds_void *)(kd + (w * 8 + r) * 1024), 16, 0, 0);
    }
  };
  // V: thread = 4 consecutive keys x 8 dims, two such groups per block.
  u32x4 vr[2][4];
  auto load_v = [&](int blk) {
    const int j0 = blk * kBN;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int u = tid + kThreads * gi;      // 0..511
      const int kq = u >> 5, c = u & 31;      // key quad 0..15, dim chunk 0..31
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int jk = min(j0 + 4 * kq + i, kend);
        vr[gi][i] = *(const u32x4 *)(vbase + (int64_t)jk * kvstride + 16 * c);
      }
    }
  };
  auto store_vt = [&](int stage) {
    uint8_t *vt = smem + stage * kStage + kKBytes;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int u = tid + kThreads * gi;
      const int kq = u >> 5, c = u & 31;
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // dim 8c + j: keys 4kq..4kq+3
        const int wsel = j >> 1, hsel = j & 1;
        const uint32_t a0 = vr[gi][0][wsel], a1 = vr[gi][1][wsel];
        const uint32_t a2 = vr[gi][2][wsel], a3 = vr[gi][3][wsel];
        const uint32_t sel = hsel ? 0x07060302u : 0x05040100u;  // high or low halves
        const uint32_t lo = __builtin_amdgcn_perm(a1, a0, sel);
        const uint32_t hi = __builtin_amdgcn_perm(a3, a2, sel);
        *(u32x2 *)(vt + (8 * c + j) * kVTStride + 8 * kq) = u32x2{lo, hi};
      }
    }
  };

  if (n_blocks > 0) {
    issue_k(0, 0);
    load_v(0);
    store_vt(0);
  }
  for (int blk = 0; blk < n_blocks; ++blk) {
    const int st = blk & 1;
    const bool more = blk + 1 < n_blocks;
    if (more) {
      issue_k(blk + 1, st ^ 1);
      load_v(blk + 1);
      __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory");  // block blk's K DMA is done
    } else {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();  // K and V^T of block blk visible to all waves

    const uint8_t *kd = smem + st * kStage;
    const uint8_t *vt = kd + kKBytes;
    const int j0 = blk * kBN;
    const bool need_mask = (j0 + kBN - 1) > wave_min_lim;

    {
      // ---- S^T for 4 key tiles x 2 slabs
      floatx4 s[2][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        s[0][kt] = floatx4{0.f, 0.f, 0.f, 0.f};
        s[1][kt] = floatx4{0.f, 0.f, 0.f, 0.f};
        const int key = 16 * kt + n;
        const uint8_t *krow = kd + key * (kHD * 2);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const half8 kf = __builtin_bit_cast(half8, *(const u32x4 *)(krow + 16 * ((4 * b + g) ^ (key & 15))));
          s[0][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[0][b], s[0][kt], 0, 0, 0);
          s[1][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[1][b], s[1][kt], 0, 0, 0);
        }
      }
      // ---- online softmax per slab: lane = row n, keys 16kt + 4g + i
      half8 pf[2][2];
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        float tmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = s[sl][kt][i] * sl2;
            if (need_mask && j0 + 16 * kt + 4 * g + i > lim_row[sl]) v = -INFINITY;
            s[sl][kt][i] = v;
            tmax = fmaxf(tmax, v);
          }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run[sl], tmax);
        // rows with no key yet keep m = -inf; exp2(-inf - -inf) must not be used
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(s[sl][kt][i] - m_use);
            s[sl][kt][i] = e;
            psum += e;
          }
        if (__any(m_new != m_run[sl])) {
          const float corr = (m_run[sl] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run[sl] - m_use);
          l_run[sl] *= corr;
#pragma unroll
          for (int i = 0; i < 16; ++i) o[sl][i] *= corr;
        }
        m_run[sl] = m_new;
        l_run[sl] += psum;
        // B operand of PV: k-slot 8h + i <-> key 32*kg + 16*(i>>2) + 4h + (i&3)
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
          for (int i = 0; i < 8; ++i) pf[sl][kg][i] = (_Float16)s[sl][2 * kg + (i >> 2)][i & 3];
      }
      // ---- O^T += V^T P^T: A = 16 dims x 32 keys of V^T (shared by both slabs)
#pragma unroll
      for (int kg = 0; kg < 2; ++kg) {
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
          const uint8_t *vrow = vt + (16 * dt + n) * kVTStride + 2 * (32 * kg + 4 * g);
          const u32x2 lo = *(const u32x2 *)vrow;         // keys 32kg + 4g .. +3
          const u32x2 hi = *(const u32x2 *)(vrow + 32);  // keys 32kg + 16 + 4g .. +3
          const half8 vf = __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[0][kg], o[0][dt], 0, 0, 0);
          o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[1][kg], o[1][dt], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // all waves are done with stage st
    if (more) store_vt(st ^ 1);
  }

  // ---- epilogue: l over the 4 key groups, normalize, gate, store
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    float L = l_run[sl];
    L += __shfl_xor(L, 16, 64);
    L += __shfl_xor(L, 32, 64);
    const int row = r0 + kRowsW * w + 16 * sl + n;
    if (row >= n_rows) continue;
    const int q = row / grp, head = kvh * grp + row % grp;
    const float inv = (m_run[sl] == -INFINITY || !(L > 0.0f)) ? 0.0f : 1.0f / L;
    const int64_t ob = ((int64_t)q * p.n_head + head) * kHD;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const int d = 16 * dt + 4 * g;
      float v[4] = {o[sl][dt][0] * inv, o[sl][dt][1] * inv, o[sl][dt][2] * inv, o[sl][dt][3] * inv};
      if (p.gate) {
        float4 gv = *(const float4 *)(p.gate + ob + d);
        float gs[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          gs[i] = 1.0f / (1.0f + expf(-gs[i]));
          v[i] *= gs[i];
        }
        *(float4 *)(p.gate + ob + d) = make_float4(gs[0], gs[1], gs[2], gs[3]);
      }
      *(float4 *)(p.out + ob + d) = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

bool prefill_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  const char *e = std::getenv("RD4_PREFILL_GENERIC");
  if (e && std::atoi(e) != 0) return false;
  return kt == F16 && vt == F16 && head_dim == kHD && n_head_kv > 0 && n_head % n_head_kv == 0;
}

hipError_t prefill_mfma_launch(const PrefillArgs &p, hipStream_t st) {
  const int grp = p.n_head / p.n_head_kv;
  const int n_rb = (p.n_q * grp + kBM - 1) / kBM;
  dim3 grid((unsigned)n_rb, (unsigned)p.n_head_kv);
  hipLaunchKernelGGL(prefill_mfma_kernel, grid, dim3(kThreads), (size_t)(2 * kStage), st, p);
  return hipGetLastError();
}

}  // namespace rd4
