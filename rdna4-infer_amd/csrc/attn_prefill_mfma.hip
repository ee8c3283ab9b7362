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
// tiles. Default CTA = 12 waves = 192 consecutive rows of one kv head; each wave
// owns 16 rows (one MFMA slab), three waves per SIMD so one wave's softmax and
// LDS waits overlap the others' MFMAs. The CTA walks 64-key blocks:
//   * K block (64 x 256 f16) arrives by global->LDS DMA (scalar base + 32-bit
//     lane offsets), row-major with the 16-byte chunks of key r permuted by
//     swz(r) (conflict-free for both read patterns below);
//   * V block arrives the same way, same swizzle; the PV operand (16 dims x
//     8 keys per lane group) is read straight out of it with the gfx950
//     transposing LDS load (ds_read_b64_tr_b16), so no transpose pass;
//   three K stages and two V stages: K two blocks ahead, V one, one CTA
//   barrier per block;
//   * S^T = K Q^T on v_mfma_f32_16x16x32_f16 (A = 16 keys x 32 dims of K from
//     LDS, B = the wave's query rows in registers), O^T += V^T P^T likewise;
//     in both phases a ring of operand fragments keeps several steps of LDS
//     reads in flight ahead of their MFMAs, and scheduling fences hold the
//     compiler to that order;
//   * online softmax in registers (exp2 domain, lazy O rescale); the C layout
//     of S^T is the B operand of O^T += V^T P^T, so p never leaves registers;
//   * causal masking only in blocks that cross a row's limit (a wave-uniform
//     branch).
// Row blocks are scheduled heaviest (latest queries) first.
#include <algorithm>
#include <cstdlib>

#include "kv_quant.hpp"
#include "prefill.hpp"

namespace rd4 {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
// 16-byte LDS reads through an explicit address-space-3 pointer. (The
// compiler waits for these with lgkmcnt(0), all outstanding LDS reads; exact
// waits through asm measured no faster here.)
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;

constexpr int kHD = 256;
constexpr int kBN = 64;                    // keys per block
constexpr int kKBytes = kBN * kHD * 2;     // K block, 32 KiB
// LDS: three K stages then two V stages (the whole 160 KiB): K streams two
// blocks ahead, V one
constexpr int kKStages = 3, kVStages = 2;
constexpr int kLdsBytes = (kKStages + kVStages) * kKBytes;
constexpr float kLog2e = 1.4426950408889634f;
// profiling knob bits of prefill_mfma_kernel (0 in production builds): 1 no K
// fragment reads, 2 no V fragment reads, 4 no softmax, 8 no DMA after the
// first blocks, 16 no block barrier, 32 no MFMA, 64 no key blocks at all
#ifndef RD4_PF_KNOB
#define RD4_PF_KNOB 0
#endif
// operand ring depth of the PV phase (steps of two MFMAs whose V^T operands
// are in registers or in flight)
#ifndef RD4_PF_PVD
#define RD4_PF_PVD 3
#endif
constexpr int kPVD0 = RD4_PF_PVD;
// QK^T operand ring: kQD steps of kQG K fragments
#ifndef RD4_PF_QKG
#define RD4_PF_QKG 2
#endif
#ifndef RD4_PF_QKD
#define RD4_PF_QKD 4
#endif
constexpr int kQG = RD4_PF_QKG, kQD0 = RD4_PF_QKD;
// the same at three waves per SIMD (12 waves per CTA)
#ifndef RD4_PF_QKD_W12
#define RD4_PF_QKD_W12 3
#endif
#ifndef RD4_PF_PVD_W12
#define RD4_PF_PVD_W12 3
#endif
// a scheduling fence after each PV step (2), so the operand reads stay as far
// ahead of their MFMAs as written (the QK^T reads are always fenced)
#ifndef RD4_PF_SB
#define RD4_PF_SB 2
#endif
// the first PV operand reads go out before the softmax (1) or after it (0)
#ifndef RD4_PF_VEARLY
#define RD4_PF_VEARLY 0
#endif
// causal mask under a wave-uniform branch (1) or applied to every block (0)
#ifndef RD4_PF_MASKBR
#define RD4_PF_MASKBR 1
#endif
// where K(j + 2) is requested (0 at the top of block j, 1 after its QK^T phase,
// 3 with V(j + 1) after it too)
// K/V DMA by inline asm (1) or by the builtin (0)
#ifndef RD4_PF_DMAASM
#define RD4_PF_DMAASM 1
#endif
#ifndef RD4_PF_DMAPOS
#define RD4_PF_DMAPOS 1
#endif
// block max by max3 asm (1) or by fmaxf (0)
#ifndef RD4_PF_SM
#define RD4_PF_SM 1
#endif
#ifndef RD4_PF_PROBE
#define RD4_PF_PROBE 0
#endif

__device__ __forceinline__ _Float16 h16(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// Max of x over lanes l, l ^ 16, l ^ 32, l ^ 48 by the gfx950 row and half-wave
// swaps (no LDS round trip): with x in both operands the two registers come out
// holding x and its partner. Asm with tied operands (the builtins mishandle equal
// operands); s_nop 1 covers the VALU-write -> swap-read hazard.
__device__ __forceinline__ float max_groups4(float x) {
  float a = x, b = x;
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  float c = fmaxf(a, b), d = c;
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return fmaxf(c, d);
}

// LDS swizzle of a K/V row: 16-byte chunk c of key r sits in slot c ^ swz(r).
// swz is the GF(2)-linear map with r's bits 0..3 -> 8, 7, 2, 4 (a permutation
// of 0..15). Plain r & 15 leaves the transposing PV reads with 2-way bank
// conflicts (each half wave's 8 keys x 2 chunks fall in 8 slots); this map,
// found by timing all 20,160 linear maps on gfx950 with this kernel's two read
// patterns, serves those reads at 1.8x the rate and the QK^T b128 reads at the
// rate of the plain swizzle. 0 selects the plain one.
#ifndef RD4_PF_SWZ
#define RD4_PF_SWZ 1
#endif
__device__ __forceinline__ int swz(int r) {
  if (!RD4_PF_SWZ) return r & 15;
  return ((r & 1) ? 8 : 0) ^ ((r & 2) ? 7 : 0) ^ ((r & 4) ? 2 : 0) ^ ((r & 8) ? 4 : 0);
}

// max3 and the group max without the compiler's canonicalizing maxes (the
// operands are finite or -inf, never NaN)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_groups4_raw(float x) {
  float a = x, b = x;
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  float c;
  __asm__("v_max_f32 %0, %1, %2" : "=v"(c) : "v"(a), "v"(b));
  float d = c;
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  float r;
  __asm__("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(c), "v"(d));
  return r;
}

// K/V block DMA through asm: the builtin makes the compiler put a vmcnt(0) in
// front of later LDS reads it cannot tell from the DMA's destination (the
// transposing V reads), i.e. wait for the next blocks' DMA; the kernel waits
// for its DMA explicitly (s_waitcnt vmcnt at the top of each block). 16 bytes
// per lane from saddr + voffset into LDS at M0 + 16 * lane.
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds) {
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(voff), "s"(sbase), "s"(lds)
                   : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p);
}

}  // namespace

#ifndef RD4_PF_TRACE
#define RD4_PF_TRACE 0
#endif
#if RD4_PF_TRACE
// timestamps (100 MHz realtime counter) of lane 0 of each wave of the first 64
// CTAs (diagnostic builds only): [cta][wave][point]; point 0 the start, then 5
// per block for the first 12 blocks (barrier passed, S^T MFMAs issued, softmax
// start, PV start, PV issued)
__device__ unsigned long long rd4_pf_trace[64 * 16 * 64];
extern "C" int rd4_pf_trace_read(void *host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(rd4_pf_trace), sizeof(rd4_pf_trace));
}
#define RD4_PFTP(pt)                                                                          \
  do {                                                                                        \
    if (lane == 0 && blockIdx.x < 64 && (pt) < 64)                                            \
      rd4_pf_trace[(blockIdx.x * 16 + w) * 64 + (pt)] = __builtin_amdgcn_s_memrealtime();     \
  } while (0)
#else
#define RD4_PFTP(pt) \
  do {               \
  } while (0)
#endif

// W waves of NSL 16-row slabs each (W * 16 * NSL rows per CTA).
template <int W, int NSL>
__global__ __launch_bounds__(64 * W, 1) void prefill_mfma_kernel(PrefillArgs p) {
  constexpr int kRowsWT = 16 * NSL;         // rows per wave
  // a K (or V) block is 32 wave-chunks of 64 x 16 bytes; wave w takes chunks
  // w*ND .. w*ND+ND-1 below 32 (nk of them)
  constexpr int ND = (32 + W - 1) / W;
  constexpr bool kEven = 32 % W == 0;
  constexpr int kBM = W * kRowsWT;          // rows per CTA
  // ring depths in steps: with two slabs every step feeds twice the MFMAs
  // (and with three waves per SIMD the registers allow shorter rings only)
  constexpr int kQD = NSL > 1 ? 2 : W > 8 ? RD4_PF_QKD_W12 : kQD0;
  constexpr int kPVD = NSL > 1 ? 2 : W > 8 ? RD4_PF_PVD_W12 : kPVD0;
  extern __shared__ __align__(16) uint8_t smem[];
  // the wave index is uniform: readfirstlane keeps DMA bases and LDS
  // destinations in scalar registers
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int grp = p.n_head / p.n_head_kv;
  RD4_PFTP(0);
  const int n_rows = p.n_q * grp;
  const int n_rb = (n_rows + kBM - 1) / kBM;
  // XCD-aware order: workgroup L runs on XCD L % 8. When the kv heads divide
  // the 8 XCDs, each kv head gets 8 / n_head_kv XCDs that take its row blocks
  // in turn (heaviest first), so an XCD's L2 serves one kv head whose CTAs
  // sweep the same keys at about the same time.
  const int total = n_rb * p.n_head_kv;
  // key split of this CTA: the splits' grids follow one another, so workgroup
  // L of a split still runs on XCD L % 8 (total is a multiple of 8 there)
  const int ksp = p.n_ksplit > 1 ? (int)blockIdx.x / total : 0;
  const int L = p.n_ksplit > 1 ? (int)blockIdx.x - ksp * total : (int)blockIdx.x;
  int kvh, rbp;
  if (8 % p.n_head_kv == 0 && total % 8 == 0) {
    const int X = 8 / p.n_head_kv, xcd = L % 8, j = L / 8;
    kvh = xcd % p.n_head_kv;
    rbp = j * X + xcd / p.n_head_kv;
  } else {
    kvh = L / n_rb;
    rbp = L - kvh * n_rb;
  }
  const int rb = n_rb - 1 - rbp;
  const int r0 = rb * kBM;

  // Fused append: the chunk's new K and V rows (2 * n_q * n_head_kv of them) are
  // spread over the CTAs, one wave per row, 8 lanes per 32-value block, with the
  // quantizer of kv_store_row_launch; the attention below reads other rows.
  if (p.app_k && ksp == 0) {  // (the first split's CTAs)
    const int nrow = p.n_q * p.n_head_kv, total_rows = 2 * nrow;
    const int rb_bytes = (int)row_bytes(p.app_type, kHD);
    for (int R = L * W + w; R < total_rows; R += total * W) {
      const bool isv = R >= nrow;
      const int rr = isv ? R - nrow : R;
      const float4 x4 = *(const float4 *)((isv ? p.app_v_src : p.app_k_src) + (int64_t)rr * kHD + 4 * lane);
      const float x[4] = {x4.x, x4.y, x4.z, x4.w};
      uint8_t *row = (isv ? p.app_v : p.app_k) + (int64_t)rr * rb_bytes;
      switch (p.app_type) {
        case F32: store_group4<F32>(x, lane & 7, row, lane >> 3); break;
        case F16: store_group4<F16>(x, lane & 7, row, lane >> 3); break;
        case Q8_0: store_group4<Q8_0>(x, lane & 7, row, lane >> 3); break;
        case Q4_0: store_group4<Q4_0>(x, lane & 7, row, lane >> 3); break;
        case Q5_0: store_group4<Q5_0>(x, lane & 7, row, lane >> 3); break;
        default: store_group4<Q4_1>(x, lane & 7, row, lane >> 3); break;
      }
    }
  }

  // Causal limit of a row: last key it may attend.
  auto limit_of = [&](int row) -> int {
    if (row >= n_rows) return -1;
    const int q = row / grp;
    const int lp = p.pos ? p.pos[q] : p.pos0 + q;
    return min(lp, p.kmax);
  };
  // Key range of the CTA: 0 .. max limit over its rows, reduced by every wave
  // over all of the CTA's rows (no LDS: the K/V stages take all of it).
  int kend;  // inclusive
  {
    int lim = -1;
    for (int r = lane; r < kBM; r += 64) lim = max(lim, limit_of(r0 + r));
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) lim = max(lim, __shfl_xor(lim, m, 64));
    kend = __builtin_amdgcn_readfirstlane(lim);
  }
  const int n_blocks = (RD4_PF_KNOB & 64) ? 0 : (kend + kBN) / kBN;
  // this CTA's blocks b0 .. b0 + nbk - 1 (all of them when the keys are not split)
  const int b0 = p.n_ksplit > 1 ? ksp * p.ksplit_blocks : 0;
  const int nbk = p.n_ksplit > 1 ? max(0, min(n_blocks, b0 + p.ksplit_blocks) - b0) : n_blocks;

  const int64_t kvstride = (int64_t)p.n_head_kv * kHD * 2;  // bytes between consecutive keys
  const uint8_t *kbase = p.k + (int64_t)kvh * kHD * 2;
  const uint8_t *vbase = p.v + (int64_t)kvh * kHD * 2;

  // ---- this wave's query rows: B operand of S^T (row n of slab s is row
  // r0 + 32w + 16s + n), f16 (f32 queries are rounded to f16)
  // q is pre-scaled by scale*log2(e) so S comes out in the exp2 domain
  const float sl2 = p.scale * kLog2e;
  half8 qf[NSL][8];
  int lim_row[NSL];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const int row = r0 + kRowsWT * w + 16 * sl + n;
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
      for (int b = 0; b < 8; ++b) {
        const half8 h = __builtin_bit_cast(half8, r[b]);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[sl][b][i] = on ? (_Float16)((float)h[i] * sl2) : (_Float16)0.0f;
      }
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
        for (int i = 0; i < 8; ++i) qf[sl][b][i] = on ? (_Float16)(v[i] * sl2) : (_Float16)0.0f;
      }
    }
  }
  // The wave's smallest row limit: blocks whose last key is <= it need no mask.
  int wave_min_lim = lim_row[0];
#pragma unroll
  for (int sl = 1; sl < NSL; ++sl) wave_min_lim = min(wave_min_lim, lim_row[sl]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) wave_min_lim = min(wave_min_lim, __shfl_xor(wave_min_lim, m, 64));

  floatx4 o[NSL][16];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[sl][i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[NSL], l_run[NSL];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    m_run[sl] = -INFINITY;
    l_run[sl] = 0.0f;
  }

  // ---- block loads. K: 2048 chunks of 16 B per block = 8 DMA instructions per
  // lane; chunk c -> key c/32, LDS slot c%32 holds global column slot^(key&15).
  // Per-lane offsets are block-invariant and computed once.
  uint32_t k_goff[ND];  // byte offset of this lane's chunk r from the block's first key (scalar base + 32-bit vector offset)
#pragma unroll
  for (int r = 0; r < ND; ++r) {
    const int c = min(w * ND + r, 31) * 64 + lane;
    const int key = c >> 5, slot = c & 31;
    k_goff[r] = (uint32_t)(key * (int)kvstride + 16 * (slot ^ swz(key)));
  }
  // The block's first key as a uniform (scalar) address and each lane's chunk
  // as a 32-bit offset from it: the DMA then takes the saddr + voffset form and
  // the loop keeps no 64-bit per-lane pointers.
  auto uniform_ptr = [](const uint8_t *ptr) {
    const uint64_t a = (uint64_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (const uint8_t *)(((uint64_t)hi << 32) | lo);
  };
  auto issue_kv = [&](const uint8_t *base, uint8_t *dst, int blk) {
    const int j0 = blk * kBN;
    const uint8_t *src = uniform_ptr(base + (int64_t)j0 * kvstride);
    if (j0 + kBN - 1 <= kend) {
#pragma unroll
      for (int r = 0; r < ND; ++r) {
        if (!kEven && w * ND + r >= 32) break;
        uint32_t off = k_goff[r];
        __asm__("" : "+v"(off));  // keeps the offset 32-bit (no hoisted 64-bit copy)
        if (RD4_PF_DMAASM) dma16(src, off, lds_addr(dst + (w * ND + r) * 1024));
        else __builtin_amdgcn_global_load_lds((const void *)(src + off), (lds_void *)(dst + (w * ND + r) * 1024), 16, 0, 0);
      }
    } else {  // last block: keys past kend re-read a valid row (masked later)
#pragma unroll
      for (int r = 0; r < ND; ++r) {
        if (!kEven && w * ND + r >= 32) break;
        const int c = (w * ND + r) * 64 + lane;
        const int key = c >> 5, slot = c & 31;
        const int jk = min(key, kend - j0);
        const uint32_t off = (uint32_t)(jk * (int)kvstride + 16 * (slot ^ swz(key)));
        if (RD4_PF_DMAASM) dma16(src, off, lds_addr(dst + (w * ND + r) * 1024));
        else __builtin_amdgcn_global_load_lds((const void *)(src + off), (lds_void *)(dst + (w * ND + r) * 1024), 16, 0, 0);
      }
    }
  };
  auto issue_k = [&](int blk, int stage) { issue_kv(kbase, smem + stage * kKBytes, blk); };
  // V: same DMA and swizzle as K, into its own stages.
  auto issue_v = [&](int blk, int stage) { issue_kv(vbase, smem + (kKStages + stage) * kKBytes, blk); };
  // PV operand by transposing load: in each 16-lane group, source lane s points
  // at key (base + s/4), dims 4(s%4)..+3 of a 16-dim tile; lane r then receives
  // dim r of those 4 keys. Key bits 0-3 select the swizzle (base is a multiple
  // of 16 apart from the lane group's 4g), so the per-lane part is fixed.
  const int tr_kx = 4 * g + (n >> 2);                       // key & 15 of this source lane
  const int tr_off = tr_kx * (kHD * 2) + 8 * (n & 1);        // row and 8-byte half
  const int tr_m = 16 * ((n >> 1 & 1) ^ swz(tr_kx));        // swizzle term of the chunk
  // lane offset of dim tile dt for dt = 0..7; tr_m < 256, so tile dt + 8 is
  // the same offset + 256 (an instruction immediate)
  int v_loff[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) v_loff[dt] = tr_off + ((32 * dt) ^ tr_m);
  // LDS read offsets of the MFMA operands (block-invariant).
  // K: key 16kt + n, dims 32b + 8g: slot (4b + g) ^ n = 4(b ^ (n>>2)) + (g ^ (n&3)).
  int k_loff[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) k_loff[b] = n * (kHD * 2) + 16 * ((4 * b + g) ^ swz(n));

  // Issue order: K0 V0 K1, then in block j: V(j+1) at the top, K(j+2) after
  // the QK^T phase.
  if (nbk > 0) {
    issue_k(b0, 0);
    issue_v(b0, 0);
  }
  if (nbk > 1) issue_k(b0 + 1, 1);
  int ks = 0;  // K stage of the current block (blk % 3)
#if RD4_PF_PROBE
  float pr_a = 0.f, pr_b = 1.f;
  floatx4 pr_c = {0.f, 0.f, 0.f, 0.f};
  u32x4 pr_d = {0, 0, 0, 0};
#endif
  for (int bi = 0; bi < nbk; ++bi) {
    const int blk = b0 + bi;
    const int vs = bi & 1;
    // every DMA this wave issued has landed: K(j), V(j) and also K(j+1), which
    // was requested a block earlier and has landed by now (waiting for it costs
    // nothing measurable). A partial count would assume that the DMA completes
    // in order with any other vector-memory load the compiler places in the loop
    // (spill reloads), which it does not know about.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's DMA for blk landed; every wave is done with blk - 1 (a CTA
    // barrier on LDS only, in asm)
#ifndef RD4_PF_FULLBAR
    if (!(RD4_PF_KNOB & 16)) __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (bi < 12) RD4_PFTP(5 * bi + 1);
#else
    __syncthreads();
#endif
    const int ks2 = ks == 0 ? 2 : ks - 1;  // stage of K(blk + 2): (blk + 2) % 3
    // DMA issue points (RD4_PF_DMAPOS, default 1): 0 both at the block top, 1 K(blk + 2)
    // after the QK^T phase, 3 both after it
    if (!(RD4_PF_KNOB & 8)) {
      if (RD4_PF_DMAPOS != 3 && bi + 1 < nbk) issue_v(blk + 1, vs ^ 1);
      if (RD4_PF_DMAPOS == 0 && bi + 2 < nbk) issue_k(blk + 2, ks2);
    }
    const uint8_t *kd = smem + ks * kKBytes;
    const uint8_t *vd = smem + (kKStages + vs) * kKBytes;
    ks = ks == 2 ? 0 : ks + 1;
    const int j0 = blk * kBN;
    const bool need_mask = (j0 + kBN - 1) > wave_min_lim;

    // ---- S^T for 4 key tiles x the wave's slabs; the next tile's K fragments
    // are read from LDS while the current tile's MFMAs run.
    floatx4 s[NSL][4];
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[sl][kt] = floatx4{0.f, 0.f, 0.f, 0.f};
    // fragment f (key tile f / 8, 32-dim step f % 8) is read kAhead fragments
    // before its MFMA, into a ring of kAhead + 1 registers; a scheduling fence
    // after every read and MFMA keeps that order (the compiler would otherwise
    // reorder the reads and wait for all of them)
    constexpr int kAhead = (kQD - 1) * kQG, kRing = kAhead + 1;
    u32x4 kr[kRing];
    auto read_kf = [&](int f) {
      kr[f % kRing] = (RD4_PF_KNOB & 1) ? __builtin_bit_cast(u32x4, qf[0][(f + 1) & 7])
                                        : *(const lds_u32x4 *)(kd + (f >> 3) * 16 * (kHD * 2) + k_loff[f & 7]);
      __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int f = 0; f < kAhead; ++f) read_kf(f);
#pragma unroll
    for (int f = 0; f < 32; ++f) {
      if (f + kAhead < 32) read_kf(f + kAhead);
      const int kt = f >> 3;
      const half8 kf = __builtin_bit_cast(half8, kr[f % kRing]);
#pragma unroll
      for (int sl = 0; sl < NSL; ++sl)
        s[sl][kt] = (RD4_PF_KNOB & 32) ? s[sl][kt] + (float)kf[0]
                    : __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[sl][f & 7], s[sl][kt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (bi < 12) RD4_PFTP(5 * bi + 2);
    half8 vb[kPVD][2];
    // step t: key group kg = t / 8, dim tiles 2(t % 8), +1
    auto read_vb = [&](int buf, int t) {
      const int kg = t >> 3, dt0 = 2 * (t & 7);
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint8_t *a0 = vd + v_loff[(dt0 + d) & 7] + (32 * kg) * (kHD * 2) + 256 * ((dt0 + d) >> 3);
        if (RD4_PF_KNOB & 2) {
          vb[buf][d] = qf[0][(dt0 + d) & 7];
          continue;
        }
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4 *)a0);
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4 *)(a0 + 16 * (kHD * 2)));
        vb[buf][d] = __builtin_bit_cast(half8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    if (RD4_PF_VEARLY) {  // the first PV operands do not depend on the softmax
#pragma unroll
      for (int t = 0; t < kPVD - 1; ++t) read_vb(t, t);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!(RD4_PF_KNOB & 8) && RD4_PF_DMAPOS != 0) {
      if (RD4_PF_DMAPOS == 3 && bi + 1 < nbk) issue_v(blk + 1, vs ^ 1);
      if (bi + 2 < nbk) issue_k(blk + 2, ks2);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (bi < 12) RD4_PFTP(5 * bi + 3);
    // ---- online softmax per slab: lane = row n, keys 16kt + 4g + i
    half8 pf[NSL][2];
    if (RD4_PF_KNOB & 4) {
#pragma unroll
      for (int kg = 0; kg < 2; ++kg)
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[0][kg][i] = (_Float16)s[0][2 * kg + (i >> 2)][i & 3];
    } else
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      float tmax = -INFINITY;
      if (!RD4_PF_MASKBR || need_mask) {  // wave-uniform: most blocks skip the per-element compares
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if ((RD4_PF_MASKBR || need_mask) && j0 + 16 * kt + 4 * g + i > lim_row[sl]) s[sl][kt][i] = -INFINITY;
      }
      // block max as a tree (max3 in asm: the compiler's fmaxf adds a
      // canonicalizing max per operand)
      if (RD4_PF_SM & 1) {
        const float a0 = max3f(s[sl][0][0], s[sl][0][1], s[sl][0][2]);
        const float a1 = max3f(s[sl][0][3], s[sl][1][0], s[sl][1][1]);
        const float a2 = max3f(s[sl][1][2], s[sl][1][3], s[sl][2][0]);
        const float a3 = max3f(s[sl][2][1], s[sl][2][2], s[sl][2][3]);
        const float a4 = max3f(s[sl][3][0], s[sl][3][1], s[sl][3][2]);
        tmax = max3f(max3f(a0, a1, a2), a3, max3f(a4, s[sl][3][3], s[sl][3][3]));
        tmax = max_groups4_raw(tmax);
      } else {
        float m4[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          m4[kt] = fmaxf(fmaxf(s[sl][kt][0], s[sl][kt][1]), fmaxf(s[sl][kt][2], s[sl][kt][3]));
        tmax = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        tmax = max_groups4(tmax);
      }
      // The reference max only moves when the block max exceeds it by more than
      // 2^8 (p <= 256 stays exact enough in f16 and l, O are f32): most blocks
      // then skip the O rescale.
      const bool bump = tmax > m_run[sl] + 8.0f;
      if (__any(bump)) {
        const float m_new = bump ? tmax : m_run[sl];
        const float corr = (m_run[sl] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run[sl] - m_new);
        l_run[sl] *= corr;
#pragma unroll
        for (int i = 0; i < 16; ++i) o[sl][i] *= corr;
        m_run[sl] = m_new;
      }
      const float m_use = (m_run[sl] == -INFINITY) ? 0.0f : m_run[sl];
      float ps4[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[sl][kt][i] = __builtin_amdgcn_exp2f(s[sl][kt][i] - m_use);
        ps4[kt] = (s[sl][kt][0] + s[sl][kt][1]) + (s[sl][kt][2] + s[sl][kt][3]);
      }
      l_run[sl] += (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
      // B operand of PV: k-slot 8h + i <-> key 32*kg + 16*(i>>2) + 4h + (i&3)
#pragma unroll
      for (int kg = 0; kg < 2; ++kg)
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[sl][kg][i] = (_Float16)s[sl][2 * kg + (i >> 2)][i & 3];
    }
    if (bi < 12) RD4_PFTP(5 * bi + 4);
    // ---- O^T += V^T P^T: A = 16 dims x 32 keys of V (k-slot 8g + j is key
    // 32kg + 16(j/4) + 4g + j%4, as in pf), two transposing loads per operand;
    // the next two dim tiles' operands are read while the current ones run.
    if (!RD4_PF_VEARLY) {
#pragma unroll
      for (int t = 0; t < kPVD - 1; ++t) read_vb(t, t);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t + kPVD - 1 < 16) read_vb((t + kPVD - 1) % kPVD, t + kPVD - 1);
      const int kg = t >> 3;
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int dt = 2 * (t & 7) + d;
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl)
          o[sl][dt] = (RD4_PF_KNOB & 32) ? o[sl][dt] + (float)vb[t % kPVD][d][0]
                      : __builtin_amdgcn_mfma_f32_16x16x32_f16(vb[t % kPVD][d], pf[sl][kg], o[sl][dt], 0, 0, 0);
      }
      if (RD4_PF_SB & 2) __builtin_amdgcn_sched_barrier(0);
    }
    if (bi < 12) RD4_PFTP(5 * bi + 5);
#if RD4_PF_PROBE
    // sensitivity probes (diagnostic builds only): extra independent work per block
    if (RD4_PF_PROBE & 1)
      __asm__ volatile(".rept 16\n\tv_add_f32 %0, %0, %2\n\tv_add_f32 %1, %1, %2\n\t.endr" : "+v"(pr_a), "+v"(pr_b) : "v"(sl2));
    if (RD4_PF_PROBE & 2)
      __asm__ volatile(".rept 16\n\tv_mfma_f32_16x16x32_f16 %0, %1, %2, %0\n\t.endr\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(pr_c) : "v"(qf[0][0]), "v"(qf[0][1]));
    if (RD4_PF_PROBE & 4)
      __asm__ volatile(".rept 16\n\tds_read_b128 %0, %1\n\t.endr\n\ts_waitcnt lgkmcnt(0)" : "=v"(pr_d) : "v"((uint32_t)(uintptr_t)smem + k_loff[0]));
#endif
  }
#if RD4_PF_PROBE
  if (p.scale == 12345.0f) p.out[tid] = pr_a + pr_b + pr_c[0] + (float)pr_d[0];
#endif

  // ---- epilogue: l over the 4 key groups, normalize, gate, store (or, for a
  // key split, the unnormalized record)
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    float L = l_run[sl];
    L += __shfl_xor(L, 16, 64);
    L += __shfl_xor(L, 32, 64);
    const int row = r0 + kRowsWT * w + 16 * sl + n;
    if (row >= n_rows) continue;
    const int q = row / grp, head = kvh * grp + row % grp;
    if (p.n_ksplit > 1) {
      const int64_t nr = (int64_t)p.n_q * p.n_head, rr = (int64_t)ksp * nr + (int64_t)q * p.n_head + head;
      float *rec = p.part + rr * kHD;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        *(floatx4 *)(rec + 16 * dt + 4 * g) = o[sl][dt];
      if (g == 0) *(float2 *)(p.part + (int64_t)p.n_ksplit * nr * kHD + 2 * rr) = make_float2(m_run[sl], L);
      continue;
    }
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

// Fold of the key splits' records (the LSE merge of the split decode, exp2
// domain), then the gate and the store of the unsplit epilogue: one wave per
// (query, head) row, 4 dims per lane.
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t nr = (int64_t)p.n_q * p.n_head;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nr) return;
  const int S = p.n_ksplit;
  const float *ml = p.part + (int64_t)S * nr * kHD;
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * (s * nr + row)]);
  float L = 0.0f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const float2 r = *(const float2 *)(ml + 2 * (s * nr + row));
    if (r.x == -INFINITY) continue;  // a split with no key of this row
    const float wgt = __builtin_amdgcn_exp2f(r.x - M);
    L = fmaf(wgt, r.y, L);
    const floatx4 v = *(const floatx4 *)(p.part + (s * nr + row) * kHD + 4 * lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(wgt, v[i], acc[i]);
  }
  const float inv = (M == -INFINITY || !(L > 0.0f)) ? 0.0f : 1.0f / L;
  const int64_t ob = row * kHD + 4 * lane;
  float v[4] = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  if (p.gate) {
    float4 gv = *(const float4 *)(p.gate + ob);
    float gs[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gs[i] = 1.0f / (1.0f + expf(-gs[i]));
      v[i] *= gs[i];
    }
    *(float4 *)(p.gate + ob) = make_float4(gs[0], gs[1], gs[2], gs[3]);
  }
  *(float4 *)(p.out + ob) = make_float4(v[0], v[1], v[2], v[3]);
}

bool prefill_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  const char *e = std::getenv("RD4_PREFILL_GENERIC");
  if (e && std::atoi(e) != 0) return false;
  return kt == F16 && vt == F16 && head_dim == kHD && n_head_kv > 0 && n_head % n_head_kv == 0;
}

// Key splits the MFMA kernel wants for this call: when its row blocks leave
// CUs idle (the reference engine's 512-query chunks: 64 CTAs on 256 CUs),
// about one CTA per CU, at most 16 and at most one per key block.
// RD4_PREFILL_KSPLIT forces a count (1: never split).
int prefill_ksplits(const PrefillArgs &p) {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    return n;
  }();
  static const int env = [] {
    const char *e = std::getenv("RD4_PREFILL_KSPLIT");
    return e ? std::atoi(e) : 0;
  }();
  const int grp = p.n_head / p.n_head_kv;
  const int total = (p.n_q * grp + 191) / 192 * p.n_head_kv;  // the default 192-row CTAs
  const int max_blocks = (p.kmax + kBN) / kBN;
  int s = env > 0 ? env : (total % 8 == 0 && 2 * total <= cus) ? cus / total : 1;
  return std::max(1, std::min(s, std::min(max_blocks, 16)));
}
int64_t prefill_part_floats(const PrefillArgs &p, int splits) {
  return (int64_t)splits * p.n_q * p.n_head * (kHD + 2);
}

hipError_t prefill_mfma_launch(const PrefillArgs &p, hipStream_t st) {
  static const int shape = [] {
    const char *e = std::getenv("RD4_PREFILL_SHAPE");
    return e ? std::atoi(e) : 0;
  }();
  const int grp = p.n_head / p.n_head_kv;
  const int bm = shape == 2 ? 256 : shape == 0 ? 192 : 128;  // rows per CTA
  const int n_rb = (p.n_q * grp + bm - 1) / bm;
  const int total = n_rb * p.n_head_kv;
  // Key splits when the row blocks alone leave CUs idle (the reference
  // engine's 512-query chunks: 64 CTAs on 256 CUs): enough splits of equal
  // block counts to give about one CTA per CU, if the records fit the scratch.
  PrefillArgs q = p;
  q.n_ksplit = 1;
  q.ksplit_blocks = 0;
  const int s = prefill_ksplits(p);
  if (s > 1 && p.part && prefill_part_floats(p, s) <= p.part_floats) {
    const int max_blocks = (p.kmax + kBN) / kBN;
    q.ksplit_blocks = (max_blocks + s - 1) / s;
    q.n_ksplit = (max_blocks + q.ksplit_blocks - 1) / q.ksplit_blocks;
  }
  dim3 grid((unsigned)(total * q.n_ksplit));
  if (shape == 1)  // 4 waves x 32 rows (one wave per SIMD)
    hipLaunchKernelGGL((prefill_mfma_kernel<4, 2>), grid, dim3(256), (size_t)kLdsBytes, st, q);
  else if (shape == 2)  // 8 waves x 32 rows (two waves per SIMD)
    hipLaunchKernelGGL((prefill_mfma_kernel<8, 2>), grid, dim3(512), (size_t)kLdsBytes, st, q);
  else if (shape == 3)  // 8 waves x 16 rows (two waves per SIMD)
    hipLaunchKernelGGL((prefill_mfma_kernel<8, 1>), grid, dim3(512), (size_t)kLdsBytes, st, q);
  else  // 12 waves x 16 rows (three waves per SIMD)
    hipLaunchKernelGGL((prefill_mfma_kernel<12, 1>), grid, dim3(768), (size_t)kLdsBytes, st, q);
  if (q.n_ksplit > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t rows = (int64_t)p.n_q * p.n_head;
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, q);
  }
  return hipGetLastError();
}

}  // namespace rd4
