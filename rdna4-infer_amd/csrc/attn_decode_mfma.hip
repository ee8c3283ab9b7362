// Split-KV GQA decode on f16 MFMA (gfx950), K and V each in f16, q8_0, q4_0,
// q5_0 or q4_1 (f32 caches take the all-types kernel).
//
// Reference semantics: attn_split_kernel + attn_merge_kernel and the batched
// forms (include/rdna4/attn.cuh:445-590, 686-845) with the output gate of
// nn.cuh:405-412 and the append of graph.cuh:1011-1031 optionally fused:
// out[h] = softmax_j(q_h . k_j * scale) . V over keys 0..t, f32 accumulation.
//
// Work decomposition: CTA = 8 waves (4 for wide tiles) = one (token, kv head,
// <=8-query-head chunk, key split). Each wave walks its own 16-key tiles of the
// split (tiles w, w+8, ...: the waves stream adjacent memory) with a private
// online-softmax state, so the main loop has no CTA barrier. Per tile:
//   1. the tile's raw K and V rows (exactly the cache bytes) arrive by
//      global->LDS DMA (16 bytes per lane) into a wave-private ring, issued
//      ahead of use; the per-block scales (and q4_1 offsets) become f32 tables;
//   2. S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K
//      converted to f16 on the fly (f16 as is; the quantized types' integers,
//      exact in f16), B = the query rows. The 16 MFMA rows carry the group's
//      query heads twice, as f16 hi and lo parts (q = hi + lo to 2^-22), so the
//      f32 query costs no precision. Quantized K is scaled by its per-(key,
//      block) d after each 32-dim block's MFMA; q4_1's offset m adds
//      m * sum(q over the block), the block sums formed once per CTA;
//   3. online softmax in registers (exp2 domain); the C layout of S^T gives each
//      lane one query row x 4 keys, exactly the B operand layout PV needs; the
//      running max moves only by more than 2^8, so O is rarely rescaled;
//   4. O^T += V^T P^T on v_mfma_f32_16x16x16_f16: A = 16 dims x 16 keys of V
//      read from LDS, B = f16(p * d) in the head rows (d = the quantized V's
//      per-block scale); q4_1's offsets contribute sum_j p_j m_j per block, kept
//      in f32 registers and added to the block's dims at the end.
// The waves' states merge through LDS into one (m, l, acc) record per query
// head and split; merge_splits_kernel (merge.hip) folds the splits and applies
// the gate in a second short launch. In pair mode (PAIR) rows 0-7 and 8-15 are
// the heads of two consecutive tokens with f16 queries, so the tiles serve both.
#include <cstdlib>

#include "kv_quant.hpp"
#include "merge.hpp"
#include "prefill.hpp"

namespace rd4 {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#ifndef RD4_DEC_TRACE
#define RD4_DEC_TRACE 0
#endif
// profiling knobs (RD4_DECODE_DBG bits 2, 4, 32, 2048 skip the QK product, the PV
// product, all tiles, all loads); off in production builds, where their
// branches cost register copies in the tile loop
#ifndef RD4_DEC_QLDS
#define RD4_DEC_QLDS 1
#endif
#ifndef RD4_DEC_KNOBS
#define RD4_DEC_KNOBS 0
#endif
#ifndef RD4_DEC_ASM_WAIT
#define RD4_DEC_ASM_WAIT 0
#endif
// Cache policy of the tile DMA (the load's aux bits): 2 = non-temporal, for one
// token per CTA over f16 / q8_0 caches (q8_0 32K -1.5%, f16 32K -6%). The
// 4-bit types keep the default policy (nt there: time within noise, 13-15%
// more fabric traffic: lines shared by neighbouring rows are fetched twice), and
// so does pair mode, whose two token-pair CTAs of a split read the same tiles
// (nt there: +5%).
#ifndef RD4_DEC_AUX
#define RD4_DEC_AUX 2
#endif
// The ring's next tile is requested after the current tile's QK product
// instead of before its wait: under a chip-wide burst of requests the DMA
// instructions hold the issuing wave (0.4-1.3 us per tile in a timeline of
// every wave), and there the hold no longer delays a tile that has landed.
#ifndef RD4_DEC_LATE
#define RD4_DEC_LATE 1
#endif
constexpr int kHD = 256;     // head_dim of this kernel
constexpr int kRowPad = kHD + 4;  // LDS row stride (floats) of per-head rows: spreads banks
constexpr int kTile = 16;    // keys per wave tile
constexpr int kG = 8;        // query heads per CTA (MFMA rows 0-7 hi, 8-15 lo)
constexpr float kLog2e = 1.4426950408889634f;
// int8 query image (q8_0 K): rows [16][8 blocks][32] padded to kQiRow bytes,
// then scales [16][8] padded to kSqRow floats per row. The padding spreads the
// 16 rows read by one lane group over distinct LDS banks (unpadded, the 256-byte
// rows put all 16 on one bank pair: 5.1e5 conflict cycles per launch, 0.45 us
// of the q8_0 32K step).
constexpr int kQiRow = kHD + 16, kSqRow = 12;
constexpr int kQiBytes = 16 * kQiRow + 16 * kSqRow * 4;
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
#if RD4_DEC_ASM_WAIT
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#else
  // the builtin (not asm) lets the compiler's wait-count tracking see the wait
  static_assert(N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
#endif
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

// Tile image in LDS: the tile's K rows then V rows, contiguous 16-byte chunks
// (the last load instruction of a tile runs with its surplus lanes off).
template <int KT, int VT>
struct TileShape {
  static constexpr int KC = chunks_per_row<KT>(), VC = chunks_per_row<VT>();
  static constexpr int KCH = kTile * KC, VCH = kTile * VC;
  static constexpr int NI = (KCH + VCH + 63) / 64;  // load instructions per tile
  static constexpr int TB = (KCH + VCH) * 16;       // bytes per ring stage
  // per-wave f32 tables [block][key] of a tile, in this order: K scales, V
  // scales (quantized types), K offsets, V offsets (q4_1)
  static constexpr int NTK = (KT != F16) + (KT == Q4_1), NTV = (VT != F16) + (VT == Q4_1);
  static constexpr int DT = 512 * (NTK + NTV);
#ifndef RD4_DEC_WAVES_SMALL
#define RD4_DEC_WAVES_SMALL 8
#endif
#ifndef RD4_DEC_RMAX
#define RD4_DEC_RMAX 3
#endif
  static constexpr int WAVES = TB <= 10240 ? RD4_DEC_WAVES_SMALL : 4;
  static constexpr int QI = KT == Q8_0 ? kQiBytes : 0;  // int8 query image (q8_0 K)
  static constexpr int R0 = ((152 * 1024 - QI) / WAVES - DT) / TB;
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

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { return *(const uint32_t *)p; }

// Dim of head_dim held in k-slot j of lane group g (lanes 16g..16g+15) for the
// 32-dim block b of the S^T = K Q^T product. Any order within a block is a
// valid MFMA contraction as long as K and Q use the same one; it is chosen so
// that every lane reads its K bytes with aligned 32-bit LDS loads. q8_0 blocks
// (34 bytes) start 2 bytes past a 4-byte boundary in every other block; there
// the lane group that would straddle the row's edges takes the block's first
// two and last two values instead. q4_0 (18-byte blocks) realigns two words.
template <int KT>
__host__ __device__ constexpr int k_dim(int b, int g, int j) {
  // q4_0 / q4_1: lane group g converts the 4 quant bytes 4g..4g+3 of the block;
  // slots 0-3 are the low nibbles of bytes 0, 2, 1, 3 (elements 4g + those),
  // slots 4-7 the high nibbles (elements 16 + the same)
  if (KT == Q4_0 || KT == Q4_1) return 32 * b + 4 * g + ((j & 1) << 1) + ((j >> 1) & 1) + 16 * (j >> 2);
  // q5_0: low nibbles (g < 2) hold elements 0..15, high nibbles 16..31, read
  // with realigned words in every block
  if (KT == Q5_0) return 32 * b + 16 * (g >> 1) + 8 * (g & 1) + j;
  if (KT == F16 || (b & 1)) return 32 * b + 8 * g + j;
  // Q8_0, even blocks
  if (g < 3) return 32 * b + 8 * g + 2 + j;
  return 32 * b + (j < 4 ? 26 + j : j == 4 ? 0 : j == 5 ? 1 : j == 6 ? 30 : 31);
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Max of a non-negative float over each group of 8 lanes (8k .. 8k + 7), in
// every lane of the group: DPP quad swaps and the half-row mirror.
// Non-negative floats order like their bit patterns.
__device__ __forceinline__ float max8_nonneg(float x) {
  int v = __builtin_bit_cast(int, x);
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  return __builtin_bit_cast(float, v);
}

// (x & m) | b in one VALU instruction (the compiler splits it into two
// literal-operand ops; VOP3 on this target takes no literal, so m comes from
// an SGPR)
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t b) {
  uint32_t r;
  __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(b));
  return r;
}
// Nibbles at bits 0-3 and 16-19 of v -> two f16 of (nibble + bias), bias -8 or 0.
template <int BIAS>
__device__ __forceinline__ uint32_t nib_lo_h2(uint32_t v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c = {(_Float16)(-1024.0f + BIAS), (_Float16)(-1024.0f + BIAS)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, and_or(v, 0x000f000fu, 0x64006400u)) + c);
}
// Nibbles at bits 4-7 and 20-23 of v: the f16 1024 + 16n, times 1/16 less 64 - bias,
// is n + bias with no rounding (one packed fma).
template <int BIAS>
__device__ __forceinline__ uint32_t nib_hi_h2(uint32_t v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 sc = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 c = {(_Float16)(-64.0f + BIAS), (_Float16)(-64.0f + BIAS)};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, and_or(v, 0x00f000f0u, 0x64006400u)), sc, c));
}

// Bytes (sel-chosen pair) of v -> two f16 holding the same signed integers:
// 0x6400 | (byte ^ 0x80) is the f16 1024 + byte + 128; subtracting 1152 is exact.
__device__ __forceinline__ uint32_t i8pair_to_h2(uint32_t v, uint32_t sel) {
  const uint32_t w = __builtin_amdgcn_perm(0u, v, sel) ^ 0x64806480u;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w) + c);
}
// Low nibbles of the two bytes sel picks -> two f16 of (nibble - 8).
__device__ __forceinline__ uint32_t nibpair_to_h2(uint32_t v, uint32_t sel) {
  const uint32_t w = (__builtin_amdgcn_perm(0u, v, sel) & 0x000f000fu) | 0x64006400u;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w) + c);
}

// Low nibbles of the two bytes sel picks -> two f16 of the unsigned nibble (q4_1).
__device__ __forceinline__ uint32_t unibpair_to_h2(uint32_t v, uint32_t sel) {
  const uint32_t w = (__builtin_amdgcn_perm(0u, v, sel) & 0x000f000fu) | 0x64006400u;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w) + c);
}
// q5_0: low nibbles of the two bytes sel picks plus high bits hb0, hb1 (0/1)
// -> two f16 of (nibble | hb << 4) - 16.
__device__ __forceinline__ uint32_t q5pair_to_h2(uint32_t v, uint32_t sel, uint32_t hb0,
                                                 uint32_t hb1) {
  const uint32_t w = (__builtin_amdgcn_perm(0u, v, sel) & 0x000f000fu) | (hb0 << 4) |
                     (hb1 << 20) | 0x64006400u;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c = {(_Float16)-1040.0f, (_Float16)-1040.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w) + c);
}

// A operand of S^T = K Q^T for block b: lane (key = l%16, g = l/16) gets the
// 8 dims k_dim<KT>(b, g, 0..7) of its key as f16. sel_edge is the per-lane
// v_perm selector that gathers the edge bytes in the unaligned blocks
// (0x05040302 in the edge lane group, identity 0x07060504 elsewhere).
template <int KT>
__device__ __forceinline__ half8 k_frag(const uint8_t *krow, int b, int g, int n_of_row,
                                        uint32_t sel_edge) {
  u32x4 r;
  if constexpr (KT == F16) {
    r = *(const u32x4 *)(krow + 16 * ((4 * b + g) ^ n_of_row));
  } else if constexpr (KT == Q4_0 || KT == Q4_1) {
    // the 4 quant bytes 4g..4g+3; q4_0's are 2 bytes off a word in even blocks
    constexpr int BB = block_bytes(KT);
    uint32_t x;
    if (KT == Q4_1) x = lds_u32(krow + BB * b + 4 + 4 * g);
    else if (b & 1) x = lds_u32(krow + BB * b + 2 + 4 * g);
    else x = __builtin_amdgcn_alignbyte(lds_u32(krow + BB * b + 4 + 4 * g), lds_u32(krow + BB * b + 4 * g), 2);
    constexpr int BIAS = KT == Q4_0 ? -8 : 0;
    const uint32_t x8 = x >> 8;
    r[0] = nib_lo_h2<BIAS>(x);
    r[1] = nib_lo_h2<BIAS>(x8);
    r[2] = nib_hi_h2<BIAS>(x);
    r[3] = nib_hi_h2<BIAS>(x8);
  } else if constexpr (KT == Q5_0) {
    constexpr int BB = block_bytes(KT);
    const int gg = g & 1, sh = (g & 2) ? 4 : 0;
    uint32_t x, y;
    if (b & 1) {  // 22-byte blocks: qs at +6 is word aligned in odd blocks
      x = lds_u32(krow + BB * b + 6 + 8 * gg);
      y = lds_u32(krow + BB * b + 10 + 8 * gg);
    } else {
      const uint32_t a0 = lds_u32(krow + BB * b + 4 + 8 * gg);
      const uint32_t a1 = lds_u32(krow + BB * b + 8 + 8 * gg);
      const uint32_t a2 = lds_u32(krow + BB * b + 12 + 8 * gg);
      x = __builtin_amdgcn_alignbyte(a1, a0, 2);
      y = __builtin_amdgcn_alignbyte(a2, a1, 2);
    }
    x >>= sh;
    y >>= sh;
    {
      // the block's 32 high bits at +2; this lane's 8 elements are bits
      // 16 * (g >> 1) + 8 * gg ..
      const uint32_t qh = lds_u16(krow + BB * b + 2) | (lds_u16(krow + BB * b + 4) << 16);
      const uint32_t hb = qh >> (16 * (g >> 1) + 8 * gg);
      r[0] = q5pair_to_h2(x, 0x0c010c00u, hb & 1u, (hb >> 1) & 1u);
      r[1] = q5pair_to_h2(x, 0x0c030c02u, (hb >> 2) & 1u, (hb >> 3) & 1u);
      r[2] = q5pair_to_h2(y, 0x0c010c00u, (hb >> 4) & 1u, (hb >> 5) & 1u);
      r[3] = q5pair_to_h2(y, 0x0c030c02u, (hb >> 6) & 1u, (hb >> 7) & 1u);
    }
  } else {
    static_assert(KT == Q8_0, "q8_0 here");
    constexpr int BB = block_bytes(KT);
    uint32_t x, y;
    if (b & 1) {
      x = lds_u32(krow + BB * b + 2 + 8 * g);
      y = lds_u32(krow + BB * b + 6 + 8 * g);
    } else {
      x = lds_u32(krow + BB * b + 4 + 8 * g);
      y = __builtin_amdgcn_perm(lds_u32(krow + BB * b + 8 + 8 * g), lds_u32(krow + BB * b), sel_edge);
    }
    r[0] = i8pair_to_h2(x, 0x0c010c00u);
    r[1] = i8pair_to_h2(x, 0x0c030c02u);
    r[2] = i8pair_to_h2(y, 0x0c010c00u);
    r[3] = i8pair_to_h2(y, 0x0c030c02u);
  }
  return __builtin_bit_cast(half8, r);
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The words of one q8_0 key row that lane group g needs for the int8 product
// S^T = K Q^T, read in one asm batch that waits for its own LDS reads (through
// ordinary loads the compiler cannot tell them from the tile DMA still in
// flight and waits for that first). kw[2b], kw[2b + 1]: the two words of block
// b at k-slots 0-3 and 4-7 (even blocks: the aligned words at +4 and +8 + 8g);
// ke[b / 2]: the first word of even block b (its d and first two quants).
__device__ __forceinline__ void k_words_q8(const uint8_t *krow, int g, uint32_t (&kw)[16], uint32_t (&ke)[4]) {
  const uint32_t kb = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)(krow + 8 * g);
  const uint32_t kr = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)krow;
  // dword offsets: even b = 2m: 17m + 1, 17m + 2; odd b = 2m + 1: 17m + 9, 17m + 10
  u32x2 r[10];
  __asm__ volatile(
      "ds_read2_b32 %0, %10 offset0:1 offset1:2\n\t"
      "ds_read2_b32 %1, %10 offset0:9 offset1:10\n\t"
      "ds_read2_b32 %2, %10 offset0:18 offset1:19\n\t"
      "ds_read2_b32 %3, %10 offset0:26 offset1:27\n\t"
      "ds_read2_b32 %4, %10 offset0:35 offset1:36\n\t"
      "ds_read2_b32 %5, %10 offset0:43 offset1:44\n\t"
      "ds_read2_b32 %6, %10 offset0:52 offset1:53\n\t"
      "ds_read2_b32 %7, %10 offset0:60 offset1:61\n\t"
      "ds_read2_b32 %8, %11 offset0:0 offset1:17\n\t"
      "ds_read2_b32 %9, %11 offset0:34 offset1:51\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
        "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9])
      : "v"(kb), "v"(kr)
      : "memory");
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kw[2 * i] = r[i][0];
    kw[2 * i + 1] = r[i][1];
  }
  ke[0] = r[8][0];
  ke[1] = r[8][1];
  ke[2] = r[9][0];
  ke[3] = r[9][1];
}
// A operand of the int8 product for block b: the same 8 bytes (k-slots 0..7 of
// k_dim<Q8_0>) that k_frag converts, left as int8.
__device__ __forceinline__ long k_op_i8(const uint32_t (&kw)[16], const uint32_t (&ke)[4], int b,
                                        uint32_t sel_edge) {
  const uint32_t x = kw[2 * b];
  const uint32_t y = (b & 1) ? kw[2 * b + 1] : __builtin_amdgcn_perm(kw[2 * b + 1], ke[b >> 1], sel_edge);
  return (long)(((uint64_t)y << 32) | x);
}

// Dim of head_dim that row r' (0..15) of PV MFMA t (0..15) accumulates. The V
// operand lane with MFMA row r reads whole aligned words of its 4 keys:
//   f16:  16-byte chunk r + 16h (dims 8(r + 16h) .. +7), one MFMA per dim, t = 8h + e;
//   q8_0: the 2 bytes at dims 32b + 2r, +1 of block b, t = 2b + e;
//   q4_0, q4_1, q5_0: byte r of block b (element r low nibble, r + 16 high;
//   q5_0 adds high bits r and r + 16), t = 2b + e;
// so every MFMA's rows lie in one quantization block and share one P' operand.
template <int VT>
__host__ __device__ constexpr int v_dim(int t, int r) {
  return VT == F16 ? 8 * (r + 16 * (t >> 3)) + (t & 7)
         : VT == Q8_0 ? 32 * (t >> 1) + 2 * r + (t & 1)
                      : 32 * (t >> 1) + r + 16 * (t & 1);
}

template <int T>
__device__ __forceinline__ float scale_of(const uint8_t *row, int b) {
  return h2f((uint16_t)lds_u16(row + block_bytes(T) * b));
}
// q4_1's per-block offset m (the f16 after d)
template <int T>
__device__ __forceinline__ float offset_of(const uint8_t *row, int b) {
  return h2f((uint16_t)lds_u16(row + block_bytes(T) * b + 2));
}

// hi/lo f16 pair of an f32 (x = hi + lo to ~2^-22 relative).
__device__ __forceinline__ _Float16 hi_part(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 lo_part(float x) { return (_Float16)(x - (float)(_Float16)x); }

// P operand of the PV product for two keys: x_i = p_i * d_i split across the
// MFMA rows, f16(x) in rows n < 8 and the f16 remainder x - f16(x) in rows
// n >= 8 (lo_mask = all ones there, 0 elsewhere). The remainder is a fused
// multiply-add of the exact product, so hi + lo carries x to ~2^-22.
__device__ __forceinline__ uint32_t split_prod2(float p0, float d0, float p1, float d1,
                                                uint32_t lo_mask) {
  // v_fma_mix{lo,hi}_f16 evaluate p*d (+ an f16 operand) in one fused step and
  // write one f16 half each: two instructions per pair for hi, two for the
  // remainder, one AND to zero the subtrahend in the hi rows. The compiler's
  // hazard tracking does not see into inline asm, so the sequence pads its
  // own wait states: p may come straight from v_exp_f32 (a transcendental
  // result read by a VALU op) and the result feeds an MFMA operand (a VALU
  // write read by an MFMA); s_nop 1 covers two wait states at each end.
#if RD4_DEC_PSPLIT_C
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const float x0 = p0 * d0, x1 = p1 * d1;
  const h2 rr = {lo_mask ? lo_part(x0) : hi_part(x0), lo_mask ? lo_part(x1) : hi_part(x1)};
  return __builtin_bit_cast(uint32_t, rr);
#endif
  uint32_t hi, r;
  __asm__("s_nop 1\n\t"
          "v_fma_mixlo_f16 %0, %1, %2, 0\n\t"
          "v_fma_mixhi_f16 %0, %3, %4, 0"
          : "=&v"(hi)
          : "v"(p0), "v"(d0), "v"(p1), "v"(d1));
  const uint32_t m = hi & lo_mask;
  __asm__("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]\n\t"
          "v_fma_mixhi_f16 %0, %4, %5, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
          "s_nop 1"
          : "=&v"(r)
          : "v"(p0), "v"(d0), "v"(m), "v"(p1), "v"(d1));
  return r;
}
// The 8 per-block float4 entries p[16 b .. 16 b + 3] of a per-tile scale table,
// read with one asm block that waits for its own LDS reads. Through ordinary
// loads the compiler places a vmcnt(0) before them (it cannot rule out that the
// tile DMA still in flight writes the table), which would stall every tile on
// the next tile's prefetch.
__device__ __forceinline__ void tbl_read8(const float *p, floatx4 (&out)[8]) {
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)p;
  __asm__ volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:64\n\t"
      "ds_read_b128 %2, %8 offset:128\n\t"
      "ds_read_b128 %3, %8 offset:192\n\t"
      "ds_read_b128 %4, %8 offset:256\n\t"
      "ds_read_b128 %5, %8 offset:320\n\t"
      "ds_read_b128 %6, %8 offset:384\n\t"
      "ds_read_b128 %7, %8 offset:448\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(out[4]), "=&v"(out[5]),
        "=&v"(out[6]), "=&v"(out[7])
      : "v"(a)
      : "memory");
}
// q4_0 / q4_1 K: the quant word of each of the 8 blocks that lane group g
// converts (bytes 4g..4g+3 of the block's nibbles, as k_frag reads them) and the
// 8 query fragments from LDS, in one asm batch that waits for its own LDS reads
// (see k_words_q8). q4_0 blocks are 18 bytes: odd blocks' words are aligned,
// even blocks' straddle two words; q4_1 blocks (20 bytes) are all aligned.
template <int KT>
__device__ __forceinline__ void k_words_q4(const uint8_t *krow, int g, const uint8_t *qfl,
                                           uint32_t (&xw)[8], u32x4 (&qf)[8]) {
  const uint32_t kb = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)(krow + 4 * g);
  const uint32_t qa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)qfl;
  u32x2 r[6];
  if constexpr (KT == Q4_0) {
    // dword offsets from krow + 4g: even b: 4.5b, +1; odd b: 4.5b + 0.5
    __asm__ volatile(
        "ds_read2_b32 %0, %14 offset0:0 offset1:1\n\t"
        "ds_read2_b32 %1, %14 offset0:9 offset1:10\n\t"
        "ds_read2_b32 %2, %14 offset0:18 offset1:19\n\t"
        "ds_read2_b32 %3, %14 offset0:27 offset1:28\n\t"
        "ds_read2_b32 %4, %14 offset0:5 offset1:14\n\t"
        "ds_read2_b32 %5, %14 offset0:23 offset1:32\n\t"
        "ds_read_b128 %6, %15\n\t"
        "ds_read_b128 %7, %15 offset:1024\n\t"
        "ds_read_b128 %8, %15 offset:2048\n\t"
        "ds_read_b128 %9, %15 offset:3072\n\t"
        "ds_read_b128 %10, %15 offset:4096\n\t"
        "ds_read_b128 %11, %15 offset:5120\n\t"
        "ds_read_b128 %12, %15 offset:6144\n\t"
        "ds_read_b128 %13, %15 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(qf[0]),
          "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]), "=&v"(qf[6]), "=&v"(qf[7])
        : "v"(kb), "v"(qa)
        : "memory");
#pragma unroll
    for (int m = 0; m < 4; ++m) xw[2 * m] = __builtin_amdgcn_alignbyte(r[m][1], r[m][0], 2);
    xw[1] = r[4][0];
    xw[3] = r[4][1];
    xw[5] = r[5][0];
    xw[7] = r[5][1];
  } else {
    static_assert(KT == Q4_1, "q4_1 here");
    // dword offsets from krow + 4g: 5b + 1
    __asm__ volatile(
        "ds_read2_b32 %0, %12 offset0:1 offset1:6\n\t"
        "ds_read2_b32 %1, %12 offset0:11 offset1:16\n\t"
        "ds_read2_b32 %2, %12 offset0:21 offset1:26\n\t"
        "ds_read2_b32 %3, %12 offset0:31 offset1:36\n\t"
        "ds_read_b128 %4, %13\n\t"
        "ds_read_b128 %5, %13 offset:1024\n\t"
        "ds_read_b128 %6, %13 offset:2048\n\t"
        "ds_read_b128 %7, %13 offset:3072\n\t"
        "ds_read_b128 %8, %13 offset:4096\n\t"
        "ds_read_b128 %9, %13 offset:5120\n\t"
        "ds_read_b128 %10, %13 offset:6144\n\t"
        "ds_read_b128 %11, %13 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]),
          "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]), "=&v"(qf[6]), "=&v"(qf[7])
        : "v"(kb), "v"(qa)
        : "memory");
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      xw[2 * m] = r[m][0];
      xw[2 * m + 1] = r[m][1];
    }
  }
}
// q5_0 K: for each of the 8 blocks the two realigned quant words that lane
// group g converts (x, y as k_frag<Q5_0> reads them) and the block's 32 high
// bits, plus the 8 query fragments from LDS, in one asm batch that waits for its
// own LDS reads (see k_words_q8). Blocks are 22 bytes; a block pair spans 11
// dwords, with the even block's words 2 bytes off alignment.
__device__ __forceinline__ void k_words_q5(const uint8_t *krow, int g, const uint8_t *qfl, uint32_t (&x)[8],
                                           uint32_t (&y)[8], uint32_t (&qh)[8], u32x4 (&qf)[8]) {
  const uint32_t b1 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)(krow + 8 * (g & 1));
  const uint32_t b0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)krow;
  const uint32_t qa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)qfl;
  u32x2 r1[10], r0[6];
  __asm__ volatile(
        "ds_read2_b32 %0, %24 offset0:1 offset1:2\n\t"
        "ds_read2_b32 %1, %24 offset0:3 offset1:7\n\t"
        "ds_read2_b32 %2, %24 offset0:8 offset1:12\n\t"
        "ds_read2_b32 %3, %24 offset0:13 offset1:14\n\t"
        "ds_read2_b32 %4, %24 offset0:18 offset1:19\n\t"
        "ds_read2_b32 %5, %24 offset0:23 offset1:24\n\t"
        "ds_read2_b32 %6, %24 offset0:25 offset1:29\n\t"
        "ds_read2_b32 %7, %24 offset0:30 offset1:34\n\t"
        "ds_read2_b32 %8, %24 offset0:35 offset1:36\n\t"
        "ds_read2_b32 %9, %24 offset0:40 offset1:41\n\t"
        "ds_read2_b32 %10, %25 offset0:0 offset1:1\n\t"
        "ds_read2_b32 %11, %25 offset0:6 offset1:11\n\t"
        "ds_read2_b32 %12, %25 offset0:12 offset1:17\n\t"
        "ds_read2_b32 %13, %25 offset0:22 offset1:23\n\t"
        "ds_read2_b32 %14, %25 offset0:28 offset1:33\n\t"
        "ds_read2_b32 %15, %25 offset0:34 offset1:39\n\t"
        "ds_read_b128 %16, %26\n\t"
        "ds_read_b128 %17, %26 offset:1024\n\t"
        "ds_read_b128 %18, %26 offset:2048\n\t"
        "ds_read_b128 %19, %26 offset:3072\n\t"
        "ds_read_b128 %20, %26 offset:4096\n\t"
        "ds_read_b128 %21, %26 offset:5120\n\t"
        "ds_read_b128 %22, %26 offset:6144\n\t"
        "ds_read_b128 %23, %26 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
      : "=&v"(r1[0]), "=&v"(r1[1]), "=&v"(r1[2]), "=&v"(r1[3]), "=&v"(r1[4]), "=&v"(r1[5]), "=&v"(r1[6]), "=&v"(r1[7]), "=&v"(r1[8]), "=&v"(r1[9]), "=&v"(r0[0]), "=&v"(r0[1]), "=&v"(r0[2]), "=&v"(r0[3]), "=&v"(r0[4]), "=&v"(r0[5]), "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]), "=&v"(qf[6]), "=&v"(qf[7])
      : "v"(b1), "v"(b0), "v"(qa)
      : "memory");
    // blocks 0 (even) and 1 (odd)
    qh[0] = __builtin_amdgcn_alignbyte(r0[0][1], r0[0][0], 2);
    x[0] = __builtin_amdgcn_alignbyte(r1[0][1], r1[0][0], 2);
    y[0] = __builtin_amdgcn_alignbyte(r1[1][0], r1[0][1], 2);
    qh[1] = r0[1][0];
    x[1] = r1[1][1];
    y[1] = r1[2][0];
    // blocks 2 (even) and 3 (odd)
    qh[2] = __builtin_amdgcn_alignbyte(r0[2][0], r0[1][1], 2);
    x[2] = __builtin_amdgcn_alignbyte(r1[3][0], r1[2][1], 2);
    y[2] = __builtin_amdgcn_alignbyte(r1[3][1], r1[3][0], 2);
    qh[3] = r0[2][1];
    x[3] = r1[4][0];
    y[3] = r1[4][1];
    // blocks 4 (even) and 5 (odd)
    qh[4] = __builtin_amdgcn_alignbyte(r0[3][1], r0[3][0], 2);
    x[4] = __builtin_amdgcn_alignbyte(r1[5][1], r1[5][0], 2);
    y[4] = __builtin_amdgcn_alignbyte(r1[6][0], r1[5][1], 2);
    qh[5] = r0[4][0];
    x[5] = r1[6][1];
    y[5] = r1[7][0];
    // blocks 6 (even) and 7 (odd)
    qh[6] = __builtin_amdgcn_alignbyte(r0[5][0], r0[4][1], 2);
    x[6] = __builtin_amdgcn_alignbyte(r1[8][0], r1[7][1], 2);
    y[6] = __builtin_amdgcn_alignbyte(r1[8][1], r1[8][0], 2);
    qh[7] = r0[5][1];
    x[7] = r1[9][0];
    y[7] = r1[9][1];
}
// f16 K: the lane's 8 K fragments (16-byte chunks of its key row at the
// swizzled LDS addresses ka[b]) and the 8 query fragments from LDS, in one asm
// batch that waits for its own LDS reads (see k_words_q8).
__device__ __forceinline__ void k_words_f16(const uint32_t (&ka)[8], const uint8_t *qfl, u32x4 (&kf)[8],
                                            u32x4 (&qf)[8]) {
  const uint32_t qa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)qfl;
  __asm__ volatile(
      "ds_read_b128 %0, %16\n\t"
      "ds_read_b128 %1, %17\n\t"
      "ds_read_b128 %2, %18\n\t"
      "ds_read_b128 %3, %19\n\t"
      "ds_read_b128 %4, %20\n\t"
      "ds_read_b128 %5, %21\n\t"
      "ds_read_b128 %6, %22\n\t"
      "ds_read_b128 %7, %23\n\t"
      "ds_read_b128 %8, %24\n\t"
      "ds_read_b128 %9, %24 offset:1024\n\t"
      "ds_read_b128 %10, %24 offset:2048\n\t"
      "ds_read_b128 %11, %24 offset:3072\n\t"
      "ds_read_b128 %12, %24 offset:4096\n\t"
      "ds_read_b128 %13, %24 offset:5120\n\t"
      "ds_read_b128 %14, %24 offset:6144\n\t"
      "ds_read_b128 %15, %24 offset:7168\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(kf[0]), "=&v"(kf[1]), "=&v"(kf[2]), "=&v"(kf[3]), "=&v"(kf[4]), "=&v"(kf[5]), "=&v"(kf[6]),
        "=&v"(kf[7]), "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]),
        "=&v"(qf[6]), "=&v"(qf[7])
      : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(ka[4]), "v"(ka[5]), "v"(ka[6]), "v"(ka[7]), "v"(qa)
      : "memory");
}
// A operand of S^T = K Q^T for a q5_0 block from its realigned words and high
// bits (as k_frag<Q5_0> builds it)
__device__ __forceinline__ half8 k_frag_q5words(uint32_t x, uint32_t y, uint32_t qh, int g) {
  const int gg = g & 1, sh = (g & 2) ? 4 : 0;
  x >>= sh;
  y >>= sh;
  const uint32_t hb = qh >> (16 * (g >> 1) + 8 * gg);
  u32x4 r;
  r[0] = q5pair_to_h2(x, 0x0c010c00u, hb & 1u, (hb >> 1) & 1u);
  r[1] = q5pair_to_h2(x, 0x0c030c02u, (hb >> 2) & 1u, (hb >> 3) & 1u);
  r[2] = q5pair_to_h2(y, 0x0c010c00u, (hb >> 4) & 1u, (hb >> 5) & 1u);
  r[3] = q5pair_to_h2(y, 0x0c030c02u, (hb >> 6) & 1u, (hb >> 7) & 1u);
  return __builtin_bit_cast(half8, r);
}
// A operand of S^T = K Q^T for a q4_0 / q4_1 block from its quant word x (as
// k_frag builds it)
template <int KT>
__device__ __forceinline__ half8 k_frag_q4word(uint32_t x) {
  constexpr int BIAS = KT == Q4_0 ? -8 : 0;
  const uint32_t x8 = x >> 8;
  u32x4 r;
  r[0] = nib_lo_h2<BIAS>(x);
  r[1] = nib_lo_h2<BIAS>(x8);
  r[2] = nib_hi_h2<BIAS>(x);
  r[3] = nib_hi_h2<BIAS>(x8);
  return __builtin_bit_cast(half8, r);
}

// A operand of the f16 product for a q8_0 block from the words k_words_q8 read
// (as k_frag<Q8_0> builds it)
__device__ __forceinline__ half8 k_frag_q8words(const uint32_t (&kw)[16], const uint32_t (&ke)[4], int b,
                                                uint32_t sel_edge) {
  const uint32_t x = kw[2 * b];
  const uint32_t y = (b & 1) ? kw[2 * b + 1] : __builtin_amdgcn_perm(kw[2 * b + 1], ke[b >> 1], sel_edge);
  u32x4 r;
  r[0] = i8pair_to_h2(x, 0x0c010c00u);
  r[1] = i8pair_to_h2(x, 0x0c030c02u);
  r[2] = i8pair_to_h2(y, 0x0c010c00u);
  r[3] = i8pair_to_h2(y, 0x0c030c02u);
  return __builtin_bit_cast(half8, r);
}
// x[i] of lane n ^ 8 within each 16-lane row (row_ror:8), for the four
// elements, as DPP moves in asm: the compiler does not fold them into the
// following adds (its DPP combine of this exchange miscompiled). s_nop 1 covers
// the VALU-write -> DPP-read hazard, which the compiler cannot see in asm.
__device__ __forceinline__ floatx4 ror8x4(floatx4 x) {
  floatx4 r;
  __asm__("s_nop 1\n\t"
          "v_mov_b32_dpp %0, %4 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
          "v_mov_b32_dpp %1, %5 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
          "v_mov_b32_dpp %2, %6 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
          "v_mov_b32_dpp %3, %7 row_ror:8 row_mask:0xf bank_mask:0xf"
          : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
          : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
  return r;
}
// x summed with its value in lane ^ 16, then in lane ^ 32 (all four lane groups),
// by the gfx950 row and half-wave swaps: with x in both operands the two
// registers come out holding x and its partner, in one order or the other. In
// asm: through the builtins the compiler added one result to itself when both
// inputs were the same value. s_nop 1 covers the VALU-write -> swap-read hazard.
__device__ __forceinline__ float sum_groups4(float x) {
  float a = x, b = x;
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  float c = a + b, d = a + b;
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return c + d;
}
// tbl_read8 plus the two float4 at q (8 consecutive floats), in one batch.
__device__ __forceinline__ void tbl_read8_q2(const float *p, const float *q, floatx4 (&out)[8], floatx4 &q0,
                                             floatx4 &q1) {
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)p;
  const uint32_t b = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)q;
  __asm__ volatile(
      "ds_read_b128 %0, %10\n\t"
      "ds_read_b128 %1, %10 offset:64\n\t"
      "ds_read_b128 %2, %10 offset:128\n\t"
      "ds_read_b128 %3, %10 offset:192\n\t"
      "ds_read_b128 %4, %10 offset:256\n\t"
      "ds_read_b128 %5, %10 offset:320\n\t"
      "ds_read_b128 %6, %10 offset:384\n\t"
      "ds_read_b128 %7, %10 offset:448\n\t"
      "ds_read_b128 %8, %11\n\t"
      "ds_read_b128 %9, %11 offset:16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(out[4]), "=&v"(out[5]),
        "=&v"(out[6]), "=&v"(out[7]), "=&v"(q0), "=&v"(q1)
      : "v"(a), "v"(b)
      : "memory");
}
// f16 of four products, the B operand of one PV MFMA. In single-token mode
// rows n and n + 8 carry the same head (the hi and lo query parts were summed
// into both), so their O columns come out identical and rows 8-15 are ignored.
__device__ __forceinline__ half4 p_op4(float x0, float x1, float x2, float x3) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 a = {(_Float16)x0, (_Float16)x1}, b = {(_Float16)x2, (_Float16)x3};
  return __builtin_bit_cast(half4, u32x2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)});
}
// Online-softmax reference max: moved only when a row's new scores exceed it
// by more than kRescaleLog2 (probabilities stay <= 2^8 against a stale max),
// so the O rescale and the cross-lane max are rare instead of per tile.
#ifndef RD4_DEC_THRESH
#define RD4_DEC_THRESH 8.0f
#endif
constexpr float kRescaleLog2 = RD4_DEC_THRESH;

}  // namespace
#if RD4_DEC_TRACE
__device__ unsigned long long rd4_dec_trace[1024 * 8 * 32];
extern "C" int rd4_dec_trace_read(void *host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(rd4_dec_trace), sizeof(rd4_dec_trace));
}
extern "C" int rd4_dec_trace_clear() {
  static unsigned long long z[1024 * 8 * 32];
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(rd4_dec_trace), z, sizeof(z));
}
#endif

// CTA barrier for LDS data only: waits for this wave's LDS operations, not for
// tile DMA still in flight (which __syncthreads would also wait for).
__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The int8 query fragments (8 x 8 bytes, 32 bytes apart from p) and, when
// wanted, the 8 row scales (from sq), in one batch of LDS reads with one wait
// (plain loads would also wait for the tile DMA in flight).
template <bool kScales>
__device__ __forceinline__ void read_qop(const uint8_t *p, const float *sq, long (&qop)[8], float *sqb) {
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
  const uint32_t b = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)sq;
#define RD4_QOP_READS                                                                                  \
  "ds_read_b64 %0, %[a]\n\tds_read_b64 %1, %[a] offset:32\n\tds_read_b64 %2, %[a] offset:64\n\t"     \
  "ds_read_b64 %3, %[a] offset:96\n\tds_read_b64 %4, %[a] offset:128\n\tds_read_b64 %5, %[a] offset:160\n\t" \
  "ds_read_b64 %6, %[a] offset:192\n\tds_read_b64 %7, %[a] offset:224\n\t"
  if constexpr (kScales) {
    uint64_t s0, s1, s2, s3;  // scale pairs (64-bit outputs: a vector type here lost its upper halves)
    __asm__ volatile(RD4_QOP_READS
                     "ds_read_b64 %8, %[b]\n\tds_read_b64 %9, %[b] offset:8\n\t"
                     "ds_read_b64 %10, %[b] offset:16\n\tds_read_b64 %11, %[b] offset:24\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(qop[0]), "=&v"(qop[1]), "=&v"(qop[2]), "=&v"(qop[3]), "=&v"(qop[4]), "=&v"(qop[5]),
                       "=&v"(qop[6]), "=&v"(qop[7]), "=&v"(s0), "=&v"(s1), "=&v"(s2), "=&v"(s3)
                     : [a] "v"(a), [b] "v"(b)
                     : "memory");
    const uint64_t sv[4] = {s0, s1, s2, s3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sqb[2 * i] = __builtin_bit_cast(float, (uint32_t)sv[i]);
      sqb[2 * i + 1] = __builtin_bit_cast(float, (uint32_t)(sv[i] >> 32));
    }
  } else {
    (void)b;
    (void)sqb;
    __asm__ volatile(RD4_QOP_READS "s_waitcnt lgkmcnt(0)"
                     : "=&v"(qop[0]), "=&v"(qop[1]), "=&v"(qop[2]), "=&v"(qop[3]), "=&v"(qop[4]), "=&v"(qop[5]),
                       "=&v"(qop[6]), "=&v"(qop[7])
                     : [a] "v"(a)
                     : "memory");
  }
#undef RD4_QOP_READS
}

template <int KT, int VT, bool PAIR>
__global__ __launch_bounds__((64 * TileShape<KT, VT>::WAVES), 1) void decode_mfma_kernel(AttnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  using TS = TileShape<KT, VT>;
  constexpr int kWaves = TS::WAVES, kThreads = 64 * kWaves;
  constexpr int KS = rowb<KT>(), VS = rowb<VT>();
  constexpr int KC = TS::KC, VC = TS::VC, KCH = TS::KCH, VCH = TS::VCH, NI = TS::NI;
  constexpr int TB = TS::TB, R = TS::R, DT = TS::DT;

  // q8_0 K in single-token mode: S^T on the int8 MFMA, the query as int8 hi and
  // lo rows with a scale pair per 32-dim block (q = s_hi q_hi + s_lo q_lo to
  // ~amax / 65000 of the block)
  constexpr bool kI8 = KT == Q8_0 && !PAIR;
  const int s = blockIdx.x;
  const int kvh = blockIdx.y / a.n_chunks;
  const int hc = blockIdx.y - kvh * a.n_chunks;
  // Pair mode: this CTA carries tokens tok and tok + 1 (ntc of them exist);
  // MFMA row n is head n & 7 of token tok + (n >> 3), queries in f16.
  constexpr bool pair = PAIR;
  const int tok = pair ? 2 * (int)blockIdx.z : (int)blockIdx.z;
  const int ntc = pair ? min(2, a.n_tok - tok) : 1;
  // the wave index is uniform across the wave: readfirstlane lets the compiler
  // keep tile bases and LDS destinations in scalar registers
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
#if RD4_DEC_TRACE
  // timestamps (100 MHz realtime counter) of lane 0 of every wave, slot
  // [cta][wave][point] of rd4_dec_trace (diagnostic builds only)
  int tpos = 0;
  const int tcta = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
#define RD4_TP()                                                                          \
  do {                                                                                    \
    if (lane == 0 && tpos < 28 && tcta < 1024)                                            \
      rd4_dec_trace[(tcta * 8 + w) * 32 + tpos++] = __builtin_amdgcn_s_memrealtime();     \
  } while (0)
#else
#define RD4_TP() \
  do {           \
  } while (0)
#endif
  RD4_TP();
  if (RD4_DEC_KNOBS && (a.dbg & 4096)) return;  // profiling: launch cost alone
  const int grp = a.n_head / a.n_head_kv;
  const int h0 = kvh * grp + hc * kG;
  const int G = min(kG, grp - hc * kG);
  const int t = a.pos ? a.pos[tok] : a.t + tok + ntc - 1;  // last key of the CTA's last token
  const int n_keys = t + 1;

#ifndef RD4_DEC_ILV
#define RD4_DEC_ILV 1
#endif
  // Keys of split s: with RD4_DEC_ILV, the 16-key tiles s, s + S, s + 2S, ...
  // (at any moment the splits of a kv head read neighbouring tiles); else a
  // contiguous range of tiles.
  int chunk = (max(n_keys, 0) + a.n_splits - 1) / a.n_splits;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  const int j_begin = RD4_DEC_ILV ? 16 * s : s * chunk;
  const int j_end = RD4_DEC_ILV ? max(n_keys, 0) : min(n_keys, j_begin + chunk);
  const int j_step = RD4_DEC_ILV ? 16 * a.n_splits : 16;  // keys between the split's tiles

  const int64_t kstride = (int64_t)a.n_head_kv * rowb<KT>();
  const int64_t vstride = (int64_t)a.n_head_kv * rowb<VT>();
  const uint8_t *kbase = a.k + (int64_t)kvh * rowb<KT>();
  const uint8_t *vbase = a.v + (int64_t)kvh * rowb<VT>();

  // Fused append: the CTA owning key t writes the new K/V row of its kv head
  // (8-lane groups per 32-element block, the store kernel's quantizer) before
  // any of its tiles is requested; every other CTA starts its loads at once.
  const bool owns_new = a.k_new && t >= 0 &&
                        (RD4_DEC_ILV ? (t >> 4) % a.n_splits == s : (j_begin <= t && t < j_end));
  if (owns_new) {
    if (tid < 128) {
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
    // the new row reaches this CU's L1 before any wave loads it (workgroup
    // scope; a CTA barrier orders it for the other waves: the one after the query
    // staging, or on the int8 query path the one after the query preparation, and
    // this CTA issues no tile before it)
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  }

  // ---- async tile ring: stage i of this wave at ring + (i % R) * TB
  uint8_t *ring = smem + w * (R * TB);
  // tables [8 blocks][16 keys]: K scales, V scales, K offsets, V offsets
  constexpr int iDK = KT != F16 ? 0 : -1;
  constexpr int iDV = VT != F16 ? (KT != F16) : -1;
  constexpr int iMK = KT == Q4_1 ? (KT != F16) + (VT != F16) : -1;
  constexpr int iMV = VT == Q4_1 ? (KT != F16) + (VT != F16) + (KT == Q4_1) : -1;
  // The scale tables live in their own static LDS array: a separate object from
  // the DMA ring, so the compiler can prove their reads do not alias tile loads
  // still in flight and inserts no vmcnt(0) wait (which would stall on the
  // next tile's prefetch) before them.
  __shared__ __align__(16) float tbl_s[kWaves][DT > 0 ? DT / 4 : 4];
  float *dk_t = tbl_s[w];
  float *dv_t = dk_t + 128 * (iDV > 0 ? iDV : 0);
  float *mk_t = dk_t + 128 * (iMK > 0 ? iMK : 0);
  float *mv_t = dk_t + 128 * (iMV > 0 ? iMV : 0);
  const int n_tiles_all = j_end > j_begin ? (j_end - j_begin - 1) / j_step + 1 : 0;
  // Tile order: with 8 waves, waves w and w + 4 share a SIMD and the older one
  // (w < 4) is issued first, so it takes more tiles: n_lo rounds go to all 8
  // waves (tile 8i + w), the rest to waves 0-3 only (4 per round).
#ifndef RD4_DEC_LO
#define RD4_DEC_LO 6
#endif
  const int n_lo = kWaves == 8 ? n_tiles_all * RD4_DEC_LO / 64 : n_tiles_all;
  const int t_rem = kWaves == 8 ? n_tiles_all - 8 * n_lo : 0;
  const int my_tiles = (RD4_DEC_KNOBS && (a.dbg & 32)) ? 0
                       : kWaves == 8 ? (w < 4 ? n_lo + (t_rem > w ? (t_rem - w + 3) / 4 : 0) : n_lo)
                                     : (n_tiles_all > w ? (n_tiles_all - w + kWaves - 1) / kWaves : 0);
  auto tile_of = [&](int i) {
    return kWaves == 8 ? (i < n_lo ? 8 * i + w : 8 * n_lo + 4 * (i - n_lo) + w) : w + i * kWaves;
  };
  // Global source of this lane's chunk in load instruction r of a tile:
  // byte offset from the tile's K (or V) base, with the f16 swizzle applied.
  // Rows past the tile's last key (partial tiles) re-read the tile's first row.
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
  // Full tiles use offsets computed once: instructions whose 64 chunks are all
  // K (or all V) address from a wave-uniform base.
  uint32_t goff[NI];  // unsigned: scalar base + 32-bit vector offset addressing
#pragma unroll
  for (int r = 0; r < NI; ++r) {
    const int c = lane + 64 * r;
    if (c < KCH) {
      const int row = c / KC, slot = c - row * KC;
      goff[r] = (uint32_t)(row * (int)kstride + 16 * swz<KT>(row, slot));
    } else {
      const int cv = c < KCH + VCH ? c - KCH : 0;
      const int row = cv / VC, slot = cv - row * VC;
      goff[r] = (uint32_t)(row * (int)vstride + 16 * swz<VT>(row, slot));
    }
  }
  constexpr int kAux = (PAIR || !(KT == F16 || KT == Q8_0) || !(VT == F16 || VT == Q8_0)) ? 0 : RD4_DEC_AUX;
  auto issue = [&](int i) {  // i-th tile of this wave
    if (RD4_DEC_KNOBS && (a.dbg & 2048)) return;
    const int j0 = j_begin + tile_of(i) * j_step;
    const int nk = min(kTile, j_end - j0);
    const uint8_t *kt0 = kbase + (int64_t)j0 * kstride;
    const uint8_t *vt0 = vbase + (int64_t)j0 * vstride;
    uint8_t *st = ring + (i % R) * TB;
    if (nk == kTile) {
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const uint8_t *base = (64 * r + 63 < KCH) ? kt0 : (64 * r >= KCH) ? vt0
                              : (lane + 64 * r < KCH ? kt0 : vt0);
        if (64 * r + 63 < KCH + VCH || lane + 64 * r < KCH + VCH)
          __builtin_amdgcn_global_load_lds((const void *)(base + goff[r]), (lds_void *)(st + 1024 * r),
                                           16, 0, kAux);
      }
    } else {
#pragma unroll
      for (int r = 0; r < NI; ++r)
        if (64 * r + 63 < KCH + VCH || lane + 64 * r < KCH + VCH)
          __builtin_amdgcn_global_load_lds((const void *)src_of(r, nk, kt0, vt0),
                                           (lds_void *)(st + 1024 * r), 16, 0, kAux);
    }
  };
  // The chunk's G query rows are copied into LDS once per CTA by the same
  // global->LDS DMA, issued before any tile so they are not queued behind the
  // tiles; rows are padded by 16 bytes so the per-row fragment reads below do
  // not collide in one bank.
  uint8_t *q_lds = smem + kWaves * (R * TB);
  const int qcw = a.q_f16 ? kHD / 8 : kHD / 4;  // 16-byte chunks per query row
  const int qsb = 16 * (qcw + 1);               // padded row stride in bytes
  auto issue_q = [&]() {  // one load instruction per 64 chunks, spread over the waves
    if (RD4_DEC_KNOBS && (a.dbg & 2048)) return;
    for (int base = 64 * w; base < G * (qcw + 1); base += 64 * kWaves) {
      const int idx = base + lane, r = idx / (qcw + 1), c = idx - r * (qcw + 1);
      if (r < G && c < qcw) {
        const uint8_t *src = (const uint8_t *)a.q +
                             (((int64_t)tok * a.n_head + h0 + r) * kHD) * (a.q_f16 ? 2 : 4) + 16 * c;
        __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(q_lds + 16 * base), 16, 0, 0);
      }
    }
  };
  // int8 query path: wave w loads the rows it quantizes straight into registers
  // (lane l: dims 4l..4l+3), ahead of its tile loads, so it waits for its own
  // rows only, with no barrier and no LDS traffic
  float xq[kI8 ? 8 / kWaves : 1][4];
  auto load_q_own = [&]() {
#pragma unroll
    for (int m = 0; m < 8 / kWaves; ++m) {
      const int r = w + kWaves * m;
      const int64_t off = ((int64_t)tok * a.n_head + h0 + (r < G ? r : 0)) * kHD + 4 * lane;
      if (a.q_f16) {
        const uint2 hv = *(const uint2 *)((const uint16_t *)a.q + off);
        xq[m][0] = h2f((uint16_t)hv.x);
        xq[m][1] = h2f((uint16_t)(hv.x >> 16));
        xq[m][2] = h2f((uint16_t)hv.y);
        xq[m][3] = h2f((uint16_t)(hv.y >> 16));
      } else {
        const float4 fv = *(const float4 *)(a.q + off);
        xq[m][0] = fv.x;
        xq[m][1] = fv.y;
        xq[m][2] = fv.z;
        xq[m][3] = fv.w;
      }
    }
  };
  if (!pair) {
    if constexpr (kI8) load_q_own();
    else issue_q();
  }
#ifndef RD4_DEC_PRE
#define RD4_DEC_PRE 0
#endif
  // Tiles issued before the query rows have landed: none. The query rows gate
  // the whole CTA, and a chip-wide burst of tile requests queued with them at
  // the memory controllers delays them (by about 2 us on q8_0 32K); the first
  // tile goes out once they have landed, the rest of the ring at the loop start.
  // (pair mode reads its query rows inside the preparation: one tile ahead)
  constexpr int kPre = PAIR ? 1 : RD4_DEC_PRE;
  int next_issue = (kPre > 0 && !owns_new) ? min(kPre, my_tiles) : 0;  // next tile to issue
  if (!owns_new) {
#pragma unroll
    for (int i = 0; i < kPre; ++i)
      if (i < my_tiles) issue(i);  // first tiles in flight right behind the query rows
  }
  // this wave's query chunk has landed once at most the tile loads issued after it remain
  if (!pair) {
    const int after = owns_new ? 0 : min(kPre, my_tiles);
    if (after >= 3) wait_vm<3 * NI>();
    else if (after == 2) wait_vm<2 * NI>();
    else if (after == 1) wait_vm<NI>();
    else wait_vm<0>();
    // every wave uses every row: the rows loaded by the other waves must land
    // (the int8 path's barrier comes after its own preparation)
    if constexpr (!kI8) __syncthreads();
  }
  RD4_TP();
  if (RD4_DEC_KNOBS && (a.dbg & 8192)) return;  // profiling: up to the query rows
  // One tile requested as soon as the query rows are in (on the LDS-staged query
  // paths, once every wave has read them), so it lands during the query
  // preparation. The preparation's barriers wait for LDS only: a CTA barrier
  // would also wait for this tile.
#ifndef RD4_DEC_POSTQ
#define RD4_DEC_POSTQ 1
#endif
  auto issue_postq = [&]() {
    if (RD4_DEC_POSTQ > 0 && !pair && !owns_new) {
      while (next_issue < min(RD4_DEC_POSTQ, R) && next_issue < my_tiles) issue(next_issue++);
    }
  };
  // (f16 K measured faster with the tile requested here and landed by the
  // preparation's CTA barriers)
  if constexpr (kI8 || KT == F16) issue_postq();

  // Query fragment (B operand of S^T = K Q^T): row n is head n (hi) or n-8
  // (lo); k-slot j of lane group g holds dim k_dim<KT>(b, g, j). Every wave
  // needs the same 8 fragments, so wave w converts blocks w, w + kWaves, ...
  // once and the CTA exchanges them through LDS (over the query rows).
  const uint32_t lo_mask = n >= 8 ? 0xffffffffu : 0u;
  half8 qf[8];
  float qblk[8];
  long qop[kI8 ? 8 : 1];    // int8 query fragments (kI8)
  // this lane's row scale per block (kI8); with q4_1 V (more live registers in
  // the tile loop) they are re-read from LDS with the K scale table instead
  constexpr bool kSqReg = VT != Q4_1;
  float sqb[kI8 && kSqReg ? 8 : 1];
  if (pair) {
    // f16 query rows straight from global memory, both tokens' heads
    const int hh = n & 7, tr = n >> 3;
    const bool on = hh < G && tr < ntc;
    const float *qrow = a.q + ((int64_t)(tok + (on ? tr : 0)) * a.n_head + h0 + (on ? hh : 0)) * kHD;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      float qs = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float2 f = on ? make_float2(qrow[k_dim<KT>(b, g, 2 * jj)], qrow[k_dim<KT>(b, g, 2 * jj + 1)])
                            : make_float2(0.f, 0.f);
        qf[b][2 * jj] = (_Float16)f.x;
        qf[b][2 * jj + 1] = (_Float16)f.y;
        if constexpr (KT == Q4_1) qs += f.x + f.y;
      }
      if constexpr (KT == Q4_1) {
        qs += xor_f(qs, 16);
        qs += xor_f(qs, 32);
        qblk[b] = qs;
      }
    }
  } else if constexpr (kI8) {
    if (RD4_DEC_KNOBS && (a.dbg & 64)) {  // profiling knob: skip the query preparation
#pragma unroll
      for (int b = 0; b < 8; ++b) qop[b] = 0;
      if constexpr (kSqReg) {
#pragma unroll
        for (int b = 0; b < 8; ++b) sqb[b] = 0.0f;
      }
    } else {
    // wave w quantizes head rows w, w + kWaves, ...: lane l holds dims 4l..4l+3
    // of block l / 8; per block s_hi = amax / 127, q_hi = rint(q / s_hi), and the
    // remainder on s_hi / 254. The int8 image lies past the query rows, so no
    // barrier is needed before it.
    uint8_t *qi = q_lds + kG * (kHD * 4 + 16) + 256;  // [16 rows][8 blocks][32 slots]
    float *sq = (float *)(qi + 16 * kQiRow);           // [16 rows][8 blocks] scales (with scale * log2 e)
#pragma unroll
    for (int m = 0; m < 8 / kWaves; ++m) {
      const int r = w + kWaves * m;
      float xr[4] = {xq[m][0], xq[m][1], xq[m][2], xq[m][3]};
      if (r >= G) xr[0] = xr[1] = xr[2] = xr[3] = 0.0f;
      const float am = max8_nonneg(fmaxf(fmaxf(fabsf(xr[0]), fabsf(xr[1])), fmaxf(fabsf(xr[2]), fabsf(xr[3]))));
      // any scales work as long as the reconstruction uses the same ones: s_hi =
      // amax / 127 and s_lo = s_hi / 254 by multiplication, the inverses from one
      // v_rcp_f32 (a q_hi off by one from rounding is absorbed by the lo part)
      const float rcp = am > 0.0f ? __builtin_amdgcn_rcpf(am) : 0.0f;
      const float s_hi = am * (1.0f / 127.0f), s_lo = am * (1.0f / (127.0f * 254.0f));
      const float i_hi = 127.0f * rcp, i_lo = (127.0f * 254.0f) * rcp;
      uint32_t bh[4], bl[4];  // the int8 hi / lo values as bytes
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float qh = __builtin_amdgcn_fmed3f(rintf(xr[i] * i_hi), -127.0f, 127.0f);
        const float rem = fmaf(-s_hi, qh, xr[i]);
        const float ql = __builtin_amdgcn_fmed3f(rintf(rem * i_lo), -127.0f, 127.0f);
        bh[i] = (uint32_t)(int)qh & 0xffu;
        bl[i] = (uint32_t)(int)ql & 0xffu;
      }
      // lane l holds dims e = 4(l & 7) + i of block b = l / 8. Their k-slots (the
      // inverse of k_dim<Q8_0>): odd blocks e (one aligned word); even blocks
      // e - 2 for 2 <= e < 30, 28 + e below, e above (two aligned 16-bit pairs)
      const int b = lane >> 3, e0 = 4 * (lane & 7);
      uint8_t *hrow = qi + r * kQiRow + b * 32, *lrow = qi + (r + 8) * kQiRow + b * 32;
      if (b & 1) {
        *(uint32_t *)(hrow + e0) = bh[0] | bh[1] << 8 | bh[2] << 16 | bh[3] << 24;
        *(uint32_t *)(lrow + e0) = bl[0] | bl[1] << 8 | bl[2] << 16 | bl[3] << 24;
      } else {
        const int s01 = e0 == 0 ? 28 : e0 - 2, s23 = e0 == 28 ? 30 : e0;
        *(uint16_t *)(hrow + s01) = (uint16_t)(bh[0] | bh[1] << 8);
        *(uint16_t *)(hrow + s23) = (uint16_t)(bh[2] | bh[3] << 8);
        *(uint16_t *)(lrow + s01) = (uint16_t)(bl[0] | bl[1] << 8);
        *(uint16_t *)(lrow + s23) = (uint16_t)(bl[2] | bl[3] << 8);
      }
      if ((lane & 7) == 0) {
        sq[r * kSqRow + b] = s_hi * a.scale * kLog2e;
        sq[(r + 8) * kSqRow + b] = s_lo * a.scale * kLog2e;
      }
    }
    lds_barrier();
    read_qop<kSqReg>(qi + n * kQiRow + 8 * g, sq + n * kSqRow, qop, sqb);
    }
  } else {
    const int hh = n & 7;
    const bool on = hh < G;
    const uint8_t *qrow = q_lds + (on ? hh : 0) * qsb;
    u32x4 mine[8 / kWaves];
    float qsum_mine[8 / kWaves];  // q4_1 K: sum of the row's q over block b
#pragma unroll
    for (int m = 0; m < 8 / kWaves; ++m) {
      const int b = w + kWaves * m;
      float qs = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int d0 = k_dim<KT>(b, g, 2 * jj), d1 = k_dim<KT>(b, g, 2 * jj + 1);
        float x0, x1;
        if (a.q_f16) {
          x0 = h2f(*(const uint16_t *)(qrow + 2 * d0));
          x1 = h2f(*(const uint16_t *)(qrow + 2 * d1));
        } else {
          x0 = *(const float *)(qrow + 4 * d0);
          x1 = *(const float *)(qrow + 4 * d1);
        }
        mine[m][jj] = on ? split_prod2(x0, 1.0f, x1, 1.0f, lo_mask) : 0u;
        if constexpr (KT == Q4_1) qs += x0 + x1;
      }
      if constexpr (KT == Q4_1) {
        qs += xor_f(qs, 16);
        qs += xor_f(qs, 32);
      }
      qsum_mine[m] = qs;
    }
    __syncthreads();  // every wave has read the query rows
    if constexpr (KT != F16) issue_postq();
    u32x4 *qf_lds = (u32x4 *)q_lds;  // [block][lane]
    float *qsum_lds = (float *)(q_lds + 8 * 64 * 16);  // [block][head]
#pragma unroll
    for (int m = 0; m < 8 / kWaves; ++m) {
      qf_lds[(w + kWaves * m) * 64 + lane] = mine[m];
      if (KT == Q4_1 && lane < 8) qsum_lds[(w + kWaves * m) * 8 + lane] = on ? qsum_mine[m] : 0.0f;
    }
    if constexpr (KT == F16) __syncthreads();
    else lds_barrier();
#pragma unroll
    for (int b = 0; b < 8; ++b) {
#if !RD4_DEC_QLDS
      qf[b] = __builtin_bit_cast(half8, qf_lds[b * 64 + lane]);
#endif
      // the offset term goes to the hi rows only (rows n and n^8 are summed)
      if constexpr (KT == Q4_1) qblk[b] = n < 8 ? qsum_lds[b * 8 + n] : 0.0f;
    }
  }
  // Query fragment of block b for the QK product: pair mode keeps its eight in
  // registers; single-token mode reads them from LDS at each use, which frees
  // 32 VGPRs in the tile loop
  auto q_frag = [&](int b) __attribute__((always_inline)) {
#if RD4_DEC_QLDS
    if constexpr (!PAIR) return __builtin_bit_cast(half8, ((const u32x4 *)q_lds)[b * 64 + lane]);
#endif
    return qf[b];
  };
  const float sl2 = a.scale * kLog2e;
  // edge gather of the unaligned q8_0 K blocks: lane group 3 takes the block's
  // first and last byte pairs
  const uint32_t sel_edge = g == 3 ? 0x05040302u : 0x07060504u;
  // f16 K: byte offset of block b's 16-byte chunk in the lane's swizzled key row
  uint32_t kf16_off[KT == F16 ? 8 : 1];
  if constexpr (KT == F16) {
#pragma unroll
    for (int b = 0; b < 8; ++b) kf16_off[b] = 16u * (uint32_t)((4 * b + g) ^ n);
  }
  // pair mode: the last key of this lane's row; the P operand fills all 16 rows
  const int row_last = pair ? a.t + tok + (n >> 3) : t;

  floatx4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float cm[8];  // q4_1 V: sum_j p_j m_j per block for this lane's row and keys
#pragma unroll
  for (int b = 0; b < 8; ++b) cm[b] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // state of the current tile, shared by the exp/PV step and the rescale
  float sc[4];
  const uint8_t *vl = nullptr;
  int i = 0;  // this wave's tile being processed
  auto finish = [&]() __attribute__((always_inline)) {
    float psum = 0.0f;
    // a row that has seen no key yet (pair mode, a split holding only the
    // second token's last key) keeps m_run = -inf; its masked scores give 0
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = __builtin_amdgcn_exp2f(sc[i] - m_use);
      psum += sc[i];
    }
    l_run += psum;

    RD4_TP();
    // ---- O^T += V^T P^T (16 keys)
    if (RD4_DEC_KNOBS && (a.dbg & 4)) {
      o[0][0] += sc[0] + sc[3];
      (void)vl;
    } else if constexpr (VT == F16) {
      const half4 pf = p_op4(sc[0], sc[1], sc[2], sc[3]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // 16-byte chunk n + 16h (dims 8(n + 16h) .. +7) of the lane's 4 keys
        u32x4 ch[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 4 * g + i;
          ch[i] = *(const u32x4 *)(vl + row * VS + 16 * ((n ^ (row & 15)) + 16 * h));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          const uint32_t lo = __builtin_amdgcn_perm(ch[1][e >> 1], ch[0][e >> 1], sel);
          const uint32_t hi = __builtin_amdgcn_perm(ch[3][e >> 1], ch[2][e >> 1], sel);
          o[8 * h + e] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4, u32x2{lo, hi}),
                                                              pf, o[8 * h + e], 0, 0, 0);
        }
      }
    } else {
      floatx4 dvs[8], mvs[VT == Q4_1 ? 8 : 1];
      // the V bytes of the lane's 4 keys for all 8 blocks are read ahead of the
      // scale table, whose asm batch then lands them in the same round trip
      // (q5_0 and q4_1, with more live registers here, read per block below)
      constexpr bool kHoistV = VT == Q8_0 || VT == Q4_0;
      uint32_t ur[kHoistV ? 8 : 1][4];
      if constexpr (kHoistV) {
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint8_t *vrow = vl + (4 * g + i) * VS + block_bytes(VT) * b + (VT == Q4_1 ? 4 : 2);
            ur[b][i] = VT == Q8_0 ? lds_u16(vrow + 2 * n) : lds_u8(vrow + n);
          }
      }
      tbl_read8(dv_t + 4 * g, dvs);
      if constexpr (VT == Q4_1) tbl_read8(mv_t + 4 * g, mvs);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const float4 dv = make_float4(dvs[b][0], dvs[b][1], dvs[b][2], dvs[b][3]);
        // P' = f16(p * d)
        const half4 pf = p_op4(sc[0] * dv.x, sc[1] * dv.y, sc[2] * dv.z, sc[3] * dv.w);
        if constexpr (VT == Q4_1) {
          if (pair || n < 8) {
            const float4 mv = make_float4(mvs[b][0], mvs[b][1], mvs[b][2], mvs[b][3]);
            cm[b] = fmaf(sc[0], mv.x, fmaf(sc[1], mv.y, fmaf(sc[2], mv.z, fmaf(sc[3], mv.w, cm[b]))));
          }
        }
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint8_t *blk = vl + (4 * g + i) * VS + block_bytes(VT) * b;
          const uint8_t *vrow = blk + (VT == Q4_1 ? 4 : VT == Q5_0 ? 6 : 2);
          if constexpr (kHoistV) u[i] = ur[b][i];
          else u[i] = VT == Q8_0 ? lds_u16(vrow + 2 * n) : lds_u8(vrow + n);
          if constexpr (VT == Q5_0) {
            // element n: low nibble + high bit n; element n + 16: high nibble +
            // high bit n + 16; as two 5-bit values in bytes 0 and 1
            const uint32_t hlo = (lds_u16(blk + 2) >> n) & 1u, hhi = (lds_u16(blk + 4) >> n) & 1u;
            u[i] = (u[i] & 0x0fu) | (hlo << 4) | ((u[i] & 0xf0u) << 4) | (hhi << 12);
          }
        }
        // [key0, key1] and [key2, key3] bytes of the lane's 2-dim (q8_0) or
        // 2-nibble (q4_0) word, one MFMA per dim
        const uint32_t w01_0 = __builtin_amdgcn_perm(u[1], u[0], 0x0c040c00u);
        const uint32_t w23_0 = __builtin_amdgcn_perm(u[3], u[2], 0x0c040c00u);
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          uint32_t a01, a23;
          if constexpr (VT == Q5_0) {
            const uint32_t sel = e ? 0x0c050c01u : 0x0c040c00u;
            const h2 c = {(_Float16)-1040.0f, (_Float16)-1040.0f};  // 1024 + 16
            a01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(u[1], u[0], sel) | 0x64006400u) + c);
            a23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(u[3], u[2], sel) | 0x64006400u) + c);
          } else if constexpr (VT == Q8_0) {
            const uint32_t sel = e ? 0x0c050c01u : 0x0c040c00u;
            const h2 c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
            a01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(u[1], u[0], sel) ^ 0x64806480u) + c);
            a23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(u[3], u[2], sel) ^ 0x64806480u) + c);
          } else {
            constexpr int BIAS = VT == Q4_1 ? 0 : -8;
            a01 = e ? nib_hi_h2<BIAS>(w01_0) : nib_lo_h2<BIAS>(w01_0);
            a23 = e ? nib_hi_h2<BIAS>(w23_0) : nib_lo_h2<BIAS>(w23_0);
          }
          o[2 * b + e] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4, u32x2{a01, a23}),
                                                              pf, o[2 * b + e], 0, 0, 0);
        }
      }
    }
  };
  auto rescale = [&]() __attribute__((always_inline)) {
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    tmax = fmaxf(tmax, xor_f(tmax, 16));
    tmax = fmaxf(tmax, xor_f(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    // a row whose max did not move (also -inf, a row with no key yet) keeps its state
    const float corr = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= corr;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] *= corr;
    if constexpr (VT == Q4_1) {
#pragma unroll
      for (int b = 0; b < 8; ++b) cm[b] *= corr;
    }
    m_run = m_new;
  };

  // The tile loop proper never rescales: a tile whose scores pass the running
  // max by the threshold leaves it, is rescaled and finished here, and the loop
  // resumes with the next tile. (With the rescale as a branch inside the loop,
  // the accumulators reach the PV MFMAs through a branch merge, and the
  // compiler gives every MFMA a result register apart from its C operand and
  // copies all 64 back on every tile.)
  RD4_TP();
  if (RD4_DEC_KNOBS && (a.dbg & 16384)) return;  // profiling: up to the tile loop
  for (;;) {
    bool rescale_due = false;
    for (; i < my_tiles; ++i) {
      RD4_TP();
      const int j_tile = j_begin + tile_of(i) * j_step;
      const int nk = min(kTile, j_end - j_tile);
      // the next tiles go out here, or with RD4_DEC_LATE after this tile's QK
      // product (then only a tile this iteration needs itself is issued here)
      const int issue_to = RD4_DEC_LATE ? i : i + R - 1;
      if (next_issue <= issue_to && next_issue < my_tiles) {
        // the stage being refilled was read by the previous iteration: those reads are done
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        do {
          issue(next_issue++);
        } while (next_issue <= issue_to && next_issue < my_tiles);
      }
#if RD4_DEC_TRACE >= 2
      RD4_TP();
#endif
      // tile i is complete once at most the loads of the tiles issued after it remain
      const int after = next_issue - 1 - i;
      if (after >= 3) wait_vm<3 * NI>();
      else if (after == 2) wait_vm<2 * NI>();
      else if (after == 1) wait_vm<NI>();
      else wait_vm<0>();
      wave_sync();
      RD4_TP();
      const uint8_t *kl = ring + (i % R) * TB;
      vl = kl + KCH * 16;
      // q8_0 K words of this lane's key row for the int8 QK product
      // (also for q8_0 K in pair mode, converted to f16 there)
      constexpr bool kQ8W = kI8 || (KT == Q8_0 && PAIR);
      uint32_t kw[kQ8W ? 16 : 1], ke[kQ8W ? 4 : 1];
      // q4_0 / q4_1 K words and the query fragments, batched the same way
      constexpr bool kQ4 = (KT == Q4_0 || KT == Q4_1) && !PAIR && RD4_DEC_QLDS;
      constexpr bool kQ5 = KT == Q5_0 && !PAIR && RD4_DEC_QLDS;
      uint32_t xw[kQ4 || kQ5 ? 8 : 1], yw[kQ5 ? 8 : 1], hw[kQ5 ? 8 : 1];
      u32x4 qfr[kQ4 || kQ5 ? 8 : 1];
      if constexpr (DT > 0) {  // f16 scales (and offsets) of the tile -> f32 tables, once per tile
        // the raw f16 words are read first, so that the K words' batch below
        // (which waits for every LDS read of the wave) lands them in the same
        // round trip
        uint16_t raw[DT / 256];
#pragma unroll
        for (int j = 0; j < DT / 256; ++j) {
          const int v = lane + 64 * j;
          const int ti = v >> 7, key = v & 15, b = (v >> 4) & 7;
          const uint8_t *src = ti == iDK   ? kl + key * KS + block_bytes(KT) * b
                               : ti == iDV ? vl + key * VS + block_bytes(VT) * b
                               : ti == iMK ? kl + key * KS + block_bytes(KT) * b + 2
                                           : vl + key * VS + block_bytes(VT) * b + 2;
          raw[j] = (uint16_t)lds_u16(src);
        }
        if constexpr ((kI8 && kSqReg) || (KT == Q8_0 && PAIR)) {
          k_words_q8(kl + n * KS, g, kw, ke);
#pragma unroll
          for (int j = 0; j < DT / 256; ++j) dk_t[lane + 64 * j] = h2f(raw[j]);
        } else if constexpr (kQ4 || kQ5) {
          if constexpr (kQ4) k_words_q4<KT>(kl + n * KS, g, q_lds + 16 * lane, xw, qfr);
          else k_words_q5(kl + n * KS, g, q_lds + 16 * lane, xw, yw, hw, qfr);
#pragma unroll
          for (int j = 0; j < DT / 256; ++j) dk_t[lane + 64 * j] = h2f(raw[j]);
        } else {
#pragma unroll
          for (int j = 0; j < DT / 256; ++j) {
            dk_t[lane + 64 * j] = h2f(raw[j]);
            __builtin_amdgcn_sched_barrier(0);  // convert each word as it lands
          }
        }
        wave_sync();
      }

      RD4_TP();
      // ---- S^T = K Q^T: lane holds keys 4g..4g+3 of row n
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      if (RD4_DEC_KNOBS && (a.dbg & 2)) {
        acc = floatx4{(float)lane, 1.f, 2.f, 3.f};
      } else {
        const uint8_t *krow = kl + n * KS;
        if constexpr (kI8) {
          floatx4 dks[8];
          float sqv[8];
          if constexpr (kSqReg) {
            tbl_read8(dk_t + 4 * g, dks);
#pragma unroll
            for (int b = 0; b < 8; ++b) sqv[b] = sqb[b];
          } else {
            // (with q4_1 V, whose tables hold more registers, the K words and the
            // block scales are read here)
            k_words_q8(krow, g, kw, ke);
            floatx4 s0, s1;
            tbl_read8_q2(dk_t + 4 * g, (const float *)(q_lds + kG * (kHD * 4 + 16) + 256 + 16 * kQiRow) + kSqRow * n,
                         dks, s0, s1);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              sqv[b] = s0[b];
              sqv[b + 4] = s1[b];
            }
          }
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const i32x4 z = {0, 0, 0, 0};
            const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(k_op_i8(kw, ke, b, sel_edge), qop[b], z, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(dks[b][e], (float)c[e] * sqv[b], acc[e]);
          }
        } else if constexpr (KT == F16) {
          if constexpr (!PAIR && RD4_DEC_QLDS) {
            uint32_t ka[8];
            const uint32_t kr = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)krow;
#pragma unroll
            for (int b = 0; b < 8; ++b) ka[b] = kr + kf16_off[b];
            u32x4 kfr[8], qfr8[8];
            k_words_f16(ka, q_lds + 16 * lane, kfr, qfr8);
#pragma unroll
            for (int b = 0; b < 8; ++b)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, kfr[b]), __builtin_bit_cast(half8, qfr8[b]), acc, 0, 0, 0);
          } else {
#pragma unroll
            for (int b = 0; b < 8; ++b)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g, n, sel_edge), q_frag(b), acc, 0, 0, 0);
          }
        } else {
          floatx4 dks[8], mks[KT == Q4_1 ? 8 : 1];
          tbl_read8(dk_t + 4 * g, dks);
          if constexpr (KT == Q4_1) tbl_read8(mk_t + 4 * g, mks);
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const floatx4 z = {0.f, 0.f, 0.f, 0.f};
            floatx4 c;
            if constexpr (KT == Q8_0 && PAIR)
              c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag_q8words(kw, ke, b, sel_edge), q_frag(b), z, 0, 0, 0);
            else if constexpr (kQ4)
              c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag_q4word<KT>(xw[b]), __builtin_bit_cast(half8, qfr[b]), z, 0, 0, 0);
            else if constexpr (kQ5)
              c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag_q5words(xw[b], yw[b], hw[b], g), __builtin_bit_cast(half8, qfr[b]), z, 0, 0, 0);
            else
              c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_frag<KT>(krow, b, g, n, sel_edge), q_frag(b), z, 0, 0, 0);
            const float4 dk = make_float4(dks[b][0], dks[b][1], dks[b][2], dks[b][3]);
            acc[0] = fmaf(dk.x, c[0], acc[0]);
            acc[1] = fmaf(dk.y, c[1], acc[1]);
            acc[2] = fmaf(dk.z, c[2], acc[2]);
            acc[3] = fmaf(dk.w, c[3], acc[3]);
            if constexpr (KT == Q4_1) {
              const float4 mk = make_float4(mks[b][0], mks[b][1], mks[b][2], mks[b][3]);
              acc[0] = fmaf(mk.x, qblk[b], acc[0]);
              acc[1] = fmaf(mk.y, qblk[b], acc[1]);
              acc[2] = fmaf(mk.z, qblk[b], acc[2]);
              acc[3] = fmaf(mk.w, qblk[b], acc[3]);
            }
          }
        }
      }
      if (RD4_DEC_LATE && next_issue <= i + R - 1 && next_issue < my_tiles) {
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        do {
          issue(next_issue++);
        } while (next_issue <= i + R - 1 && next_issue < my_tiles);
      }
      RD4_TP();
      // Rows n and n^8 are the hi and lo halves of the same head. (A DPP
      // row_ror:8 add was tried here; the compiler's DPP combine fed acc[0] to
      // all four adds, so the exchange stays a plain lane shuffle.)
      bool over = false;
      // last key this lane's row may see, relative to the tile: pair mode masks the
      // second token's last key in the first token's rows
      const int lim = pair ? min(nk - 1, row_last - j_tile) : nk - 1;
      // hi + lo rows: lane n ^ 8 by a DPP rotate (no LDS round trip) for q8_0 and
      // f16 K; the nibble types keep the lane shuffle, which measured faster there
      floatx4 acc8 = acc;
      if constexpr (!PAIR) {
        if constexpr (KT == Q8_0 || KT == F16) {
          acc8 = ror8x4(acc);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc8[i] = xor_f(acc[i], 8);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v;
        if constexpr (kI8) {
          v = acc[i] + acc8[i];
        } else {
          v = pair ? acc[i] * sl2 : (acc[i] + acc8[i]) * sl2;
        }
        if (4 * g + i > lim) v = -INFINITY;
        sc[i] = v;
        over |= v > m_run + kRescaleLog2;
      }
      // The running max moves only when some score passed it by the threshold
      // (a wave vote); only then is the tile's row max reduced across lanes, in
      // the rare path after this loop.
      if (__any(over)) {
        rescale_due = true;
        break;
      }
      finish();
    }
    if (!rescale_due) break;
    rescale();
    finish();
    ++i;
  }

  RD4_TP();
  if (RD4_DEC_KNOBS && (a.dbg & 32768)) {  // profiling: no epilogue (a store keeps the loop live)
    if (m_run == 1.2345f) a.out[lane] = l_run + o[0][0] + o[15][3];
    return;
  }
  // ---- wave state: l summed over the 4 key groups; the hi (n < 8) and lo
  // (n >= 8) rows of O go to LDS as separate rows and are added by the reader
  l_run = sum_groups4(l_run);

  // ---- merge the waves through LDS (reuses the tile buffers). Row slots are
  // the 16 MFMA rows: single-token mode uses rows 0-7 (heads) and adds the lo
  // rows 8-15 into them; pair mode keeps all 16 (two tokens' heads).
  __syncthreads();
  constexpr int kR = 16;
  float *wm = (float *)smem;                 // [kWaves][kR] m, then [kWaves][kR] l
  float *wo = wm + 2 * kWaves * kR;          // [kWaves][16 rows][kRowPad]
  if (lane < kR) {
    wm[w * kR + lane] = m_run;
    wm[kWaves * kR + w * kR + lane] = l_run;
  }
  {
    // o[t][i] holds dim v_dim<VT>(t, 4g + i); written back as 4-dim runs
    float *dst = wo + (w * 16 + n) * kRowPad;
    const bool wr = pair || n < 8;  // single-token rows 8-15 duplicate rows 0-7
    if constexpr (VT == F16) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = v_dim<VT>(8 * h, 4 * g + i);
          if (wr) *(floatx4 *)(dst + d0) = floatx4{o[8 * h][i], o[8 * h + 1][i], o[8 * h + 2][i], o[8 * h + 3][i]};
          if (wr) *(floatx4 *)(dst + d0 + 4) = floatx4{o[8 * h + 4][i], o[8 * h + 5][i], o[8 * h + 6][i], o[8 * h + 7][i]};
        }
    } else if constexpr (VT == Q8_0) {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int d0 = v_dim<VT>(2 * b, 4 * g);
        if (wr) *(floatx4 *)(dst + d0) = floatx4{o[2 * b][0], o[2 * b + 1][0], o[2 * b][1], o[2 * b + 1][1]};
        if (wr) *(floatx4 *)(dst + d0 + 4) = floatx4{o[2 * b][2], o[2 * b + 1][2], o[2 * b][3], o[2 * b + 1][3]};
      }
    } else {
      if constexpr (VT == Q4_1) {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          cm[b] += xor_f(cm[b], 16);
          cm[b] += xor_f(cm[b], 32);
        }
      }
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        floatx4 v = o[t];
        if constexpr (VT == Q4_1) v += cm[t >> 1];
        if (wr) *(floatx4 *)(dst + v_dim<VT>(t, 4 * g)) = v;
      }
    }
  }
  __syncthreads();
  RD4_TP();

  // output rows: (token tr, head hh) in MFMA row r = hh + 8 tr. Each thread
  // weighs the 8 wave states of its row itself (one LDS round trip for their m
  // and l, no lane exchanges and no further barrier).
  const int nrow = pair ? ntc * G : G;
  for (int i = tid; i < nrow * kHD / 4; i += kThreads) {
    const int ri = i / (kHD / 4), d = 4 * (i - ri * (kHD / 4));
    const int tr = pair ? ri / G : 0, hh = ri - tr * G, r = hh + 8 * tr;
    float mw[kWaves], lw[kWaves];
    float mm = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      mw[ww] = wm[ww * kR + r];
      lw[ww] = wm[kWaves * kR + ww * kR + r];
      mm = fmaxf(mm, mw[ww]);
    }
    floatx4 acc4 = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const float wt = (mm == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw[ww] - mm);
      L = fmaf(wt, lw[ww], L);
      acc4 += wt * *(const floatx4 *)(wo + (ww * 16 + r) * kRowPad + d);
    }
    const int64_t hrow_r = (int64_t)(tok + tr) * a.n_head + h0 + hh;
    if (a.n_splits == 1) {
      const float inv = (mm == -INFINITY) ? 0.0f : ((L > 0.0f) ? 1.0f / L : 0.0f);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float o1 = acc4[k] * inv;
        const int64_t oi = hrow_r * kHD + d + k;
        if (a.gate) {
          const float sg = sigmoid_dev(a.gate[oi]);
          a.gate[oi] = sg;
          o1 = o1 * sg;
        }
        a.out[oi] = o1;
      }
    } else {
// the split records leave through non-temporal stores (read once, by the
// merge launch): q8_0 32K -1.3% (non-temporal loads in the merge: +8%)
#ifndef RD4_DEC_RECNT
#define RD4_DEC_RECNT 1
#endif
      if (RD4_DEC_RECNT) {
        __builtin_nontemporal_store(acc4, (floatx4 *)(rec_acc(a, hrow_r, s) + d));
      } else {
        *(floatx4 *)(rec_acc(a, hrow_r, s) + d) = acc4;
      }
      if (d == 0) {
        float *ml = rec_ml(a, hrow_r, s);
        ml[0] = (mm == -INFINITY) ? -INFINITY : mm * 0.6931471805599453f;  // log2 -> ln units
        ml[1] = L;
      }
    }
  }
  RD4_TP();
}

namespace {

template <int KT, int VT>
size_t decode_lds() {
  using TS = TileShape<KT, VT>;
  // query rows (later the shared fragments and the q4_1 block sums)
  const size_t qreg = (size_t)kG * (kHD * 4 + 16) + 256 + TS::QI;
  const size_t tiles = (size_t)TS::WAVES * TS::R * TS::TB + qreg;  // scale tables are static LDS
  // the wave states of the epilogue reuse the ring
  const size_t merge = (2 * TS::WAVES * 16 + TS::WAVES * 16 * kRowPad) * 4;
  return tiles > merge ? tiles : merge;
}

template <int KT, int VT, bool PAIR = false>
hipError_t launch(const AttnArgs &a, int n_tok, hipStream_t st) {
  dim3 grid((unsigned)a.n_splits, (unsigned)(a.n_head_kv * a.n_chunks), (unsigned)n_tok);
  hipLaunchKernelGGL((decode_mfma_kernel<KT, VT, PAIR>), grid, dim3(64 * TileShape<KT, VT>::WAVES),
                     (decode_lds<KT, VT>()), st, a);
  return hipGetLastError();
}

// pair mode is built for the cache types a verify step is likely to use
bool pair_type(int kt, int vt) {
  return (kt == vt && (kt == F16 || kt == Q8_0 || kt == Q4_0 || kt == Q5_0 || kt == Q4_1)) ||
         (kt == Q5_0 && vt == Q4_1);
}

bool hot_k(int t) { return t == F16 || t == Q8_0 || t == Q4_0 || t == Q5_0 || t == Q4_1; }
bool hot_v(int t) { return t == F16 || t == Q8_0 || t == Q4_0 || t == Q5_0 || t == Q4_1; }

}  // namespace

bool decode_mfma_supported(int kt, int vt, int n_head, int n_head_kv, int head_dim) {
  // read per call: the tests switch paths inside one process
  const char *e = std::getenv("RD4_DECODE_GENERIC");
  if (e && std::atoi(e) != 0) return false;
  return hot_k(kt) && hot_v(vt) && head_dim == kHD && n_head_kv > 0 &&
         n_head % n_head_kv == 0;
}

bool decode_mfma_pairs(int kt, int vt) { return pair_type(kt, vt); }

hipError_t decode_mfma_launch(int kt, int vt, const AttnArgs &a0, int n_tok, hipStream_t st) {
  AttnArgs a = a0;
  a.n_chunks = (a.n_head / a.n_head_kv + kG - 1) / kG;
  a.n_tok = n_tok;
  // pair mode needs host positions, f32 queries, no fused append and one head
  // chunk per kv head (the rows of two tokens share one 16-row tile)
  if (a.tok_pair && (a.pos || a.k_new || a.q_f16 || a.n_chunks != 1 || n_tok < 2 ||
                     !pair_type(kt, vt)))
    a.tok_pair = 0;
  // split records are folded by the merge launch on the same stream
  a.ext_merge = a.n_splits > 1 ? 1 : 0;
  const int grid_tok = a.tok_pair ? (n_tok + 1) / 2 : n_tok;
  hipError_t err = hipErrorInvalidValue;
#define RD4_D(K, V) \
  if (kt == K && vt == V && !a.tok_pair) err = launch<K, V>(a, grid_tok, st);
#define RD4_P(K, V) \
  if (kt == K && vt == V && a.tok_pair) err = launch<K, V, true>(a, grid_tok, st);
  RD4_P(F16, F16) RD4_P(Q8_0, Q8_0) RD4_P(Q4_0, Q4_0) RD4_P(Q5_0, Q5_0) RD4_P(Q4_1, Q4_1)
  RD4_P(Q5_0, Q4_1)
#undef RD4_P
  RD4_D(F16, F16) RD4_D(F16, Q8_0) RD4_D(F16, Q4_0)
  RD4_D(Q8_0, F16) RD4_D(Q8_0, Q8_0) RD4_D(Q8_0, Q4_0)
  RD4_D(Q4_0, F16) RD4_D(Q4_0, Q8_0) RD4_D(Q4_0, Q4_0)
  RD4_D(Q5_0, F16) RD4_D(Q5_0, Q8_0) RD4_D(Q5_0, Q4_0) RD4_D(Q5_0, Q4_1)
  RD4_D(Q4_1, F16) RD4_D(Q4_1, Q8_0) RD4_D(Q4_1, Q4_0) RD4_D(Q4_1, Q4_1)
  RD4_D(F16, Q4_1) RD4_D(Q8_0, Q4_1) RD4_D(Q4_0, Q4_1)
  RD4_D(F16, Q5_0) RD4_D(Q8_0, Q5_0) RD4_D(Q4_0, Q5_0) RD4_D(Q5_0, Q5_0) RD4_D(Q4_1, Q5_0)
#undef RD4_D
  if (err != hipSuccess || !a.ext_merge) return err;
  return merge_splits_launch(a, n_tok, st);
}

}  // namespace rd4
