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
// output. The records live in uncached device memory, so CTAs on different XCDs
// (whose L2s are not coherent with each other) exchange them with plain 16-byte
// loads and stores; a writer only waits for its stores to complete before the
// counter increment, and a merger issues all of its record loads at once.
#pragma once
#include "attn_generic.hpp"

namespace rd4 {

constexpr int kMergeFan = 16;
constexpr int kCtrStride = 1 + kMaxSplits / kMergeFan;  // level-2 + level-1 counters
constexpr int kGMaxMerge = 8;

// Wait until this thread's vector memory stores are acknowledged; also a
// compiler barrier for memory.
__device__ __forceinline__ void stores_done() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float sigmoid_dev(float x) { return 1.0f / (1.0f + expf(-x)); }

// Fold n (<= kMergeFan) records per head for G heads. acc: head 0's first
// record, heads acc_hs floats apart, records hd floats apart; ml likewise with
// (m, l) pairs. final: normalize, gate and write a.out/a.gate at qoff; else
// write one record per head to dacc/dml. w_s: LDS [kGMaxMerge][kMergeFan];
// ml_s: LDS [kGMaxMerge][2]. All NT threads of the CTA call it.
template <int NT>
__device__ __forceinline__ void merge_records(const float *acc, const float *ml, int64_t acc_hs,
                                              int64_t ml_hs, int n, int G, int hd, bool final,
                                              const AttnArgs &a, int64_t qoff, float *dacc,
                                              float *dml, int64_t dacc_hs, int64_t dml_hs,
                                              float *w_s, float *ml_s) {
  const int tid = threadIdx.x;
  // Record loads first (one item of 4 dims per thread when G*hd/4 <= NT), so the
  // (m, l) round trip and the record round trip overlap.
  const int nq = hd / 4;
  const int it0 = tid;
  const bool have0 = it0 < G * nq;
  const int g0 = have0 ? it0 / nq : 0, d0 = have0 ? 4 * (it0 - g0 * nq) : 0;
  float4 v0[kMergeFan];
  {
    const float *r = acc + g0 * acc_hs + d0;
#pragma unroll
    for (int si = 0; si < kMergeFan; ++si)
      v0[si] = (have0 && si < n) ? *(const float4 *)(r + (int64_t)si * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid < kGMaxMerge * kMergeFan) {
    const int g = tid / kMergeFan, si = tid % kMergeFan;
    const bool on = g < G && si < n;
    const float ms = on ? ml[g * ml_hs + 2 * si] : -INFINITY;
    const float ls = on ? ml[g * ml_hs + 2 * si + 1] : 0.0f;
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
    dml[tid * dml_hs] = ml_s[2 * tid];
    dml[tid * dml_hs + 1] = ml_s[2 * tid + 1];
  }
  for (int it = tid; it < G * nq; it += NT) {
    const int g = it / nq, d = 4 * (it - g * nq);
    float4 v[kMergeFan];
    if (it == it0) {
#pragma unroll
      for (int si = 0; si < kMergeFan; ++si) v[si] = v0[si];
    } else {
      const float *r = acc + g * acc_hs + d;
#pragma unroll
      for (int si = 0; si < kMergeFan; ++si)
        v[si] = si < n ? *(const float4 *)(r + (int64_t)si * hd) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int si = 0; si < kMergeFan; ++si) {
      const float w = w_s[g * kMergeFan + si];
      o.x += v[si].x * w;
      o.y += v[si].y * w;
      o.z += v[si].z * w;
      o.w += v[si].w * w;
    }
    if (final) {
      const float mm = ml_s[2 * g], L = ml_s[2 * g + 1];
      const float inv = (mm == -INFINITY) ? 0.0f : ((L > 0.0f) ? 1.0f / L : 0.0f);
      float ov[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
      const int64_t oi = qoff + (int64_t)g * hd + d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (a.gate) {
          const float sg = sigmoid_dev(a.gate[oi + i]);
          a.gate[oi + i] = sg;
          ov[i] = ov[i] * sg;
        }
        a.out[oi + i] = ov[i];
      }
    } else {
      *(float4 *)(dacc + g * dacc_hs + d) = o;
    }
  }
}

// Called by every CTA after it has written its level-0 records for heads
// h0..h0+G-1 of token tok, split s. flag: LDS int. Returns after the merge (or
// at once for CTAs that are not the last of their group).
template <int NT>
__device__ __forceinline__ void split_tail(const AttnArgs &a, int tok, int kvh, int hc, int h0,
                                           int G, int s, int *flag, float *w_s, float *ml_s) {
  const int tid = threadIdx.x;
  const int hd = a.head_dim, S = a.n_splits;
  const int NG = (S + kMergeFan - 1) / kMergeFan;
  const int group = s / kMergeFan;
  const int n_in = min(kMergeFan, S - group * kMergeFan);
  unsigned *ctr = a.counters + (((int64_t)tok * a.n_head_kv + kvh) * a.n_chunks + hc) * kCtrStride;

  stores_done();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr + 1 + group, 1u);
    flag[0] = (done == (unsigned)(n_in - 1));
    if (flag[0]) atomicExch(ctr + 1 + group, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;

  const int64_t qoff = ((int64_t)tok * a.n_head + h0) * hd;
  const int64_t hrow = (int64_t)tok * a.n_head + h0;  // first head row of this chunk
  const float *acc0 = a.partial + (hrow * S + group * kMergeFan) * hd;
  const float *ml0 = a.partial + a.ml0_off + (hrow * S + group * kMergeFan) * 2;
  if (NG == 1) {
    merge_records<NT>(acc0, ml0, (int64_t)S * hd, (int64_t)S * 2, n_in, G, hd, true, a, qoff,
                      nullptr, nullptr, 0, 0, w_s, ml_s);
    return;
  }
  float *acc1 = a.partial + a.acc1_off + hrow * NG * hd;
  float *ml1 = a.partial + a.ml1_off + hrow * NG * 2;
  merge_records<NT>(acc0, ml0, (int64_t)S * hd, (int64_t)S * 2, n_in, G, hd, false, a, qoff,
                    acc1 + group * hd, ml1 + group * 2, (int64_t)NG * hd, (int64_t)NG * 2, w_s,
                    ml_s);
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(ctr, 1u);
    flag[0] = (done == (unsigned)(NG - 1));
    if (flag[0]) atomicExch(ctr, 0u);
  }
  __syncthreads();
  if (!flag[0]) return;
  merge_records<NT>(acc1, ml1, (int64_t)NG * hd, (int64_t)NG * 2, NG, G, hd, true, a, qoff,
                    nullptr, nullptr, 0, 0, w_s, ml_s);
}

// Lane exchanges without LDS round trips: DPP within 16-lane rows (xor 1, xor 2,
// then the half-row and row mirrors, which pair the 4- and 8-lane groups), and
// the gfx950 row / half-wave swaps for lanes ^ 16 and ^ 32 (asm with tied
// operands; s_nop 1 covers the VALU-write -> swap-read hazard).
__device__ __forceinline__ float dpp_f(float x, int ctrl_sel) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  switch (ctrl_sel) {  // the DPP control must be a constant
    case 0: r = __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    case 1: r = __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
    case 2: r = __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: r = __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ void swap16(float &a, float &b) {
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float &a, float &b) {
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// max / sum over the 64 lanes of the wave, in every lane
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int c = 0; c < 4; ++c) x = fmaxf(x, dpp_f(x, c));
  float a = x, b = x;
  swap16(a, b);
  float c = fmaxf(a, b), d = c;
  swap32(c, d);
  return fmaxf(c, d);
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int c = 0; c < 4; ++c) x += dpp_f(x, c);
  float a = x, b = x;
  swap16(a, b);
  float c = a + b, d = c;
  swap32(c, d);
  return c + d;
}

// In-kernel slice merge of the MFMA decode (single-token CTAs). Group gi (one
// token's kv head and head chunk: G heads x hd values) has S split CTAs; its
// values are cut into a.merge_slices slices of Z = a.merge_z values (Z % 4 ==
// 0), and CTA s merges slice s. A slice's records are 1 + Z/4 quads per split,
// stored quad-major: float4 mrec[gi][slice][quad][split], quad 0 = {m_a, l_a,
// m_b, l_b} (a: the head of the slice's first value, b: the next head when the
// slice straddles two; m in log2 units), quad 1 + k = values 4k..4k+3. A
// writer's quad is one 16-byte store; a reader's load of one quad for all
// splits is one contiguous run. Every slot holds kPoison until its writer
// stores it; the reader polls until its slots hold no kPoison, merges, and
// stores kPoison back over every slot it read, so the region is all kPoison
// between launches (HIP graph replays included). The region is uncached
// memory: stores reach memory and loads read it, across XCDs. The launcher
// guarantees that all CTAs of the launch are resident at once (grid <= CUs,
// one CTA per CU), so the wait ends.
__device__ __forceinline__ bool is_poison(float x) { return __builtin_bit_cast(uint32_t, x) == kPoison; }
// A relaxed device-scope atomic load: re-issued on every poll (never hoisted
// out of the loop), and several of them fly at once (no wait between them).
__device__ __forceinline__ float poll_load(const float *p) {
  const uint32_t v = __hip_atomic_load((const __attribute__((address_space(1))) uint32_t *)p, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_bit_cast(float, v);
}
__device__ __forceinline__ float *slice_quad(const AttnArgs &a, int gi, int sl, int q, int split) {
  const int nq = 1 + a.merge_z / 4;
  return a.mrec + ((((int64_t)gi * a.merge_slices + sl) * nq + q) * a.n_splits + split) * 4;
}

// Writer: values [v, v+4) of the group (v = head * hd + d, v % 4 == 0) with its
// head's (m, l) of split s.
__device__ __forceinline__ void slice_record_store(const AttnArgs &a, int gi, int s, int v, int hd,
                                                   float4 acc, float m, float l) {
  const int Z = a.merge_z;
  const int sl = v / Z, p = v - sl * Z;
  *(float4 *)slice_quad(a, gi, sl, 1 + p / 4, s) = acc;
  const int d = v % hd;
  if (p == 0 || d == 0) *(float2 *)(slice_quad(a, gi, sl, 0, s) + (p == 0 ? 0 : 2)) = make_float2(m, l);
}

// Reader: CTA s merges slice s of group gi (NT threads, all of them call it).
// Output element (tok, h0 + head, d) of a.out, gated like merge_splits_kernel.
// Wave w takes value quads w, w + NT/64, ...; lane = split.
// (trace: diagnostic builds pass this wave's timestamp slots; slots 28-31 get
// the merge's start, the end of the (m, l) poll, the end of the value loads and
// the end of the merge)
#ifndef RD4_MERGE_SLEEP
#define RD4_MERGE_SLEEP 8
#endif
#ifndef RD4_MERGE_POLL
#define RD4_MERGE_POLL 0
#endif
template <int NT>
__device__ __forceinline__ void slice_merge(const AttnArgs &a, int gi, int tok, int h0, int G, int s,
                                            float *ml_lds, unsigned long long *trace = nullptr) {
  constexpr int kW = NT / 64, kPer = (kInMergeMaxZ / 4 + kW - 1) / kW;
  const int Z = a.merge_z, S = a.n_splits, hd = a.head_dim;
  if (s >= a.merge_slices) return;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int first = s * Z, nv = min(Z, G * hd - first);
  if (nv <= 0) return;  // a head chunk with fewer heads needs fewer slices
  const int nquad = nv / 4;
  const int ha = first / hd, hb = (first + nv - 1) / hd;
  const bool on = lane < S;
  const int sp = on ? lane : 0;
  const float *mlp = slice_quad(a, gi, s, 0, sp);
  float ml[4];
  float4 av[kPer];
  for (int i = 0; i < 4; ++i) ml[i] = 0.0f;
  auto pending_ml = [&]() {
    return on && (is_poison(ml[0]) || is_poison(ml[1]) || (hb != ha && (is_poison(ml[2]) || is_poison(ml[3]))));
  };
  // The gate logits this CTA gates are loaded ahead of the wait.
  float4 gl[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int q = w + kW * k;
    const int v = first + 4 * q, h = v / hd;
    gl[k] = (a.gate && lane == 0 && q < nquad)
                ? *(const float4 *)(a.gate + ((int64_t)tok * a.n_head + h0 + h) * hd + (v - h * hd))
                : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
  bool timed_out = false;
  // 100 MHz realtime clock: give up after 200 ms (never reached when the
  // launcher's residency guarantee holds); the output is then NaN
  auto expired = [&]() { return __builtin_amdgcn_s_memrealtime() - t_start > 20000000ull; };
  auto load_quads = [&]() {
    bool pending = false;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int q = w + kW * k;
      if (q < nquad) {
        const float *qp = slice_quad(a, gi, s, 1 + q, sp);
        av[k] = make_float4(poll_load(qp), poll_load(qp + 1), poll_load(qp + 2), poll_load(qp + 3));
        pending |= on && (is_poison(av[k].x) || is_poison(av[k].y) || is_poison(av[k].z) || is_poison(av[k].w));
      }
    }
    return pending;
  };
#if RD4_MERGE_POLL == 1
  // Every wave polls its value quads (wave 0 also the (m, l) quads) until none
  // holds kPoison, pausing between polls.
  for (;;) {
    bool pending = false;
    if (w == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ml[i] = poll_load(mlp + i);
      pending = pending_ml();
    }
    pending |= load_quads();
    if (!__any(pending)) break;
    if (expired()) {
      timed_out = true;
      break;
    }
    __builtin_amdgcn_s_sleep(RD4_MERGE_SLEEP);
  }
#else
  // Wave 0 polls the (m, l) quads of every split, pausing between polls, while
  // the other waves wait at the barrier and issue nothing (waiting CTAs add
  // little traffic while the last splits still stream their keys). A writer
  // stores its values with its (m, l), so they are then read in one more round
  // trip (and polled again in the rare case they trail their (m, l)).
  // The sigmoids of the gate elements this wave's lane 0 writes are computed
  // while the wave waits (off the path from the last record to the output).
  float4 sg[kPer];
  auto gate_sigmoids = [&]() {
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      sg[k] = make_float4(sigmoid_dev(gl[k].x), sigmoid_dev(gl[k].y), sigmoid_dev(gl[k].z), sigmoid_dev(gl[k].w));
  };
  if (w == 0) {
    bool first = true;
    for (;;) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ml[i] = poll_load(mlp + i);
      if (first && a.gate) gate_sigmoids();  // waits for the gate loads only (issued first)
      first = false;
      if (!__any(pending_ml())) break;
      if (expired()) {
        timed_out = true;
        break;
      }
      __builtin_amdgcn_s_sleep(RD4_MERGE_SLEEP);
    }
  } else if (a.gate) {
    gate_sigmoids();
  }
  // (LDS-only barrier: a plain one would also wait for the gate loads)
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  while (!timed_out && __any(load_quads())) {
    if (expired()) timed_out = true;
    else __builtin_amdgcn_s_sleep(2);
  }
#endif
  // wave 0's (m, l) and time-out flag to every wave through LDS
  if (w == 0) {
    ((float4 *)ml_lds)[lane] = make_float4(ml[0], ml[1], ml[2], ml[3]);
    if (lane == 0) ((int *)ml_lds)[256] = timed_out ? 1 : 0;
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (w != 0) {
    const float4 m4 = ((const float4 *)ml_lds)[lane];
    ml[0] = m4.x;
    ml[1] = m4.y;
    ml[2] = m4.z;
    ml[3] = m4.w;
  }
  timed_out = timed_out || ((const int *)ml_lds)[256] != 0;
  if (trace && lane == 0) trace[28] = __builtin_amdgcn_s_memrealtime();
  const float ma = on ? ml[0] : -INFINITY, la = on ? ml[1] : 0.0f;
  const float mb = (on && hb != ha) ? ml[2] : -INFINITY, lb = (on && hb != ha) ? ml[3] : 0.0f;
  const float Ma = wave_max(ma), Mb = wave_max(mb);
  const float wa = ma == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ma - Ma);
  const float wb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - Mb);
  const float La = wave_sum(wa * la), Lb = wave_sum(wb * lb);
  const float ia = (Ma == -INFINITY || !(La > 0.0f)) ? 0.0f : __builtin_amdgcn_rcpf(La);
  const float ib = (Mb == -INFINITY || !(Lb > 0.0f)) ? 0.0f : __builtin_amdgcn_rcpf(Lb);
  if (trace && lane == 0) trace[29] = __builtin_amdgcn_s_memrealtime() + (uint64_t)(ia + ib > 1e30f);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int q = w + kW * k;
    if (q >= nquad) break;  // wave-uniform
    const int v = first + 4 * q, h = v / hd;  // a quad never straddles heads (hd % 4 == 0)
    const float wt = on ? (h == ha ? wa : wb) : 0.0f;
    const float s0 = wave_sum(wt * av[k].x), s1 = wave_sum(wt * av[k].y);
    const float s2 = wave_sum(wt * av[k].z), s3 = wave_sum(wt * av[k].w);
    if (lane == 0) {
      const int64_t oi = ((int64_t)tok * a.n_head + h0 + h) * hd + (v - h * hd);
      const float inv = h == ha ? ia : ib;
      float o[4] = {s0 * inv, s1 * inv, s2 * inv, s3 * inv};
      if (a.gate) {
        *(float4 *)(a.gate + oi) = sg[k];
        o[0] *= sg[k].x;
        o[1] *= sg[k].y;
        o[2] *= sg[k].z;
        o[3] *= sg[k].w;
      }
      const float nan = __builtin_nanf("");
      *(float4 *)(a.out + oi) = timed_out ? make_float4(nan, nan, nan, nan) : make_float4(o[0], o[1], o[2], o[3]);
    }
  }
  if (trace && lane == 0) trace[30] = __builtin_amdgcn_s_memrealtime();
  // restore kPoison over what this wave read from memory: its value quads, and
  // for wave 0 the (m, l) quads (the other waves took (m, l) from LDS), so no
  // barrier is needed first
  if (on) {
    const float pz = __builtin_bit_cast(float, kPoison);
    const float4 pz4 = make_float4(pz, pz, pz, pz);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int q = w + kW * k;
      if (q < nquad) *(float4 *)slice_quad(a, gi, s, 1 + q, sp) = pz4;
    }
    if (w == 0) *(float4 *)mlp = pz4;
  }
  if (trace && lane == 0) trace[31] = __builtin_amdgcn_s_memrealtime();
}

// Level-0 record of head row `hrow` (= tok * n_head + head), split s.
__device__ __forceinline__ float *rec_acc(const AttnArgs &a, int64_t hrow, int s) {
  return a.partial + (hrow * a.n_splits + s) * a.head_dim;
}
__device__ __forceinline__ float *rec_ml(const AttnArgs &a, int64_t hrow, int s) {
  return a.partial + a.ml0_off + (hrow * a.n_splits + s) * 2;
}

}  // namespace rd4
