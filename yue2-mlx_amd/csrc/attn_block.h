// Workgroup body of the split-K flash-decode attention (head_dim 128),
// shared by the per-op kernel (attention.hip) and the fused QKV + attention +
// o_proj layer kernel (fused.hip).
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, cache append,
// SDPA with fp32 softmax/accumulation, bf16 output) and ar.cpp:88-91.
//
// Workgroup (s, kvh, b) owns keys [s*chunk, min(L, (s+1)*chunk)) of kv head
// kvh of branch b, L = pos[b] + 1 (chunk a multiple of the 32-key V block),
// and all G = Hq/Hkv query heads sharing that kv head, so each K/V byte is
// read from HBM exactly once per step. The per-split math (prologue, MFMA
// passes, online softmax, wave combine) is attn_core.h. The q/k/v inputs are
// issued first, then the split's first 128-key pass of K/V, so the prologue
// (q/k RMSNorm + RoPE) overlaps the K/V stream; the workgroup whose range
// contains slot pos[b] appends the new K/V once its partials are out. Partials (m, l, o) go to a global
// buffer with write-through stores; the last of the `nsplit` workgroups to
// arrive on a kv head (device-scope counter) merges the splits exactly.
//
// WORDS: q/k/v are activation words of the same launch (gemv_core.h), re-read
// until fresh while the first K/V pass is in flight, and the output is stored
// as activation words; otherwise plain bf16 rows in and out.
// TAGGED (implied by WORDS): the split partials are stored tagged (io.tag32,
// unique per step and layer) without waiting, and the workgroup of split 0
// re-reads them until fresh and merges in the same order as the counter
// merge; otherwise partials are followed by a store-completion wait and a
// device-scope counter whose last arrival merges.
#pragma once
#include "attn_core.h"
#include "common.h"
#include "gemv_core.h"
#include "kernels.h"

namespace yuear {

constexpr int kAttnMaxSplits = 64;

template <int G, int W>
struct AttnShared {
  attn::Lds<G, W> sh;
  float s_w[kAttnMaxSplits][G];  // merge weights
  int is_last;
};

namespace attn_detail {
constexpr int D = attn::D;
// Load coherent at device (agent) scope: served past any stale per-XCD L2 line.
__device__ __forceinline__ float coherent_load(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
}  // namespace attn_detail

using attn_detail::coherent_load;

// Tagged split partials of the fused layer kernel: u32x4 {tag, v0, tag, v1}
// per output pair, then {tag, m, tag, l} per head (kPartVecs per split).
template <int G>
constexpr int part_vecs() { return G * attn::D / 2 + G; }

// Agent-scope write-through 16-byte store (sc1) at vector index i of a
// workgroup-uniform resource.
__device__ __forceinline__ void part_store(__amdgpu_buffer_rsrc_t r, int i, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, uint32_t(i) * 16, 0, 16);
}
__device__ __forceinline__ bool part_fresh(u32x4 v, uint32_t tag) {
  return ((v.x ^ tag) | (v.z ^ tag)) == 0;
}
// The two payload floats of a tagged vector. The elements are copied out by
// value first: this clang reads element 0 when __builtin_bit_cast is applied
// directly to an ext_vector element lvalue.
__device__ __forceinline__ float part_lo(u32x4 v) {
  const uint32_t w = v.y;
  return __builtin_bit_cast(float, w);
}
__device__ __forceinline__ float part_hi(u32x4 v) {
  const uint32_t w = v.w;
  return __builtin_bit_cast(float, w);
}

// Merge of the n_active tagged partials of (b, kv head) by one workgroup,
// the same arithmetic and order as the counter-based merge below. One memory
// round: the (m, l) of all splits (wave w: heads w + W j, lane t: split t)
// and this thread's output pairs of the first kRound splits are re-read
// together until every vector is fresh; further splits (more than kRound) are
// read afterwards. Output: activation words (WORDS) or bf16 pairs at p.out.
template <int G, int W, bool WORDS>
__device__ __forceinline__ void merge_tagged(const AttnDecodeParams &p, int b, int kvh,
                                             size_t part, int n_active, AttnShared<G, W> &sm,
                                             const WordIO &io) {
  constexpr int D = attn::D, NT = 64 * W;
  constexpr int kPairs = G * D / 2;
  constexpr int kRounds = (kPairs + NT - 1) / NT;
  constexpr int kRound = kRounds == 1 ? 24 : 12;  // splits per memory round (registers)
  constexpr int kMergeHeads = (G + W - 1) / W;
  constexpr int kVecs = part_vecs<G>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const u32x4 *pt = io.part + part * kVecs;
  const auto rp = word_rsrc(pt, uint32_t(n_active * kVecs) * 16);
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  float mm[kMergeHeads], ll[kMergeHeads];
  u32x4 ov[kRounds][kRound];
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kMergeHeads; ++j) {
      const int h = min(wave + W * j, G - 1), t = min(lane, n_active - 1);
      const u32x4 v = word_load4(rp, uint32_t(t * kVecs + kPairs + h) * 16);
      ok = ok && part_fresh(v, io.tag32);
      mm[j] = part_lo(v);
      ll[j] = part_hi(v);
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int q = min(int(threadIdx.x) + NT * r, kPairs - 1);
#pragma unroll
      for (int j = 0; j < kRound; ++j) {
        ov[r][j] = word_load4(rp, uint32_t(min(j, n_active - 1) * kVecs + q) * 16);
        ok = ok && part_fresh(ov[r][j], io.tag32);
      }
    }
    if (__syncthreads_and(ok))
      break;
    const bool give_up = threadIdx.x == 0 && wait_expired(io, t0);
    if (__syncthreads_or(give_up))
      break;
    __builtin_amdgcn_s_sleep(1);
  }
  stamp_ready(io, 5);
#pragma unroll
  for (int j = 0; j < kMergeHeads; ++j) {
    const int h = wave + W * j;
    if (h < G) {
      const float w = merge_weight(mm[j], ll[j], lane < n_active);
      if (lane < n_active)
        sm.s_w[lane][h] = w;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int q = min(int(threadIdx.x) + NT * r, kPairs - 1);
    const int h = (2 * q) / D;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      if (j < n_active) {  // sequential over splits
        a0 = fmaf(sm.s_w[j][h], part_lo(ov[r][j]), a0);
        a1 = fmaf(sm.s_w[j][h], part_hi(ov[r][j]), a1);
      }
    }
    for (int j = kRound; j < n_active; ++j) {  // more splits than one round
      u32x4 v;
      for (;;) {
        v = word_load4(rp, uint32_t(j * kVecs + q) * 16);
        if (part_fresh(v, io.tag32) || wait_expired(io, t0))
          break;
        __builtin_amdgcn_s_sleep(1);
      }
      a0 = fmaf(sm.s_w[j][h], part_lo(v), a0);
      a1 = fmaf(sm.s_w[j][h], part_hi(v), a1);
    }
    if (int(threadIdx.x) + NT * r < kPairs) {
      if constexpr (WORDS) {
        const unsigned long long w2 =
            (static_cast<unsigned long long>((io.tag << 16) | f2bf(a1)) << 32) |
            ((io.tag << 16) | f2bf(a0));
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(
                               io.out + size_t(b) * io.out_stride + size_t(kvh * G) * D) + q,
                           w2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        reinterpret_cast<uint32_t *>(p.out + size_t(b) * p.out_stride + size_t(kvh * G) * D)[q] =
            uint32_t(f2bf(a0)) | (uint32_t(f2bf(a1)) << 16);
      }
    }
  }
  stamp_ready(io, 2);
}

template <int G, int W, bool WORDS, bool TAGGED = WORDS>
__device__ __forceinline__ void attn_block(const AttnDecodeParams &p, float scale, int s, int kvh,
                                           int b, int nsplit, AttnShared<G, W> &sm,
                                           const WordIO &io) {
  constexpr int NT = 64 * W;
  constexpr int kHeadsPerWave = (G + 2 + W - 1) / W;  // prologue heads (q heads, k, v)
  constexpr int kPartVecs = part_vecs<G>();
  attn::Lds<G, W> &sh = sm.sh;
  float(&s_w)[kAttnMaxSplits][G] = sm.s_w;
  int &is_last = sm.is_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int D = attn::D;
  const int Hkv = p.kv_heads;
  const int pos = p.pos[b];
  if (pos < 0 || pos >= p.capacity)
    return;  // uniform for the grid slice of this branch: nothing to append
  const int L = pos + 1;
  const int per = (L + p.max_splits - 1) / p.max_splits;
  const int chunk = (per + attn::kBlock - 1) & ~(attn::kBlock - 1);
  const int s0 = s * chunk, s1 = min(L, s0 + chunk);
  const bool active = s0 < s1;
  const size_t head_base = (size_t(b) * Hkv + kvh) * p.capacity;  // slot index base
  const u32x4 *kc = reinterpret_cast<const u32x4 *>(p.k_cache) + head_base * (D / 8);
  const u32x4 *vc = reinterpret_cast<const u32x4 *>(p.v_cache) + head_base * (D / 8);
  const size_t part = (size_t(b) * Hkv + kvh) * p.max_splits;

  if (active) {
    const int last_cached = pos > 0 ? pos - 1 : 0;
    // q/k/v inputs of this wave's heads (h = wave + W j < G + 2) and
    // their norm gains / RoPE rows first, then the first pass of K/V: the
    // prologue waits only for the former (all loads branch-free)
    const uint16_t *row = p.qkv + size_t(b) * p.qkv_stride;
    const uint16_t *cs = p.rope_cos + size_t(pos) * (D / 2);
    const uint16_t *sn = p.rope_sin + size_t(pos) * (D / 2);
    uint32_t pair[kHeadsPerWave];
    unsigned long long wpair[kHeadsPerWave];
    uint32_t wcol[kHeadsPerWave];
    NormRope nr[kHeadsPerWave];
    bool has_gain[kHeadsPerWave];
    const auto rin = WORDS ? word_rsrc(io.in, uint32_t(p.batch * io.in_stride) * 4)
                           : word_rsrc(nullptr, 0);
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; ++j) {
      const int h = min(wave + W * j, G + 1);
      const size_t col = h < G ? size_t(kvh * G + h) * D
                               : size_t(p.heads + (h - G) * Hkv + kvh) * D;
      if constexpr (WORDS) {
        wcol[j] = uint32_t(b * io.in_stride + int(col) + 2 * lane) * 4;
        wpair[j] = word_load2(rin, wcol[j]);
      } else {
        pair[j] = reinterpret_cast<const uint32_t *>(row + col)[lane];
      }
      const uint16_t *gain = h < G ? p.q_norm : p.k_norm;
      has_gain[j] = gain != nullptr;
      load_rope(nr[j], cs, sn, lane);
      load_gain(nr[j], has_gain[j] ? gain : cs, lane);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the prologue inputs ahead of K/V
    u32x4 kr[8], vr[8];
    attn::load_k(kc, s0, wave, lane, last_cached, kr);
    attn::load_v(vc, s0, wave, lane, last_cached, vr);
    if constexpr (WORDS) {
      // q/k/v words of this launch: re-read until every one is fresh (the
      // K/V of the first pass are already in flight)
      const long long t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < kHeadsPerWave; ++j)
          ok = ok && word_fresh(uint32_t(wpair[j]), io.tag) &&
               word_fresh(uint32_t(wpair[j] >> 32), io.tag);
        if (__all(ok))
          break;
        bool give_up = false;
        if (lane == 0)
          give_up = wait_expired(io, t0);
        if (__any(give_up))
          break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < kHeadsPerWave; ++j)
          wpair[j] = word_load2(rin, wcol[j]);
      }
#pragma unroll
      for (int j = 0; j < kHeadsPerWave; ++j)
        pair[j] = (uint32_t(wpair[j]) & 0xffffu) | (uint32_t(wpair[j] >> 32) << 16);
      stamp_ready(io);
    }

    // ---- prologue: q heads, current k, current v ----
    if constexpr (WORDS)
      stamp_ready(io, 6);
    const float qscale = scale * attn::kLog2e;
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; ++j) {
      const int h = wave + W * j;
      if (h < G + 2)
        attn::prologue_head<G>(sh, h, pair[j], has_gain[j], p.eps, nr[j], lane);
    }
    __syncthreads();
    if constexpr (WORDS)
      stamp_ready(io, 1);
    // ---- passes over the split, then the W-wave combine ----
    attn::split<G>(sh, kc, vc, s0, s1, pos, last_cached, lane, wave, qscale, kr, vr);
    __syncthreads();
    if constexpr (TAGGED) {
      stamp_ready(io, 3);
      // tagged partials {tag, o0, tag, o1} per output pair and {tag, m, tag, l}
      // per head, stored without waiting: the merger re-reads until fresh
      const auto pt = word_rsrc(io.part + (part + s) * kPartVecs, kPartVecs * 16);
      for (int q = threadIdx.x; q < G * D / 2; q += NT) {
        float o0, o1, M, l;
        attn::combine<G>(sh, 2 * q, o0, M, l);
        attn::combine<G>(sh, 2 * q + 1, o1, M, l);
        part_store(pt, q, u32x4{io.tag32, __builtin_bit_cast(uint32_t, o0), io.tag32,
                                __builtin_bit_cast(uint32_t, o1)});
        if ((2 * q) % D == 0)
          part_store(pt, G * D / 2 + (2 * q) / D,
                     u32x4{io.tag32, __builtin_bit_cast(uint32_t, M), io.tag32,
                           __builtin_bit_cast(uint32_t, l)});
      }
    } else {
      for (int e = threadIdx.x; e < G * D; e += NT) {
        float o, M, l;
        attn::combine<G>(sh, e, o, M, l);
        // write-through (agent-scope) stores: visible to every XCD once complete
        __hip_atomic_store(&p.part_o[(part + s) * (G * D) + e], o, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (e % D == 0) {
          const int h = e / D;
          __hip_atomic_store(&p.part_ml[((part + s) * G + h) * 2], M, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(&p.part_ml[((part + s) * G + h) * 2 + 1], l, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    // Append of the current token's K/V (ar.cpp:119-123), after the partials:
    // this launch reads the current key from LDS, and a store's source
    // registers cannot be reused before the store completes, so an early
    // append would stall the split on a store round trip.
    if (pos >= s0 && pos < s1 && threadIdx.x < D / 8 + D) {
      if (threadIdx.x < D / 8) {  // K row: 16 bytes per thread
        reinterpret_cast<u32x4 *>(p.k_cache)[(head_base + pos) * (D / 8) + threadIdx.x] =
            sh.kv_new[0][threadIdx.x];
      } else {  // V: one dim per thread into its block column
        const int d = threadIdx.x - D / 8;
        p.v_cache[head_base * D + attn::v_index(pos, d)] =
            reinterpret_cast<const uint16_t *>(&sh.kv_new[1][0])[d];
      }
    }
  }
  if constexpr (TAGGED) {
    stamp_ready(io, 4);
    if (s == 0)
      merge_tagged<G, W, WORDS>(p, b, kvh, part, (L + chunk - 1) / chunk, sm, io);
    return;
  }

  // ---- arrival. Every wave waits for its write-through partial stores to
  // complete (vmcnt(0); a workgroup barrier alone does not wait for memory),
  // then one counter increment per workgroup. The last workgroup of this
  // (b, kv head) reads the partials with agent-scope loads and merges. No
  // cache-wide write-back or invalidate is needed on this path. ----
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&p.counters[b * Hkv + kvh], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == nsplit - 1;
  }
  __syncthreads();
  if (!is_last)
    return;
  const int n_active = (L + chunk - 1) / chunk;
  // One memory round: the (m, l) of all splits first (wave w: heads w + W j,
  // lane t: split t), then thread x's 8-byte partials of outputs (2 q,
  // 2 q + 1), q = x + NT r, for up to kRound splits (clamped to the active
  // ones); the merge weights are formed while the partials arrive.
  constexpr int kPairs = G * D / 2;
  constexpr int kRounds = (kPairs + NT - 1) / NT;
  constexpr int kRound = 32;
  constexpr int kMergeHeads = (G + W - 1) / W;
  float mm[kMergeHeads], ll[kMergeHeads];
#pragma unroll
  for (int j = 0; j < kMergeHeads; ++j) {
    const int h = min(wave + W * j, G - 1), t = min(lane, n_active - 1);
    mm[j] = coherent_load(&p.part_ml[((part + t) * G + h) * 2]);
    ll[j] = coherent_load(&p.part_ml[((part + t) * G + h) * 2 + 1]);
  }
  for (int r = 0; r < kRounds; ++r) {
    const int q = min(int(threadIdx.x) + NT * r, kPairs - 1);
    const unsigned long long *po =
        reinterpret_cast<const unsigned long long *>(p.part_o + part * (G * D)) + q;
    unsigned long long ov[kRound];
#pragma unroll
    for (int j = 0; j < kRound; ++j)
      ov[j] = __hip_atomic_load(po + size_t(min(j, n_active - 1)) * (G * D / 2), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
    if (r == 0) {
#pragma unroll
      for (int j = 0; j < kMergeHeads; ++j) {
        const int h = wave + W * j;
        if (h < G) {
          const float w = merge_weight(mm[j], ll[j], lane < n_active);
          if (lane < n_active)
            s_w[lane][h] = w;
        }
      }
      __syncthreads();
    }
    if (int(threadIdx.x) + NT * r < kPairs) {
      const int h = (2 * q) / D;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int j = 0; j < kRound; ++j) {
        if (j < n_active) {  // sequential over splits
          const float o0 = __builtin_bit_cast(float, uint32_t(ov[j]));
          const float o1 = __builtin_bit_cast(float, uint32_t(ov[j] >> 32));
          a0 = fmaf(s_w[j][h], o0, a0);
          a1 = fmaf(s_w[j][h], o1, a1);
        }
      }
      for (int j = kRound; j < n_active; ++j) {  // more splits than one round
        const unsigned long long v = __hip_atomic_load(po + size_t(j) * (G * D / 2),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a0 = fmaf(s_w[j][h], __builtin_bit_cast(float, uint32_t(v)), a0);
        a1 = fmaf(s_w[j][h], __builtin_bit_cast(float, uint32_t(v >> 32)), a1);
      }
      reinterpret_cast<uint32_t *>(p.out + size_t(b) * p.out_stride + size_t(kvh * G) * D)[q] =
          uint32_t(f2bf(a0)) | (uint32_t(f2bf(a1)) << 16);
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&p.counters[b * Hkv + kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


}  // namespace yuear
