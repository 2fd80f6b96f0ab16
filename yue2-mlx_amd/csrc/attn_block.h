// Workgroup body of the split-K flash-decode attention (head_dim 128).
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, cache append,
// SDPA with fp32 softmax/accumulation, bf16 output) and ar.cpp:88-91.
//
// Workgroup (s, bh) owns keys [s*chunk, min(L, (s+1)*chunk)) of kv head kvh
// of branch b (bh = b * Hkv + kvh), L = pos[b] + 1, chunk a multiple of the
// 32-key V block, and all G = Hq/Hkv query heads sharing that kv head, so
// each K/V byte is read from HBM exactly once per step. The per-split math
// (prologue, MFMA passes, online softmax, wave combine) is attn_core.h. The
// q/k/v inputs are issued first, then every K/V operand of the split's first
// pass (with chunk <= 32 W keys the whole split is in flight at once), so
// the q/k RMSNorm + RoPE prologue overlaps the K/V stream; the workgroup
// whose range contains slot pos[b] appends the new K/V once its partials are
// out. Partials (m, l, o) go to a global buffer with write-through stores;
// the last of the `nsplit` workgroups to arrive on (b, kvh) (device-scope
// counter) reads them back from memory (agent-scope loads) and merges the
// splits exactly.
#pragma once
#include "attn_core.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

constexpr int kAttnMaxSplits = 64;

template <int G, int W>
struct AttnShared {
  attn::Lds<G, W> sh;
  alignas(16) float s_w[G][kAttnMaxSplits];  // merge weights per head, 0 past the active splits
  int is_last;
};

// Loads of the split partials past any stale per-XCD L2 line (sc1): the
// partials were written by workgroups on other XCDs with write-through stores.
__device__ __forceinline__ unsigned long long part_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16);
  return (static_cast<unsigned long long>(v.y) << 32) | v.x;
}
__device__ __forceinline__ float part_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 16));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

template <int G, int W>
__device__ __forceinline__ void attn_block(const AttnDecodeParams &p, float scale, int s, int bh,
                                           int nsplit, AttnShared<G, W> &sm) {
  constexpr int NT = 64 * W;
  constexpr int kHeadsPerWave = (G + 2 + W - 1) / W;  // prologue heads (q heads, k, v)
  attn::Lds<G, W> &sh = sm.sh;

  // the wave index is uniform: as a scalar, the per-wave head choice below
  // selects kernel arguments instead of loading them through a vector address
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int D = attn::D;
  const int Hkv = p.kv_heads;
  const int b = bh / Hkv, kvh = bh % Hkv;
  const int pos = p.pos[b];
  if (pos < 0 || pos >= p.capacity)
    return;  // uniform for the grid slice of this branch: nothing to append
  const int L = pos + 1;
  const int per = (L + nsplit - 1) / nsplit;
  const int chunk = (per + attn::kBlock - 1) & ~(attn::kBlock - 1);
  const int s0 = s * chunk, s1 = min(L, s0 + chunk);
  const bool active = s0 < s1;
  const size_t head_base = size_t(bh) * p.capacity;  // slot index base
  const u32x4 *kc = reinterpret_cast<const u32x4 *>(p.k_cache) + head_base * (D / 8);
  const u32x4 *vc = reinterpret_cast<const u32x4 *>(p.v_cache) + head_base * (D / 8);
  const size_t part = size_t(bh) * p.max_splits;

  if (active) {
    const int last_cached = pos > 0 ? pos - 1 : 0;
    // q/k/v inputs of this wave's heads (h = wave + W j < G + 2) and their
    // norm gains / RoPE rows first, then the first pass of K/V: the prologue
    // waits only for the former (all loads branch-free)
    const uint16_t *row = p.qkv + size_t(b) * p.qkv_stride;
    const uint16_t *cs = p.rope_cos + size_t(pos) * (D / 2);
    const uint16_t *sn = p.rope_sin + size_t(pos) * (D / 2);
    uint32_t pair[kHeadsPerWave];
    NormRope nr[kHeadsPerWave];
    bool has_gain[kHeadsPerWave];
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; ++j) {
      const int h = min(wave + W * j, G + 1);
      const size_t col = h < G ? size_t(kvh * G + h) * D
                               : size_t(p.heads + (h - G) * Hkv + kvh) * D;
      pair[j] = reinterpret_cast<const uint32_t *>(row + col)[lane];
      const uint16_t *gain = h < G ? p.q_norm : p.k_norm;
      has_gain[j] = gain != nullptr;
      load_rope(nr[j], cs, sn, lane);
      // without a gain the (unused) load reads the head's own 128 inputs,
      // which are always in bounds
      load_gain(nr[j], has_gain[j] ? gain : row + col, lane);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the prologue inputs ahead of K/V
    u32x4 kr[8], vr[8];
    attn::load_k(kc, s0, wave, lane, last_cached, kr);
    attn::load_v(vc, s0, wave, lane, last_cached, vr);

    // ---- prologue: q heads, current k, current v ----
    const float qscale = scale * attn::kLog2e;
#pragma unroll
    for (int j = 0; j < kHeadsPerWave; ++j) {
      const int h = wave + W * j;
      if (h < G + 2)
        attn::prologue_head<G>(sh, h, pair[j], has_gain[j], p.eps, nr[j], lane);
    }
    __syncthreads();
    // ---- passes over the split, then the W-wave combine ----
    attn::split<G>(sh, kc, vc, s0, s1, pos, last_cached, lane, wave, qscale, kr, vr);
    __syncthreads();
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

  // ---- arrival. Every wave waits for its write-through partial stores to
  // complete (vmcnt(0); a workgroup barrier alone does not wait for memory),
  // then one counter increment per workgroup. The last workgroup of this
  // (b, kv head) merges. No cache-wide write-back or invalidate is needed. ----
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&p.counters[bh * kCounterStride], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    sm.is_last = prev == nsplit - 1;
  }
  __syncthreads();
  if (!sm.is_last)
    return;
  const int n_active = (L + chunk - 1) / chunk;
  // One memory round: the (m, l) of all splits (wave w: heads w + W j, lane
  // t: split t) and thread x's 8-byte partials of outputs (2 q, 2 q + 1),
  // q = x + NT r, of every active split; the merge weights are formed while
  // the partials arrive and go to LDS per head ([G][splits], zero past the
  // active splits), so the weighted sum reads them four at a time and runs
  // without branches (adding 0 * 0 leaves the sum unchanged).
  constexpr int kPairs = G * D / 2;
  constexpr int kRounds = (kPairs + NT - 1) / NT;
  constexpr int kRound = kAttnMaxSplits;
  constexpr int kMergeHeads = (G + W - 1) / W;
  const auto rml = part_rsrc(p.part_ml + part * G * 2, uint32_t(n_active * G * 2) * 4);
  const auto ro = part_rsrc(p.part_o + part * (G * D), uint32_t(n_active * G * D) * 4);
  float mm[kMergeHeads], ll[kMergeHeads];
#pragma unroll
  for (int j = 0; j < kMergeHeads; ++j) {
    const int h = min(wave + W * j, G - 1), t = min(lane, n_active - 1);
    mm[j] = part_load1(rml, uint32_t((t * G + h) * 2) * 4);
    ll[j] = part_load1(rml, uint32_t((t * G + h) * 2 + 1) * 4);
  }
  for (int r = 0; r < kRounds; ++r) {
    const int q = min(int(threadIdx.x) + NT * r, kPairs - 1);
    unsigned long long ov[kRound];
#pragma unroll
    for (int j = 0; j < kRound; ++j)
      ov[j] = j < n_active ? part_load2(ro, uint32_t(j * (G * D) + 2 * q) * 4) : 0ull;
    if (r == 0) {
#pragma unroll
      for (int j = 0; j < kMergeHeads; ++j) {
        const int h = wave + W * j;
        if (h < G) {
          const float w = merge_weight(mm[j], ll[j], lane < n_active);
          sm.s_w[h][lane] = lane < n_active ? w : 0.f;
        }
      }
      __syncthreads();
    }
    if (int(threadIdx.x) + NT * r < kPairs) {
      const int h = (2 * q) / D;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int j4 = 0; j4 < kRound / 4; ++j4) {
        if (4 * j4 >= n_active)  // uniform: the rest adds 0 * 0
          break;
        const float4 w4 = reinterpret_cast<const float4 *>(&sm.s_w[h][0])[j4];
        const float wj[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // sequential over splits
          const unsigned long long v = ov[4 * j4 + t];
          a0 = fmaf(wj[t], __builtin_bit_cast(float, uint32_t(v)), a0);
          a1 = fmaf(wj[t], __builtin_bit_cast(float, uint32_t(v >> 32)), a1);
        }
      }
      reinterpret_cast<uint32_t *>(p.out + size_t(b) * p.out_stride + size_t(kvh * G) * D)[q] =
          uint32_t(f2bf(a0)) | (uint32_t(f2bf(a1)) << 16);
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&p.counters[bh * kCounterStride], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace yuear
