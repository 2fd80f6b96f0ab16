// Split-K flash-decode attention for one layer on gfx950 (head_dim 128).
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, cache append,
// SDPA with fp32 softmax/accumulation, bf16 output) and ar.cpp:88-91.
//
// Grid (max_splits, Hkv, batch), 256 threads. Workgroup (s, h, b) owns keys
// [s*chunk, min(L, (s+1)*chunk)) of kv head h of branch b, L = pos[b] + 1
// (chunk a multiple of the 32-key V block), and
// all G = Hq/Hkv query heads sharing that kv head, so each K/V byte is read
// from HBM exactly once per step. The chunk length is derived on device from
// pos[b], so one captured graph serves every KV length up to capacity.
//
// The per-split math (prologue, MFMA passes, online softmax, wave combine) is
// attn_core.h, shared with the persistent step; it also fixes the cache
// layout (K row-major, V in dim-major 32-key blocks). Here: the q/k/v inputs are
// issued first, then the split's first 128-key pass of K/V, so the prologue
// (q/k RMSNorm + RoPE) overlaps the K/V stream; the workgroup whose range
// contains slot pos[b] appends the new K/V. Partials (m, l, o) go to a
// global buffer with write-through stores; the last workgroup to arrive on a
// kv head (device-scope counter) merges the splits exactly and writes bf16.
#include <cmath>

#include "attn_core.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int D = attn::D;
constexpr int kMaxSplits = 64;
constexpr int kWaves = 4;  // 128 keys per pass (8 waves measured no faster on MI355X)

// Load coherent at device (agent) scope: served past any stale per-XCD L2 line.
__device__ __forceinline__ float coherent_load(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int G, int W>
__global__ __launch_bounds__(64 * W) void attn_decode_kernel(AttnDecodeParams p, float scale) {
  constexpr int NT = 64 * W;
  constexpr int kHeadsPerWave = (G + 2 + W - 1) / W;  // prologue heads (q heads, k, v)
  __shared__ attn::Lds<G, W> sh;
  __shared__ float s_w[kMaxSplits][G];  // merge weights
  __shared__ int is_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
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
      load_gain(nr[j], has_gain[j] ? gain : cs, lane);
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
    if (pos >= s0 && pos < s1 && threadIdx.x < D / 8 + D) {  // append (ar.cpp:119-123)
      if (threadIdx.x < D / 8) {  // K row: 16 bytes per thread
        reinterpret_cast<u32x4 *>(p.k_cache)[(head_base + pos) * (D / 8) + threadIdx.x] =
            sh.kv_new[0][threadIdx.x];
      } else {  // V: one dim per thread into its block column
        const int d = threadIdx.x - D / 8;
        p.v_cache[head_base * D + attn::v_index(pos, d)] =
            reinterpret_cast<const uint16_t *>(&sh.kv_new[1][0])[d];
      }
    }

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
    is_last = prev == int(gridDim.x) - 1;
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

template <int G>
hipError_t launch_g(const AttnDecodeParams &p, hipStream_t s) {
  const float scale = float(std::pow(double(D), -0.5));  // ar.cpp:283
  hipLaunchKernelGGL((attn_decode_kernel<G, kWaves>), dim3(p.max_splits, p.kv_heads, p.batch),
                     dim3(64 * kWaves), 0,
                     s, p, scale);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_decode(const AttnDecodeParams &p, hipStream_t s) {
  if (p.head_dim != D || p.kv_heads < 1 || p.heads % p.kv_heads || p.max_splits < 1 ||
      p.max_splits > kMaxSplits || p.batch < 1 || p.capacity < 1 ||
      p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  switch (p.heads / p.kv_heads) {
  case 1: return launch_g<1>(p, s);
  case 2: return launch_g<2>(p, s);
  case 3: return launch_g<3>(p, s);
  case 4: return launch_g<4>(p, s);
  case 6: return launch_g<6>(p, s);
  case 8: return launch_g<8>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace yuear
