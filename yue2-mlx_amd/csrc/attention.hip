// Split-K flash-decode attention for one layer on gfx950 (head_dim 128).
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, cache append,
// SDPA with fp32 softmax/accumulation, bf16 output) and ar.cpp:88-91.
//
// Grid (max_splits, Hkv, batch), 256 threads. Workgroup (s, h, b) owns keys
// [s*chunk, min(L, (s+1)*chunk)) of kv head h of branch b, L = pos[b] + 1, and
// all G = Hq/Hkv query heads sharing that kv head, so each K/V byte is read
// from HBM exactly once per step. The chunk length is derived on device from
// pos[b], so one captured graph serves every KV length up to capacity.
//
// Prologue: every workgroup normalises and rotates its G query heads and the
// current key in registers (q_norm/k_norm and the half-split RoPE with the
// reference's bf16 rounding points); the workgroup whose range contains slot
// pos[b] appends the new K/V to the cache and takes that key from LDS.
//
// Main loop: 64 keys per pass, 16 per wave; a 16-lane group reads one 256-byte
// key row per 16-byte lane load, four rows per wave-wide load (1 KiB
// contiguous). Online softmax in fp32 (exp2 with log2(e) folded into q).
// Partials (m, l, o) go to a global buffer; the last workgroup to arrive on a
// kv head (device-scope counter) merges the splits exactly and writes bf16.
#include <cmath>

#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int D = 128;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ void unpack8(u32x4 v, float *f) {
  f[0] = bflo(v.x); f[1] = bfhi(v.x);
  f[2] = bflo(v.y); f[3] = bfhi(v.y);
  f[4] = bflo(v.z); f[5] = bfhi(v.z);
  f[6] = bflo(v.w); f[7] = bfhi(v.w);
}

constexpr int kMaxSplits = 64;

// s_waitcnt vmcnt(0): this wave's outstanding vector memory operations
// (including stores) have completed. gfx9 encoding: vmcnt in bits [3:0] and
// [15:14] (zero here), expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 (no wait).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Load coherent at device (agent) scope: served past any stale per-XCD L2 line.
__device__ __forceinline__ float coherent_load(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void load_tile(const u32x4 *kc, const u32x4 *vc, int t0, int wave,
                                          int grp, int sub, int last_cached, u32x4 *kr,
                                          u32x4 *vr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // keys at or beyond the current slot come from LDS (or are masked); the
    // clamp keeps every address inside the written part of the cache
    const int kk = min(t0 + wave * 16 + i * 4 + grp, last_cached);
    kr[i] = kc[size_t(kk) * (D / 8) + sub];
    vr[i] = vc[size_t(kk) * (D / 8) + sub];
  }
}

template <int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeParams p, float scale) {
  __shared__ float q_lds[G][D];        // scaled query (fp32), log2(e) folded in
  __shared__ u32x4 kv_new[2][D / 8];   // current key / value (bf16)
  __shared__ float w_m[4][G], w_l[4][G];
  __shared__ float w_o[4][G][D];
  __shared__ float s_m[kMaxSplits][G], s_w[kMaxSplits][G], s_den[G];
  __shared__ int is_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int Hkv = p.kv_heads;
  const int pos = p.pos[b];
  if (pos < 0 || pos >= p.capacity)
    return;  // uniform for the grid slice of this branch: nothing to append
  const int L = pos + 1;
  const int per = (L + p.max_splits - 1) / p.max_splits;
  const int chunk = (per + 15) & ~15;
  const int s0 = s * chunk, s1 = min(L, s0 + chunk);
  const bool active = s0 < s1;
  const size_t head_base = (size_t(b) * Hkv + kvh) * p.capacity;  // row index base
  const u32x4 *kc = reinterpret_cast<const u32x4 *>(p.k_cache) + head_base * (D / 8);
  const u32x4 *vc = reinterpret_cast<const u32x4 *>(p.v_cache) + head_base * (D / 8);
  const size_t part = (size_t(b) * Hkv + kvh) * p.max_splits;

  if (active) {
    const int grp = lane >> 4, sub = lane & 15;
    const int last_cached = pos > 0 ? pos - 1 : 0;
    // first K/V tile in flight before the prologue's dependent work
    u32x4 kr[4], vr[4];
    load_tile(kc, vc, s0, wave, grp, sub, last_cached, kr, vr);

    // ---- prologue: q heads, current k, current v ----
    const uint16_t *row = p.qkv + size_t(b) * p.qkv_stride;
    const uint16_t *cs = p.rope_cos + size_t(pos) * (D / 2);
    const uint16_t *sn = p.rope_sin + size_t(pos) * (D / 2);
    for (int h = wave; h < G + 2; h += 4) {
      const uint16_t *src;
      if (h < G)
        src = row + size_t(kvh * G + h) * D;
      else if (h == G)
        src = row + size_t(p.heads) * D + size_t(kvh) * D;
      else
        src = row + size_t(p.heads + Hkv) * D + size_t(kvh) * D;
      const uint32_t pair = reinterpret_cast<const uint32_t *>(src)[lane];
      float y0 = bflo(pair), y1 = bfhi(pair);
      if (h <= G)
        norm_rope_head(y0, y1, h < G ? p.q_norm : p.k_norm, p.eps, cs, sn, lane, y0, y1);
      if (h < G) {
        q_lds[h][2 * lane] = y0 * (scale * kLog2e);
        q_lds[h][2 * lane + 1] = y1 * (scale * kLog2e);
      } else {
        reinterpret_cast<uint32_t *>(&kv_new[h - G][0])[lane] =
            uint32_t(f2bf(y0)) | (uint32_t(f2bf(y1)) << 16);
      }
    }
    __syncthreads();
    if (pos >= s0 && pos < s1 && threadIdx.x < 2 * (D / 8)) {  // append (ar.cpp:119-123)
      const int which = threadIdx.x / (D / 8), c = threadIdx.x % (D / 8);
      u32x4 *dst = reinterpret_cast<u32x4 *>(which ? p.v_cache : p.k_cache) +
                   (head_base + pos) * (D / 8) + c;
      *dst = kv_new[which][c];
    }

    // ---- main loop: 64 keys per pass, next tile prefetched ----
    float q[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        q[h][e] = q_lds[h][sub * 8 + e];
    float m_run[G], l_run[G], o_run[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m_run[h] = -__builtin_inff();
      l_run[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o_run[h][e] = 0.f;
    }
    for (int t0 = s0; t0 < s1; t0 += 64) {
      u32x4 kn[4], vn[4];
      load_tile(kc, vc, t0 + 64, wave, grp, sub, last_cached, kn, vn);
      float sc[4][G];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = t0 + wave * 16 + i * 4 + grp;
        if (key == pos) {
          kr[i] = kv_new[0][sub];
          vr[i] = kv_new[1][sub];
        }
        float kf[8];
        unpack8(kr[i], kf);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            acc = fmaf(q[h][e], kf[e], acc);
          acc += __shfl_xor(acc, 8, 64);
          acc += __shfl_xor(acc, 4, 64);
          acc += __shfl_xor(acc, 2, 64);
          acc += __shfl_xor(acc, 1, 64);
          sc[i][h] = key < s1 ? acc : -__builtin_inff();
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float mx = fmaxf(fmaxf(sc[0][h], sc[1][h]), fmaxf(sc[2][h], sc[3][h]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[h], mx);
        if (m_new == -__builtin_inff())
          continue;  // nothing visible yet in this wave
        const float corr = __builtin_amdgcn_exp2f(m_run[h] - m_new);
        float lsum = 0.f;
        float pw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pw[i] = __builtin_amdgcn_exp2f(sc[i][h] - m_new);
          lsum += pw[i];
        }
        l_run[h] = l_run[h] * corr + lsum;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          o_run[h][e] *= corr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float vf[8];
          unpack8(vr[i], vf);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            o_run[h][e] = fmaf(pw[i], vf[e], o_run[h][e]);
        }
        m_run[h] = m_new;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kr[i] = kn[i];
        vr[i] = vn[i];
      }
    }
    // reduce the four 16-lane groups of the wave
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float l = l_run[h];
      l += __shfl_xor(l, 16, 64);
      l += __shfl_xor(l, 32, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float o = o_run[h][e];
        o += __shfl_xor(o, 16, 64);
        o += __shfl_xor(o, 32, 64);
        o_run[h][e] = o;
      }
      if (lane < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          w_o[wave][h][sub * 8 + e] = o_run[h][e];
      }
      if (lane == 0) {
        w_m[wave][h] = m_run[h];
        w_l[wave][h] = l;
      }
    }
    __syncthreads();
    // merge the four waves; write the split partial
    for (int e = threadIdx.x; e < G * D; e += 256) {
      const int h = e / D, d = e % D;
      float M = fmaxf(fmaxf(w_m[0][h], w_m[1][h]), fmaxf(w_m[2][h], w_m[3][h]));
      float o = 0.f, l = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = w_m[w][h] == -__builtin_inff() ? 0.f
                                                        : __builtin_amdgcn_exp2f(w_m[w][h] - M);
        o = fmaf(f, w_o[w][h][d], o);
        l = fmaf(f, w_l[w][h], l);
      }
      // write-through (agent-scope) stores: visible to every XCD once complete
      __hip_atomic_store(&p.part_o[(part + s) * (G * D) + e], o, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
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
  // One memory round: this thread's partial-o loads (up to kMergeBatch splits
  // per output) are issued together with the (m, l) staging loads.
  constexpr int kMergeBatch = 32;
  constexpr int kOutPerThread = (G * D + 255) / 256;
  float ov[kOutPerThread][kMergeBatch];
#pragma unroll
  for (int r = 0; r < kOutPerThread; ++r) {
    const int e = min(int(threadIdx.x) + 256 * r, G * D - 1);
    const float *po = p.part_o + part * (G * D) + e;
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j)
      ov[r][j] = coherent_load(po + size_t(min(j, n_active - 1)) * (G * D));
  }
  for (int i = threadIdx.x; i < n_active * G; i += 256) {
    const int t = i / G, h = i - t * G;
    s_m[t][h] = coherent_load(&p.part_ml[((part + t) * G + h) * 2]);
    s_w[t][h] = coherent_load(&p.part_ml[((part + t) * G + h) * 2 + 1]);  // l, made a weight below
  }
  __syncthreads();
  if (threadIdx.x < G) {
    const int h = threadIdx.x;
    float M = -__builtin_inff();
    for (int t = 0; t < n_active; ++t)
      M = fmaxf(M, s_m[t][h]);
    float den = 0.f;
    for (int t = 0; t < n_active; ++t) {
      const float f = s_m[t][h] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(s_m[t][h] - M);
      s_m[t][h] = f;
      den = fmaf(f, s_w[t][h], den);
    }
    s_den[h] = den;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_active * G; i += 256) {
    const int t = i / G, h = i - t * G;
    s_w[t][h] = s_m[t][h] / s_den[h];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kOutPerThread; ++r) {
    const int e = int(threadIdx.x) + 256 * r;
    if (e >= G * D)
      break;
    const int h = e / D;
    const float *po = p.part_o + part * (G * D) + e;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j)
      acc = j < n_active ? fmaf(s_w[j][h], ov[r][j], acc) : acc;
    for (int t = kMergeBatch; t < n_active; ++t)  // more than kMergeBatch splits
      acc = fmaf(s_w[t][h], coherent_load(po + size_t(t) * (G * D)), acc);
    p.out[size_t(b) * p.out_stride + size_t(kvh * G) * D + e] = f2bf(acc);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&p.counters[b * Hkv + kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int G>
hipError_t launch_g(const AttnDecodeParams &p, hipStream_t s) {
  const float scale = float(std::pow(double(D), -0.5));  // ar.cpp:283
  hipLaunchKernelGGL(attn_decode_kernel<G>, dim3(p.max_splits, p.kv_heads, p.batch), dim3(256), 0,
                     s, p, scale);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_decode(const AttnDecodeParams &p, hipStream_t s) {
  if (p.head_dim != D || p.kv_heads < 1 || p.heads % p.kv_heads || p.max_splits < 1 ||
      p.max_splits > kMaxSplits || p.batch < 1 || p.capacity < 1)
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
