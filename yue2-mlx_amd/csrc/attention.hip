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

template <int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeParams p, float scale) {
  __shared__ float q_lds[G][D];        // scaled query (fp32), log2(e) folded in
  __shared__ u32x4 kv_new[2][D / 8];   // current key / value (bf16)
  __shared__ float w_m[4][G], w_l[4][G];
  __shared__ float w_o[4][G][D];
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
    // ---- prologue: q heads (waves 0..), current k, current v ----
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

    // ---- main loop ----
    const int grp = lane >> 4, sub = lane & 15;
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
      u32x4 kr[4], vr[4];
      int key[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        key[i] = t0 + wave * 16 + i * 4 + grp;
        const int kk = min(key[i], pos > 0 ? pos - 1 : 0);
        kr[i] = kc[size_t(kk) * (D / 8) + sub];
        vr[i] = vc[size_t(kk) * (D / 8) + sub];
      }
      float sc[4][G];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (key[i] == pos) {
          kr[i] = kv_new[0][sub];
          vr[i] = kv_new[1][sub];
        }
        float kf[8];
        unpack8(kr[i], kf);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float a = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            a = fmaf(q[h][e], kf[e], a);
          a += __shfl_xor(a, 8, 64);
          a += __shfl_xor(a, 4, 64);
          a += __shfl_xor(a, 2, 64);
          a += __shfl_xor(a, 1, 64);
          sc[i][h] = key[i] < s1 ? a : -__builtin_inff();
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
      p.part_o[(part + s) * (G * D) + e] = o;
      if (d == 0) {
        p.part_ml[((part + s) * G + h) * 2] = M;
        p.part_ml[((part + s) * G + h) * 2 + 1] = l;
      }
    }
  }

  // ---- arrival; the last workgroup of this (b, kv head) merges ----
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&p.counters[b * Hkv + kvh], 1);
    is_last = prev == int(gridDim.x) - 1;
  }
  __syncthreads();
  if (!is_last)
    return;
  __threadfence();
  const int n_active = (L + chunk - 1) / chunk;
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int h = e / D, d = e % D;
    float M = -__builtin_inff();
    for (int t = 0; t < n_active; ++t)
      M = fmaxf(M, p.part_ml[((part + t) * G + h) * 2]);
    float num = 0.f, den = 0.f;
    for (int t = 0; t < n_active; ++t) {
      const float m = p.part_ml[((part + t) * G + h) * 2];
      const float l = p.part_ml[((part + t) * G + h) * 2 + 1];
      const float f = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - M);
      num = fmaf(f, p.part_o[(part + t) * (G * D) + e], num);
      den = fmaf(f, l, den);
    }
    p.out[size_t(b) * p.out_stride + size_t(kvh * G + h) * D + d] = f2bf(num / den);
  }
  if (threadIdx.x == 0)
    atomicExch(&p.counters[b * Hkv + kvh], 0);
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
      p.batch < 1 || p.capacity < 1)
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
