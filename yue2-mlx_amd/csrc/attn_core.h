// Split-K decode attention core for head_dim 128 on gfx950, shared by the
// per-op kernel (attention.hip) and the persistent step (decode.hip): both
// call these functions, so the two decode paths compute the same bits.
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, SDPA with fp32
// softmax and accumulation) and ar.cpp:88-91.
//
// A workgroup (4 waves) owns keys [s0, s1) of one kv head and the G query
// heads sharing it. A pass covers kPass = 128 keys: wave w takes keys
// t0 + 32 w + [0, 32), its four 16-lane groups one key row each per step
// (row i of group g is key t0 + 32 w + 4 i + g), each lane 8 of the 128
// dims, so a wave-wide load is 1 KiB of 4 consecutive key rows. Scores and
// the online softmax run in fp32 with log2(e) folded into q (exp2).
#pragma once
#include "common.h"

namespace yuear {
namespace attn {

constexpr int D = 128;
constexpr int kRows = 8;                  // key rows per lane group per pass
constexpr int kPass = 4 * 4 * kRows;      // keys per workgroup pass
constexpr float kLog2e = 1.4426950408889634f;

template <int G>
struct Lds {
  float q[G][D];            // normalised, rotated, scaled q (fp32)
  u32x4 kv_new[2][D / 8];   // current key / value (bf16)
  float w_m[4][G], w_l[4][G];
  float w_o[4][G][D];
};

__device__ __forceinline__ int key_of(int t0, int wave, int i, int grp) {
  return t0 + wave * (4 * kRows) + i * 4 + grp;
}

__device__ __forceinline__ void unpack8(u32x4 v, float *f) {
  f[0] = bflo(v.x); f[1] = bfhi(v.x);
  f[2] = bflo(v.y); f[3] = bfhi(v.y);
  f[4] = bflo(v.z); f[5] = bfhi(v.z);
  f[6] = bflo(v.w); f[7] = bfhi(v.w);
}

// Keys of a pass (all K rows first, then all V rows, so that the scores wait
// only for K). Keys at or beyond the current slot come from LDS or are
// masked; the clamp keeps every address inside the written part of the
// cache (last_cached = max(pos - 1, 0)).
__device__ __forceinline__ void load_k(const u32x4 *kc, int t0, int wave, int grp, int sub,
                                       int last_cached, u32x4 (&kr)[kRows]) {
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    kr[i] = kc[size_t(min(key_of(t0, wave, i, grp), last_cached)) * (D / 8) + sub];
}
__device__ __forceinline__ void load_v(const u32x4 *vc, int t0, int wave, int grp, int sub,
                                       int last_cached, u32x4 (&vr)[kRows]) {
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    vr[i] = vc[size_t(min(key_of(t0, wave, i, grp), last_cached)) * (D / 8) + sub];
}

// Prologue for head h of the workgroup (h < G: query head, h == G: key,
// h == G + 1: value), one head per wave, lane l holding dims 2l and 2l + 1:
// RMSNorm with the q/k gain and half-split RoPE (ar.cpp:268-277), then LDS.
template <int G, class GainPtr>
__device__ __forceinline__ void prologue_head(Lds<G> &sh, int h, uint32_t pair, GainPtr gain,
                                              float eps, const uint16_t *cs, const uint16_t *sn,
                                              float qscale, int lane) {
  float y0 = bflo(pair), y1 = bfhi(pair);
  if (h <= G)
    norm_rope_head(y0, y1, gain, eps, cs, sn, lane, y0, y1);
  if (h < G) {
    sh.q[h][2 * lane] = y0 * qscale;
    sh.q[h][2 * lane + 1] = y1 * qscale;
  } else {
    reinterpret_cast<uint32_t *>(&sh.kv_new[h - G][0])[lane] =
        uint32_t(f2bf(y0)) | (uint32_t(f2bf(y1)) << 16);
  }
}

// One pass over keys [t0, t0 + kPass) ∩ [s0, s1) with the online softmax
// state of this lane (m, l per head; o: 8 dims per head). kr / vr hold the
// pass's rows on entry; when `more`, the next pass's K rows are issued into
// kr as soon as the scores are formed, and its V rows into vr after P.V.
template <int G>
__device__ __forceinline__ void pass(const Lds<G> &sh, const u32x4 *kc, const u32x4 *vc, int t0,
                                     int s1, int pos, int last_cached, bool more, int wave,
                                     int grp, int sub, u32x4 (&kr)[kRows], u32x4 (&vr)[kRows],
                                     float (&m_run)[G], float (&l_run)[G], float (&o_run)[G][8]) {
  float sc[kRows][G];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int key = key_of(t0, wave, i, grp);
    if (key == pos)
      kr[i] = sh.kv_new[0][sub];
    float kf[8];
    unpack8(kr[i], kf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float *q = &sh.q[h][sub * 8];  // LDS broadcast within a lane group
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        acc = fmaf(q[e], kf[e], acc);
      acc = row_sum16(acc);  // the 16 lanes of this key row
      sc[i][h] = key < s1 ? acc : -__builtin_inff();
    }
  }
  if (more)
    load_k(kc, t0 + kPass, wave, grp, sub, last_cached, kr);
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    if (key_of(t0, wave, i, grp) == pos)
      vr[i] = sh.kv_new[1][sub];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mx = sc[0][h];
#pragma unroll
    for (int i = 1; i < kRows; ++i)
      mx = fmaxf(mx, sc[i][h]);
    mx = max_halves(max_row_pairs(mx));  // over the 4 lane groups
    const float m_new = fmaxf(m_run[h], mx);
    if (m_new == -__builtin_inff())
      continue;  // nothing visible yet in this wave
    const float corr = __builtin_amdgcn_exp2f(m_run[h] - m_new);
    float lsum = 0.f;
    float pw[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      pw[i] = __builtin_amdgcn_exp2f(sc[i][h] - m_new);
      lsum += pw[i];
    }
    l_run[h] = l_run[h] * corr + lsum;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o_run[h][e] *= corr;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      float vf[8];
      unpack8(vr[i], vf);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o_run[h][e] = fmaf(pw[i], vf[e], o_run[h][e]);
    }
    m_run[h] = m_new;
  }
  if (more)
    load_v(vc, t0 + kPass, wave, grp, sub, last_cached, vr);
}

// All passes of [s0, s1) for this wave, starting from kr / vr holding the
// first pass; leaves the wave's (m, l, o) in LDS (w_m, w_l, w_o).
template <int G>
__device__ __forceinline__ void split(Lds<G> &sh, const u32x4 *kc, const u32x4 *vc, int s0,
                                      int s1, int pos, int last_cached, int lane, int wave,
                                      u32x4 (&kr)[kRows], u32x4 (&vr)[kRows]) {
  const int grp = lane >> 4, sub = lane & 15;
  float m_run[G], l_run[G], o_run[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -__builtin_inff();
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o_run[h][e] = 0.f;
  }
  for (int t0 = s0;; t0 += kPass) {
    const bool more = t0 + kPass < s1;  // uniform
    pass<G>(sh, kc, vc, t0, s1, pos, last_cached, more, wave, grp, sub, kr, vr, m_run, l_run,
            o_run);
    if (!more)
      break;
  }
  // reduce the four 16-lane groups of the wave
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float l = sum_halves(sum_row_pairs(l_run[h]));
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o_run[h][e] = sum_halves(sum_row_pairs(o_run[h][e]));
    if (lane < 16) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        sh.w_o[wave][h][sub * 8 + e] = o_run[h][e];
    }
    if (lane == 0) {
      sh.w_m[wave][h] = m_run[h];
      sh.w_l[wave][h] = l;
    }
  }
}

// Combine the four waves for element e = h * D + d of the split partial
// (after a barrier): running max M, weighted o and l.
template <int G>
__device__ __forceinline__ void combine(const Lds<G> &sh, int e, float &o, float &M,
                                        float &lsum) {
  const int h = e / D, d = e % D;
  M = fmaxf(fmaxf(sh.w_m[0][h], sh.w_m[1][h]), fmaxf(sh.w_m[2][h], sh.w_m[3][h]));
  o = 0.f;
  lsum = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f =
        sh.w_m[w][h] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(sh.w_m[w][h] - M);
    o = fmaf(f, sh.w_o[w][h][d], o);
    lsum = fmaf(f, sh.w_l[w][h], lsum);
  }
}

}  // namespace attn
}  // namespace yuear
