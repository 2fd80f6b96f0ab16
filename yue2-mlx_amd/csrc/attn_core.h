// Split-K decode attention core for head_dim 128 on gfx950 MFMA: the
// per-split math of the decode attention kernel (attention.hip, whose
// workgroup body is attn_block.h).
//
// Reference: native/src/ar.cpp:268-291 (q/k RMSNorm, RoPE, SDPA with fp32
// softmax and accumulation) and ar.cpp:88-91.
//
// A workgroup (W waves) owns keys [s0, s1) of one kv head and the G <= 16
// query heads sharing it. A pass covers 32 W keys: wave w takes the 32-key
// block t0 + 32 w. Both products run on v_mfma_f32_16x16x32_bf16 with
// the G heads as the 16 MFMA columns (columns >= G are zero):
//
//   S^T[key][head] = K[key][:] . q[head][:]   two 16-key tiles x 4 k-steps
//   O^T[dim][head] += V^T[dim][key] . P^T[key][head]   8 dim tiles
//
// The rows of the two S^T tiles are permuted (row i of tile T is key
// 8 (i / 4) + 4 T + i % 4 of the block) so that lane (head j, row group r)
// ends up holding the scores of keys 8 r + [0, 8): exactly the B operand of
// P.V, with no data movement between the products. P (fp32) is fed as the
// sum of three bf16 pieces (hi, mid, lo: 24 significant bits, three MFMAs),
// q and K are bf16 already, so every product is exact and every sum is fp32
// like the reference's opmath.
//
// V cache layout (per branch and kv head): blocks of 32 keys, each stored
// dim-major [128][32] (v_index below), so the A operand of P.V -- 8
// consecutive keys of one dim per lane -- is one 16-byte load, and a wave's
// load of a dim tile is 1 KiB contiguous. K stays row-major [slot][128].
#pragma once
#include "common.h"

namespace yuear {
namespace attn {

constexpr int D = 128;
constexpr int kBlock = 32;           // keys per V block = keys per wave per pass
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Element (slot t, dim d) of one head's V cache, in elements.
__host__ __device__ __forceinline__ size_t v_index(int t, int d) {
  return size_t(t >> 5) * (kBlock * D) + size_t(d) * kBlock + (t & (kBlock - 1));
}

template <int G, int W = 4>
struct Lds {
  u32x4 q[G][D / 8];        // normalised, rotated q heads (bf16, unscaled)
  u32x4 kv_new[2][D / 8];   // current key / value (bf16)
  float w_m[W][G], w_l[W][G];
  float w_o[W][G][D];
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Offset in its 32-key block of row i of S^T tile T.
__device__ __forceinline__ int key_ofs(int T, int i) { return 8 * (i >> 2) + 4 * T + (i & 3); }

// K rows of this wave's block starting at t0 + 32 wave (A operands of S^T):
// kr[4 T + s] = key key_ofs(T, lane % 16), dims 32 s + 8 (lane / 16) + [0, 8).
// Rows beyond the written part of the cache are clamped to last_cached
// (their scores are masked; the current key comes from LDS).
__device__ __forceinline__ void load_k(const u32x4 *kc, int t0, int wave, int lane,
                                       int last_cached, u32x4 (&kr)[8]) {
  const int r = lane >> 4, i = lane & 15;
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    const int key = min(t0 + kBlock * wave + key_ofs(T, i), last_cached);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      kr[4 * T + s] = kc[size_t(key) * (D / 8) + 4 * s + r];
  }
}

// V^T of the same block (A operands of O^T): vr[dt] = dim 16 dt + lane % 16,
// keys 8 (lane / 16) + [0, 8). A block past last_cached's block holds only
// masked keys (and the current key, taken from LDS), so it is clamped.
__device__ __forceinline__ void load_v(const u32x4 *vc, int t0, int wave, int lane,
                                       int last_cached, u32x4 (&vr)[8]) {
  const int r = lane >> 4, d = lane & 15;
  const int blk = min((t0 >> 5) + wave, last_cached >> 5);
  const u32x4 *base = vc + size_t(blk) * (kBlock * D / 8);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    vr[dt] = base[(16 * dt + d) * (kBlock / 8) + r];
}

// Prologue for head h of the workgroup (h < G: query head, h == G: key,
// h == G + 1: value), one head per wave, lane l holding dims 2l and 2l + 1:
// RMSNorm with the q/k gain and half-split RoPE (ar.cpp:268-277; operands
// preloaded in nr), then LDS.
template <int G, int W>
__device__ __forceinline__ void prologue_head(Lds<G, W> &sh, int h, uint32_t pair, bool has_gain,
                                              float eps, const NormRope &nr, int lane) {
  float y0 = bflo(pair), y1 = bfhi(pair);
  if (h <= G)
    norm_rope_apply(y0, y1, has_gain, eps, nr, lane, y0, y1);
  const uint32_t packed = uint32_t(f2bf(y0)) | (uint32_t(f2bf(y1)) << 16);
  if (h < G)
    reinterpret_cast<uint32_t *>(&sh.q[h][0])[lane] = packed;
  else
    reinterpret_cast<uint32_t *>(&sh.kv_new[h - G][0])[lane] = packed;
}

// bf16 element e of a 16-byte vector replaced by `val`.
__device__ __forceinline__ u32x4 with_elem(u32x4 v, int e, uint32_t val) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (q == (e >> 1))
      w[q] = (e & 1) ? (w[q] & 0xffffu) | (val << 16) : (w[q] & 0xffff0000u) | val;
  return u32x4{w[0], w[1], w[2], w[3]};
}

// One pass over keys [t0, t0 + 32 W) ∩ [s0, s1) with the online softmax
// state of this lane (head lane % 16): m, l (over this lane's keys), o (O^T
// tiles: dims 16 dt + 4 (lane / 16) + [0, 4)). kr / vr hold the pass's
// operands on entry; when `more`, the next pass's K rows are issued into kr
// right after the S^T products and its V^T rows into vr after P.V.
template <int G, int W>
__device__ __forceinline__ void pass(const Lds<G, W> &sh, const u32x4 *kc, const u32x4 *vc, int t0,
                                     int s1, int pos, int last_cached, bool more, int wave,
                                     int lane, const u32x4 (&qb)[4], float qscale,
                                     u32x4 (&kr)[8], u32x4 (&vr)[8], float &m_run, float &l_run,
                                     f32x4 (&o)[8]) {
  const int r = lane >> 4, i = lane & 15;
  const int blk0 = t0 + kBlock * wave;
#pragma unroll
  for (int T = 0; T < 2; ++T)
    if (blk0 + key_ofs(T, i) == pos) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        kr[4 * T + s] = sh.kv_new[0][4 * s + r];
    }
  f32x4 st[2];
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    st[T] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      st[T] = mfma(kr[4 * T + s], qb[s], st[T]);
  }
  if (more)
    load_k(kc, t0 + kBlock * W, wave, lane, last_cached, kr);
  // the current key's values (dim 16 dt + i) into element pos - (blk0 + 8 r)
  const int ep = pos - (blk0 + 8 * r);
  if (ep >= 0 && ep < 8) {
    const uint16_t *vn = reinterpret_cast<const uint16_t *>(&sh.kv_new[1][0]);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      vr[dt] = with_elem(vr[dt], ep, vn[16 * dt + i]);
  }
  // Values of keys at or past s1 are zeroed: their P is exactly 0, but a slot
  // never written (or rewound) must not bring an Inf or NaN into P.V.
  if (blk0 + kBlock > s1) {  // wave-uniform
    const int nv = min(max(s1 - (blk0 + 8 * r), 0), 8);
    uint32_t keep[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      keep[w] = (nv > 2 * w ? 0x0000ffffu : 0u) | (nv > 2 * w + 1 ? 0xffff0000u : 0u);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      vr[dt] = u32x4{vr[dt].x & keep[0], vr[dt].y & keep[1], vr[dt].z & keep[2],
                     vr[dt].w & keep[3]};
  }
  // scores of keys blk0 + 8 r + e, e = 4 T + t
  float sc[8];
#pragma unroll
  for (int T = 0; T < 2; ++T)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      sc[4 * T + t] = blk0 + 8 * r + 4 * T + t < s1 ? st[T][t] * qscale : -__builtin_inff();
  float mx = sc[0];
#pragma unroll
  for (int e = 1; e < 8; ++e)
    mx = fmaxf(mx, sc[e]);
  mx = max_halves(max_row_pairs(mx));  // over the 4 row groups: all 32 keys
  const float m_new = fmaxf(m_run, mx);
  const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;  // nothing visible yet
  const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
  float ps = 0.f;
  uint32_t pw[3][4];  // p = hi + mid + lo, each bf16 (the residuals are exact)
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float p0 = __builtin_amdgcn_exp2f(sc[2 * q] - m_use);
    float p1 = __builtin_amdgcn_exp2f(sc[2 * q + 1] - m_use);
    ps += p0;
    ps += p1;
    // Each piece rounds to nearest even (one v_cvt_pk_bf16_f32 per pair on
    // the device); the remainder is exact.
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const uint16_t b0 = f2bf(p0), b1 = f2bf(p1);
      pw[k][q] = uint32_t(b0) | (uint32_t(b1) << 16);
      p0 -= bf2f(b0);
      p1 -= bf2f(b1);
    }
  }
  l_run = l_run * corr + ps;
  m_run = m_new;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    o[dt] *= corr;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      o[dt] = mfma(vr[dt], u32x4{pw[k][0], pw[k][1], pw[k][2], pw[k][3]}, o[dt]);
  }
  if (more)
    load_v(vc, t0 + kBlock * W, wave, lane, last_cached, vr);
}

// All passes of [s0, s1) for this wave (s0 a multiple of 32), starting from
// kr / vr holding the first pass; leaves the wave's (m, l, o) in LDS (w_m,
// w_l, w_o). Needs the prologue's q in LDS (after a barrier).
template <int G, int W>
__device__ __forceinline__ void split(Lds<G, W> &sh, const u32x4 *kc, const u32x4 *vc, int s0,
                                      int s1, int pos, int last_cached, int lane, int wave,
                                      float qscale, u32x4 (&kr)[8], u32x4 (&vr)[8]) {
  const int r = lane >> 4, i = lane & 15;
  u32x4 qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x4 v = sh.q[i < G ? i : 0][4 * s + r];
    qb[s] = i < G ? v : u32x4{0u, 0u, 0u, 0u};
  }
  float m_run = -__builtin_inff(), l_run = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int t0 = s0;; t0 += kBlock * W) {
    const bool more = t0 + kBlock * W < s1;  // uniform
    pass<G, W>(sh, kc, vc, t0, s1, pos, last_cached, more, wave, lane, qb, qscale, kr, vr, m_run,
            l_run, o);
    if (!more)
      break;
  }
  const float l = sum_halves(sum_row_pairs(l_run));  // over the 4 row groups
  if (i < G) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<f32x4 *>(&sh.w_o[wave][i][16 * dt + 4 * r]) = o[dt];
    if (r == 0) {
      sh.w_m[wave][i] = m_run;
      sh.w_l[wave][i] = l;
    }
  }
}

// Combine the W waves for element e = h * D + d of the split partial
// (after a barrier): running max M, weighted o and l.
template <int G, int W>
__device__ __forceinline__ void combine(const Lds<G, W> &sh, int e, float &o, float &M,
                                        float &lsum) {
  const int h = e / D, d = e % D;
  M = sh.w_m[0][h];
#pragma unroll
  for (int w = 1; w < W; ++w)
    M = fmaxf(M, sh.w_m[w][h]);
  o = 0.f;
  lsum = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float f =
        sh.w_m[w][h] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(sh.w_m[w][h] - M);
    o = fmaf(f, sh.w_o[w][h][d], o);
    lsum = fmaf(f, sh.w_l[w][h], lsum);
  }
}

}  // namespace attn
}  // namespace yuear
