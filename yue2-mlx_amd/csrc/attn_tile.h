// One 32-query tile of multi-query attention with head_dim 128 on gfx950
// MFMA, shared by the causal prefill attention (prefill.hip, ar.cpp:284-291)
// and the acoustic-model attention (nar_attention.hip,
// nar_attention.cpp:63-218): fp32 scores of bf16 operands, an exp2 online
// softmax in fp32, P fed to P.V as three truncated bf16 pieces (its 24
// significant bits: every product exact), fp32 sums, bf16(o / l).
//
// The workgroup's 4 waves split the tile's key range: wave w walks the
// 32-key blocks w, w + 4, w + 8, ... with the next block's K loads in flight
// (and the block's own V issued at its start), then the four (m, l, O)
// partials are merged through LDS. Each wave holds both 16-query MFMA column
// tiles:
//
//   S^T[key][query] = K[key][:] . q[query][:]            (attn_core.h rows)
//   O^T[dim][query] += V^T[dim][key] . P^T[key][query]
//
// Splitting the keys over the waves (rather than the queries) shortens each
// wave's dependent chain of blocks four times and gives four times more
// workgroups; both matter because a block step is a latency-bound chain
// (MFMA accumulations, cross-lane max / sum, the exp2 and the P split).
#pragma once
#include <type_traits>

#include "attn_core.h"
#include "common.h"

namespace yuear {
namespace attn {

struct TileLds {
  float m[4][2][16], l[4][2][16];
  f32x4 o[4][2][8][64];  // [wave][column tile][dim tile][lane]
};

struct QueryTile {
  const u32x4 *kc = nullptr;  // this kv head's K rows, row-major [slot][128]
  const u32x4 *vc = nullptr;  // its V in 32-key dim-major blocks (v_index)
  int kend = 0;               // keys [0, kend) are read
  int kv_len = 0;             // non-causal: keys [0, kv_len) are visible
  int causal_pos = -1;        // >= 0: query t sees keys <= causal_pos + t
  const uint16_t *q = nullptr;  // query 0 of the tile
  size_t q_stride = 0;          // elements between consecutive queries
  int nq = 0;                   // valid queries (1..32)
  uint16_t *out = nullptr;      // output row of query 0
  size_t out_stride = 0;
  // attn_query_tile64 only: key blocks [blk0, blk1) of the tile (blk1 0: all)
  // and, when set, an unnormalised partial per query instead of out: 132
  // floats {o[128], m, l, pad} at part + query * 132 (m the running maximum in
  // the exp2 domain, l the sum of exp2(s - m), o the sum of exp2(s - m) v)
  int blk0 = 0, blk1 = 0;
  float *part = nullptr;
};

__device__ __forceinline__ void attn_query_tile(const QueryTile &t, float qscale, TileLds &sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, i = lane & 15;
  const int nblk = (t.kend + kBlock - 1) / kBlock;
  const int last = t.kend - 1;

  // Q^T operands: column tile c, query 16 c + i (clamped), dims 32 s + 8 r
  u32x4 qb[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int qi = min(16 * c + i, t.nq - 1);
    const u32x4 *src = reinterpret_cast<const u32x4 *>(t.q + size_t(qi) * t.q_stride);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[c][s] = src[4 * s + r];
  }
  float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      o[c][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wave < nblk) {  // uniform per wave
    u32x4 kr[8];
    load_k(t.kc, wave * kBlock, 0, lane, last, kr);
    for (int blk = wave; blk < nblk; blk += 4) {
      const int kb = blk * kBlock;
      const bool more = blk + 4 < nblk;  // uniform
      // this block's V lands during S^T and the softmax; the next block's K
      // is in flight during the whole step (two waves per SIMD hide the rest)
      u32x4 vr[8], kn[8];
      load_v(t.vc, kb, 0, lane, last, vr);
      if (more)
        load_k(t.kc, kb + 4 * kBlock, 0, lane, last, kn);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f32x4 st[2];
#pragma unroll
        for (int T = 0; T < 2; ++T) {
          st[T] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s)
            st[T] = mfma(kr[4 * T + s], qb[c][s], st[T]);
        }
        // lane (query 16 c + i, r): keys kb + 8 r + 4 T + u
        const int kmax = t.causal_pos >= 0 ? t.causal_pos + 16 * c + i : t.kv_len - 1;
        float sc[8];
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            sc[4 * T + u] = kb + 8 * r + 4 * T + u <= kmax ? st[T][u] * qscale : -__builtin_inff();
        float mx = sc[0];
#pragma unroll
        for (int e = 1; e < 8; ++e)
          mx = fmaxf(mx, sc[e]);
        mx = max_halves(max_row_pairs(mx));
        const float m_new = fmaxf(m_run[c], mx);
        const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
        const float corr = __builtin_amdgcn_exp2f(m_run[c] - m_use);
        float ps = 0.f;
        uint32_t pw[3][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float p0 = __builtin_amdgcn_exp2f(sc[2 * q] - m_use);
          float p1 = __builtin_amdgcn_exp2f(sc[2 * q + 1] - m_use);
          ps += p0;
          ps += p1;
          // three truncated bf16 pieces: the top 8, next 8 and last 8
          // significant bits of p; each remainder is exact, so p is their sum
#pragma unroll
          for (int k = 0; k < 3; ++k) {
            const uint32_t u0 = __builtin_bit_cast(uint32_t, p0);
            const uint32_t u1 = __builtin_bit_cast(uint32_t, p1);
            pw[k][q] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);  // hi16(u0) | hi16(u1) << 16
            p0 -= __builtin_bit_cast(float, u0 & 0xffff0000u);
            p1 -= __builtin_bit_cast(float, u1 & 0xffff0000u);
          }
        }
        l_run[c] = l_run[c] * corr + ps;
        m_run[c] = m_new;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          o[c][dt] *= corr;
#pragma unroll
          for (int k = 0; k < 3; ++k)
            o[c][dt] = mfma(vr[dt], u32x4{pw[k][0], pw[k][1], pw[k][2], pw[k][3]}, o[c][dt]);
        }
      }
      if (more) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          kr[j] = kn[j];
      }
    }
  }

  // Merge the four waves' partials: wave w finishes column tile w / 2, dim
  // tiles 4 (w % 2) .. + 3. A wave that saw no visible key of a query has
  // m = -inf and weight 0 (key 0 is in wave 0's first block and visible to
  // every query, so the maximum is finite).
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float l = sum_halves(sum_row_pairs(l_run[c]));
    if (r == 0) {
      sh.m[wave][c][i] = m_run[c];
      sh.l[wave][c][i] = l;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      sh.o[wave][c][dt][lane] = o[c][dt];
  }
  __syncthreads();
  const int c = wave >> 1, d0 = 4 * (wave & 1);
  float f[4], M = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < 4; ++w)
    M = fmaxf(M, sh.m[w][c][i]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float m = sh.m[w][c][i];
    f[w] = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - M);
    L += f[w] * sh.l[w][c][i];
  }
  const int qi = 16 * c + i;
  if (qi < t.nq) {
    uint16_t *dst = t.out + size_t(qi) * t.out_stride;
#pragma unroll
    for (int dt = d0; dt < d0 + 4; ++dt) {
      f32x4 acc = sh.o[0][c][dt][lane] * f[0];
#pragma unroll
      for (int w = 1; w < 4; ++w)
        acc += sh.o[w][c][dt][lane] * f[w];
      // lane (query, r) holds dims 16 dt + 4 r + [0, 4): out = bf16(o / l)
      const uint32_t lo = uint32_t(f2bf(acc[0] / L)) | (uint32_t(f2bf(acc[1] / L)) << 16);
      const uint32_t hi = uint32_t(f2bf(acc[2] / L)) | (uint32_t(f2bf(acc[3] / L)) << 16);
      *reinterpret_cast<uint2 *>(dst + 16 * dt + 4 * r) = uint2{lo, hi};
    }
  }
}

// ---------------------------------------------------------------------------
// 64-query tile with K/V shared through LDS: wave w owns queries 16 w + i and
// all four waves walk the same 32-key blocks. Each block's K and V are
// fetched once per workgroup (each wave loads a quarter: K pieces and V dim
// tiles 2 w, 2 w + 1 in the MFMA operand layout of load_k / load_v) into an
// LDS ring ahead of the block being computed; every wave then reads its
// operands from LDS. Same arithmetic per query as
// attn_query_tile (fp32 scores, exp2 online softmax, P as three truncated
// bf16 pieces, fp32 sums, bf16(o / l)), with no merge across waves.
// Workgroups of the 64-query tile below which the 32-query key-split tile
// is faster on MI355X's 256 CUs (measured, causal self-attention at 24/8
// heads: 288 workgroups of 64 queries (768 tokens) lose to 576 of 32, 23.3
// against 22.1 us; 384 (1024 tokens) win, 30.5 against 33.5 us, and the gap
// grows with the length: 66.6 against 85 us at 1984 tokens).
constexpr int kTile64MinGroups = 384;
// Key splits of a non-causal launch aim at this many workgroups.
constexpr int kSplitTargetGroups = 768;

// LDS ring of two stages (32 KiB: one block ahead), filled by direct-to-LDS
// loads, so the next block needs no registers: 96 VGPRs, five waves per SIMD
// and five workgroups per CU (160 KiB of LDS). Three stages with register
// staging (48 KiB, 131 VGPRs, three waves) measured 2-4% slower than two.
constexpr int kTile64Stages = 2;
constexpr int kTile64Waves = 5;  // waves per SIMD (LDS, registers)

struct Tile64Lds {
  u32x4 k[kTile64Stages][8][64];  // [stage][piece][lane]
  u32x4 v[kTile64Stages][8][64];
};

__device__ __forceinline__ void attn_query_tile64(const QueryTile &t, float qscale,
                                                  Tile64Lds &sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, i = lane & 15;
  const int b_lo = t.blk0;
  const int nblk = t.blk1 ? t.blk1 : (t.kend + kBlock - 1) / kBlock;  // blocks [b_lo, nblk)
  const int last = t.kend - 1;
  u32x4 qb[4];
  {
    const int qi = min(16 * wave + i, t.nq - 1);
    const u32x4 *src = reinterpret_cast<const u32x4 *>(t.q + size_t(qi) * t.q_stride);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[s] = src[4 * s + r];
  }
  const int kmax = t.causal_pos >= 0 ? t.causal_pos + 16 * wave + i : t.kv_len - 1;
  // this wave's quarter of the block at kb into `stage`: K pieces 2 w, 2 w + 1
  // (T = w / 2, s = 2 (w % 2) + {0, 1}) and V dim tiles 2 w, 2 w + 1, each a
  // direct-to-LDS buffer load that puts lane l's 16 bytes in slot l of the
  // piece row (the MFMA operand layout; no registers in between). Keys and
  // blocks are clamped to the last visible one, inside both ranges.
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4 *>(t.kc), 0,
                                                    uint32_t(t.kend) * (D * 2), 0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4 *>(t.vc), 0, uint32_t((last >> 5) + 1) * (kBlock * D * 2), 0x00020000);
  auto fetch = [&](int kb, int stage) {
    const int key = min(kb + key_ofs(wave >> 1, i), last);
    const uint32_t ko = uint32_t(key * (D / 8) + 8 * (wave & 1) + r) * 16;
    const uint32_t vo = uint32_t(min(kb >> 5, last >> 5)) * (kBlock * D * 2) +
                        uint32_t((32 * wave + i) * (kBlock / 8) + r) * 16;
    typedef __attribute__((address_space(3))) void *lds_ptr_t;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)&sh.k[stage][2 * wave][0], 16, ko, 0,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)&sh.k[stage][2 * wave + 1][0], 16,
                                             ko + 64, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)&sh.v[stage][2 * wave][0], 16, vo, 0,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)&sh.v[stage][2 * wave + 1][0], 16,
                                             vo + 16 * kBlock * 2, 0, 0, 0);
  };

  float m_run = -__builtin_inff(), l_run = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int S = kTile64Stages;
  fetch(b_lo * kBlock, b_lo % S);
  __builtin_amdgcn_s_waitcnt(0);  // (a barrier waits for no load)
  __syncthreads();
  // one block; kMask: the causal / key-length mask, needed only from the
  // first block with a key past the smallest kmax of the tile's queries (the
  // blocks before it are visible to every query: same scores, no compares)
  auto block = [&](int b, auto mask_tag) {
    constexpr bool kMask = decltype(mask_tag)::value;
    const int stage = b % S, kb = b * kBlock;
    // block b + 1 into the stage every wave finished reading before the
    // previous barrier; in flight during this block's products
    if (b + 1 < nblk)  // uniform
      fetch(kb + kBlock, (b + 1) % S);
    u32x4 kr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      kr[j] = sh.k[stage][j][lane];
    f32x4 st[2];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      st[T] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        st[T] = mfma(kr[4 * T + s], qb[s], st[T]);
    }
    // lane (query 16 w + i, r): keys kb + 8 r + 4 T + u
    float sc[8];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        sc[4 * T + u] = !kMask || kb + 8 * r + 4 * T + u <= kmax ? st[T][u] * qscale
                                                                : -__builtin_inff();
    float mx = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e)
      mx = fmaxf(mx, sc[e]);
    mx = max_halves(max_row_pairs(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    float ps = 0.f;
    uint32_t pw[3][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float p0 = __builtin_amdgcn_exp2f(sc[2 * q] - m_use);
      float p1 = __builtin_amdgcn_exp2f(sc[2 * q + 1] - m_use);
      ps += p0;
      ps += p1;
      // three truncated bf16 pieces: the top 8, next 8 and last 8
      // significant bits of p; each remainder is exact, so p is their sum
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const uint32_t u0 = __builtin_bit_cast(uint32_t, p0);
        const uint32_t u1 = __builtin_bit_cast(uint32_t, p1);
        pw[k][q] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);  // hi16(u0) | hi16(u1) << 16
        p0 -= __builtin_bit_cast(float, u0 & 0xffff0000u);
        p1 -= __builtin_bit_cast(float, u1 & 0xffff0000u);
      }
    }
    l_run = l_run * corr + ps;
    m_run = m_new;
    u32x4 vr[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      vr[dt] = sh.v[stage][dt][lane];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      o[dt] *= corr;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        o[dt] = mfma(vr[dt], u32x4{pw[k][0], pw[k][1], pw[k][2], pw[k][3]}, o[dt]);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's part of block b + 1
    __syncthreads();
  };
  const int kfull = (t.causal_pos >= 0 ? t.causal_pos + 1 : t.kv_len) / kBlock;
  int b = b_lo;
  for (; b < min(kfull, nblk); ++b)
    block(b, std::false_type{});
  for (; b < nblk; ++b)
    block(b, std::true_type{});
  // lane (query 16 w + i, r) holds dims 16 dt + 4 r + [0, 4): out = bf16(o / l)
  const float L = sum_halves(sum_row_pairs(l_run));
  const int qi = 16 * wave + i;
  if (t.part) {
    if (qi < t.nq) {
      float *pq = t.part + size_t(qi) * 132;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<f32x4 *>(pq + 16 * dt + 4 * r) = o[dt];
      if (r == 0) {
        pq[128] = m_run;
        pq[129] = L;
      }
    }
    return;
  }
  if (qi < t.nq) {
    uint16_t *dst = t.out + size_t(qi) * t.out_stride;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint32_t lo = uint32_t(f2bf(o[dt][0] / L)) | (uint32_t(f2bf(o[dt][1] / L)) << 16);
      const uint32_t hi = uint32_t(f2bf(o[dt][2] / L)) | (uint32_t(f2bf(o[dt][3] / L)) << 16);
      *reinterpret_cast<uint2 *>(dst + 16 * dt + 4 * r) = uint2{lo, hi};
    }
  }
}

}  // namespace attn
}  // namespace yuear
