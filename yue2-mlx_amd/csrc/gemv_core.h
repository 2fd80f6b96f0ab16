// Workgroup body of the batch 1..8 bf16 GEMV (y[b, r] = sum_k x[b, k] *
// W[row(r), k], fp32 accumulation, native/src/ar.cpp:20-29).
//
// Streaming design: every wave owns R consecutive weight rows. Its lanes read
// 16-byte chunks at k = 8 * (64 j + lane), so each wave-wide load is 1 KiB of
// one row, fully coalesced, marked non-temporal (weights are read once per
// step and must not evict the activations from L2). The activation rows
// (optionally gathered from the embedding table and/or RMS-normalised,
// ar.cpp:30-35) are staged once per workgroup in LDS; products use
// v_dot2_f32_bf16 and a 64-lane butterfly finishes each row. The activation
// loads go first, then the weight stream, so the prologue waits only for the
// small activation loads.
#pragma once
#include "common.h"
#include "kernels.h"

namespace yuear {

// Embedding row of branch b; ids outside the table are clamped so that a bad
// id can never address memory outside it (the host validates ids).
__device__ __forceinline__ int gemv_token_row(const GemvParams &p, int b) {
  const int t = p.tokens[b];
  return p.embed_rows > 0 ? min(max(t, 0), p.embed_rows - 1) : t;
}

// One workgroup (256 threads) of the GEMV: rows [blk * 4 R, blk * 4 R + 4 R).
// xs: B * (k / 8) chunks of LDS; red: [B][4] floats of LDS.
template <int B, int KC, int R, int EPI>
__device__ __forceinline__ void gemv_block(const GemvParams &p, int blk, u32x4 *xs,
                                           float (*red)[4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.k >> 3;
  const int row_base = (blk * 4 + wave) * R;
  constexpr int XPT = (KC + 3) / 4;  // activation chunks per thread
  constexpr bool kRegStage = B * XPT <= 8;

  // 1. Activation (and RMSNorm gain) loads first: the vector-memory counter
  // drains in issue order, so the prologue below then waits only for these.
  // Loads are branch-free (indices clamped, values masked later) so the
  // waitcnt pass can count them precisely across the prologue.
  u32x4 xr[kRegStage ? B : 1][kRegStage ? XPT : 1];
  u32x4 gr[XPT];
  if constexpr (kRegStage) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int bb = min(b, p.batch - 1);
      const uint16_t *src = p.embed ? p.embed + size_t(gemv_token_row(p, bb)) * p.k
                                    : p.x + size_t(bb) * p.x_stride;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = min(int(threadIdx.x) + 256 * i, nch - 1);
        xr[b][i] = reinterpret_cast<const u32x4 *>(src)[c];
      }
    }
  }
  if (p.norm_w) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int c = min(int(threadIdx.x) + 256 * i, nch - 1);
      gr[i] = reinterpret_cast<const u32x4 *>(p.norm_w)[c];
    }
  }
  // 2. The weight stream of this wave's rows.
  u32x4 wv[R][KC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int lr = min(row_base + r, p.n - 1);
    const int row = lr < p.seg0_len ? p.seg0_start + lr : p.seg1_start + (lr - p.seg0_len);
    const u32x4 *wrow = reinterpret_cast<const u32x4 *>(p.w + size_t(row) * p.k);
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int c = j * 64 + lane;
      const u32x4 v = __builtin_nontemporal_load(wrow + min(c, nch - 1));
      wv[r][j] = c < nch ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // 3. Stage activations (gather copy-out, RMSNorm) into LDS. Every one of
  // the B template rows is processed without a branch on p.batch (rows past
  // it repeat the last real row and are never read back), so the rows'
  // reduction and normalisation chains interleave instead of running one
  // after the other (batch 2: 0.8-0.9 us less per normed launch on MI355X).
  float ss[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    ss[b] = 0.f;
    const int bb = min(b, p.batch - 1);
    const uint16_t *src = p.embed ? p.embed + size_t(gemv_token_row(p, bb)) * p.k
                                  : p.x + size_t(bb) * p.x_stride;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int c = threadIdx.x + 256 * i;
      if (c >= nch)
        continue;
      u32x4 v;
      if constexpr (kRegStage)
        v = xr[b][i];
      else
        v = reinterpret_cast<const u32x4 *>(src)[c];
      if (p.x_out && blk == 0 && b < p.batch)
        reinterpret_cast<u32x4 *>(p.x_out + size_t(b) * p.x_stride)[c] = v;
      if (p.norm_w) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bflo(w4[q]), hi = bfhi(w4[q]);
          ss[b] += lo * lo;
          ss[b] += hi * hi;
        }
      } else {
        xs[b * nch + c] = v;
      }
    }
  }
  if (p.norm_w) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float t = wave_sum(ss[b]);
      if (lane == 0)
        red[b][wave] = t;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float total = (red[b][0] + red[b][1]) + (red[b][2] + red[b][3]);
      const float scale = rbf(1.0f / __builtin_sqrtf(total / float(p.k) + p.eps));
      const int bb = min(b, p.batch - 1);
      const uint16_t *src = p.embed ? p.embed + size_t(gemv_token_row(p, bb)) * p.k
                                    : p.x + size_t(bb) * p.x_stride;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c >= nch)
          continue;
        u32x4 v;
        if constexpr (kRegStage)
          v = xr[b][i];
        else
          v = reinterpret_cast<const u32x4 *>(src)[c];
        const u32x4 g = gr[i];
        const uint32_t vi[4] = {v.x, v.y, v.z, v.w}, gi[4] = {g.x, g.y, g.z, g.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = f2bf(rbf(bflo(vi[q]) * scale) * bflo(gi[q]));
          const uint32_t hi = f2bf(rbf(bfhi(vi[q]) * scale) * bfhi(gi[q]));
          o[q] = lo | (hi << 16);
        }
        xs[b * nch + c] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
  __syncthreads();

  // 4. Dot products.
  float acc[B][R];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[b][r] = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int c = j * 64 + lane;
    if (c < nch) {
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const u32x4 xv = xs[(b < p.batch ? b : 0) * nch + c];
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[b][r] = dot8(wv[r][j], xv, acc[b][r]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[b][r] = wave_sum(acc[b][r]);

  // 5. Epilogue (lane 0 of each wave).
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (b >= p.batch)
        continue;
      uint16_t *yb = p.y + size_t(b) * p.y_stride;
      if constexpr (EPI == kEpiSwiGLU) {
#pragma unroll
        for (int r = 0; r + 1 < R; r += 2) {
          const int row = row_base + r;
          if (row + 1 < p.n) {
            const float g = rbf(acc[b][r]), u = rbf(acc[b][r + 1]);
            const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
            yb[row >> 1] = f2bf(act * u);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = row_base + r;
          if (row < p.n) {
            float v = acc[b][r];
            if constexpr (EPI == kEpiResidual)
              v = bf2f(yb[row]) + rbf(v);
            yb[row] = f2bf(v);
          }
        }
      }
    }
  }
  if (p.advance && blk == 0 && threadIdx.x < p.batch)
    p.advance[threadIdx.x] += 1;
}

}  // namespace yuear
