// Workgroup body of the batch 1..8 bf16 GEMV (y[b, r] = sum_k x[b, k] *
// W[row(r), k], fp32 accumulation, native/src/ar.cpp:20-29), shared by the
// per-op kernel (gemv.hip) and the fused QKV + attention + o_proj layer
// kernel (fused.hip), so both compute the same bits.
//
// Streaming design: every wave owns R consecutive weight rows. Its lanes read
// 16-byte chunks at k = 8 * (64 j + lane), so each wave-wide load is 1 KiB of
// one row, fully coalesced, marked non-temporal (weights are read once per
// step and must not evict the activations from L2). The activation rows
// (optionally gathered from the embedding table and/or RMS-normalised,
// ar.cpp:30-35) are staged once per workgroup in LDS; products use
// v_dot2_f32_bf16 and a 64-lane butterfly finishes each row.
//
// Modes:
//   kGemvPlain     activations from memory written by an earlier kernel; their
//                  loads go first, then the weight stream, so the prologue
//                  waits only for the small activation loads.
//   kGemvProduce   as kGemvPlain, but the outputs are stored as activation
//                  words (tag << 16 | bf16) with agent-scope write-through
//                  stores for consumers in the same launch.
//   kGemvConsume   the input rows are activation words produced in the same
//                  launch: the weight stream is issued first, then the words
//                  are re-read until every one carries the launch tag (a
//                  bounded wait). The residual epilogue adds the token's
//                  embedding row when p.embed is set (the first layer: it is
//                  x itself) and y otherwise.
#pragma once
#include "common.h"
#include "kernels.h"

namespace yuear {

enum GemvMode : int { kGemvPlain = 0, kGemvProduce = 1, kGemvConsume = 2 };

// Same-launch activation words: (tag << 16) | bf16 payload. A word with
// another tag is stale (an earlier launch) and is read again.
struct WordIO {
  uint32_t tag = 0;
  const uint32_t *in = nullptr;  // consume: [batch][in_stride] words
  int in_stride = 0;
  uint32_t *out = nullptr;       // produce: [batch][out_stride] words
  int out_stride = 0;
  int32_t *err = nullptr;        // sticky error word (expired wait)
  long long max_ticks = 0;       // bound of one wait, s_memrealtime ticks (100 MHz)
  unsigned long long *ready = nullptr;  // optional: time the inputs were ready
  bool late_weights = false;     // consume: issue the weight stream after the inputs are fresh
  uint32_t tag32 = 0;            // attention split partials: unique per (step, layer), not 0
  u32x4 *part = nullptr;         // attention split partials (attn_block.h)
};
__device__ __forceinline__ void stamp_ready(const WordIO &io, int slot = 0) {
  if (io.ready && threadIdx.x == 0)
    io.ready[slot] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ bool word_fresh(uint32_t w, uint32_t tag) { return (w >> 16) == tag; }
// All eight words of two 16-byte loads fresh (branch-free).
__device__ __forceinline__ bool words8_fresh(u32x4 a, u32x4 e, uint32_t tag) {
  const uint32_t t = tag;
  const uint32_t bad = ((a.x >> 16) ^ t) | ((a.y >> 16) ^ t) | ((a.z >> 16) ^ t) |
                       ((a.w >> 16) ^ t) | ((e.x >> 16) ^ t) | ((e.y >> 16) ^ t) |
                       ((e.z >> 16) ^ t) | ((e.w >> 16) ^ t);
  return bad == 0;
}

// Buffer resource over [base, base + bytes): loads outside read as 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t word_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
// 16 bytes past the caches (sc1): a stale line is never served.
__device__ __forceinline__ u32x4 word_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}
__device__ __forceinline__ unsigned long long word_load2(__amdgpu_buffer_rsrc_t r,
                                                         uint32_t off) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16);
  return (static_cast<unsigned long long>(v.y) << 32) | v.x;
}
__device__ __forceinline__ void word_store(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool wait_expired(const WordIO &io, long long t0) {
  if (__builtin_amdgcn_s_memrealtime() - t0 > io.max_ticks ||
      __hip_atomic_load(io.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
    __hip_atomic_store(io.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  return false;
}

// Embedding row of branch b; ids outside the table are clamped so that a bad
// id can never address memory outside it (the host validates ids).
__device__ __forceinline__ int gemv_token_row(const GemvParams &p, int b) {
  const int t = p.tokens[b];
  return p.embed_rows > 0 ? min(max(t, 0), p.embed_rows - 1) : t;
}

// One workgroup (256 threads) of the GEMV: rows [blk * 4 R, blk * 4 R + 4 R).
// xs: B * (k / 8) chunks of LDS; red: [B][4] floats of LDS.
template <int B, int KC, int R, int EPI, int MODE>
__device__ __forceinline__ void gemv_block(const GemvParams &p, int blk, u32x4 *xs,
                                           float (*red)[4], const WordIO &io) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.k >> 3;
  const int row_base = (blk * 4 + wave) * R;
  constexpr int XPT = (KC + 3) / 4;  // activation chunks per thread
  constexpr bool kRegStage = MODE != kGemvConsume && B * XPT <= 8;

  // Weight stream of this wave's rows (issued first when consuming).
  u32x4 wv[R][KC];
  auto issue_weights = [&]() {
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
  };

  u32x4 xr[kRegStage ? B : 1][kRegStage ? XPT : 1];
  u32x4 gr[XPT];
  // consume + residual: lane 0's residual inputs are loaded before the wait
  // (x from an earlier kernel, or the token's embedding row in the first
  // layer, which is x itself)
  float resid[B][R];
  if constexpr (MODE == kGemvConsume) {
    if (!io.late_weights)
      issue_weights();
    if constexpr (EPI == kEpiResidual) {
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int bb = min(b, p.batch - 1);
        const uint16_t *res = p.embed ? p.embed + size_t(gemv_token_row(p, bb)) * p.n
                                      : p.y + size_t(bb) * p.y_stride;
#pragma unroll
        for (int r = 0; r < R; ++r)
          resid[b][r] = bf2f(res[min(row_base + r, p.n - 1)]);
      }
    }
  } else {
    // 1. Activation (and RMSNorm gain) loads first: the vector-memory counter
    // drains in issue order, so the prologue below then waits only for these.
    // Loads are branch-free (indices clamped, values masked later) so the
    // waitcnt pass can count them precisely across the prologue.
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
    // 2. Issue the weight stream for this wave's rows.
    issue_weights();
  }

  // 3. Stage activations (gather copy-out, RMSNorm) into LDS.
  float ss[B];
  if constexpr (MODE == kGemvConsume) {
    // activation words of this launch: re-read until all are fresh
    const auto rin = word_rsrc(io.in, uint32_t((p.batch - 1) * io.in_stride + p.k) * 4);
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      bool ok = true;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        if (b >= p.batch)
          continue;
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          if (c >= nch)
            continue;
          const uint32_t off = uint32_t(b * io.in_stride + c * 8) * 4;
          const u32x4 a = word_load4(rin, off), e = word_load4(rin, off + 16);
          ok = ok && words8_fresh(a, e, io.tag);
          xs[b * nch + c] = u32x4{(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                                  (e.x & 0xffffu) | (e.y << 16), (e.z & 0xffffu) | (e.w << 16)};
        }
      }
      if (__syncthreads_and(ok))
        break;
      const bool give_up = threadIdx.x == 0 && wait_expired(io, t0);
      if (__syncthreads_or(give_up))
        break;
      __builtin_amdgcn_s_sleep(1);
    }
    stamp_ready(io);
    if (io.late_weights)
      issue_weights();
  } else {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      ss[b] = 0.f;
      if (b >= p.batch)
        continue;
      const uint16_t *src = p.embed ? p.embed + size_t(gemv_token_row(p, b)) * p.k
                                    : p.x + size_t(b) * p.x_stride;
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
        xs[b * nch + c] = v;
        if (p.x_out && blk == 0)
          reinterpret_cast<u32x4 *>(p.x_out + size_t(b) * p.x_stride)[c] = v;
        if (p.norm_w) {
          const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float lo = bflo(w4[q]), hi = bfhi(w4[q]);
            ss[b] += lo * lo;
            ss[b] += hi * hi;
          }
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
        if (b >= p.batch)
          continue;
        const float total = (red[b][0] + red[b][1]) + (red[b][2] + red[b][3]);
        const float scale = rbf(1.0f / __builtin_sqrtf(total / float(p.k) + p.eps));
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          if (c >= nch)
            continue;
          const u32x4 v = xs[b * nch + c], g = gr[i];
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
  }

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
            if constexpr (EPI == kEpiResidual) {
              if constexpr (MODE == kGemvConsume) {
                v = resid[b][r] + rbf(v);
              } else {
                v = bf2f(yb[row]) + rbf(v);
              }
            }
            if constexpr (MODE == kGemvProduce)
              word_store(io.out + size_t(b) * io.out_stride + row,
                         (io.tag << 16) | uint32_t(f2bf(v)));
            else
              yb[row] = f2bf(v);
          }
        }
      }
    }
  }
  if (p.advance && blk == 0 && threadIdx.x < p.batch)
    p.advance[threadIdx.x] += 1;
  if (p.epoch && blk == 0 && threadIdx.x == 0)
    *p.epoch += 1;
}

}  // namespace yuear
