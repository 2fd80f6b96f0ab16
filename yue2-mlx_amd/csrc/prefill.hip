// Prompt prefill kernels on gfx950 (the projections are MFMA GEMMs in
// gemm.hip, SwiGLU in the gate/up GEMM's epilogue): row-wise RMSNorm and
// embedding, q/k RMSNorm + RoPE + KV append, and an MFMA causal attention
// with fp32 opmath.
//
// Reference: native/src/ar.cpp:246-301 (hidden() over T > 1 tokens) and
// native/src/sampling.cpp:152-183 (prefill). The reference upcasts Q/K/V to
// fp32 for the causal SDPA (ar.cpp:284-291); the attention kernel here forms
// exact products on MFMA, keeps scores, softmax and all sums in fp32 and
// rounds only the output to bf16.
#include <cmath>
#include <type_traits>

#include "attn_core.h"
#include "attn_tile.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {


// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint16_t *table, const int32_t *ids,
                                                         int width, uint16_t *out) {
  const int r = blockIdx.x;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(table + size_t(ids[r]) * width);
  u32x4 *dst = reinterpret_cast<u32x4 *>(out + size_t(r) * width);
  for (int c = threadIdx.x; c < width / 8; c += 256)
    dst[c] = src[c];
}

// ar.cpp:30-35 per row. Thread t takes the row's 8-feature chunks t, t + 256,
// ... (at most kRowChunks, rows up to 8192 features), held in registers
// between the squares' sum and the scaling (one read of the row).
constexpr int kRowChunks = 4;
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const uint16_t *x, int width,
                                                            const uint16_t *w, float eps,
                                                            uint16_t *y) {
  __shared__ float red[4];
  const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = width / 8;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(x + size_t(r) * width);
  u32x4 xv[kRowChunks];
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = int(threadIdx.x) + 256 * i;
    xv[i] = c < chunks ? src[c] : u32x4{0u, 0u, 0u, 0u};
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    if (int(threadIdx.x) + 256 * i >= chunks)
      break;
    const uint32_t vi[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = bflo(vi[q]), hi = bfhi(vi[q]);
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = rbf(1.0f / __builtin_sqrtf(total / float(width) + eps));
  const u32x4 *g4 = reinterpret_cast<const u32x4 *>(w);
  u32x4 *dst = reinterpret_cast<u32x4 *>(y + size_t(r) * width);
#pragma unroll
  for (int i = 0; i < kRowChunks; ++i) {
    const int c = int(threadIdx.x) + 256 * i;
    if (c >= chunks)
      break;
    const u32x4 g = g4[c];
    const uint32_t vi[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w}, gi[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = f2bf(rbf(bflo(vi[q]) * scale) * bflo(gi[q]));
      const uint32_t hi = f2bf(rbf(bfhi(vi[q]) * scale) * bfhi(gi[q]));
      o[q] = lo | (hi << 16);
    }
    dst[c] = u32x4{o[0], o[1], o[2], o[3]};
  }
}


// q/k RMSNorm + RoPE for T tokens, K/V append (ar.cpp:268-282).
// Workgroup (block, head): the positions of one 32-key cache block (the
// block layout's unit) that this call covers, for one head (q heads, then
// k heads, then v heads); wave w takes the block's positions 8w .. 8w + 7
// and issues all 8 row loads (256 bytes each) before the first reduction.
// q / k rows: RMSNorm + RoPE per row (a short dependent chain: cross-lane
// sum, rotate), stored row-major. V rows: staged in LDS, then written as the
// block's dim-major rows (64 bytes of 32 keys per dim) in 16-byte pieces;
// keys of a partly covered block outside the call's positions keep their
// cache contents (2-byte stores for those pieces only).
__global__ __launch_bounds__(256) void qk_prep_kernel(QkPrepParams p) {
  __shared__ uint32_t vrow[attn::kBlock][65];  // V tile: [key in block][dim pair], padded
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.y;
  const int blk = p.pos0 / attn::kBlock + int(blockIdx.x);
  const int lo = max(blk * attn::kBlock, p.pos0);
  const int hi = min(blk * attn::kBlock + attn::kBlock, p.pos0 + p.tokens);  // positions [lo, hi)
  const int base = blk * attn::kBlock + 8 * wave;
  uint32_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // clamped rows: always a valid address
    const int t = min(max(base + j, lo), hi - 1) - p.pos0;
    v[j] = reinterpret_cast<const uint32_t *>(p.qkv + size_t(t) * p.qkv_stride)[h * 64 + lane];
  }
  if (h < p.heads + p.kv_heads) {
    const bool is_q = h < p.heads;
    const uint16_t *gain = is_q ? p.q_norm : p.k_norm;
    // the gains (without a gain the unused load reads this head's 128 inputs
    // of the block's first row, always in bounds), then every row's RoPE
    // entries (positions clamped into [lo, hi)), all issued together so no
    // row waits for its own round trip
    NormRope g;
    load_gain(g, gain ? gain : p.qkv + size_t(lo - p.pos0) * p.qkv_stride + size_t(h) * 128, lane);
    NormRope r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pos = min(max(base + j, lo), hi - 1);
      load_rope(r[j], p.rope_cos + size_t(pos) * 64, p.rope_sin + size_t(pos) * 64, lane);
      r[j].g0 = g.g0;
      r[j].g1 = g.g1;
    }
    // norm_rope_apply's arithmetic for the 8 rows, with the per-row scale
    // rbf(1 / sqrt(ssq / 128 + eps)) evaluated once for all rows (row j in
    // lane j, read back as a scalar) instead of once per row across the
    // wave, and the RoPE halves without a branch: lanes 0-31 add the
    // negated partner product, which rounds to exactly minus the product
    // (round-to-nearest-even is symmetric), so every result is the same bits
    float x0[8], x1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x0[j] = bflo(v[j]);
      x1[j] = bfhi(v[j]);
    }
    if (gain != nullptr) {
      float mine = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float ssq = wave_sum(x0[j] * x0[j] + x1[j] * x1[j]);
        mine = lane == j ? ssq : mine;
      }
      const float sc_lane = rbf(1.0f / __builtin_sqrtf(mine / 128.0f + p.eps));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sc = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_lane), j));
        x0[j] = rbf(rbf(x0[j] * sc) * r[j].g0);
        x1[j] = rbf(rbf(x1[j] * sc) * r[j].g1);
      }
    }
    const float sgn = lane < 32 ? -1.0f : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pos = base + j;
      const float p0 = sgn * xor32(x0[j], lane), p1 = sgn * xor32(x1[j], lane);
      const float y0 = rbf(rbf(x0[j] * r[j].c0) + rbf(p0 * r[j].s0));
      const float y1 = rbf(rbf(x1[j] * r[j].c1) + rbf(p1 * r[j].s1));
      if (pos < lo || pos >= hi)  // uniform per wave
        continue;
      uint32_t *dst =
          is_q ? reinterpret_cast<uint32_t *>(p.q_out + (size_t(pos - p.pos0) * p.heads + h) * 128)
               : reinterpret_cast<uint32_t *>(p.k_cache +
                                              (size_t(h - p.heads) * p.capacity + pos) * 128);
      dst[lane] = uint32_t(f2bf(y0)) | (uint32_t(f2bf(y1)) << 16);
    }
    return;
  }
  // V: [key][dim pair] into LDS, then piece (d, c) = keys 8c .. 8c + 7 of dim d
#pragma unroll
  for (int j = 0; j < 8; ++j)
    vrow[8 * wave + j][lane] = v[j];
  __syncthreads();
  uint16_t *vh = p.v_cache + size_t(h - p.heads - p.kv_heads) * p.capacity * 128;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int piece = int(threadIdx.x) + 256 * i;  // 512 pieces: 128 dims x 4
    const int d = piece >> 2, c = piece & 3;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t a = vrow[8 * c + 2 * e][d >> 1], b2 = vrow[8 * c + 2 * e + 1][d >> 1];
      w[e] = (d & 1) ? ((a >> 16) | (b2 & 0xffff0000u)) : ((a & 0xffffu) | (b2 << 16));
    }
    const int k0 = blk * attn::kBlock + 8 * c;
    uint16_t *dst = vh + attn::v_index(k0, d);
    if (k0 >= lo && k0 + 8 <= hi) {
      *reinterpret_cast<u32x4 *>(dst) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (k0 + e >= lo && k0 + e < hi)
          dst[e] = uint16_t(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------------------
// Causal attention on MFMA (ar.cpp:284-291: fp32 scores, softmax and P.V,
// bf16 output): one workgroup per (q head, 32-query tile), the tile's keys
// [0, pos0 + last query] split over the 4 waves and merged in LDS
// (attn_tile.h). Query t sits at position pos0 + t. Tiles are dispatched
// longest causal range first, and all heads of a tile run together so the
// K/V blocks are shared in L2.
// ---------------------------------------------------------------------------
// T64: the 64-query tile with K/V shared through LDS (attn_query_tile64),
// chosen when it yields enough workgroups to fill the GPU; otherwise the
// 32-query tile whose four waves split the keys.
template <bool T64>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(T64 ? attn::kTile64Waves : 2, T64 ? attn::kTile64Waves : 2))) void attn_prefill_kernel(AttnPrefillParams p, float qscale) {
  constexpr int kQ = T64 ? 64 : 32;  // queries per workgroup
  __shared__ std::conditional_t<T64, attn::Tile64Lds, attn::TileLds> sh;
  using attn::D;
  const int h = blockIdx.x;
  const int tile = gridDim.y - 1 - blockIdx.y;  // longest causal range first
  const int q0 = tile * kQ;
  const int kvh = h / (p.heads / p.kv_heads);
  attn::QueryTile t;
  t.kc = reinterpret_cast<const u32x4 *>(p.k_cache) + size_t(kvh) * p.capacity * (D / 8);
  t.vc = reinterpret_cast<const u32x4 *>(p.v_cache) + size_t(kvh) * p.capacity * (D / 8);
  t.nq = min(kQ, p.tokens - q0);
  t.kend = p.pos0 + q0 + t.nq;
  t.causal_pos = p.pos0 + q0;
  t.q = p.q + (size_t(q0) * p.heads + h) * D;
  t.q_stride = size_t(p.heads) * D;
  t.out = p.out + (size_t(q0) * p.heads + h) * D;
  t.out_stride = size_t(p.heads) * D;
  if constexpr (T64)
    attn::attn_query_tile64(t, qscale, sh);
  else
    attn::attn_query_tile(t, qscale, sh);
}

}  // namespace

hipError_t launch_embed_rows(const uint16_t *table, const int32_t *ids, int rows, int width,
                             uint16_t *out, hipStream_t s) {
  if (rows < 1 || width % 8)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_rows_kernel, dim3(rows), dim3(256), 0, s, table, ids, width, out);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rows(const uint16_t *x, int rows, int width, const uint16_t *w,
                                float eps, uint16_t *y, hipStream_t s) {
  if (rows < 1 || width < 8 || width % 8 || width > 8 * 256 * kRowChunks)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(rows), dim3(256), 0, s, x, width, w, eps, y);
  return hipGetLastError();
}


hipError_t launch_qk_prep(const QkPrepParams &p, hipStream_t s) {
  if (p.head_dim != 128 || p.tokens < 1 || p.pos0 < 0 || p.pos0 + p.tokens > p.capacity ||
      p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  const int blocks = (p.pos0 + p.tokens - 1) / attn::kBlock - p.pos0 / attn::kBlock + 1;
  hipLaunchKernelGGL(qk_prep_kernel, dim3(blocks, p.heads + 2 * p.kv_heads), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const AttnPrefillParams &p, hipStream_t s) {
  if (p.head_dim != 128 || p.tokens < 1 || p.kv_heads < 1 || p.heads < p.kv_heads ||
      p.heads % p.kv_heads || p.pos0 < 0 || p.pos0 + p.tokens > p.capacity ||
      p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  const float qscale = float(std::pow(128.0, -0.5)) * 1.4426950408889634f;
  if (p.heads * ((p.tokens + 63) / 64) >= attn::kTile64MinGroups)
    hipLaunchKernelGGL(attn_prefill_kernel<true>, dim3(p.heads, (p.tokens + 63) / 64), dim3(256),
                       0, s, p, qscale);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<false>, dim3(p.heads, (p.tokens + 31) / 32), dim3(256),
                       0, s, p, qscale);
  return hipGetLastError();
}

}  // namespace yuear
