// Prompt prefill kernels on gfx950: MFMA bf16 GEMM for the projections,
// row-wise RMSNorm / embedding / SwiGLU, q/k RMSNorm + RoPE + KV append, and
// an MFMA causal attention with fp32 opmath.
//
// Reference: native/src/ar.cpp:246-301 (hidden() over T > 1 tokens) and
// native/src/sampling.cpp:152-183 (prefill). The reference upcasts Q/K/V to
// fp32 for the causal SDPA (ar.cpp:284-291); the attention kernel here forms
// exact products on MFMA, keeps scores, softmax and all sums in fp32 and
// rounds only the output to bf16.
#include <cmath>

#include "attn_core.h"
#include "attn_tile.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// GEMM: C[m][n] = sum_k A[m][k] W[n][k] (A tokens x hidden, W row-major
// weights), fp32 accumulation on v_mfma_f32_32x32x16_bf16, bf16 output.
// Block tile 128 x 128 x 64, four waves in a 2 x 2 arrangement of 64 x 64
// wave tiles (2 x 2 MFMA tiles each). LDS holds one A and one W tile with
// rows padded to 72 elements; the next K slab is prefetched into registers
// while the current one feeds the MFMAs. Blocks are renumbered so that the
// blocks sharing a weight tile land on the same XCD (shared L2).
// ---------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64, LDSW = BK + 8;

__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  __shared__ uint16_t As[BM * LDSW];
  __shared__ uint16_t Bs[BN * LDSW];
  const int tiles_m = (p.m + BM - 1) / BM;
  const int nb = gridDim.x;
  const int bid = blockIdx.x;
  const int per = nb / 8, rem = nb % 8, xcd = bid % 8, slot = bid / 8;
  const int logical = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = logical / tiles_m, m_tile = logical % tiles_m;
  const int m0 = m_tile * BM, n0 = n_tile * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global -> register staging: 4 x 16 B of A and of W per thread
  u32x4 ra[4], rb[4];
  auto load = [&](int k0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c, row = idx >> 3, col = (idx & 7) * 8;
      const int am = m0 + row, bn = n0 + row;
      ra[c] = am < p.m ? *reinterpret_cast<const u32x4 *>(p.a + size_t(am) * p.lda + k0 + col)
                       : u32x4{0u, 0u, 0u, 0u};
      rb[c] = bn < p.n ? __builtin_nontemporal_load(
                             reinterpret_cast<const u32x4 *>(p.w + size_t(bn) * p.k + k0 + col))
                       : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c, row = idx >> 3, col = (idx & 7) * 8;
      *reinterpret_cast<u32x4 *>(&As[row * LDSW + col]) = ra[c];
      *reinterpret_cast<u32x4 *>(&Bs[row * LDSW + col]) = rb[c];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  load(0);
  for (int k0 = 0; k0 < p.k; k0 += BK) {
    __syncthreads();
    store();
    __syncthreads();
    if (k0 + BK < p.k)
      load(k0 + BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      bf16x8_t af[2], bf[2];
      const int kk = ks + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t *>(&As[(wm * 64 + i * 32 + (lane & 31)) * LDSW + kk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const bf16x8_t *>(&Bs[(wn * 64 + j * 32 + (lane & 31)) * LDSW + kk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: lane holds column (lane % 32), rows 8(r/4) + 4(lane/32) + r%4
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= p.n)
        continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m) {
          uint16_t *dst = p.c + size_t(row) * p.ldc + col;
          float v = acc[i][j][r];
          if (p.residual)
            v = bf2f(*dst) + rbf(v);
          *dst = f2bf(v);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Large GEMM (prefill chunks with at least ~240 such tiles, e.g. QKV and
// gate/up at 3000 tokens): block tile 256 x 256 x 64,
// eight waves (two per SIMD) in a 2 x 4 arrangement of 128 x 64 wave tiles
// (4 x 2 MFMA 32x32x16 tiles, 128 fp32 accumulators per lane), so each A
// fragment read from LDS feeds two MFMAs and each W fragment four. LDS is
// double-buffered (2 x (A + W) x 256 rows x 72 elements = 144 KiB of the
// 160 KiB): the next K slab's global loads are in flight while the current
// slab feeds the MFMAs, and one barrier per slab suffices.
// ---------------------------------------------------------------------------
constexpr int GM = 256, GN = 256, GK = 64, GP = GK + 8;
constexpr size_t kGemm256Lds = size_t(2) * 2 * 256 * GP * sizeof(uint16_t);

__global__ __launch_bounds__(512) void gemm256_kernel(GemmParams p) {
  extern __shared__ uint16_t glds[];
  const int tiles_m = (p.m + GM - 1) / GM;
  const int nb = gridDim.x;
  const int bid = blockIdx.x;
  const int per = nb / 8, rem = nb % 8, xcd = bid % 8, slot = bid / 8;
  const int logical = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = logical / tiles_m, m_tile = logical % tiles_m;
  const int m0 = m_tile * GM, n0 = n_tile * GN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;  // rows wm * 128, cols wn * 64
  auto abuf = [&](int b) { return glds + size_t(b) * (2 * 256 * GP); };
  auto bbuf = [&](int b) { return glds + size_t(b) * (2 * 256 * GP) + 256 * GP; };

  // global -> register staging: 4 x 16 B of A and of W per thread
  u32x4 ra[4], rb[4];
  auto load = [&](int k0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 512 * c, row = idx >> 3, col = (idx & 7) * 8;
      const int am = m0 + row, bn = n0 + row;
      ra[c] = am < p.m ? *reinterpret_cast<const u32x4 *>(p.a + size_t(am) * p.lda + k0 + col)
                       : u32x4{0u, 0u, 0u, 0u};
      rb[c] = bn < p.n ? __builtin_nontemporal_load(
                             reinterpret_cast<const u32x4 *>(p.w + size_t(bn) * p.k + k0 + col))
                       : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int b) {
    uint16_t *As = abuf(b), *Bs = bbuf(b);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 512 * c, row = idx >> 3, col = (idx & 7) * 8;
      *reinterpret_cast<u32x4 *>(&As[row * GP + col]) = ra[c];
      *reinterpret_cast<u32x4 *>(&Bs[row * GP + col]) = rb[c];
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  const int nk = p.k / GK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more)
      load((kt + 1) * GK);
    const uint16_t *As = abuf(cur), *Bs = bbuf(cur);
#pragma unroll
    for (int ks = 0; ks < GK; ks += 16) {
      bf16x8_t af[4], bf[2];
      const int kk = ks + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t *>(&As[(wm * 128 + i * 32 + (lane & 31)) * GP + kk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const bf16x8_t *>(&Bs[(wn * 64 + j * 32 + (lane & 31)) * GP + kk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more)
      store(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column (lane % 32), rows 8(r/4) + 4(lane/32) + r%4
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= p.n)
        continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m) {
          uint16_t *dst = p.c + size_t(row) * p.ldc + col;
          float v = acc[i][j][r];
          if (p.residual)
            v = bf2f(*dst) + rbf(v);
          *dst = f2bf(v);
        }
      }
    }
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint16_t *table, const int32_t *ids,
                                                         int width, uint16_t *out) {
  const int r = blockIdx.x;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(table + size_t(ids[r]) * width);
  u32x4 *dst = reinterpret_cast<u32x4 *>(out + size_t(r) * width);
  for (int c = threadIdx.x; c < width / 8; c += 256)
    dst[c] = src[c];
}

// ar.cpp:30-35 per row.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const uint16_t *x, int width,
                                                            const uint16_t *w, float eps,
                                                            uint16_t *y) {
  __shared__ float red[4];
  const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(x + size_t(r) * width);
  float ss = 0.f;
  for (int c = threadIdx.x; c < width / 8; c += 256) {
    const u32x4 v = src[c];
    const uint32_t vi[4] = {v.x, v.y, v.z, v.w};
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
  for (int c = threadIdx.x; c < width / 8; c += 256) {
    const u32x4 v = src[c], g = g4[c];
    const uint32_t vi[4] = {v.x, v.y, v.z, v.w}, gi[4] = {g.x, g.y, g.z, g.w};
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

// ar.cpp:36-51 on interleaved (gate_i, up_i) columns.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const uint16_t *gu, int f,
                                                          uint16_t *out) {
  const int r = blockIdx.x;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(gu + size_t(r) * 2 * f);
  for (int i = threadIdx.x; i < f; i += 256) {
    const uint32_t pair = src[i];
    const float g = bflo(pair), u = bfhi(pair);
    const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
    out[size_t(r) * f + i] = f2bf(act * u);
  }
}

// q/k RMSNorm + RoPE for T tokens, K/V append (ar.cpp:268-282).
__global__ __launch_bounds__(256) void qk_prep_kernel(QkPrepParams p) {
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos = p.pos0 + t;
  const uint16_t *row = p.qkv + size_t(t) * p.qkv_stride;
  const uint16_t *cs = p.rope_cos + size_t(pos) * 64;
  const uint16_t *sn = p.rope_sin + size_t(pos) * 64;
  const int nh = p.heads + 2 * p.kv_heads;
  for (int h = wave + 4 * blockIdx.y; h < nh; h += 4 * gridDim.y) {
    const uint32_t pair = reinterpret_cast<const uint32_t *>(row + size_t(h) * 128)[lane];
    float y0 = bflo(pair), y1 = bfhi(pair);
    uint32_t *dst;
    if (h < p.heads) {
      norm_rope_head(y0, y1, p.q_norm, p.eps, cs, sn, lane, y0, y1);
      dst = reinterpret_cast<uint32_t *>(p.q_out + (size_t(t) * p.heads + h) * 128);
    } else if (h < p.heads + p.kv_heads) {
      const int kvh = h - p.heads;
      norm_rope_head(y0, y1, p.k_norm, p.eps, cs, sn, lane, y0, y1);
      dst = reinterpret_cast<uint32_t *>(p.k_cache + (size_t(kvh) * p.capacity + pos) * 128);
    } else {  // V: dims 2 lane, 2 lane + 1 into the slot's 32-key block column
      const int kvh = h - p.heads - p.kv_heads;
      uint16_t *vh = p.v_cache + size_t(kvh) * p.capacity * 128;
      vh[attn::v_index(pos, 2 * lane)] = f2bf(y0);
      vh[attn::v_index(pos, 2 * lane + 1)] = f2bf(y1);
      continue;
    }
    dst[lane] = uint32_t(f2bf(y0)) | (uint32_t(f2bf(y1)) << 16);
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
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_prefill_kernel(AttnPrefillParams p, float qscale) {
  __shared__ attn::TileLds sh;
  using attn::D;
  const int h = blockIdx.x;
  const int tile = gridDim.y - 1 - blockIdx.y;  // longest causal range first
  const int q0 = tile * 32;
  const int kvh = h / (p.heads / p.kv_heads);
  attn::QueryTile t;
  t.kc = reinterpret_cast<const u32x4 *>(p.k_cache) + size_t(kvh) * p.capacity * (D / 8);
  t.vc = reinterpret_cast<const u32x4 *>(p.v_cache) + size_t(kvh) * p.capacity * (D / 8);
  t.nq = min(32, p.tokens - q0);
  t.kend = p.pos0 + q0 + t.nq;
  t.causal_pos = p.pos0 + q0;
  t.q = p.q + (size_t(q0) * p.heads + h) * D;
  t.q_stride = size_t(p.heads) * D;
  t.out = p.out + (size_t(q0) * p.heads + h) * D;
  t.out_stride = size_t(p.heads) * D;
  attn::attn_query_tile(t, qscale, sh);
}

}  // namespace

hipError_t launch_gemm(const GemmParams &p, hipStream_t s) {
  if (p.m < 1 || p.n < 1 || p.k % BK || p.lda % 8 || p.ldc < p.n)
    return hipErrorInvalidValue;
  const int big_blocks = ((p.m + GM - 1) / GM) * ((p.n + GN - 1) / GN);
  if (big_blocks >= 240) {  // enough 256 x 256 tiles to fill the GPU (K % 64 == 0 here)
    static bool lds_set = false;
    if (!lds_set) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm256_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         int(kGemm256Lds));
      if (e != hipSuccess)
        return e;
      lds_set = true;
    }
    hipLaunchKernelGGL(gemm256_kernel, dim3(big_blocks), dim3(512), kGemm256Lds, s, p);
    return hipGetLastError();
  }
  const int blocks = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  hipLaunchKernelGGL(gemm_kernel, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_embed_rows(const uint16_t *table, const int32_t *ids, int rows, int width,
                             uint16_t *out, hipStream_t s) {
  if (rows < 1 || width % 8)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_rows_kernel, dim3(rows), dim3(256), 0, s, table, ids, width, out);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rows(const uint16_t *x, int rows, int width, const uint16_t *w,
                                float eps, uint16_t *y, hipStream_t s) {
  if (rows < 1 || width % 8)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(rows), dim3(256), 0, s, x, width, w, eps, y);
  return hipGetLastError();
}

hipError_t launch_swiglu_rows(const uint16_t *gu, int rows, int f, uint16_t *out, hipStream_t s) {
  if (rows < 1 || f < 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3(rows), dim3(256), 0, s, gu, f, out);
  return hipGetLastError();
}

hipError_t launch_qk_prep(const QkPrepParams &p, hipStream_t s) {
  if (p.head_dim != 128 || p.tokens < 1 || p.pos0 < 0 || p.pos0 + p.tokens > p.capacity ||
      p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  const int nh = p.heads + 2 * p.kv_heads;
  const int gy = (nh + 3) / 4;
  hipLaunchKernelGGL(qk_prep_kernel, dim3(p.tokens, gy), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const AttnPrefillParams &p, hipStream_t s) {
  if (p.head_dim != 128 || p.tokens < 1 || p.kv_heads < 1 || p.heads % p.kv_heads ||
      p.pos0 + p.tokens > p.capacity || p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  const float qscale = float(std::pow(128.0, -0.5)) * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(p.heads, (p.tokens + 31) / 32), dim3(256), 0, s,
                     p, qscale);
  return hipGetLastError();
}

}  // namespace yuear
