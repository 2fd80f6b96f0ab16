// Batched decode projections (3..8 independent rows) on MFMA, gfx950.
//
// y[b, r] = x[b, :] . W[row(r), :] with fp32 accumulation and one bf16
// rounding (native/src/ar.cpp:20-29), for the batched-sequence decode where
// a VALU GEMV would do 8 dot products per weight element. The weight stream
// is still read exactly once: the work is HBM-bound, v_mfma_f32_16x16x32_bf16
// only keeps the arithmetic off the VALU.
//
// Workgroup: 16 consecutive weight rows; its WAVES waves split K, wave w
// owning k in [w KW, (w + 1) KW), KW = KSTEPS * 32. MFMA operands per k-step
// (layouts of the 16x16x32 bf16 form): A = 16 weight rows x 32 k, lane l
// holding row l % 16, k 8 (l / 16) + [0, 8) (one 16-byte load); B = 32 k x
// 16 batch columns, lane l holding column l % 16 (zero beyond the batch)
// from the staged activations; D = 16 rows x 16 columns, lane l holding
// column l % 16, rows 4 (l / 16) + [0, 4).
//
// Rows that need a gather (layer 0's embedding) or an RMSNorm prologue
// (ar.cpp:30-35) are prepared once by a small row kernel into p.stage;
// re-normalising all rows in every workgroup costs more than the weight
// stream it hides behind. In the main kernel each thread first loads one
// 16-byte activation column of all rows, then all KSTEPS weight loads of its
// wave (non-temporal), so the staging waits only for the former (the
// vector-memory counter drains in issue order). Rows are staged in LDS
// padded by 16 bytes (conflict-free 16-byte reads across the 16 batch
// columns). The waves' D tiles are summed through LDS in wave order, then
// the epilogue (store / residual / SwiGLU) runs one thread per (row, column).
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Row preparation for the batched form (grid = batch rows, 256 threads):
// gather from the embedding (copy-out to x_out) and/or RMSNorm with the
// rounding points of ar.cpp:30-35, written to p.stage.
__global__ __launch_bounds__(256) void stage_rows_kernel(GemvParams p) {
  __shared__ float red[4];
  constexpr int kMaxChunks = 4;  // k <= 8192
  const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.k >> 3;
  const uint16_t *src;
  if (p.embed) {
    const int t = min(max(p.tokens[b], 0), p.embed_rows - 1);
    src = p.embed + size_t(t) * p.k;
  } else {
    src = p.x + size_t(b) * p.x_stride;
  }
  const u32x4 *s4 = reinterpret_cast<const u32x4 *>(src);
  const u32x4 *g4 = reinterpret_cast<const u32x4 *>(p.norm_w ? p.norm_w : src);
  u32x4 *dst = reinterpret_cast<u32x4 *>(p.stage + size_t(b) * p.k);
  // one round of loads: this thread's chunks c = t + 256 i and their gains
  u32x4 v[kMaxChunks], g[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = min(int(threadIdx.x) + 256 * i, nch - 1);
    v[i] = s4[c];
    g[i] = g4[c];
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c >= nch)
      continue;
    if (p.x_out)
      reinterpret_cast<u32x4 *>(p.x_out + size_t(b) * p.x_stride)[c] = v[i];
    const uint32_t w4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = bflo(w4[q]), hi = bfhi(w4[q]);
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  if (!p.norm_w) {
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) {
      const int c = threadIdx.x + 256 * i;
      if (c < nch)
        dst[c] = v[i];
    }
    return;
  }
  ss = wave_sum(ss);
  if (lane == 0)
    red[wave] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = rbf(1.0f / __builtin_sqrtf(total / float(p.k) + p.eps));
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c >= nch)
      continue;
    const uint32_t vi[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    const uint32_t gi[4] = {g[i].x, g[i].y, g[i].z, g[i].w};
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

template <int WAVES, int KSTEPS, int EPI>
__global__ __launch_bounds__(WAVES * 64) void gemv_mfma_kernel(GemvParams p) {
  extern __shared__ u32x4 lds[];
  constexpr int NT = WAVES * 64;
  constexpr int K = WAVES * KSTEPS * 32;
  constexpr int NCH = K / 8;           // 16-byte chunks per activation row
  constexpr int ROWC = NCH + 1;        // staged row stride (chunks): +16 bytes of padding
  static_assert(NCH <= NT, "one activation column per thread");
  float *red = reinterpret_cast<float *>(lds + 8 * ROWC);  // [WAVES][16][16]

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int B = p.batch;
  const int n0 = blockIdx.x * 16;
  const int c = min(int(threadIdx.x), NCH - 1);  // this thread's activation column

  // 1. activation column c of every row first (rows past the batch clamped)
  u32x4 xr[8];
#pragma unroll
  for (int b = 0; b < 8; ++b)
    xr[b] = reinterpret_cast<const u32x4 *>(p.x + size_t(min(b, B - 1)) * p.x_stride)[c];
  // keep these loads ahead of the weight stream (the scheduler may otherwise
  // sink some below it, and the staging would then wait for every weight)
  __builtin_amdgcn_sched_barrier(0);

  // 2. this wave's weight stream: row n0 + l % 16 (clamped; mapped for the
  // lm_head phases), k = wave * KW + 32 s + 8 (l / 16); from the tiled copy
  // when there is one (the 16-byte piece of (row, k-step) sits at
  // ((row / 16) (K / 32) + k-step) 64 + row % 16 + 16 (l / 16))
  u32x4 a[KSTEPS];
  {
    const int lr = min(n0 + (lane & 15), p.n - 1);
    const int row = lr < p.seg0_len ? p.seg0_start + lr : p.seg1_start + (lr - p.seg0_len);
    const bool tiled = p.w_tiled != nullptr;
    const u32x4 *w =
        tiled ? reinterpret_cast<const u32x4 *>(p.w_tiled) +
                    (size_t(row >> 4) * (K / 32) + wave * KSTEPS) * 64 + (row & 15) + 16 * (lane >> 4)
              : reinterpret_cast<const u32x4 *>(p.w + size_t(row) * K) + wave * (KSTEPS * 4) +
                    (lane >> 4);
    const int step = tiled ? 64 : 4;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      a[s] = __builtin_nontemporal_load(w + step * s);
  }

  // 3. stage the activations in LDS
  if (int(threadIdx.x) < NCH) {
#pragma unroll
    for (int b = 0; b < 8; ++b)
      if (b < B)
        lds[b * ROWC + c] = xr[b];
  }
  __syncthreads();

  // 4. MFMA over this wave's K slice
  const int col = lane & 15;
  const bool live = col < B;
  const u32x4 *xrow = lds + min(col, B - 1) * ROWC + wave * (KSTEPS * 4) + (lane >> 4);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    const u32x4 bv = live ? xrow[4 * s] : u32x4{0u, 0u, 0u, 0u};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[s]), as_bf16x8(bv), acc, 0, 0, 0);
  }

  // 5. sum the waves' tiles (wave order), epilogue per (row, column)
#pragma unroll
  for (int t = 0; t < 4; ++t)
    red[(wave * 16 + 4 * (lane >> 4) + t) * 16 + col] = acc[t];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int i = threadIdx.x >> 4, j = threadIdx.x & 15;  // row n0 + i, column j
    float y = 0.f, y1 = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      y += red[(w * 16 + i) * 16 + j];
      if constexpr (EPI == kEpiSwiGLU)
        y1 += red[(w * 16 + (i | 1)) * 16 + j];
    }
    const int row = n0 + i;
    if (j < B && row < p.n) {
      uint16_t *yb = p.y + size_t(j) * p.y_stride;
      if constexpr (EPI == kEpiSwiGLU) {
        if ((i & 1) == 0) {  // rows (2m, 2m + 1) = (gate_m, up_m)
          const float g = rbf(y), u = rbf(y1);
          const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
          yb[row >> 1] = f2bf(act * u);
        }
      } else if constexpr (EPI == kEpiResidual) {
        yb[row] = f2bf(bf2f(yb[row]) + rbf(y));
      } else {
        yb[row] = f2bf(y);
      }
    }
  }
  if (p.advance && blockIdx.x == 0 && threadIdx.x < p.batch)
    p.advance[threadIdx.x] += 1;
}

template <int WAVES, int KSTEPS, int EPI>
hipError_t launch_wke(const GemvParams &p, hipStream_t s) {
  constexpr int K = WAVES * KSTEPS * 32;
  const size_t lds = size_t(8) * (K / 8 + 1) * 16 + size_t(WAVES) * 256 * 4;
  auto kern = gemv_mfma_kernel<WAVES, KSTEPS, EPI>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
  if (e != hipSuccess)
    return e;
  hipLaunchKernelGGL(kern, dim3((p.n + 15) / 16), dim3(WAVES * 64), lds, s, p);
  return hipGetLastError();
}

template <int WAVES, int KSTEPS>
hipError_t launch_wk(const GemvParams &p, hipStream_t s) {
  switch (p.epilogue) {
  case kEpiStore: return launch_wke<WAVES, KSTEPS, kEpiStore>(p, s);
  case kEpiResidual: return launch_wke<WAVES, KSTEPS, kEpiResidual>(p, s);
  case kEpiSwiGLU: return launch_wke<WAVES, KSTEPS, kEpiSwiGLU>(p, s);
  }
  return hipErrorInvalidValue;
}

__global__ __launch_bounds__(256) void tile_rows_kernel(const uint16_t *w, int n, int k,
                                                        uint16_t *out, size_t total) {
  const size_t o = size_t(blockIdx.x) * 256 + threadIdx.x;  // 16-byte piece of out
  if (o >= total)
    return;
  const int l = int(o & 63);
  const size_t blk = o >> 6;
  const int ks = k / 32;
  const size_t t = blk / ks;
  const int s = int(blk % ks);
  const size_t row = t * 16 + (l & 15);
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (row < size_t(n))
    v = reinterpret_cast<const u32x4 *>(w + row * k + 32 * s + 8 * (l >> 4))[0];
  reinterpret_cast<u32x4 *>(out)[o] = v;
}

}  // namespace

hipError_t launch_tile_rows(const uint16_t *w, int n, int k, uint16_t *out, hipStream_t s) {
  if (n < 1 || k < 32 || k % 32)
    return hipErrorInvalidValue;
  const size_t total = size_t((n + 15) / 16) * (k / 32) * 64;
  hipLaunchKernelGGL(tile_rows_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, w, n,
                     k, out, total);
  return hipGetLastError();
}

bool gemv_mfma_supported(const GemvParams &p) {
  return p.batch >= 3 && p.batch <= 8 && (p.x_stride % 8 == 0 || p.embed) &&
         (p.k == 3072 || p.k == 8192 || p.k == 2048 || p.k == 6144) &&
         (p.epilogue != kEpiSwiGLU || p.n % 2 == 0) &&
         (p.stage || (!p.norm_w && !p.embed && !p.x_out));
}

hipError_t launch_gemv_mfma(const GemvParams &p, hipStream_t s) {
  if (!gemv_mfma_supported(p) || p.n < 1)
    return hipErrorInvalidValue;
  GemvParams q = p;
  if (p.norm_w || p.embed || p.x_out) {  // prepare the rows once
    hipLaunchKernelGGL(stage_rows_kernel, dim3(p.batch), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      return e;
    q.x = p.stage;
    q.x_stride = p.k;
    q.norm_w = nullptr;
    q.embed = nullptr;
    q.x_out = nullptr;
  }
  switch (q.k) {
  case 3072: return launch_wk<8, 12>(q, s);   // 8 waves x 384 k (one column per thread)
  case 8192: return launch_wk<16, 16>(q, s);  // 16 waves x 512 k
  case 2048: return launch_wk<4, 16>(q, s);   // 4 waves x 512 k
  case 6144: return launch_wk<16, 12>(q, s);  // 16 waves x 384 k
  }
  return hipErrorInvalidValue;
}

}  // namespace yuear
