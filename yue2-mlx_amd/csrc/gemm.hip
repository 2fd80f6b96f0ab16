// Prefill projections on gfx950 MFMA: C[m][n] = bf16(sum_k A[m][k] W[n][k])
// (A: token rows, W: row-major weights, both K-contiguous), fp32 accumulation
// with one rounding, or the residual form C = bf16(C + bf16(acc)) with both
// of the reference's rounding points (native/src/ar.cpp:20-29, 292-298).
//
// Tiling: a workgroup owns a BM x BN tile of C and walks K in 64-wide steps.
// Its WM x WN waves each own a (BM / WM) x (BN / WN) sub-tile of 32 x 32
// v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators). Each K step's A and W
// slabs (BM x 64 and BN x 64 bf16) are loaded from global memory with
// 16-byte buffer loads (rows past M or N read as zero), parked in registers
// while the previous step computes, then written to the other half of a
// two-stage LDS ring (rows padded to 72 elements against bank conflicts):
// one barrier per K step. MFMA operands are read from LDS as 16-byte
// fragments: lane l holds row (l % 32), k 8 (l / 32) + [0, 8) of a 16-wide K
// sub-step; the 32 x 32 result leaves lane l with column (l % 32), rows
// 8 (r / 4) + 4 (l / 32) + r % 4 for its 16 values r.
//
// Shapes: 256 x 256 tiles (8 waves, 147 KiB of LDS, one workgroup per CU)
// when they give at least one tile per CU, else 128 x 128 tiles (4 waves,
// 74 KiB, two per CU).
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int LDSK = BK + 8;  // LDS row stride in elements (144 bytes)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           uint32_t(bytes > 0xffffffffu ? 0xffffffffu : bytes),
                                           0x00020000);
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // MFMA tiles per wave
  constexpr int CPR = BK / 8;                          // 16-byte chunks per slab row
  constexpr int ACH = BM * CPR / NT, BCH = BN * CPR / NT;
  static_assert(ACH * NT == BM * CPR && BCH * NT == BN * CPR, "slab chunks per thread");
  extern __shared__ uint16_t lds[];
  // stage st: A slab at lds + st (BM + BN) LDSK, W slab BM LDSK after it
  auto as = [&](int st) { return lds + st * (BM + BN) * LDSK; };
  auto bs = [&](int st) { return lds + st * (BM + BN) * LDSK + BM * LDSK; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const auto ra = rows_rsrc(p.a + size_t(m0) * p.lda, size_t(max(p.m - m0, 0)) * p.lda * 2);
  const auto rw = rows_rsrc(p.w + size_t(n0) * p.k, size_t(max(p.n - n0, 0)) * p.k * 2);

  u32x4 sa[ACH], sb[BCH];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      sa[i] = __builtin_amdgcn_raw_buffer_load_b128(
          ra, uint32_t((size_t(row) * p.lda + k0 + kc * 8) * 2), 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      sb[i] = __builtin_amdgcn_raw_buffer_load_b128(
          rw, uint32_t((size_t(row) * p.k + k0 + kc * 8) * 2), 0, 0);
    }
  };
  auto stash = [&](int st) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4 *>(as(st) + (c / CPR) * LDSK + (c % CPR) * 8) = sa[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4 *>(bs(st) + (c / CPR) * LDSK + (c % CPR) * 8) = sb[i];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  const int steps = p.k / BK;
  load(0);
  stash(0);
  __syncthreads();
  const int frow = lane & 31, fk = 8 * (lane >> 5);
  for (int kt = 0; kt < steps; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < steps)
      load((kt + 1) * BK);
    const uint16_t *a_s = as(st) + (wm * (BM / WM) + frow) * LDSK + fk;
    const uint16_t *b_s = bs(st) + (wn * (BN / WN) + frow) * LDSK + fk;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8_t af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t *>(a_s + i * 32 * LDSK + s * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const bf16x8_t *>(b_s + j * 32 * LDSK + s * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < steps)
      stash(st ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column (lane % 32), rows 8 (r / 4) + 4 (lane / 32) + r % 4
  const int col = lane & 31, rsub = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + j * 32 + col;
      if (n >= p.n)
        continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * (BM / WM) + i * 32 + 8 * (r >> 2) + rsub + (r & 3);
        if (m < p.m) {
          uint16_t *c = p.c + size_t(m) * p.ldc + n;
          const float v = acc[i][j][r];
          *c = p.residual ? f2bf(bf2f(*c) + rbf(v)) : f2bf(v);
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_tile(const GemmParams &p, hipStream_t s) {
  auto kern = gemm_kernel<BM, BN, WM, WN>;
  const size_t lds = size_t(2) * (BM + BN) * LDSK * 2;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
  if (e != hipSuccess)
    return e;
  hipLaunchKernelGGL(kern, dim3((p.n + BN - 1) / BN, (p.m + BM - 1) / BM), dim3(WM * WN * 64),
                     lds, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const GemmParams &p, hipStream_t s) {
  if (p.m < 1 || p.n < 1 || p.k < BK || p.k % BK || p.lda < p.k || p.ldc < p.n || p.lda % 8 ||
      !p.a || !p.w || !p.c)
    return hipErrorInvalidValue;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  const long tiles256 = long((p.m + 255) / 256) * ((p.n + 255) / 256);
  if (tiles256 >= cus)
    return launch_tile<256, 256, 2, 4>(p, s);
  return launch_tile<128, 128, 2, 2>(p, s);
}

}  // namespace yuear
