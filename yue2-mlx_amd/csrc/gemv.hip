// bf16 GEMV for batch 1..8 decode projections on gfx950: one kernel per
// projection (the workgroup body is gemv_core.h). Batches of 3..8 rows go to
// the MFMA form (gemv_mfma.hip).
#include "common.h"
#include "gemv_core.h"
#include "kernels.h"

namespace yuear {

namespace {

template <int B, int KC, int R, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  extern __shared__ u32x4 xs[];  // [B][nch] activation chunks (bf16 x 8)
  __shared__ float red[B][4];
  gemv_block<B, KC, R, EPI>(p, blockIdx.x, xs, red);
}

template <int B, int KC, int R, int EPI>
hipError_t launch_bkre(const GemvParams &p, hipStream_t s) {
  const int rows_per_block = 4 * R;
  const int blocks = (p.n + rows_per_block - 1) / rows_per_block;
  const size_t lds = size_t(B) * (p.k >> 3) * sizeof(u32x4);
  auto kern = gemv_kernel<B, KC, R, EPI>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess)
      return e;
  }
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, p);
  return hipGetLastError();
}

template <int B, int KC, int R>
hipError_t launch_bkr(const GemvParams &p, hipStream_t s) {
  switch (p.epilogue) {
  case kEpiStore: return launch_bkre<B, KC, R, kEpiStore>(p, s);
  case kEpiResidual: return launch_bkre<B, KC, R, kEpiResidual>(p, s);
  case kEpiSwiGLU:
    if constexpr (R % 2 == 0)
      return launch_bkre<B, KC, R, kEpiSwiGLU>(p, s);
    break;
  }
  return hipErrorInvalidValue;
}

template <int B, int R>
hipError_t launch_b(const GemvParams &p, hipStream_t s) {
  const int kc = ((p.k >> 3) + 63) / 64;
  if (kc <= 1) return launch_bkr<B, 1, R>(p, s);
  if (kc <= 2) return launch_bkr<B, 2, R>(p, s);
  if (kc <= 4) return launch_bkr<B, 4, R>(p, s);
  if (kc <= 6) return launch_bkr<B, 6, R>(p, s);
  if (kc <= 8) return launch_bkr<B, 8, R>(p, s);
  if (kc <= 12) return launch_bkr<B, 12, R>(p, s);
  if (kc <= 16) return launch_bkr<B, 16, R>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemv(const GemvParams &p, hipStream_t s) {
  // rows must not overlap: activation rows (read, or written as the gather's
  // copy-out) at least k apart, output rows at least the output width apart
  const int out_n = p.epilogue == kEpiSwiGLU ? p.n / 2 : p.n;
  if (p.k < 8 || p.k % 8 || p.k > 8192 || p.n < 1 || p.batch < 1 || p.batch > 8 ||
      (p.x_stride % 8 && !p.embed) || (p.epilogue == kEpiSwiGLU && p.n % 2) ||
      ((!p.embed || p.x_out) && p.x_stride < p.k) || p.y_stride < out_n)
    return hipErrorInvalidValue;
  if (p.bits && p.batch <= 2)  // quantized weights (qgemv.hip)
    return launch_qgemv(p, s);
  if (gemv_mfma_supported(p))  // 3..8 rows: MFMA (gemv_mfma.hip)
    return launch_gemv_mfma(p, s);
  // Rows per wave. Batch 1: one row (QKV 5120 rows = 1280 workgroups, o_proj
  // 768, lm_head 20992: whole multiples of the 256 CUs, measured 4-7% faster
  // per launch than two rows on MI355X); the SwiGLU epilogue needs its
  // (gate, up) pair in one wave. Batch 2: one row as well (QKV 9.1 against
  // 9.4 us, o_proj 6.1 against 6.8), except for the lm_head-sized grids,
  // where two rows keep ~12 KiB of weight loads in flight per wave
  // (73 against 77 us); K = 8192 uses one row.
  const bool wide = p.k > 4096;
  const bool two = p.epilogue == kEpiSwiGLU ||
                   (!wide && (p.batch > 2 || (p.batch == 2 && p.n >= 32768)));
  if (p.batch == 1) return two ? launch_b<1, 2>(p, s) : launch_b<1, 1>(p, s);
  if (p.batch == 2) return two ? launch_b<2, 2>(p, s) : launch_b<2, 1>(p, s);
  if (p.batch <= 4) return two ? launch_b<4, 2>(p, s) : launch_b<4, 1>(p, s);
  return two ? launch_b<8, 2>(p, s) : launch_b<8, 1>(p, s);
}

}  // namespace yuear
