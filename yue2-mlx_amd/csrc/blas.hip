// Prefill projections (plain bf16 GEMMs, fp32 accumulation, one bf16
// rounding: ar.cpp:20-29 over T tokens) on hipBLASLt, the vendor GEMM
// library: at the 3B prefill shapes it runs 1.1-1.3 PFLOP/s against
// 0.6-0.8 for the MFMA GEMM this file replaced, with bit-identical outputs.
//
// Row-major C[m][ldc] = A[m][lda] . W[n][k]^T is the column-major product
// C^T (n x m) = op_T(W as k x n, ld k) . (A as k x m, ld lda). The residual
// form (o_proj, down: x = bf16(x + bf16(acc)), ar.cpp:292-298) writes the
// product to a scratch matrix first and adds it in a second kernel, keeping
// the reference's two rounding points.
//
// One library handle per device, created on first use; the algorithm chosen
// by the library's heuristic (allowed up to kGemmWorkspace bytes of
// workspace) is cached per shape. The workspace belongs to the caller (one
// per stream that runs GEMMs), so concurrent streams never share one.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

struct Algo {
  hipblasLtMatmulAlgo_t algo;
  size_t workspace;  // bytes the algorithm needs
};

struct Lt {
  hipblasLtHandle_t handle = nullptr;
  std::map<std::tuple<int, int, int, int, int>, Algo> algos;
};

std::mutex g_mu;
std::map<int, Lt> g_lt;  // per device

hipError_t status_error(hipblasStatus_t st) {
  return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorUnknown;
}

// x[i] = bf16(x[i] + t[i]) over rows [m][ld] (n columns), 8 columns per thread.
__global__ __launch_bounds__(256) void add_rows_kernel(uint16_t *x, const uint16_t *t, int m, int n,
                                                       int ld) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const int per_row = n / 8;
  if (idx >= (long long)m * per_row)
    return;
  const int r = int(idx / per_row), c = int(idx % per_row) * 8;
  u32x4 *xp = reinterpret_cast<u32x4 *>(x + size_t(r) * ld + c);
  const u32x4 tv = *reinterpret_cast<const u32x4 *>(t + size_t(r) * ld + c);
  const u32x4 xv = *xp;
  const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w}, ts[4] = {tv.x, tv.y, tv.z, tv.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = uint32_t(f2bf(bflo(xs[q]) + bflo(ts[q]))) |
           (uint32_t(f2bf(bfhi(xs[q]) + bfhi(ts[q]))) << 16);
  *xp = u32x4{o[0], o[1], o[2], o[3]};
}

// Validates p, creates the device's handle on first use and finds (or
// caches) the algorithm for p's shape; desc / layouts are created for the
// caller, who destroys them. Called with g_mu held.
hipblasStatus_t prepare(const GemmParams &p, Lt *&lt, const Algo *&algo, hipblasLtMatmulDesc_t &desc,
                        hipblasLtMatrixLayout_t &la, hipblasLtMatrixLayout_t &lb,
                        hipblasLtMatrixLayout_t &lc) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return HIPBLAS_STATUS_INTERNAL_ERROR;
  lt = &g_lt[dev];
  if (!lt->handle && hipblasLtCreate(&lt->handle) != HIPBLAS_STATUS_SUCCESS) {
    lt->handle = nullptr;
    return HIPBLAS_STATUS_NOT_INITIALIZED;
  }
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasStatus_t st = hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, p.k, p.n, p.k);
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, p.k, p.m, p.lda);
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatrixLayoutCreate(&lc, HIP_R_16BF, p.n, p.m, p.ldc);
  if (st != HIPBLAS_STATUS_SUCCESS)
    return st;
  const auto key = std::make_tuple(p.m, p.n, p.k, p.lda, p.ldc);
  auto it = lt->algos.find(key);
  if (it == lt->algos.end()) {
    hipblasLtMatmulPreference_t pref = nullptr;
    st = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t ws = kGemmWorkspace;
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                 &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t result[1];
    int found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulAlgoGetHeuristic(lt->handle, desc, la, lb, lc, lc, pref, 1, result, &found);
    if (pref)
      hipblasLtMatmulPreferenceDestroy(pref);
    if (st == HIPBLAS_STATUS_SUCCESS && found < 1)
      st = HIPBLAS_STATUS_NOT_SUPPORTED;
    if (st != HIPBLAS_STATUS_SUCCESS)
      return st;
    it = lt->algos.emplace(key, Algo{result[0].algo, result[0].workspaceSize}).first;
  }
  algo = &it->second;
  return HIPBLAS_STATUS_SUCCESS;
}

void destroy(hipblasLtMatmulDesc_t desc, hipblasLtMatrixLayout_t la, hipblasLtMatrixLayout_t lb,
             hipblasLtMatrixLayout_t lc) {
  if (lc) hipblasLtMatrixLayoutDestroy(lc);
  if (lb) hipblasLtMatrixLayoutDestroy(lb);
  if (la) hipblasLtMatrixLayoutDestroy(la);
  if (desc) hipblasLtMatmulDescDestroy(desc);
}

bool valid(const GemmParams &p) {
  return p.m >= 1 && p.n >= 1 && p.k >= 1 && p.lda >= p.k && p.ldc >= p.n && p.a && p.w && p.c;
}

}  // namespace

hipError_t gemm_workspace_bytes(const GemmParams &p, size_t *bytes) {
  if (!valid(p) || !bytes)
    return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lock(g_mu);
  Lt *lt = nullptr;
  const Algo *algo = nullptr;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  const hipblasStatus_t st = prepare(p, lt, algo, desc, la, lb, lc);
  destroy(desc, la, lb, lc);
  if (st != HIPBLAS_STATUS_SUCCESS)
    return status_error(st);
  *bytes = algo->workspace;
  return hipSuccess;
}

hipError_t launch_gemm(const GemmParams &p, uint16_t *scratch, void *workspace,
                       size_t workspace_bytes, hipStream_t s) {
  if (!valid(p) || (p.residual && (!scratch || p.n % 8 || p.ldc % 8)))
    return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lock(g_mu);
  Lt *lt = nullptr;
  const Algo *algo = nullptr;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasStatus_t st = prepare(p, lt, algo, desc, la, lb, lc);
  if (st == HIPBLAS_STATUS_SUCCESS && algo->workspace > (workspace ? workspace_bytes : 0)) {
    destroy(desc, la, lb, lc);
    return hipErrorInvalidValue;  // the caller's workspace is too small
  }
  if (st == HIPBLAS_STATUS_SUCCESS) {
    const float alpha = 1.f, beta = 0.f;
    uint16_t *d = p.residual ? scratch : p.c;
    st = hipblasLtMatmul(lt->handle, desc, &alpha, p.w, la, p.a, lb, &beta, d, lc, d, lc,
                         &algo->algo, workspace, workspace ? workspace_bytes : 0, s);
  }
  destroy(desc, la, lb, lc);
  if (st != HIPBLAS_STATUS_SUCCESS)
    return status_error(st);
  if (p.residual) {
    const long long threads = (long long)p.m * (p.n / 8);
    hipLaunchKernelGGL(add_rows_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s,
                       p.c, scratch, p.m, p.n, p.ldc);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace yuear
