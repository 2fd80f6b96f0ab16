// Acoustic-model attention on gfx950 MFMA: the drop-in for nar_attention()
// (native/src/nar_attention.cpp:224-270) and its custom Metal kernel
// lyra_nar_precise_attention (nar_attention.cpp:63-218).
//
// Tensors are [batch, heads, tokens, 128] bf16 (q: Hq heads, Lq tokens; k, v:
// Hkv heads, Lk tokens; query head h reads kv head h / (Hq / Hkv)); the
// output has q's shape. Arithmetic of the reference kernel: fp32 scores of
// the bf16 operands scaled by scale * log2(e) (one fp32 constant), an exp2
// online softmax in fp32, P kept in fp32 for P.V ("precise" left operand),
// fp32 sums, bf16(o / l). causal (Lq == Lk, the conditioning prefill of
// nar.cpp:176) hides the keys after each query's own position.
//
// Structure: one workgroup per (batch, q head, 32-query tile); its 4 waves
// split the keys and merge in LDS (attn_tile.h, shared with the causal
// prefill attention). K is read row-major as given. The V^T operand wants 8 consecutive keys of one dim per lane, so V is first
// rewritten (nar_v_blocks_kernel) into 32-key blocks stored dim-major, the
// layout of the KV cache, in a caller-provided workspace; keys past Lk in the
// last block are zero there (and masked in the scores).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "attn_core.h"
#include "attn_tile.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

using attn::D;
using attn::f32x4;
using attn::kBlock;

// One 32-key block of one (batch, kv head): [32][128] row-major in, [128][32]
// out, through an LDS tile (rows padded to 136 elements: 272-byte rows keep
// the 16-byte stores aligned and spread the column reads over the banks).
__global__ __launch_bounds__(256) void nar_v_blocks_kernel(const uint16_t *v, int lk, int lkp,
                                                           uint16_t *vb) {
  __shared__ __align__(16) uint16_t tile[kBlock][D + 8];
  const size_t head = blockIdx.y;
  const int t0 = blockIdx.x * kBlock;
  for (int c = threadIdx.x; c < kBlock * D / 8; c += 256) {
    const int t = c / (D / 8), d8 = (c % (D / 8)) * 8;
    u32x4 val{0u, 0u, 0u, 0u};
    if (t0 + t < lk)
      val = *reinterpret_cast<const u32x4 *>(v + (head * lk + t0 + t) * D + d8);
    *reinterpret_cast<u32x4 *>(&tile[t][d8]) = val;
  }
  __syncthreads();
  uint16_t *dst = vb + (head * lkp + t0) * D;
  for (int c = threadIdx.x; c < kBlock * D / 8; c += 256) {
    const int d = c / (kBlock / 8), k8 = (c % (kBlock / 8)) * 8;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = uint32_t(tile[k8 + 2 * j][d]) | (uint32_t(tile[k8 + 2 * j + 1][d]) << 16);
    *reinterpret_cast<u32x4 *>(dst + d * kBlock + k8) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// T64: the 64-query tile with K/V shared through LDS (attn_query_tile64),
// chosen when it yields enough workgroups to fill the GPU; otherwise the
// 32-query tile whose four waves split the keys.
template <bool T64>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(T64 ? attn::kTile64Waves : 2, T64 ? attn::kTile64Waves : 2))) void nar_attn_kernel(NarAttnParams p, float qscale) {
  constexpr int kQ = T64 ? 64 : 32;  // queries per workgroup
  __shared__ std::conditional_t<T64, attn::Tile64Lds, attn::TileLds> sh;
  const int bh = blockIdx.x;  // batch * heads + head
  const int h = bh % p.heads, b = bh / p.heads;
  const int tile = p.causal ? gridDim.y - 1 - blockIdx.y : blockIdx.y;  // causal: longest first
  const int q0 = tile * kQ;
  const int kvh = h / (p.heads / p.kv_heads);
  const size_t kvhead = size_t(b) * p.kv_heads + kvh;
  attn::QueryTile t;
  t.kc = reinterpret_cast<const u32x4 *>(p.k) + kvhead * p.kv_len * (D / 8);
  t.vc = reinterpret_cast<const u32x4 *>(p.vb) + kvhead * p.kv_pad * (D / 8);
  t.nq = min(kQ, p.q_len - q0);
  t.kv_len = p.kv_len;
  t.kend = p.causal ? q0 + t.nq : p.kv_len;
  t.causal_pos = p.causal ? q0 : -1;
  t.q = p.q + (size_t(bh) * p.q_len + q0) * D;
  t.q_stride = D;
  t.out = p.out + (size_t(bh) * p.q_len + q0) * D;
  t.out_stride = D;
  if constexpr (T64) {
    if (p.splits > 1) {  // keys split over gridDim.z workgroups (non-causal)
      const int nb = (p.kv_len + attn::kBlock - 1) / attn::kBlock;
      const int per = (nb + p.splits - 1) / p.splits;
      t.blk0 = int(blockIdx.z) * per;
      t.blk1 = min(nb, t.blk0 + per);
      t.part = p.part + (size_t(blockIdx.z) * p.batch * p.heads * p.q_len +
                         size_t(bh) * p.q_len + q0) * 132;
    }
    attn::attn_query_tile64(t, qscale, sh);
  } else
    attn::attn_query_tile(t, qscale, sh);
}

// out[row][d] = bf16(sum_s w_s o_s[d] / sum_s w_s l_s), w_s = exp2(m_s - max m)
// over the split partials of each query row; one thread per (row, 4 dims).
__global__ __launch_bounds__(256) void nar_merge_kernel(const float *part, int splits, long long rows,
                                                        uint16_t *out) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * 32)
    return;
  const long long row = idx / 32;
  const int d4 = int(idx % 32) * 4;
  float M = -__builtin_inff();
  for (int s = 0; s < splits; ++s)
    M = fmaxf(M, part[(s * rows + row) * 132 + 128]);
  float L = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const float *ps = part + (s * rows + row) * 132;
    const float m = ps[128];
    const float w = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - M);
    L += w * ps[129];
    const f32x4 v = *reinterpret_cast<const f32x4 *>(ps + d4);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] += w * v[j];
  }
  const uint32_t lo = uint32_t(f2bf(o[0] / L)) | (uint32_t(f2bf(o[1] / L)) << 16);
  const uint32_t hi = uint32_t(f2bf(o[2] / L)) | (uint32_t(f2bf(o[3] / L)) << 16);
  *reinterpret_cast<uint2 *>(out + row * 128 + d4) = uint2{lo, hi};
}

// Inverse of nar_v_blocks_kernel for a cache head: keys [0, n) of each head
// (blocked, kv_stride slots apart) -> row-major [heads][n][128]; one thread
// per 8 dims of one key.
__global__ __launch_bounds__(256) void v_rows_kernel(const uint16_t *vb, int kv_stride, int heads,
                                                     int n, uint16_t *out) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)heads * n * (D / 8))
    return;
  const int d8 = int(idx % (D / 8)) * 8;
  const long long row = idx / (D / 8);
  const int t = int(row % n), h = int(row / n);
  const uint16_t *src = vb + size_t(h) * kv_stride * D;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = uint32_t(src[attn::v_index(t, d8 + 2 * j)]) |
           (uint32_t(src[attn::v_index(t, d8 + 2 * j + 1)]) << 16);
  *reinterpret_cast<u32x4 *>(out + size_t(row) * D + d8) = u32x4{w[0], w[1], w[2], w[3]};
}

}  // namespace

hipError_t launch_v_rows(const uint16_t *vb, int kv_stride, int heads, int n, uint16_t *out,
                         hipStream_t s) {
  if (heads < 1 || n < 1 || n > kv_stride)
    return hipErrorInvalidValue;
  const long long threads = (long long)heads * n * (D / 8);
  hipLaunchKernelGGL(v_rows_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, vb,
                     kv_stride, heads, n, out);
  return hipGetLastError();
}

namespace {
// Key splits for a non-causal launch whose 64-query workgroups do not fill
// the GPU: enough to reach kSplitTargetGroups, each split at least 8 blocks.
// The kernel gives split z the blocks [z * per, min(nb, (z + 1) * per)),
// per = ceil(nb / splits); the count is recomputed from per so that no
// split is left without blocks (nb 81 over 10 splits: per 9, 9 splits).
int nar_splits(int batch, int heads, int q_len, int kv_len, int causal) {
  const long long g64 = (long long)batch * heads * ((q_len + 63) / 64);
  const int nb = (kv_len + attn::kBlock - 1) / attn::kBlock;
  if (causal || g64 >= attn::kSplitTargetGroups)
    return 1;
  const int want = int((attn::kSplitTargetGroups + g64 - 1) / g64);
  const int s = std::max(1, std::min(want, nb / 8));
  const int per = (nb + s - 1) / s;
  return (nb + per - 1) / per;
}
}  // namespace

size_t nar_attention_part_floats(int batch, int heads, int q_len, int kv_len, int causal) {
  const int s = nar_splits(batch, heads, q_len, kv_len, causal);
  return s > 1 ? size_t(s) * batch * heads * q_len * 132 : 0;
}

size_t nar_attention_workspace_elems(int batch, int kv_heads, int kv_len) {
  return size_t(batch) * kv_heads * size_t((kv_len + kBlock - 1) / kBlock * kBlock) * D;
}

hipError_t launch_nar_attention(NarAttnParams p, hipStream_t s) {
  if (p.batch < 1 || p.heads < 1 || p.kv_heads < 1 || p.heads % p.kv_heads || p.q_len < 1 ||
      p.kv_len < 1 || (p.causal && p.q_len != p.kv_len) || !p.q || !p.k || !p.v || !p.vb ||
      !p.out)
    return hipErrorInvalidValue;
  p.kv_pad = (p.kv_len + kBlock - 1) / kBlock * kBlock;
  hipLaunchKernelGGL(nar_v_blocks_kernel, dim3(p.kv_pad / kBlock, p.batch * p.kv_heads), dim3(256),
                     0, s, p.v, p.kv_len, p.kv_pad, p.vb);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return e;
  // scale * log2(e) as in the reference kernel (nar_attention.cpp:95)
  const float qscale = 0.08838834764831845f * 1.4426950408889634f;
  const int splits = nar_splits(p.batch, p.heads, p.q_len, p.kv_len, p.causal);
  if (splits > 1 && p.part &&
      p.part_floats >= nar_attention_part_floats(p.batch, p.heads, p.q_len, p.kv_len, p.causal)) {
    p.splits = splits;
    hipLaunchKernelGGL(nar_attn_kernel<true>, dim3(p.batch * p.heads, (p.q_len + 63) / 64, splits),
                       dim3(256), 0, s, p, qscale);
    e = hipGetLastError();
    if (e != hipSuccess)
      return e;
    const long long rows = (long long)p.batch * p.heads * p.q_len;
    hipLaunchKernelGGL(nar_merge_kernel, dim3(unsigned((rows * 32 + 255) / 256)), dim3(256), 0, s,
                       p.part, splits, rows, p.out);
    return hipGetLastError();
  }
  p.splits = 1;
  if (p.batch * p.heads * ((p.q_len + 63) / 64) >= attn::kTile64MinGroups)
    hipLaunchKernelGGL(nar_attn_kernel<true>, dim3(p.batch * p.heads, (p.q_len + 63) / 64),
                       dim3(256), 0, s, p, qscale);
  else
    hipLaunchKernelGGL(nar_attn_kernel<false>, dim3(p.batch * p.heads, (p.q_len + 31) / 32),
                       dim3(256), 0, s, p, qscale);
  return hipGetLastError();
}

}  // namespace yuear
