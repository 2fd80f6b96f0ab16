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
// Structure: the causal prefill attention of prefill.hip generalised to
// separate query and key sequences. Workgroup = 4 independent waves on one
// (batch, q head); wave w owns queries 128 y + 32 w + [0, 32) as two
// 16-query MFMA column tiles and walks the keys in 32-key blocks with the
// next block's loads in flight:
//
//   S^T[key][query] = K[key][:] . q[query][:]          (K row-major, as given)
//   O^T[dim][query] += V^T[dim][key] . P^T[key][query]  P as hi + mid + lo bf16
//
// The V^T operand wants 8 consecutive keys of one dim per lane, so V is first
// rewritten (nar_v_blocks_kernel) into 32-key blocks stored dim-major, the
// layout of the KV cache, in a caller-provided workspace; keys past Lk in the
// last block are zero there (and masked in the scores).
#include <cmath>

#include "attn_core.h"
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

__global__ __launch_bounds__(256) void nar_attn_kernel(NarAttnParams p, float qscale) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane >> 4, i = lane & 15;
  const int bh = blockIdx.x;  // batch * heads + head
  const int h = bh % p.heads, b = bh / p.heads;
  const int tile = p.causal ? gridDim.y - 1 - blockIdx.y : blockIdx.y;  // causal: longest first
  const int qbase = tile * 128 + wave * 32;
  if (qbase >= p.q_len)
    return;  // whole wave idle (no barriers in this kernel)
  const int kvh = h / (p.heads / p.kv_heads);
  const int kend = p.causal ? min(qbase + 32, p.q_len) : p.kv_len;  // keys [0, kend)
  const int last = kend - 1;
  const size_t kvhead = size_t(b) * p.kv_heads + kvh;
  const u32x4 *kc = reinterpret_cast<const u32x4 *>(p.k) + kvhead * p.kv_len * (D / 8);
  const u32x4 *vc = reinterpret_cast<const u32x4 *>(p.vb) + kvhead * p.kv_pad * (D / 8);

  // Q^T operands: column tile c, query qbase + 16 c + i (clamped), dims 32 s + 8 r
  u32x4 qb[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int qi = min(qbase + 16 * c + i, p.q_len - 1);
    const u32x4 *src = reinterpret_cast<const u32x4 *>(p.q + (size_t(bh) * p.q_len + qi) * D);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[c][s] = src[4 * s + r];
  }
  u32x4 kr[8], vr[8];
  attn::load_k(kc, 0, 0, lane, last, kr);
  attn::load_v(vc, 0, 0, lane, last, vr);

  float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      o[c][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < kend; kb += kBlock) {
    const bool more = kb + kBlock < kend;  // uniform
    u32x4 kn[8], vn[8];
    if (more) {
      attn::load_k(kc, kb + kBlock, 0, lane, last, kn);
      attn::load_v(vc, kb + kBlock, 0, lane, last, vn);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      f32x4 st[2];
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        st[T] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
          st[T] = attn::mfma(kr[4 * T + s], qb[c][s], st[T]);
      }
      // lane (query qbase + 16 c + i, r): keys kb + 8 r + 4 T + t
      const int qpos = qbase + 16 * c + i;
      const int kmax = p.causal ? qpos : p.kv_len - 1;
      float sc[8];
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          sc[4 * T + t] = kb + 8 * r + 4 * T + t <= kmax ? st[T][t] * qscale : -__builtin_inff();
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
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const uint16_t b0 = f2bf(p0), b1 = f2bf(p1);
          pw[k][q] = uint32_t(b0) | (uint32_t(b1) << 16);
          p0 -= bf2f(b0);
          p1 -= bf2f(b1);
        }
      }
      l_run[c] = l_run[c] * corr + ps;
      m_run[c] = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        o[c][dt] *= corr;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          o[c][dt] = attn::mfma(vr[dt], u32x4{pw[k][0], pw[k][1], pw[k][2], pw[k][3]}, o[c][dt]);
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kr[j] = kn[j];
        vr[j] = vn[j];
      }
    }
  }
  // lane (query, r) holds dims 16 dt + 4 r + [0, 4): out = bf16(o / l)
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float l = sum_halves(sum_row_pairs(l_run[c]));
    const int qi = qbase + 16 * c + i;
    if (qi < p.q_len) {
      uint16_t *dst = p.out + (size_t(bh) * p.q_len + qi) * D;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint32_t lo = uint32_t(f2bf(o[c][dt][0] / l)) | (uint32_t(f2bf(o[c][dt][1] / l)) << 16);
        const uint32_t hi = uint32_t(f2bf(o[c][dt][2] / l)) | (uint32_t(f2bf(o[c][dt][3] / l)) << 16);
        *reinterpret_cast<uint2 *>(dst + 16 * dt + 4 * r) = uint2{lo, hi};
      }
    }
  }
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
  hipLaunchKernelGGL(nar_attn_kernel, dim3(p.batch * p.heads, (p.q_len + 127) / 128), dim3(256),
                     0, s, p, qscale);
  return hipGetLastError();
}

}  // namespace yuear
