// Affine group-64 quantized GEMV for 1-2 branches, and dequantization, on
// gfx950.
//
// Reference: native/src/ar.cpp:20-29 and 306-312, mx::quantized_matmul(x, w,
// scales, biases, transpose=true, group_size=64, bits, "affine"):
//   y[b, r] = bf16(sum_g (s_g * sum_{i in g} x_i q_i + b_g * sum_{i in g} x_i))
// with codes q in [0, 2^bits) packed 32 / bits per uint32, code j of a word at
// bits [bits * j, bits * j + bits) (the checkpoint layout written by
// native/src/conversion.cpp:470-532 through MLX quantize).
//
// Device layout: codes [rows][k * bits / 32] uint32 as in the checkpoint; one
// uint32 per group, scale | bias << 16 (bf16 halves), [rows][k / 64].
//
// Streaming: a row is NP = k * bits / 128 16-byte pieces (32 codes at 4 bits,
// 16 at 8). L lanes share a row (64 / L rows per wave), lane li reading the P
// pieces li + p L, so each wave-wide load covers whole 16-byte pieces of
// 64 / L rows; a wave owns R such row sets and issues all its loads (codes
// non-temporal, group words with them) before the first use. The activation
// rows, gathered and RMS-normalised exactly as in the bf16 GEMV, are staged
// once per workgroup in LDS, permuted so that every code pair meets its
// activation pair, together with each piece's activation sum.
//
// Codes are never converted to float: a pair of codes moved into the low
// mantissa bits of two bf16 with exponent 2^7, ((w >> 4 s) & 0x000f000f) |
// 0x43004300, is exactly the pair (128 + q_a, 128 + q_b), so a shift, one
// and-or and one v_dot2_f32_bf16 consume two codes. At 4 bits the shifts
// s = 0..3 give the pairs (n_s, n_{s+4}) of a word's nibbles; at 8 bits the
// same four masks give the low (s = 0, 2) and high (s = 1, 3) nibbles of
// bytes (0, 2) and (1, 3), q = lo + 16 hi. With D the dot product with the
// offset pairs and Sx the activation sum of the piece:
//   4 bits: s (D - 128 Sx) + b Sx          = s D + (b - 128 s) Sx
//   8 bits: s (Dlo + 16 Dhi - 2176 Sx) + b Sx = s (Dlo + 16 Dhi) + (b - 2176 s) Sx
// fp32 throughout, one bf16 rounding per output (plus the epilogue's).
#include <cmath>

#include "common.h"
#include "gemv_core.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr uint32_t kPairMask = 0x000f000fu, kPairBias = 0x43004300u;
constexpr uint32_t kOnes = 0x3f803f80u;  // bf16 pair (1, 1)

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a), as_bf16x2(b), acc, false);
}

// Sum over the L lanes of a row group (every lane of the group gets it).
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L == 64) {
    return wave_sum(v);
  } else if constexpr (L == 32) {
    return sum_row_pairs(row_sum16(v));
  } else if constexpr (L == 16) {
    return row_sum16(v);
  } else {
    static_assert(L == 8, "lanes per row");
    v += dpp<0xB1>(v);          // lane ^ 1
    v += dpp<0x4E>(v);          // lane ^ 2
    return v + dpp<0x141>(v);   // the other quad of the 8 lanes
  }
}

// One 8-element activation chunk {(x0,x1),(x2,x3),(x4,x5),(x6,x7)} in the
// pair order of the codes: 4 bits {(x0,x4),(x1,x5),(x2,x6),(x3,x7)},
// 8 bits {(x0,x2),(x1,x3),(x4,x6),(x5,x7)}. v_perm_b32 selectors 0-3 pick
// bytes of the second operand, 4-7 of the first.
template <int BITS>
__device__ __forceinline__ u32x4 pair_order(u32x4 v) {
  const uint32_t a = v.x, b = v.y, c = v.z, d = v.w;
  if constexpr (BITS == 4)
    return u32x4{__builtin_amdgcn_perm(c, a, 0x05040100u), __builtin_amdgcn_perm(c, a, 0x07060302u),
                 __builtin_amdgcn_perm(d, b, 0x05040100u), __builtin_amdgcn_perm(d, b, 0x07060302u)};
  else
    return u32x4{__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(b, a, 0x07060302u),
                 __builtin_amdgcn_perm(d, c, 0x05040100u), __builtin_amdgcn_perm(d, c, 0x07060302u)};
}

template <int B, int BITS, int L, int P, int R>
__global__ __launch_bounds__(256) void qgemv_kernel(GemvParams p) {
  constexpr int EP = 128 / BITS;          // codes per 16-byte piece
  constexpr int RW = 64 / L;              // rows per wave and row set
  constexpr int ROWS = 4 * R * RW;        // rows per workgroup
  constexpr int K = L * P * EP;
  constexpr int NP = K / EP;              // pieces per row
  constexpr int NCH = K / 8;              // 8-element activation chunks
  constexpr int XPT = (NCH + 255) / 256;  // chunks per thread when staging
  constexpr int CPP = EP / 8;             // chunks per piece (4 or 2)
  constexpr int GPR = K / 64;             // groups per row
  __shared__ u32x4 xs[B][NCH];
  __shared__ float psum[B][NP];
  __shared__ float red[B][4];
  __shared__ float res[B][ROWS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane % L, sub = lane / L;
  const int blk = blockIdx.x;

  // 1. Activation rows and RMSNorm gains first (branch-free, clamped): the
  // prologue then waits only for these, not for the weight stream.
  u32x4 xr[B][XPT], gr[XPT];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const uint16_t *src = p.embed ? p.embed + size_t(gemv_token_row(p, b)) * K
                                  : p.x + size_t(b) * p.x_stride;
#pragma unroll
    for (int i = 0; i < XPT; ++i)
      xr[b][i] = reinterpret_cast<const u32x4 *>(src)[min(tid + 256 * i, NCH - 1)];
  }
  if (p.norm_w) {
#pragma unroll
    for (int i = 0; i < XPT; ++i)
      gr[i] = reinterpret_cast<const u32x4 *>(p.norm_w)[min(tid + 256 * i, NCH - 1)];
  }

  // 2. Code and group-word stream of this wave's rows.
  u32x4 wv[R][P];
  uint32_t sbv[R][P];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int lr = min(blk * ROWS + (wave * R + r) * RW + sub, p.n - 1);
    const int row = lr < p.seg0_len ? p.seg0_start + lr : p.seg1_start + (lr - p.seg0_len);
    const u32x4 *wrow = reinterpret_cast<const u32x4 *>(p.qw) + size_t(row) * NP;
    const uint32_t *srow = p.qsb + size_t(row) * GPR;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int piece = li + q * L;
      wv[r][q] = __builtin_nontemporal_load(wrow + piece);
      sbv[r][q] = __builtin_nontemporal_load(srow + piece / (64 / EP));
    }
  }

  // 3. Stage: RMSNorm (the bf16 GEMV's arithmetic and order), the gathered
  // rows to x_out, piece sums, pair order.
  float scale[B];
#pragma unroll
  for (int b = 0; b < B; ++b)
    scale[b] = 1.f;
  if (p.norm_w) {
    float ss[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      ss[b] = 0.f;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        if (tid + 256 * i >= NCH)
          continue;
        const u32x4 v = xr[b][i];
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bflo(w4[q]), hi = bfhi(w4[q]);
          ss[b] += lo * lo;
          ss[b] += hi * hi;
        }
      }
      const float t = wave_sum(ss[b]);
      if (lane == 0)
        red[b][wave] = t;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float total = (red[b][0] + red[b][1]) + (red[b][2] + red[b][3]);
      scale[b] = rbf(1.0f / __builtin_sqrtf(total / float(K) + p.eps));
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int c = tid + 256 * i;
      u32x4 v = xr[b][i];
      if (p.x_out && blk == 0 && c < NCH)
        reinterpret_cast<u32x4 *>(p.x_out + size_t(b) * p.x_stride)[c] = v;
      if (p.norm_w) {
        const u32x4 g = gr[i];
        const uint32_t vi[4] = {v.x, v.y, v.z, v.w}, gi[4] = {g.x, g.y, g.z, g.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = f2bf(rbf(bflo(vi[q]) * scale[b]) * bflo(gi[q]));
          const uint32_t hi = f2bf(rbf(bfhi(vi[q]) * scale[b]) * bfhi(gi[q]));
          o[q] = lo | (hi << 16);
        }
        v = u32x4{o[0], o[1], o[2], o[3]};
      }
      // chunk sum, then the sum of the CPP chunks of a piece (consecutive
      // lanes; whole pieces are valid or invalid together)
      float cs = dot2(v.x, kOnes, 0.f);
      cs = dot2(v.y, kOnes, cs);
      cs = dot2(v.z, kOnes, cs);
      cs = dot2(v.w, kOnes, cs);
      cs += dpp<0xB1>(cs);
      if constexpr (CPP == 4)
        cs += dpp<0x4E>(cs);
      if (c < NCH) {
        xs[b][c] = pair_order<BITS>(v);
        if (c % CPP == 0)
          psum[b][c / CPP] = cs;
      }
    }
  }
  __syncthreads();

  // 4. Dot products.
  float acc[R][B];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b)
      acc[r][b] = 0.f;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int piece = li + q * L;
    uint32_t xw[B][CPP * 4];
    float sx[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
      for (int j = 0; j < CPP; ++j) {
        const u32x4 v = xs[b][piece * CPP + j];
        xw[b][4 * j] = v.x;
        xw[b][4 * j + 1] = v.y;
        xw[b][4 * j + 2] = v.z;
        xw[b][4 * j + 3] = v.w;
      }
      sx[b] = psum[b][piece];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4 w = wv[r][q];
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
      uint32_t pr[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          pr[j][s] = ((wd[j] >> (4 * s)) & kPairMask) | kPairBias;
      const float sc = bflo(sbv[r][q]), bias = bfhi(sbv[r][q]);
#pragma unroll
      for (int b = 0; b < B; ++b) {
        if constexpr (BITS == 4) {
          float d0 = 0.f, d1 = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {  // word j <-> chunk j
            d0 = dot2(pr[j][0], xw[b][4 * j], d0);
            d1 = dot2(pr[j][1], xw[b][4 * j + 1], d1);
            d0 = dot2(pr[j][2], xw[b][4 * j + 2], d0);
            d1 = dot2(pr[j][3], xw[b][4 * j + 3], d1);
          }
          const float cb = __builtin_fmaf(-128.f, sc, bias);
          acc[r][b] = __builtin_fmaf(sc, d0 + d1, __builtin_fmaf(cb, sx[b], acc[r][b]));
        } else {
          float lo = 0.f, hi = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {  // word j: elements 4j..4j+3, pairs (0,2), (1,3)
            const uint32_t x02 = xw[b][2 * j], x13 = xw[b][2 * j + 1];
            lo = dot2(pr[j][0], x02, lo);
            hi = dot2(pr[j][1], x02, hi);
            lo = dot2(pr[j][2], x13, lo);
            hi = dot2(pr[j][3], x13, hi);
          }
          const float cb = __builtin_fmaf(-2176.f, sc, bias);
          acc[r][b] = __builtin_fmaf(sc, __builtin_fmaf(16.f, hi, lo),
                                     __builtin_fmaf(cb, sx[b], acc[r][b]));
        }
      }
    }
  }

  // 5. Row sums, then the epilogue over the workgroup's rows.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float t = group_sum<L>(acc[r][b]);
      if (li == 0)
        res[b][(wave * R + r) * RW + sub] = t;
    }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < B; ++b) {
    uint16_t *yb = p.y + size_t(b) * p.y_stride;
    if (p.epilogue == kEpiSwiGLU) {
      for (int i = tid; i < ROWS / 2; i += 256) {
        const int row = blk * ROWS + 2 * i;
        if (row + 1 < p.n) {
          const float g = rbf(res[b][2 * i]), u = rbf(res[b][2 * i + 1]);
          const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
          yb[row >> 1] = f2bf(act * u);
        }
      }
    } else {
      for (int i = tid; i < ROWS; i += 256) {
        const int row = blk * ROWS + i;
        if (row < p.n) {
          float v = res[b][i];
          if (p.epilogue == kEpiResidual)
            v = bf2f(yb[row]) + rbf(v);
          yb[row] = f2bf(v);
        }
      }
    }
  }
  if (p.advance && blk == 0 && tid < p.batch)
    p.advance[tid] += 1;
}

struct Shape {
  int lanes, pieces;
};
// Lanes per row and pieces per lane for k codes of `bits`: the widest row
// group whose pieces per lane have an instance.
bool qgemv_shape(int bits, int k, Shape &s) {
  if ((bits != 4 && bits != 8) || k % 64 || k > 8192)
    return false;
  const int np = k * bits / 128;
  const Shape options[] = {{64, 1}, {64, 2}, {64, 3}, {64, 4}, {64, 6}, {64, 8},
                           {32, 1}, {32, 3}, {16, 1}, {8, 1}};
  for (const Shape &o : options)
    if (o.lanes * o.pieces == np) {
      s = o;
      return true;
    }
  return false;
}

template <int B, int BITS, int L, int P, int R>
hipError_t launch_r(const GemvParams &p, hipStream_t s) {
  constexpr int rows = 4 * R * (64 / L);
  hipLaunchKernelGGL((qgemv_kernel<B, BITS, L, P, R>), dim3((p.n + rows - 1) / rows), dim3(256),
                     0, s, p);
  return hipGetLastError();
}

template <int B, int BITS, int L, int P>
hipError_t launch_lp(const GemvParams &p, hipStream_t s) {
  // more row sets per wave for the long GEMVs (lm_head, gate/up) while that
  // still leaves >= 1024 workgroups: each workgroup's activation staging is
  // then shared by more rows (4-bit lm_head: 47.7 / 36.1 / 31.9 us with
  // 1 / 2 / 4 sets); one set for the short ones, whose time is latency
  if constexpr (P <= 3) {
    constexpr int rows4 = 16 * (64 / L);
    if ((p.n + rows4 - 1) / rows4 >= 1024)
      return launch_r<B, BITS, L, P, 4>(p, s);
  }
  if constexpr (P <= 4) {
    constexpr int rows2 = 8 * (64 / L);
    if ((p.n + rows2 - 1) / rows2 >= 1024)
      return launch_r<B, BITS, L, P, 2>(p, s);
  }
  return launch_r<B, BITS, L, P, 1>(p, s);
}

template <int B, int BITS>
hipError_t launch_bb(const GemvParams &p, const Shape &sh, hipStream_t s) {
  switch (sh.lanes * 16 + sh.pieces) {
  case 64 * 16 + 1: return launch_lp<B, BITS, 64, 1>(p, s);
  case 64 * 16 + 2: return launch_lp<B, BITS, 64, 2>(p, s);
  case 64 * 16 + 3: return launch_lp<B, BITS, 64, 3>(p, s);
  case 64 * 16 + 4: return launch_lp<B, BITS, 64, 4>(p, s);
  case 64 * 16 + 6: return launch_lp<B, BITS, 64, 6>(p, s);
  case 64 * 16 + 8: return launch_lp<B, BITS, 64, 8>(p, s);
  case 32 * 16 + 1: return launch_lp<B, BITS, 32, 1>(p, s);
  case 32 * 16 + 3: return launch_lp<B, BITS, 32, 3>(p, s);
  case 16 * 16 + 1: return launch_lp<B, BITS, 16, 1>(p, s);
  case 8 * 16 + 1: return launch_lp<B, BITS, 8, 1>(p, s);
  }
  return hipErrorInvalidValue;
}

// out[r][i] = bf16(s q + b) (s q is exact in fp32, then one fp32 add); one
// thread per 8 codes.
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *codes, const uint32_t *sb,
                                                      int bits, long long chunks, int k,
                                                      uint16_t *out) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks)
    return;
  const int per_row = k / 8;
  const long long r = i / per_row;
  const int c = int(i % per_row);
  const uint32_t g = sb[r * (k / 64) + (c * 8) / 64];
  const float s = bflo(g), b = bfhi(g);
  uint32_t q[8];
  if (bits == 4) {
    const uint32_t w = codes[r * (k / 8) + c];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      q[j] = (w >> (4 * j)) & 15u;
  } else {
    const uint32_t w0 = codes[r * (k / 4) + 2 * c], w1 = codes[r * (k / 4) + 2 * c + 1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[j] = (w0 >> (8 * j)) & 255u;
      q[j + 4] = (w1 >> (8 * j)) & 255u;
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = s * float(q[2 * j]) + b, hi = s * float(q[2 * j + 1]) + b;
    o[j] = uint32_t(f2bf(lo)) | (uint32_t(f2bf(hi)) << 16);
  }
  reinterpret_cast<u32x4 *>(out)[i] = u32x4{o[0], o[1], o[2], o[3]};
}

}  // namespace

bool qgemv_supported(int bits, int k, int batch) {
  Shape sh;
  return batch >= 1 && batch <= 2 && qgemv_shape(bits, k, sh);
}

hipError_t launch_qgemv(const GemvParams &p, hipStream_t s) {
  Shape sh;
  const int out_n = p.epilogue == kEpiSwiGLU ? p.n / 2 : p.n;  // rows must not overlap
  if (!qgemv_shape(p.bits, p.k, sh) || p.batch < 1 || p.batch > 2 || p.n < 1 || !p.qw ||
      !p.qsb || (p.x_stride % 8 && !p.embed) || (p.epilogue == kEpiSwiGLU && p.n % 2) ||
      ((!p.embed || p.x_out) && p.x_stride < p.k) || p.y_stride < out_n)
    return hipErrorInvalidValue;
  if (p.bits == 4)
    return p.batch == 1 ? launch_bb<1, 4>(p, sh, s) : launch_bb<2, 4>(p, sh, s);
  return p.batch == 1 ? launch_bb<1, 8>(p, sh, s) : launch_bb<2, 8>(p, sh, s);
}

hipError_t launch_dequantize(const uint32_t *codes, const uint32_t *sb, int bits, int rows, int k,
                             uint16_t *out, hipStream_t s) {
  if ((bits != 4 && bits != 8) || k % 64 || rows < 1)
    return hipErrorInvalidValue;
  const long long chunks = (long long)rows * (k / 8);
  hipLaunchKernelGGL(dequant_kernel, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0, s, codes,
                     sb, bits, chunks, k, out);
  return hipGetLastError();
}

}  // namespace yuear
