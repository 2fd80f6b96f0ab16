// Shared host/device helpers for the gfx950 AR decode library.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define YHD __host__ __device__ __forceinline__

namespace yuear {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Protocol constants of the reference (native/include/lyra/types.hpp:14-19).
constexpr int kEOD = 151643, kAbcEnd = 151848, kMusicEnd = 151852,
              kCodecOffset = 151853, kCodecSize = 32768, kContext = 24576;

enum Phase : int { kPhaseFull = 0, kPhaseAbc = 1, kPhaseSemantic = 2 };

YHD float bf2f(uint16_t b) { return __builtin_bit_cast(float, uint32_t(b) << 16); }
YHD float bflo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
YHD float bfhi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (quiet NaN preserved), in integer
// operations.
YHD uint16_t f2bf_int(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
// The same rounding; on gfx950 the device form is one v_cvt_pk_bf16_f32,
// which equals f2bf_int on all 2^32 inputs (denormals, infinities and NaNs
// included, checked exhaustively on MI355X) in a dozen fewer VALU operations.
YHD uint16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
#else
  return f2bf_int(f);
#endif
}
YHD float rbf(float f) { return bf2f(f2bf(f)); }

// Monotone map of fp32 onto uint32 (larger float -> larger key).
YHD uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
YHD float key_value(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, u);
}

// Philox4x32-10 counter-based generator (Salmon et al., SC'11).
struct Philox4 {
  uint32_t v[4];
};
YHD Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                          uint32_t k0, uint32_t k1) {
  for (int round = 0; round < 10; ++round) {
    const uint64_t p0 = uint64_t(0xD2511F53u) * c0;
    const uint64_t p1 = uint64_t(0xCD9E8D57u) * c2;
    const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
    c1 = uint32_t(p1);
    c3 = uint32_t(p0);
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return Philox4{{c0, c1, c2, c3}};
}

// Sampling uniform of the shared-draw protocol: u(seed, step, i) in (0,1),
// the top 24 bits of the first Philox word centred in their bin.
YHD float draw_uniform(uint64_t seed, int step, int index) {
  const Philox4 r = philox4x32_10(uint32_t(index), uint32_t(step), 0x59554541u,
                                  0u, uint32_t(seed), uint32_t(seed >> 32));
  return (float(r.v[0] >> 8) + 0.5f) * 5.9604644775390625e-08f;
}

// Natural log built from IEEE binary32 add/mul/div only (bit-identical on
// host and device when compiled without contraction): significand reduced to
// [sqrt(1/2), sqrt(2)), atanh series in f=(m-1)/(m+1), Cody-Waite ln 2.
YHD float portable_log(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  int e = int((b >> 23) & 0xffu) - 127;
  float m = __builtin_bit_cast(float, (b & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = (m - 1.0f) / (m + 1.0f);
  const float f2 = f * f;
  float p = 0.07692307692f;
  p = p * f2 + 0.09090909091f;
  p = p * f2 + 0.11111111111f;
  p = p * f2 + 0.14285714286f;
  p = p * f2 + 0.2f;
  p = p * f2 + 0.33333333333f;
  p = p * f2 + 1.0f;
  const float lm = 2.0f * f * p;
  const float fe = float(e);
  return fe * 0.693145751953125f + (lm + fe * 1.428606765330187045e-06f);
}

// exp for softmax arguments: Cody-Waite reduction, degree-8 Taylor
// polynomial, exact power-of-two scaling; 0 below -87.
YHD float portable_exp(float x) {
  if (!(x >= -87.0f))
    return 0.0f;
  if (x > 88.0f)
    return __builtin_inff();
  const float n = __builtin_floorf(x * 1.44269504089f + 0.5f);
  const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045e-06f;
  float p = 2.4801587302e-05f;
  p = p * r + 1.9841269841e-04f;
  p = p * r + 1.3888888889e-03f;
  p = p * r + 8.3333333333e-03f;
  p = p * r + 4.1666666667e-02f;
  p = p * r + 1.6666666667e-01f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const int ni = int(n);
  if (ni < -126)
    return (p * __builtin_bit_cast(float, uint32_t(ni + 127 + 64) << 23)) *
           5.421010862427522e-20f;
  return p * __builtin_bit_cast(float, uint32_t(ni + 127) << 23);
}

YHD float gumbel(float u) { return -portable_log(-portable_log(u)); }

#if defined(__HIP__)  // HIP translation units (host and device passes)
// Cross-lane reductions without the LDS crossbar (ds_bpermute costs an LDS
// round trip per step, and the decode kernels run one wave per SIMD, so
// nothing hides it): DPP permutations inside 16-lane rows, then the gfx950
// v_permlane16_swap / v_permlane32_swap across rows. Every lane of the
// reduced group receives bit-identical results (each step adds the same two
// operands on both sides).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum / max over the 16 lanes of a row.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp<0x141>(v);  // row_half_mirror: the other quad of the half-row
  v += dpp<0x140>(v);  // row_mirror: the other half of the row
  return v;
}
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return v;
}
// v_permlane16_swap_b32 a, b swaps the odd rows of a with the even rows of
// b; v_permlane32_swap_b32 a, b swaps the high half of a with the low half of
// b. With a = b = v on entry:
//   permlane16: a = rows (0,0,2,2) of v, b = rows (1,1,3,3);
//   permlane32: a = low half twice,     b = high half twice.
// Through the compiler builtins, so that its hazard recognizer sees the
// instruction (gfx950: two wait states after a VALU write of an operand,
// four after a v_cmpx write of exec) and schedules around it. The two
// results are read as plain element values (a bit cast of a vector element
// lvalue reads element 0 with this clang; see as_bf16x2 below).
__device__ __forceinline__ void permlane16_swap(uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ void permlane32_swap(uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ float sum_row_pairs(float v) {  // rows 2k + 2k+1
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane16_swap(a, b);
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_row_pairs(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane16_swap(a, b);
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float sum_halves(float v) {  // lanes 0-31 + lanes 32-63
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane32_swap(a, b);
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_halves(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane32_swap(a, b);
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
// Value held by lane ^ 32.
__device__ __forceinline__ float xor32(float v, int lane) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane32_swap(a, b);
  return __builtin_bit_cast(float, lane & 32 ? a : b);
}
__device__ __forceinline__ float wave_sum(float v) {
  return sum_halves(sum_row_pairs(row_sum16(v)));
}
__device__ __forceinline__ float wave_max(float v) {
  return max_halves(max_row_pairs(row_max16(v)));
}
// Split-K merge weight of split t, held by lane t (active: t < n_active):
// f_t / sum_s f_s l_s with f_t = exp2(m_t - max_s m_s) (log2(e) is folded
// into the scores) and l_t the split's softmax denominator (the decode
// attention's last-arriving workgroup, attn_block.h).
__device__ __forceinline__ float merge_weight(float m, float l, bool active) {
  const float mm = active ? m : -__builtin_inff();
  const float M = wave_max(mm);
  const float f = mm == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(mm - M);
  const float den = wave_sum(active ? f * l : 0.f);
  return f / den;
}

// Reinterpret one packed bf16 pair. The element must arrive by value: this
// clang reads element 0 when __builtin_bit_cast is applied directly to an
// ext_vector element lvalue such as v.y or v[3] (the by-value helpers below
// exist for that reason).
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) {
  return __builtin_bit_cast(bf16x2_t, v);
}
__device__ __forceinline__ uint32_t f32_bits(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float bits_f32(uint32_t v) { return __builtin_bit_cast(float, v); }
// dot of 8 bf16 pairs packed in two u32x4 registers, fp32 accumulate.
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.x), as_bf16x2(b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.y), as_bf16x2(b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.z), as_bf16x2(b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.w), as_bf16x2(b.w), acc, false);
  return acc;
}

// s_waitcnt vmcnt(0): this wave's outstanding vector memory operations
// (including stores) have completed. gfx9 encoding: vmcnt in bits [3:0] and
// [15:14] (zero here), expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 (no wait).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Per-lane operands of the q/k RMSNorm + RoPE of one head (lane l: dims 2l
// and 2l + 1): the gain pair and the cos/sin pairs of its rotation index, so
// that callers can issue these loads ahead of a larger stream.
struct NormRope {
  float g0 = 1.f, g1 = 1.f, c0, c1, s0, s1;
};
__device__ __forceinline__ void load_rope(NormRope &r, const uint16_t *cs, const uint16_t *sn,
                                          int lane) {
  const int j = (2 * lane) & 63;  // ar.cpp:52-87: pair (j, j + D/2)
  const uint32_t c = reinterpret_cast<const uint32_t *>(cs)[j >> 1];
  const uint32_t s = reinterpret_cast<const uint32_t *>(sn)[j >> 1];
  r.c0 = bflo(c);
  r.c1 = bfhi(c);
  r.s0 = bflo(s);
  r.s1 = bfhi(s);
}
template <class GainPtr>
__device__ __forceinline__ void load_gain(NormRope &r, GainPtr gain, int lane) {
  r.g0 = bf2f(gain[2 * lane]);
  r.g1 = bf2f(gain[2 * lane + 1]);
}

// q/k RMSNorm over a 128-wide head (ar.cpp:268-275, 30-35; skipped without
// a gain) followed by the half-split RoPE (ar.cpp:52-87), one head per wave,
// lane l holding dims 2l and 2l+1; lanes l and l ^ 32 hold the partners.
__device__ __forceinline__ void norm_rope_apply(float x0, float x1, bool has_gain, float eps,
                                                const NormRope &r, int lane, float &y0,
                                                float &y1) {
  if (has_gain) {
    const float ssq = wave_sum(x0 * x0 + x1 * x1);
    const float scale = rbf(1.0f / __builtin_sqrtf(ssq / 128.0f + eps));
    x0 = rbf(rbf(x0 * scale) * r.g0);
    x1 = rbf(rbf(x1 * scale) * r.g1);
  }
  const float p0 = xor32(x0, lane), p1 = xor32(x1, lane);
  if (lane < 32) {  // first half: first*c - second*s
    y0 = rbf(rbf(x0 * r.c0) - rbf(p0 * r.s0));
    y1 = rbf(rbf(x1 * r.c1) - rbf(p1 * r.s1));
  } else {  // second half: second*c + first*s
    y0 = rbf(rbf(x0 * r.c0) + rbf(p0 * r.s0));
    y1 = rbf(rbf(x1 * r.c1) + rbf(p1 * r.s1));
  }
}

#endif

}  // namespace yuear
