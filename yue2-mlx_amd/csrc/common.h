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

// fp32 -> bf16, round to nearest even (quiet NaN preserved).
YHD uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
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
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Reinterpret one packed bf16 pair. The element must arrive by value: this
// clang reads element 0 when __builtin_bit_cast is applied directly to an
// ext_vector element lvalue such as v.y.
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) {
  return __builtin_bit_cast(bf16x2_t, v);
}
// dot of 8 bf16 pairs packed in two u32x4 registers, fp32 accumulate.
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.x), as_bf16x2(b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.y), as_bf16x2(b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.z), as_bf16x2(b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.w), as_bf16x2(b.w), acc, false);
  return acc;
}

// q/k RMSNorm over a 128-wide head (ar.cpp:268-275, 30-35) followed by the
// half-split RoPE (ar.cpp:52-87), one head per wave, lane l holding dims
// 2l and 2l+1; cs/sn point at the bf16 cos/sin row of the position.
// (GainPtr: a plain or an address-space-qualified pointer to the [D] gain.)
template <class GainPtr>
__device__ __forceinline__ void norm_rope_head(float x0, float x1, GainPtr gain,
                                               float eps, const uint16_t *cs,
                                               const uint16_t *sn, int lane, float &y0,
                                               float &y1) {
  if (gain) {  // ar.cpp:268-275 / ar.cpp:30-35 over D
    const float ssq = wave_sum(x0 * x0 + x1 * x1);
    const float scale = rbf(1.0f / __builtin_sqrtf(ssq / 128.0f + eps));
    x0 = rbf(rbf(x0 * scale) * bf2f(gain[2 * lane]));
    x1 = rbf(rbf(x1 * scale) * bf2f(gain[2 * lane + 1]));
  }
  // ar.cpp:52-87: pair (j, j + D/2); lanes l and l ^ 32 hold the partners.
  const float p0 = __shfl_xor(x0, 32, 64), p1 = __shfl_xor(x1, 32, 64);
  const int j = (2 * lane) & 63;
  const float c0 = bf2f(cs[j]), c1 = bf2f(cs[j + 1]);
  const float s0 = bf2f(sn[j]), s1 = bf2f(sn[j + 1]);
  if (lane < 32) {  // first half: first*c - second*s
    y0 = rbf(rbf(x0 * c0) - rbf(p0 * s0));
    y1 = rbf(rbf(x1 * c1) - rbf(p1 * s1));
  } else {  // second half: second*c + first*s
    y0 = rbf(rbf(x0 * c0) + rbf(p0 * s0));
    y1 = rbf(rbf(x1 * c1) + rbf(p1 * s1));
  }
}

#endif

}  // namespace yuear
