// cpu_ref — CPU restatement of the reference AR decode path. TEST
// INFRASTRUCTURE ONLY: loaded by tests, the smoke check and the benchmark's
// CPU-baseline leg; never linked into the product library.
//
// Build: oracle/Makefile (g++ -O3 -fopenmp -ffp-contract=off). Contraction is
// off so every bf16 rounding point below is a real fp32 operation followed by
// round-to-nearest-even, as in the reference graph (CMakeLists.txt:66-68 also
// builds the reference host code with -ffp-contract=off).
#include "cpu_ref.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// Protocol constants, native/include/lyra/types.hpp:14-19.
constexpr int EOD = 151643, ABC_END = 151848, MUSIC_END = 151852,
              CODEC_OFFSET = 151853, CODEC_SIZE = 32768;

inline float bf2f(uint16_t b) {
  uint32_t u = uint32_t(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
// Round-to-nearest-even fp32 -> bf16 (the astype(bfloat16) of every rounding
// point in ar.cpp / ar.py).
inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
inline float rbf(float f) { return bf2f(f2bf(f)); }

// Accumulation mode of the dot products: 0 = fp32 in a fixed blocked order
// (the default), 1 = fp64 (a more accurate restatement, used to measure how
// far two valid fp32 accumulation orders can drift apart over many layers).
int g_accumulate = 0;

// fp32 dot product in a fixed blocked order (16 partial sums, pairwise).
float dot_f32_bf16(const float *x, const uint16_t *w, int k) {
  if (g_accumulate == 1) {
    double acc[8] = {0};
    int i = 0;
    for (; i + 8 <= k; i += 8)
      for (int j = 0; j < 8; ++j)
        acc[j] += double(x[i + j]) * double(bf2f(w[i + j]));
    double s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < k; ++i)
      s += double(x[i]) * double(bf2f(w[i]));
    return float(s);
  }
  float acc[16] = {0};
  int i = 0;
  for (; i + 16 <= k; i += 16)
    for (int j = 0; j < 16; ++j)
      acc[j] += x[i + j] * bf2f(w[i + j]);
  float tail = 0.f;
  for (; i < k; ++i)
    tail += x[i] * bf2f(w[i]);
  for (int width = 8; width; width >>= 1)
    for (int j = 0; j < width; ++j)
      acc[j] += acc[j + width];
  return acc[0] + tail;
}

struct Phase {
  int size;             // phase-local vocabulary
  int end;              // local end index, or -1
  int seg0_start, seg0_len, seg1_start, seg1_len;  // native lm_head rows
};

// sampling.cpp:8-18 and ar.cpp:302-323. The FULL phase is this build's
// identity projection for vocabularies that do not hold the YuE2 protocol rows
// (the 3B-shaped random models); it has no end token.
bool phase_of(int phase, int vocab, Phase &p) {
  switch (phase) {
  case ORACLE_PHASE_FULL:
    p = {vocab, -1, 0, vocab, 0, 0};
    return true;
  case ORACLE_PHASE_ABC:
    if (vocab <= ABC_END)
      return false;
    p = {EOD + 1, EOD, 0, EOD, ABC_END, 1};
    return true;
  case ORACLE_PHASE_SEMANTIC:
    if (vocab < CODEC_OFFSET + CODEC_SIZE)
      return false;
    p = {CODEC_SIZE + 1, 0, MUSIC_END, CODEC_SIZE + 1, 0, 0};
    return true;
  }
  return false;
}

} // namespace

struct oracle_model {
  oracle_config c;
  oracle_weights w;
  oracle_quant q;  // q.bits == 0: bf16 linears
};

struct oracle_cache {
  int capacity = 0, offset = 0, layers = 0;
  size_t per_layer = 0;  // Hkv * capacity * D
  std::vector<uint16_t> keys, values;  // [layers][Hkv][cap][D]
};

extern "C" {

uint16_t oracle_f2bf(float x) { return f2bf(x); }
float oracle_bf2f(uint16_t x) { return bf2f(x); }

void oracle_set_accumulation(int mode) { g_accumulate = mode; }

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0)
    omp_set_num_threads(n);
#else
  (void)n;
#endif
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC'11): 10 rounds of the 4x32 S-box with Weyl key bumps.
void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2],
                          uint32_t out[4]) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int round = 0; round < 10; ++round) {
    uint64_t p0 = uint64_t(M0) * c0, p1 = uint64_t(M1) * c2;
    uint32_t hi0 = uint32_t(p0 >> 32), lo0 = uint32_t(p0);
    uint32_t hi1 = uint32_t(p1 >> 32), lo1 = uint32_t(p1);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

// Shared-uniform protocol of this build: u(seed, step, i) in (0, 1) from the
// first Philox word, 24 significant bits, centred in its bin.
float oracle_uniform(uint64_t seed, int32_t step, int32_t index) {
  const uint32_t ctr[4] = {uint32_t(index), uint32_t(step), 0x59554541u, 0u};
  const uint32_t key[2] = {uint32_t(seed), uint32_t(seed >> 32)};
  uint32_t out[4];
  oracle_philox4x32_10(ctr, key, out);
  return (float(out[0] >> 8) + 0.5f) * 5.9604644775390625e-08f;
}

// Portable natural log from IEEE add/mul/div only: exponent extraction, a
// reduction of the significand to [sqrt(1/2), sqrt(2)), and the atanh series
// log(m) = 2(f + f^3/3 + f^5/5 + ...), f = (m-1)/(m+1). Valid for finite
// x > 0 in the normal range; identical on every IEEE binary32 machine.
float oracle_plog(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  int e = int((b >> 23) & 0xffu) - 127;
  uint32_t mb = (b & 0x7fffffu) | 0x3f800000u;
  float m;
  std::memcpy(&m, &mb, 4);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = (m - 1.0f) / (m + 1.0f);
  const float f2 = f * f;
  float p = 0.07692307692f;            // 1/13
  p = p * f2 + 0.09090909091f;         // 1/11
  p = p * f2 + 0.11111111111f;         // 1/9
  p = p * f2 + 0.14285714286f;         // 1/7
  p = p * f2 + 0.2f;                   // 1/5
  p = p * f2 + 0.33333333333f;         // 1/3
  p = p * f2 + 1.0f;
  const float lm = 2.0f * f * p;
  const float fe = float(e);
  // ln 2 split so that fe * LN2_HI is exact for |e| < 2^8 (Cody-Waite).
  return fe * 0.693145751953125f + (lm + fe * 1.428606765330187045e-06f);
}

// Portable exp for softmax arguments (x <= 0 after the max shift): Cody-Waite
// reduction x = n ln2 + r, degree-8 Taylor polynomial for e^r on |r| <= ln2/2,
// exact power-of-two scaling. Returns 0 below -87 (results under FLT_MIN).
float oracle_pexp(float x) {
  if (!(x >= -87.0f))
    return 0.0f;  // also -inf
  if (x > 88.0f)
    return std::numeric_limits<float>::infinity();
  const float n = std::floor(x * 1.44269504089f + 0.5f);
  const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045e-06f;
  float p = 2.4801587302e-05f;          // 1/8!
  p = p * r + 1.9841269841e-04f;        // 1/7!
  p = p * r + 1.3888888889e-03f;        // 1/6!
  p = p * r + 8.3333333333e-03f;        // 1/5!
  p = p * r + 4.1666666667e-02f;        // 1/4!
  p = p * r + 1.6666666667e-01f;        // 1/3!
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const int ni = int(n);
  uint32_t sb = uint32_t(ni + 127) << 23;
  float scale;
  if (ni < -126) {  // two-step scaling into the subnormal range
    sb = uint32_t(ni + 127 + 64) << 23;
    std::memcpy(&scale, &sb, 4);
    return (p * scale) * 5.421010862427522e-20f;  // 2^-64
  }
  std::memcpy(&scale, &sb, 4);
  return p * scale;
}

// ---- model_ops ----

// ar.cpp:30-35 (ar.py:64-68): variance = mean(f32(x)^2);
// scale = bf16(rsqrt(variance + eps)); y = bf16(bf16(x * scale) * w).
void oracle_rms_norm(const uint16_t *x, int rows, int n, const uint16_t *w,
                     float eps, uint16_t *y) {
#pragma omp parallel for schedule(static) if (rows > 8)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + size_t(r) * n;
    float acc[16] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
      for (int j = 0; j < 16; ++j) {
        float v = bf2f(xr[i + j]);
        acc[j] += v * v;
      }
    float tail = 0.f;
    for (; i < n; ++i) {
      float v = bf2f(xr[i]);
      tail += v * v;
    }
    for (int width = 8; width; width >>= 1)
      for (int j = 0; j < width; ++j)
        acc[j] += acc[j + width];
    const float variance = (acc[0] + tail) / float(n);
    const float scale = rbf(1.0f / std::sqrt(variance + eps));
    uint16_t *yr = y + size_t(r) * n;
    for (int k = 0; k < n; ++k)
      yr[k] = f2bf(rbf(bf2f(xr[k]) * scale) * bf2f(w[k]));
  }
}

// ar.cpp:20-29, bf16 path: y = bf16(x @ W^T), W row-major [n][k], fp32
// accumulation, one rounding. No bias (the AR linears are bias-free).
void oracle_linear(const uint16_t *x, int rows, int k, const uint16_t *w,
                   int n, uint16_t *y) {
  std::vector<float> xf(size_t(rows) * k);
  for (size_t i = 0; i < xf.size(); ++i)
    xf[i] = bf2f(x[i]);
#pragma omp parallel for schedule(static)
  for (int o = 0; o < n; ++o) {
    const uint16_t *wr = w + size_t(o) * k;
    for (int r = 0; r < rows; ++r)
      y[size_t(r) * n + o] = f2bf(dot_f32_bf16(xf.data() + size_t(r) * k, wr, k));
  }
}

// Code j of a packed row (MLX quantize layout: 32 / bits codes per uint32,
// code j of a word at bits [bits * j, bits * j + bits)).
static inline uint32_t qcode(const uint32_t *row, int j, int bits) {
  const int per = 32 / bits;
  return (row[j / per] >> ((j % per) * bits)) & ((1u << bits) - 1u);
}

// ar.cpp:22-24: mx::quantized_matmul(x, w, scales, biases, transpose=true,
// group_size=64, bits, "affine"). Per group g of 64 inputs, fp32 sums of
// x_i q_i and of x_i; y = bf16(sum_g (s_g * dq_g + b_g * sx_g)).
void oracle_qlinear(const uint16_t *x, int rows, int k, const uint32_t *w,
                    const uint16_t *scales, const uint16_t *biases, int bits,
                    int n, uint16_t *y) {
  std::vector<float> xf(size_t(rows) * k);
  for (size_t i = 0; i < xf.size(); ++i)
    xf[i] = bf2f(x[i]);
  const int groups = k / 64, words = k * bits / 32;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < n; ++o) {
    const uint32_t *wr = w + size_t(o) * words;
    const uint16_t *sr = scales + size_t(o) * groups, *br = biases + size_t(o) * groups;
    for (int r = 0; r < rows; ++r) {
      const float *xr = xf.data() + size_t(r) * k;
      if (g_accumulate == 1) {
        double acc = 0.0;
        for (int i = 0; i < k; ++i)
          acc += double(xr[i]) * (double(bf2f(sr[i / 64])) * double(qcode(wr, i, bits)) +
                                  double(bf2f(br[i / 64])));
        y[size_t(r) * n + o] = f2bf(float(acc));
        continue;
      }
      float acc = 0.f;
      for (int g = 0; g < groups; ++g) {
        float dq[4] = {0.f, 0.f, 0.f, 0.f}, sx[4] = {0.f, 0.f, 0.f, 0.f};
        for (int i = 0; i < 64; ++i) {
          const float xv = xr[g * 64 + i];
          dq[i & 3] += xv * float(qcode(wr, g * 64 + i, bits));
          sx[i & 3] += xv;
        }
        const float d = (dq[0] + dq[1]) + (dq[2] + dq[3]);
        const float sum = (sx[0] + sx[1]) + (sx[2] + sx[3]);
        acc += bf2f(sr[g]) * d + bf2f(br[g]) * sum;
      }
      y[size_t(r) * n + o] = f2bf(acc);
    }
  }
}

void oracle_dequantize(const uint32_t *w, const uint16_t *scales,
                       const uint16_t *biases, int bits, int n, int k,
                       uint16_t *out) {
  const int groups = k / 64, words = k * bits / 32;
  for (int o = 0; o < n; ++o)
    for (int i = 0; i < k; ++i) {
      const float s = bf2f(scales[size_t(o) * groups + i / 64]);
      const float b = bf2f(biases[size_t(o) * groups + i / 64]);
      out[size_t(o) * k + i] = f2bf(s * float(qcode(w + size_t(o) * words, i, bits)) + b);
    }
}

// RoPE tables, ar.cpp:62-74: inv_j = 1 / pow(f32 theta, f32(2j)/f32(D)) in
// fp32; angle = f32(position) * inv_j; cos/sin rounded to bf16.
void oracle_rope_table(int positions, int d, double theta, uint16_t *cos_out,
                       uint16_t *sin_out) {
  const int half = d / 2;
  std::vector<float> inv(half);
  for (int j = 0; j < half; ++j) {
    const float exponent = float(2 * j) / float(d);
    inv[j] = 1.0f / std::pow(float(theta), exponent);
  }
  for (int p = 0; p < positions; ++p)
    for (int j = 0; j < half; ++j) {
      const float angle = float(p) * inv[j];
      cos_out[size_t(p) * half + j] = f2bf(std::cos(angle));
      sin_out[size_t(p) * half + j] = f2bf(std::sin(angle));
    }
}

// ar.cpp:52-87 (ar.py:71-106): half-split rotation with every product and
// sum rounded to bf16. x is [T][heads][D], positions offset + t.
void oracle_rope(uint16_t *x, int T, int heads, int d, int offset,
                 double theta) {
  const int half = d / 2;
  std::vector<uint16_t> c(size_t(T) * half), s(size_t(T) * half);
  {
    std::vector<uint16_t> ct(size_t(offset + T) * half),
        st(size_t(offset + T) * half);
    oracle_rope_table(offset + T, d, theta, ct.data(), st.data());
    std::memcpy(c.data(), ct.data() + size_t(offset) * half, c.size() * 2);
    std::memcpy(s.data(), st.data() + size_t(offset) * half, s.size() * 2);
  }
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < heads; ++h) {
      uint16_t *v = x + (size_t(t) * heads + h) * d;
      for (int j = 0; j < half; ++j) {
        const float cj = bf2f(c[size_t(t) * half + j]),
                    sj = bf2f(s[size_t(t) * half + j]);
        const float first = bf2f(v[j]), second = bf2f(v[j + half]);
        const float fc = rbf(first * cj), ss = rbf(second * sj);
        const float sc = rbf(second * cj), fs = rbf(first * sj);
        v[j] = f2bf(fc - ss);
        v[j + half] = f2bf(sc + fs);
      }
    }
}

// ar.cpp:36-51 (ar.py:109-128): g = bf16(v * sigmoid(v)) with fp32 v, then
// the bf16 product with the up projection.
void oracle_silu_mul(const uint16_t *g, const uint16_t *u, int n,
                     uint16_t *out) {
  for (int i = 0; i < n; ++i) {
    const float v = bf2f(g[i]);
    const float act = rbf(v * (1.0f / (1.0f + std::exp(-v))));
    out[i] = f2bf(act * bf2f(u[i]));
  }
}

// ar.cpp:88-96 and 284-291: softmax(scale * q K^T) V with fp32 opmath, GQA
// head map h -> h / (Hq / Hkv), output rounded to bf16.
void oracle_attention(const uint16_t *q, const uint16_t *keys,
                      const uint16_t *values, int T, int Hq, int Hkv, int D,
                      int cap, int offset, uint16_t *out) {
  const int group = Hq / Hkv;
  const float scale = float(std::pow(double(D), -0.5));
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / group, L = offset + t + 1;
      const uint16_t *K = keys + size_t(kvh) * cap * D;
      const uint16_t *V = values + size_t(kvh) * cap * D;
      std::vector<float> qs(D), sc(L), acc(D, 0.f);
      for (int d = 0; d < D; ++d)
        qs[d] = scale * bf2f(q[(size_t(t) * Hq + h) * D + d]);
      float m = -std::numeric_limits<float>::infinity();
      for (int j = 0; j < L; ++j) {
        sc[j] = dot_f32_bf16(qs.data(), K + size_t(j) * D, D);
        m = std::max(m, sc[j]);
      }
      float l = 0.f;
      for (int j = 0; j < L; ++j) {
        const float p = std::exp(sc[j] - m);
        l += p;
        const uint16_t *vr = V + size_t(j) * D;
        for (int d = 0; d < D; ++d)
          acc[d] += p * bf2f(vr[d]);
      }
      for (int d = 0; d < D; ++d)
        out[(size_t(t) * Hq + h) * D + d] = f2bf(acc[d] / l);
    }
}

// The acoustic model's attention (nar_attention.cpp:224-270): q [B][Hq][Lq][D],
// keys / values [B][Hkv][Lk][D] (the [batch, heads, tokens, dim] tensors),
// query head h reads kv head h / (Hq / Hkv). Restated from the non-causal
// kernel lyra_nar_precise_attention (nar_attention.cpp:63-218): fp32 scores
// of the bf16 operands, times scale * log2(e) as one fp32 constant, exp2
// softmax in fp32, fp32 P times bf16 V summed in fp32, bf16(o / l). causal
// (Lq == Lk, the conditioning prefill, nar.cpp:176) hides keys after the
// query's own position.
void oracle_nar_attention(const uint16_t *q, const uint16_t *keys, const uint16_t *values,
                          int B, int Hq, int Hkv, int Lq, int Lk, int D, int causal,
                          uint16_t *out) {
  const int group = Hq / Hkv;
  const float scale2 = float(std::pow(double(D), -0.5)) * 1.4426950408889634f;
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h)
      for (int t = 0; t < Lq; ++t) {
        const int kvh = h / group, L = causal ? t + 1 : Lk;
        const uint16_t *K = keys + (size_t(b) * Hkv + kvh) * Lk * D;
        const uint16_t *V = values + (size_t(b) * Hkv + kvh) * Lk * D;
        const uint16_t *qr = q + ((size_t(b) * Hq + h) * Lq + t) * D;
        std::vector<float> qs(D), sc(L), acc(D, 0.f);
        for (int d = 0; d < D; ++d)
          qs[d] = bf2f(qr[d]);
        float m = -std::numeric_limits<float>::infinity();
        for (int j = 0; j < L; ++j) {
          sc[j] = dot_f32_bf16(qs.data(), K + size_t(j) * D, D) * scale2;
          m = std::max(m, sc[j]);
        }
        float l = 0.f;
        for (int j = 0; j < L; ++j) {
          const float p = std::exp2(sc[j] - m);
          l += p;
          const uint16_t *vr = V + size_t(j) * D;
          for (int d = 0; d < D; ++d)
            acc[d] += p * bf2f(vr[d]);
        }
        uint16_t *o = out + ((size_t(b) * Hq + h) * Lq + t) * D;
        for (int d = 0; d < D; ++d)
          o[d] = f2bf(acc[d] / l);
      }
}

// ---- model / cache ----

oracle_model *oracle_model_new(const oracle_config *c, const oracle_weights *w) {
  if (!c || !w || c->heads % c->kv_heads || c->head_dim % 2)
    return nullptr;
  return new oracle_model{*c, *w, oracle_quant{}};
}
oracle_model *oracle_model_new_quantized(const oracle_config *c, const oracle_weights *w,
                                         const oracle_quant *q) {
  if (!q || (q->bits != 8 && q->bits != 4) || c->hidden % 64 || c->intermediate % 64 ||
      (c->heads * c->head_dim) % 64)
    return nullptr;
  oracle_model *m = oracle_model_new(c, w);
  if (m)
    m->q = *q;
  return m;
}
void oracle_model_free(oracle_model *m) { delete m; }

// ar.cpp:98-101: capacity in [1, 24576]; storage zero-filled, as mx::zeros.
oracle_cache *oracle_cache_new(const oracle_model *m, int capacity) {
  if (!m || capacity < 1 || capacity > 24576)
    return nullptr;
  auto *c = new oracle_cache;
  c->capacity = capacity;
  c->layers = m->c.layers;
  c->per_layer = size_t(m->c.kv_heads) * capacity * m->c.head_dim;
  c->keys.assign(c->per_layer * c->layers, 0);
  c->values.assign(c->per_layer * c->layers, 0);
  return c;
}
void oracle_cache_free(oracle_cache *c) { delete c; }
int oracle_cache_offset(const oracle_cache *c) { return c->offset; }
void oracle_cache_set_offset(oracle_cache *c, int offset) { c->offset = offset; }
int oracle_cache_capacity(const oracle_cache *c) { return c->capacity; }
uint16_t *oracle_cache_keys(oracle_cache *c, int layer) {
  return c->keys.data() + c->per_layer * layer;
}
uint16_t *oracle_cache_values(oracle_cache *c, int layer) {
  return c->values.data() + c->per_layer * layer;
}

// Projection `kind` (0..6 = q, k, v, o, gate, up, down) of one layer.
static void layer_linear(const oracle_model *m, int layer, int kind, const uint16_t *x, int T,
                         int k, int n, uint16_t *y) {
  const oracle_weights &w = m->w;
  const uint16_t *const *tables[7] = {w.wq, w.wk, w.wv, w.wo, w.wg, w.wu, w.wd};
  const uint16_t *wt = tables[kind][layer];
  if (m->q.bits)
    oracle_qlinear(x, T, k, reinterpret_cast<const uint32_t *>(wt), m->q.scales[kind][layer],
                   m->q.biases[kind][layer], m->q.bits, n, y);
  else
    oracle_linear(x, T, k, wt, n, y);
}

// One decoder layer, ar.cpp:265-298.
int oracle_layer(oracle_model *m, oracle_cache *cache, int layer, uint16_t *x,
                 int T) {
  const oracle_config &c = m->c;
  const oracle_weights &w = m->w;
  const int H = c.hidden, Hq = c.heads, Hkv = c.kv_heads, D = c.head_dim,
            F = c.intermediate;
  const int offset = cache->offset;
  if (T < 1 || offset + T > cache->capacity)
    return 2;  // ar.cpp:109-112: overflow throws before any mutation
  std::vector<uint16_t> h(size_t(T) * H), q(size_t(T) * Hq * D),
      k(size_t(T) * Hkv * D), v(size_t(T) * Hkv * D), att(size_t(T) * Hq * D),
      o(size_t(T) * H), g(size_t(T) * F), u(size_t(T) * F), mm(size_t(T) * F),
      dn(size_t(T) * H), qn(q.size()), kn(k.size());
  oracle_rms_norm(x, T, H, w.input_ln[layer], c.rms_eps, h.data());
  layer_linear(m, layer, 0, h.data(), T, H, Hq * D, q.data());
  layer_linear(m, layer, 1, h.data(), T, H, Hkv * D, k.data());
  layer_linear(m, layer, 2, h.data(), T, H, Hkv * D, v.data());
  if (c.qk_norm) {  // ar.cpp:268-275: RMSNorm over D per head
    oracle_rms_norm(q.data(), T * Hq, D, w.q_norm[layer], c.rms_eps, qn.data());
    oracle_rms_norm(k.data(), T * Hkv, D, w.k_norm[layer], c.rms_eps, kn.data());
    q.swap(qn);
    k.swap(kn);
  }
  oracle_rope(q.data(), T, Hq, D, offset, c.rope_theta);  // ar.cpp:276-277
  oracle_rope(k.data(), T, Hkv, D, offset, c.rope_theta);
  // ar.cpp:119-123: append at the absolute slot `offset`.
  uint16_t *K = oracle_cache_keys(cache, layer), *V = oracle_cache_values(cache, layer);
  for (int t = 0; t < T; ++t)
    for (int hh = 0; hh < Hkv; ++hh)
      for (int d = 0; d < D; ++d) {
        const size_t slot = (size_t(hh) * cache->capacity + offset + t) * D + d;
        K[slot] = k[(size_t(t) * Hkv + hh) * D + d];
        V[slot] = v[(size_t(t) * Hkv + hh) * D + d];
      }
  oracle_attention(q.data(), K, V, T, Hq, Hkv, D, cache->capacity, offset,
                   att.data());
  layer_linear(m, layer, 3, att.data(), T, Hq * D, H, o.data());
  for (size_t i = 0; i < size_t(T) * H; ++i)  // ar.cpp:292-294
    x[i] = f2bf(bf2f(x[i]) + bf2f(o[i]));
  oracle_rms_norm(x, T, H, w.post_ln[layer], c.rms_eps, h.data());
  layer_linear(m, layer, 4, h.data(), T, H, F, g.data());
  layer_linear(m, layer, 5, h.data(), T, H, F, u.data());
  oracle_silu_mul(g.data(), u.data(), T * F, mm.data());
  layer_linear(m, layer, 6, mm.data(), T, F, H, dn.data());
  for (size_t i = 0; i < size_t(T) * H; ++i)  // ar.cpp:295-298
    x[i] = f2bf(bf2f(x[i]) + bf2f(dn[i]));
  return 0;
}

// ARModel::hidden, ar.cpp:246-301.
int oracle_hidden(oracle_model *m, oracle_cache *cache, const int32_t *ids,
                  int T, uint16_t *out) {
  const oracle_config &c = m->c;
  if (T < 1 || cache->offset + T > cache->capacity)
    return 2;
  for (int t = 0; t < T; ++t)
    if (ids[t] < 0 || ids[t] >= c.vocab)
      return 2;
  const int H = c.hidden;
  std::vector<uint16_t> x(size_t(T) * H);
  for (int t = 0; t < T; ++t)  // ar.cpp:259, take(embed_tokens, ids)
    std::memcpy(x.data() + size_t(t) * H, m->w.embed + size_t(ids[t]) * H, 2 * H);
  for (int l = 0; l < c.layers; ++l)
    if (int rc = oracle_layer(m, cache, l, x.data(), T))
      return rc;
  cache->offset += T;
  oracle_rms_norm(x.data(), T, H, m->w.final_norm, c.rms_eps, out);  // ar.cpp:300
  return 0;
}

int oracle_phase_size(const oracle_model *m, int phase) {
  Phase p;
  return phase_of(phase, m->c.vocab, p) ? p.size : -1;
}

// ARModel::project, ar.cpp:302-323: bf16(h @ lm_head[rows]^T).
int oracle_project(oracle_model *m, const uint16_t *h, int phase,
                   uint16_t *logits) {
  Phase p;
  if (!phase_of(phase, m->c.vocab, p))
    return 2;
  const int H = m->c.hidden;
  if (m->q.bits) {  // ar.cpp:306-312: quantized rows, one row range at a time
    const uint32_t *qw = reinterpret_cast<const uint32_t *>(m->w.lm_head);
    const size_t words = size_t(H) * m->q.bits / 32, groups = H / 64;
    auto range = [&](int start, int len, uint16_t *out) {
      oracle_qlinear(h, 1, H, qw + start * words, m->q.lm_scales + start * groups,
                     m->q.lm_biases + start * groups, m->q.bits, len, out);
    };
    range(p.seg0_start, p.seg0_len, logits);
    if (p.size > p.seg0_len)
      range(p.seg1_start, p.size - p.seg0_len, logits + p.seg0_len);
    return 0;
  }
  std::vector<float> hf(H);
  for (int i = 0; i < H; ++i)
    hf[i] = bf2f(h[i]);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < p.size; ++r) {
    const int row = r < p.seg0_len ? p.seg0_start + r : p.seg1_start + (r - p.seg0_len);
    logits[r] = f2bf(dot_f32_bf16(hf.data(), m->w.lm_head + size_t(row) * H, H));
  }
  return 0;
}

// ---- sampling ----

// sampling.cpp:100-115: delta = bf16(c - u); scaled = bf16(f32(delta) *
// f32(scale)); bf16(u + scaled).
void oracle_guided_logits(const uint16_t *c, const uint16_t *u, int n,
                          double scale, uint16_t *out) {
  const float s = float(scale);
  for (int i = 0; i < n; ++i) {
    const float delta = rbf(bf2f(c[i]) - bf2f(u[i]));
    const float scaled = rbf(delta * s);
    out[i] = f2bf(bf2f(u[i]) + scaled);
  }
}

// sampling.cpp:19-32.
int oracle_native_to_local(int token, int phase, int vocab) {
  switch (phase) {
  case ORACLE_PHASE_FULL:
    return token >= 0 && token < vocab ? token : -1;
  case ORACLE_PHASE_ABC:
    if (token >= 0 && token < EOD)
      return token;
    return token == ABC_END ? EOD : -1;
  case ORACLE_PHASE_SEMANTIC:
    if (token == MUSIC_END)
      return 0;
    if (token >= CODEC_OFFSET && token < CODEC_OFFSET + CODEC_SIZE)
      return token - MUSIC_END;
    return -1;
  }
  return -1;
}
// sampling.cpp:33-37.
int oracle_local_to_native(int token, int phase) {
  switch (phase) {
  case ORACLE_PHASE_ABC:
    return token < EOD ? token : ABC_END;
  case ORACLE_PHASE_SEMANTIC:
    return MUSIC_END + token;
  }
  return token;
}

// sampling.cpp:38-99 (sampling.py:78-134). Normal mode computes in fp32;
// legacy_off keeps every intermediate in bf16 (each op rounds). Returns 0, or
// 2 on a vocabulary mismatch.
int oracle_distribution(const uint16_t *logits, int n, const oracle_sampling *s,
                        const int32_t *history, int history_len, int step,
                        int phase, int legacy_off, float *scores) {
  const float inf = std::numeric_limits<float>::infinity();
  auto cast = [&](float v) { return legacy_off ? rbf(v) : v; };
  int end = -1;
  if (phase == ORACLE_PHASE_ABC)
    end = EOD;
  else if (phase == ORACLE_PHASE_SEMANTIC)
    end = 0;
  for (int i = 0; i < n; ++i)
    scores[i] = bf2f(logits[i]);
  if (step < s->min_tokens && end >= 0 && end < n)  // sampling.cpp:47-50
    scores[end] = -inf;
  if (s->repetition_penalty != 1.0 && history_len > 0) {  // sampling.cpp:51-75
    const int count = s->penalty_window == 0
                          ? history_len
                          : std::min(history_len, s->penalty_window);
    std::vector<int> freq_ids;
    std::vector<float> freq(n, 0.f);
    for (int i = history_len - count; i < history_len; ++i) {
      const int local = oracle_native_to_local(history[i], phase, n);
      if (local >= 0 && local < n)
        freq[local] += 1.f;
    }
    const float base = float(s->repetition_penalty);
    for (int i = 0; i < n; ++i) {
      if (freq[i] == 0.f)
        continue;  // alpha = pow(p, 0) = 1 leaves the score unchanged
      const float alpha = cast(std::pow(base, freq[i]));
      const float v = scores[i];
      scores[i] = v < 0.f ? cast(v * alpha) : cast(v / alpha);
    }
  }
  if (s->temperature == 0)
    return 0;
  if (s->temperature != 1) {  // sampling.cpp:78-81
    const float t = float(s->temperature);
    for (int i = 0; i < n; ++i)
      scores[i] = cast(scores[i] / t);
  }
  // sampling.cpp:82-84: threshold = k-th largest value (with multiplicity);
  // entries strictly below it are removed, so ties at the cut survive.
  const int k = std::min(s->top_k, n);
  {
    std::vector<float> tmp(scores, scores + n);
    std::nth_element(tmp.begin(), tmp.begin() + (k - 1), tmp.end(),
                     std::greater<float>());
    const float threshold = tmp[k - 1];
    for (int i = 0; i < n; ++i)
      if (scores[i] < threshold)
        scores[i] = -inf;
  }
  if (s->top_p < 1) {  // sampling.cpp:85-97
    // Order: value descending, equal values by ascending index (this build's
    // definition; MLX argsort's order among equal values is unspecified).
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return scores[a] > scores[b]; });
    const float m = scores[order[0]];
    std::vector<float> e(n), p(n);
    float total = 0.f;
    for (int r = 0; r < n; ++r) {  // sequential sum in sorted order
      e[r] = m == -inf ? 0.f : oracle_pexp(scores[order[r]] - m);
      total += e[r];
    }
    for (int r = 0; r < n; ++r)
      p[r] = legacy_off ? rbf(e[r] / total) : e[r] / total;
    const float top_p = float(s->top_p);
    const int minimum = legacy_off ? 3 : 1;
    float cumulative = 0.f;
    for (int r = 0; r < n; ++r) {
      cumulative = cast(cumulative + p[r]);
      const float preceding = cast(cumulative - p[r]);
      if (preceding > top_p && r >= minimum)
        scores[order[r]] = -inf;
    }
  }
  return 0;
}

// Draw: sampling.cpp:247-248. Greedy = argmax with the lowest index on ties.
// Categorical = this build's shared-uniform protocol: argmax over finite
// scores of s_i + g_i, g_i = -log(-log(u(seed, step, i))) with the portable
// log above (MLX categorical is likewise a Gumbel-max draw).
int oracle_draw(const float *scores, int n, double temperature, uint64_t seed,
                int step) {
  int best = -1;
  float best_key = -std::numeric_limits<float>::infinity();
  for (int i = 0; i < n; ++i) {
    if (!(scores[i] > -std::numeric_limits<float>::infinity()))
      continue;
    float key = scores[i];
    if (temperature != 0) {
      const float u = oracle_uniform(seed, step, i);
      key = scores[i] + (-oracle_plog(-oracle_plog(u)));
    }
    if (best < 0 || key > best_key) {
      best = i;
      best_key = key;
    }
  }
  return best < 0 ? 0 : best;
}

} // extern "C"
