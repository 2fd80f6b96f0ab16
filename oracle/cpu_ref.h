/*
 * cpu_ref — CPU restatement of the reference AR decode path (TEST INFRASTRUCTURE).
 *
 * This library is the oracle: it restates, in plain C++ on the host, the
 * arithmetic of the reference's autoregressive decode loop so that the HIP
 * product can be checked against it. Only tests, the smoke check and the CPU
 * baseline leg of the benchmark may load it; the product never links it.
 *
 * Followed reference files (paths relative to the reference checkout):
 *   native/src/ar.cpp:19-132, 246-323     model ops, KV cache, hidden(), project()
 *   native/src/sampling.cpp:8-183          phase maps, distribution, CFG, prefill
 *   oracle/port/lyra/ar.py:56-145          rounding points of every op (docstrings)
 *   oracle/port/lyra/sampling.py:58-152    window penalty, distribution, CFG
 *   vendor/yue/src/yue2/fast.py:123-136    windowed penalty lookup-table form
 *
 * All bf16 tensors are passed as uint16_t bit patterns. Accumulation is fp32.
 * Every bf16 rounding point of the reference graph is reproduced.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   bf16 RNE, Philox4x32-10 ....... published Random123 KAT + rocRAND fixture
 *   rms_norm ...................... closed form; constant-row special case
 *   linear ........................ fp64 brute force; one-hot weights
 *   qlinear / dequantize .......... fp64 brute force over the unpacked codes;
 *                                   equality with linear when every s q + b is
 *                                   a bf16 value; zero codes give the bias
 *                                   term alone. The U32 packing order (MLX
 *                                   quantize: element j of a word at bits
 *                                   bits * j) is parity unpinned: MLX is
 *                                   absent and the reference holds no
 *                                   quantized fixture.
 *   rope .......................... position 0 identity; norm preservation
 *   silu_mul ...................... reference test_ar.py known answers
 *   attention ..................... fp64 brute force; split-merge identity;
 *                                   causal chunk == full
 *   nar_attention ................. fp64 brute force; key permutation
 *                                   invariance; causal == the AR prefill
 *                                   attention; equal keys give the mean of V
 *   layer / model composition ..... golden vectors from the upstream torch model
 *   guided_logits ................. reference test_sampling.py known answers
 *   distribution .................. reference test_sampling.py / test_fast.py
 *                                   known answers (top-k ties, shifted nucleus,
 *                                   legacy floor, windowed penalty)
 *   sample (Philox/Gumbel draw) ... a protocol of this build: the reference's
 *                                   MLX threefry stream is parity unpinned.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oracle_config {
  int32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  float rms_eps;
  double rope_theta;
  int32_t qk_norm; /* 1: per-head q/k RMSNorm (ar.cpp:268-275) */
} oracle_config;

/* Borrowed host pointers; per-layer arrays have `layers` entries. */
typedef struct oracle_weights {
  const uint16_t *embed, *final_norm, *lm_head;
  const uint16_t *const *input_ln, *const *post_ln, *const *q_norm,
      *const *k_norm;
  const uint16_t *const *wq, *const *wk, *const *wv, *const *wo;
  const uint16_t *const *wg, *const *wu, *const *wd;
} oracle_weights;

/* Affine group-64 quantized linears (ar.cpp:20-29, 209-214; the
 * conversion.cpp:470-532 layout): when bits is 8 or 4, the seven projection
 * pointers of oracle_weights and lm_head point to packed uint32 codes
 * [rows][k * bits / 32] and scales / biases hold [rows][k / 64] bf16 per
 * linear (index 0..6 = q, k, v, o, gate, up, down; [layers] each). */
typedef struct oracle_quant {
  int32_t bits;
  const uint16_t *lm_scales, *lm_biases;
  const uint16_t *const *scales[7];
  const uint16_t *const *biases[7];
} oracle_quant;

typedef struct oracle_sampling {
  double temperature, top_p;
  int32_t top_k;
  double repetition_penalty;
  int32_t penalty_window, min_tokens, max_tokens;
} oracle_sampling;

enum { ORACLE_PHASE_FULL = 0, ORACLE_PHASE_ABC = 1, ORACLE_PHASE_SEMANTIC = 2 };

typedef struct oracle_model oracle_model;
typedef struct oracle_cache oracle_cache;

/* ---- scalar helpers ---- */
uint16_t oracle_f2bf(float x);
float oracle_bf2f(uint16_t x);
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2],
                          uint32_t out[4]);
float oracle_uniform(uint64_t seed, int32_t step, int32_t index);
float oracle_plog(float x);
float oracle_pexp(float x);
void oracle_set_threads(int n);
/* 0: fp32 blocked accumulation (default); 1: fp64 accumulation. */
void oracle_set_accumulation(int mode);

/* ---- model_ops (ar.cpp:19-96) ---- */
void oracle_rms_norm(const uint16_t *x, int rows, int n, const uint16_t *w,
                     float eps, uint16_t *y);
void oracle_linear(const uint16_t *x, int rows, int k, const uint16_t *w,
                   int n, uint16_t *y);
/* mx::quantized_matmul(x, w, scales, biases, transpose=true, 64, bits,
 * "affine") (ar.cpp:22-24): y = bf16(sum_g (s_g * sum_{i in g} x_i q_i +
 * b_g * sum_{i in g} x_i)), fp32 sums per group and over groups. */
void oracle_qlinear(const uint16_t *x, int rows, int k, const uint32_t *w,
                    const uint16_t *scales, const uint16_t *biases, int bits,
                    int n, uint16_t *y);
/* bf16(s * q + b) per element (s * q is exact in fp32; one fp32 add). */
void oracle_dequantize(const uint32_t *w, const uint16_t *scales,
                       const uint16_t *biases, int bits, int n, int k,
                       uint16_t *out);
void oracle_rope(uint16_t *x, int T, int heads, int d, int offset,
                 double theta);
void oracle_silu_mul(const uint16_t *g, const uint16_t *u, int n,
                     uint16_t *out);
/* q [T][Hq][D]; keys/values [Hkv][cap][D]; attends to slots [0, offset+t]
 * for query t (bottom-right causal); out [T][Hq*D]. T==1 uses the decode
 * formulation (ar.cpp:88-91), T>1 the fp32 causal one (ar.cpp:286-290). */
void oracle_attention(const uint16_t *q, const uint16_t *keys,
                      const uint16_t *values, int T, int Hq, int Hkv, int D,
                      int cap, int offset, uint16_t *out);
/* nar_attention (nar_attention.cpp:63-270): q [B][Hq][Lq][D], keys/values
 * [B][Hkv][Lk][D], out [B][Hq][Lq][D]; fp32 scores times scale * log2(e),
 * exp2 softmax, fp32 P.V, bf16(o / l); causal needs Lq == Lk. */
void oracle_nar_attention(const uint16_t *q, const uint16_t *keys, const uint16_t *values,
                          int B, int Hq, int Hkv, int Lq, int Lk, int D, int causal,
                          uint16_t *out);
void oracle_rope_table(int positions, int d, double theta, uint16_t *cos_out,
                       uint16_t *sin_out);

/* ---- model / cache (ar.cpp:98-132, 246-323) ---- */
oracle_model *oracle_model_new(const oracle_config *c, const oracle_weights *w);
/* As oracle_model_new with affine-quantized linears (q->bits 8 or 4). */
oracle_model *oracle_model_new_quantized(const oracle_config *c, const oracle_weights *w,
                                         const oracle_quant *q);
void oracle_model_free(oracle_model *m);
oracle_cache *oracle_cache_new(const oracle_model *m, int capacity);
void oracle_cache_free(oracle_cache *c);
int oracle_cache_offset(const oracle_cache *c);
void oracle_cache_set_offset(oracle_cache *c, int offset);
int oracle_cache_capacity(const oracle_cache *c);
uint16_t *oracle_cache_keys(oracle_cache *c, int layer);
uint16_t *oracle_cache_values(oracle_cache *c, int layer);
/* One decoder layer over x [T][H] (in place), appending K/V at the cache
 * offset without advancing it. Returns 0, or 2 on capacity overflow. */
int oracle_layer(oracle_model *m, oracle_cache *c, int layer, uint16_t *x,
                 int T);
/* ARModel::hidden: embedding, all layers, final norm; advances the offset.
 * out [T][H]. Returns 0, or 2 (ValueError) without mutating on overflow or
 * bad ids. */
int oracle_hidden(oracle_model *m, oracle_cache *c, const int32_t *ids, int T,
                  uint16_t *out);
/* ARModel::project for one hidden row; logits length = phase size. */
int oracle_project(oracle_model *m, const uint16_t *h, int phase,
                   uint16_t *logits);
int oracle_phase_size(const oracle_model *m, int phase);

/* ---- sampling (sampling.cpp:8-134) ---- */
void oracle_guided_logits(const uint16_t *c, const uint16_t *u, int n,
                          double scale, uint16_t *out);
int oracle_distribution(const uint16_t *logits, int n,
                        const oracle_sampling *s, const int32_t *history,
                        int history_len, int step, int phase, int legacy_off,
                        float *scores);
/* Greedy argmax (lowest index on ties) when temperature == 0, else the
 * Philox/Gumbel categorical draw over finite scores. Returns local index. */
int oracle_draw(const float *scores, int n, double temperature, uint64_t seed,
                int step);
int oracle_native_to_local(int token, int phase, int vocab);
int oracle_local_to_native(int token, int phase);

#ifdef __cplusplus
}
#endif
