// Kernel parameter blocks and host launchers for the gfx950 AR decode path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace yuear {

enum GemvEpilogue : int {
  kEpiStore = 0,     // y = bf16(acc)
  kEpiResidual = 1,  // y = bf16(y + bf16(acc))                 (ar.cpp:292-298)
  kEpiSwiGLU = 2,    // rows (2i, 2i+1) = (gate_i, up_i):
                     // y[i] = bf16(bf16(silu(bf16(g))) * bf16(u)) (ar.cpp:36-51)
};

// y[b, r] = x[b, :] . W[row(r), :], bf16 in, fp32 accumulate.
struct GemvParams {
  const uint16_t *w = nullptr;  // [rows][k]
  int n = 0;                    // output rows (phase-local rows for lm_head)
  int k = 0;
  int batch = 1;
  const uint16_t *x = nullptr;  // [batch][x_stride]
  int x_stride = 0;
  const uint16_t *embed = nullptr;  // optional gather table [vocab][k]
  const int32_t *tokens = nullptr;  // [batch] rows of `embed`
  int embed_rows = 0;               // token ids are clamped to [0, embed_rows)
  uint16_t *x_out = nullptr;        // gathered rows are stored here (block 0)
  const uint16_t *norm_w = nullptr; // optional RMSNorm prologue gain [k]
  float eps = 1e-6f;
  uint16_t *y = nullptr;
  int y_stride = 0;
  int epilogue = kEpiStore;
  int seg0_start = 0, seg0_len = 1 << 30, seg1_start = 0;  // row map
  int32_t *advance = nullptr;  // block 0 increments advance[0..batch)
  // [batch][k] scratch for the batched (MFMA) form: with a gather or an
  // RMSNorm prologue, a row kernel first writes the prepared rows here once
  // instead of every workgroup re-normalising them.
  uint16_t *stage = nullptr;
  // The same weight rows in the MFMA-tiled layout of launch_tile_rows, read
  // by the batched form when given (1 KiB contiguous per wave-load instead of
  // 16 row pieces of 64 bytes).
  const uint16_t *w_tiled = nullptr;
  // Affine group-64 quantized weights (bits 8 or 4; 0: bf16 only): codes
  // [rows][k * bits / 32] and one scale | bias << 16 word per group
  // [rows][k / 64] (qgemv.hip). launch_gemv reads them for 1-2 branches;
  // the batched form reads `w`, which then holds the dequantized rows.
  const uint32_t *qw = nullptr;
  const uint32_t *qsb = nullptr;
  int bits = 0;
};
hipError_t launch_gemv(const GemvParams &p, hipStream_t s);
// Quantized GEMV for 1-2 branches (qgemv.hip); k a multiple of 64 whose
// pieces map onto 8..64 lanes per row.
bool qgemv_supported(int bits, int k, int batch);
hipError_t launch_qgemv(const GemvParams &p, hipStream_t s);
// out [rows][k] = bf16(s q + b) of quantized rows (codes / group words as in
// GemvParams::qw / qsb).
hipError_t launch_dequantize(const uint32_t *codes, const uint32_t *sb, int bits, int rows, int k,
                             uint16_t *out, hipStream_t s);
// Host: affine group-64 quantization of bf16 rows [rows][k] into codes
// [rows][k * bits / 32] and bf16 scales / biases [rows][k / 64]
// (quantize.hip).
void quantize_affine(const uint16_t *w, int64_t rows, int k, int bits, uint32_t *codes,
                     uint16_t *scales, uint16_t *biases);
// MFMA form for 3..8 independent rows (batched sequences); launch_gemv
// dispatches to it when gemv_mfma_supported(p).
bool gemv_mfma_supported(const GemvParams &p);
hipError_t launch_gemv_mfma(const GemvParams &p, hipStream_t s);
// Copy W [n][k] (k a multiple of 32) into the MFMA-tiled layout: for each
// 16-row tile t and 32-column step s, 1 KiB whose 16-byte piece l is row
// 16 t + l % 16, columns 32 s + 8 (l / 16) + [0, 8) (rows past n zero);
// out holds ceil(n / 16) * 16 * k elements.
hipError_t launch_tile_rows(const uint16_t *w, int n, int k, uint16_t *out, hipStream_t s);

// KV cache layout of one (branch, kv head), `capacity` slots (a multiple of
// 32): K row-major [capacity][128]; V in 32-slot blocks stored dim-major,
// element (t, d) at attn::v_index(t, d) = (t / 32) * 4096 + d * 32 + t % 32.

// Arrival counters of the decode attention sit kCounterStride ints (256
// bytes) apart: the atomics of different (branch, kv head) pairs then land on
// different memory channels instead of queueing on one cache line.
constexpr int kCounterStride = 64;

// Split-K flash-decode attention for one layer, all branches, with the
// q/k RMSNorm + RoPE prologue, the KV append of the current token and the
// last-block merge of the split partials fused in.
struct AttnDecodeParams {
  const uint16_t *qkv = nullptr;  // [batch][qkv_stride] raw projections
  int qkv_stride = 0;
  const uint16_t *q_norm = nullptr, *k_norm = nullptr;  // [D] or null
  float eps = 1e-6f;
  const uint16_t *rope_cos = nullptr, *rope_sin = nullptr;  // [positions][D/2]
  uint16_t *k_cache = nullptr, *v_cache = nullptr;  // [batch][Hkv] x (capacity slots)
  const int32_t *pos = nullptr;  // [batch] slot of the current token
  int heads = 0, kv_heads = 0, head_dim = 128, capacity = 0, batch = 1;
  int max_splits = 1;
  float *part_o = nullptr;   // [batch][Hkv][max_splits][G][D]
  float *part_ml = nullptr;  // [batch][Hkv][max_splits][G][2]
  int32_t *counters = nullptr;  // [batch][Hkv] x kCounterStride ints, zero between launches
  uint16_t *out = nullptr;      // [batch][out_stride]
  int out_stride = 0;
};
hipError_t launch_attn_decode(const AttnDecodeParams &p, hipStream_t s);
// Splits per (branch, kv head) for a session (max_splits above).
int attn_decode_splits(int batch, int kv_heads, int kv_stride);

// Acoustic-model attention (nar_attention.hip, nar_attention.cpp:63-270):
// q [batch][heads][q_len][128], k / v [batch][kv_heads][kv_len][128], out
// like q; vb: workspace of nar_attention_workspace_elems() bf16 (V in 32-key
// dim-major blocks). causal needs q_len == kv_len.
struct NarAttnParams {
  const uint16_t *q = nullptr, *k = nullptr, *v = nullptr;
  uint16_t *vb = nullptr;
  uint16_t *out = nullptr;
  int batch = 1, heads = 0, kv_heads = 0, q_len = 0, kv_len = 0, causal = 0;
  int kv_pad = 0;  // set by launch_nar_attention: kv_len rounded up to 32
  // optional split-key scratch (nar_attention_part_floats() floats): with it,
  // launches too small to fill the GPU split the keys over workgroups
  float *part = nullptr;
  size_t part_floats = 0;
  int splits = 1;  // set by launch_nar_attention
};
// Floats of split-key partials that let launch_nar_attention split this
// launch's keys (0: it never splits this shape).
size_t nar_attention_part_floats(int batch, int heads, int q_len, int kv_len, int causal);
size_t nar_attention_workspace_elems(int batch, int kv_heads, int kv_len);
// Keys [0, n) of `heads` cache heads (V in 32-key dim-major blocks, heads
// kv_stride slots apart) to row-major out [heads][n][128].
hipError_t launch_v_rows(const uint16_t *vb, int kv_stride, int heads, int n, uint16_t *out,
                         hipStream_t s);
hipError_t launch_nar_attention(NarAttnParams p, hipStream_t s);

// Device sampler: CFG merge + distribution() + draw, one token per call.
struct SamplerParams {
  const uint16_t *logits = nullptr;  // [branches][ls] phase-local bf16
  int n = 0;
  int ls = 0;  // logits row stride (multiple of 8 elements)
  int branches = 1;
  float cfg_scale = 1.0f;  // applied when branches == 2 and != 1
  float temperature = 0.f, top_p = 1.f;
  int top_k = 1;
  int min_tokens = 0;
  int penalty_window = 0;
  const float *alphas = nullptr;  // [window+1] pow(penalty, count), or null
  int phase = kPhaseFull;
  int vocab = 0;
  uint64_t seed = 0;
  int legacy_off = 0;
  int32_t *state = nullptr;   // [0]=step counter, [1]=done flag
  int32_t *history = nullptr; // [max_tokens] native tokens emitted so far
  int hist_len = -1;          // history length; < 0: the step counter
  int max_tokens = 0;         // appends history[step] while step < max_tokens
  int32_t *tokens_out = nullptr;  // [branches] next input token (native)
  float *scratch = nullptr;       // [n] fp32 scores
  uint32_t *scratch_u = nullptr;  // [2 * n] survivor keys / indices
  // Independent branches (batched sequences): workgroup b samples branch b
  // from its own logits row with its own state[2b..2b+1], history row
  // (history + b * history_stride), scratch (+ b * scratch_stride /
  // scratch_u_stride) and seed + b; no CFG. Otherwise one draw is shared by
  // all branches (a request, or a CFG pair).
  int independent = 0;
  int history_stride = 0, scratch_stride = 0, scratch_u_stride = 0;
  // [1] arrival counter, zero between launches: with it a shared draw
  // (greedy, or top k up to 128) over more than 8192 rows is spread over one
  // workgroup per ~8192 rows; null keeps one workgroup.
  int32_t *sync = nullptr;
  int split_rows = 0;  // set by launch_sampler
};
// scratch_u must hold n 8-byte candidate words (2n entries) when sync is set.
hipError_t launch_sampler(const SamplerParams &p, hipStream_t s);

// ---- prefill ----
struct GemmParams {
  const uint16_t *a = nullptr;  // [m][k] activations
  int lda = 0;
  const uint16_t *w = nullptr;  // [n][k] weights
  int m = 0, n = 0, k = 0;
  uint16_t *c = nullptr;        // [m][ldc]
  int ldc = 0;
  int residual = 0;             // 1: c = bf16(c + bf16(acc)); 2: SwiGLU pairs, c [m][n / 2]
  // split-K workspace: fp32 partials [splits][m][n]; null: K is never split
  float *part = nullptr;
  size_t part_bytes = 0;
  // split-K: leave the partials to the caller's reduce (launch_gemm_reduce_norm)
  bool defer_reduce = false;
};
// MFMA GEMM (gemm.hip); k a multiple of 64, lda a multiple of 8. With a
// workspace it may split K over workgroups (gemm_plan picks the tile shape
// and split count together), summing the splits in a fixed order.
hipError_t launch_gemm(const GemmParams &p, hipStream_t s);
// One of the GEMM's tile shapes (0..5, see gemm.hip) with K in `splits`
// ranges (splits > 1 needs p.part of splits * m * n floats, k / 64 a multiple
// of splits), the shape launch_gemm would pick for m x n on `cus` CUs, and
// its split count.
hipError_t launch_gemm_tile(const GemmParams &p, int shape, hipStream_t s, int splits = 1);
int gemm_tile_choice(int m, int n, int cus);
int gemm_cus();  // CUs of the current device (256 if it cannot be read)
// The reduce of a residual GEMM launched with defer_reduce and splits > 1
// (c = bf16(c + bf16(sum of the splits in split order)), as
// gemm_reduce_kernel) fused with the RMSNorm of the updated rows into y
// (rms_norm_rows): one workgroup per row, bit-identical to the two kernels.
// residual 1, n a multiple of 8 up to 8192, ldc == n.
hipError_t launch_gemm_reduce_norm(const GemmParams &p, int splits, const uint16_t *norm_w,
                                   float eps, uint16_t *y, hipStream_t s);
void gemm_plan(int m, int n, int k, int cus, size_t part_bytes, int *shape, int *splits);

hipError_t launch_embed_rows(const uint16_t *table, const int32_t *ids, int rows,
                             int width, uint16_t *out, hipStream_t s);
hipError_t launch_rms_norm_rows(const uint16_t *x, int rows, int width,
                                const uint16_t *w, float eps, uint16_t *y,
                                hipStream_t s);

// q/k RMSNorm + RoPE for T tokens at absolute positions pos0 + t; writes q
// [T][Hq][D] and appends K/V at slots pos0 + t of one branch's cache.
struct QkPrepParams {
  const uint16_t *qkv = nullptr;  // [T][qkv_stride]
  int qkv_stride = 0;
  int tokens = 0;
  const uint16_t *q_norm = nullptr, *k_norm = nullptr;
  float eps = 1e-6f;
  const uint16_t *rope_cos = nullptr, *rope_sin = nullptr;
  int pos0 = 0;
  int heads = 0, kv_heads = 0, head_dim = 128, capacity = 0;
  uint16_t *q_out = nullptr;  // [T][Hq][D]
  uint16_t *k_cache = nullptr, *v_cache = nullptr;  // this branch, [Hkv] x (capacity slots)
};
hipError_t launch_qk_prep(const QkPrepParams &p, hipStream_t s);

// Causal attention for T queries at positions pos0 + t over keys [0, pos0+t]
// with fp32 opmath (ar.cpp:284-291). out [T][Hq*D].
struct AttnPrefillParams {
  const uint16_t *q = nullptr;  // [T][Hq][D]
  const uint16_t *k_cache = nullptr, *v_cache = nullptr;  // [Hkv] x (capacity slots)
  int tokens = 0, pos0 = 0;
  int heads = 0, kv_heads = 0, head_dim = 128, capacity = 0;
  uint16_t *out = nullptr;
};
hipError_t launch_attn_prefill(const AttnPrefillParams &p, hipStream_t s);

}  // namespace yuear
