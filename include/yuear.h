/*
 * yuear.h — C ABI of the gfx950 (MI355X) autoregressive decode library.
 *
 * Drop-in boundary for the reference's AR decode loop. The reference engine
 * API it replaces is native/include/lyra/ar.hpp:8-48 (ARModel, KVCache,
 * generate_tokens), whose only caller is Pipeline::generate_phase
 * (native/src/pipeline.cpp:186-211); the GraphAR decode-step pattern it
 * mirrors is vendor/yue/src/yue2/cuda_graph.py:35-240. ABI conventions follow
 * native/include/CLyraCore/lyra.h:8-54: opaque handles, UTF-8 JSON for results
 * and errors, caller-owned output strings freed with yuear_string_free, status
 * codes 0/1/2/130, no exception crosses the boundary, one call at a time per
 * handle, synchronous execution on the calling thread.
 *
 * All bf16 data crossing the boundary is passed as uint16_t bit patterns.
 * Host pointers unless a name says `dev_` (device pointers, for the op-level
 * entry points that mirror the reference's model_ops namespace).
 */
#ifndef YUEAR_H
#define YUEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* lyra.h:18-23 */
typedef enum yuear_status {
  YUEAR_SUCCESS = 0,
  YUEAR_FAILURE = 1,
  YUEAR_INVALID_INPUT = 2,
  YUEAR_CANCELLED = 130
} yuear_status;

/* Architectural config (the fields ar.cpp:164-192 validates). */
typedef struct yuear_model_config {
  int32_t hidden_size, intermediate_size, num_hidden_layers;
  int32_t num_attention_heads, num_key_value_heads, head_dim;
  int32_t vocab_size, max_position_embeddings;
  float rms_norm_eps;
  double rope_theta;
  int32_t qk_norm; /* 1 = Qwen3 per-head q/k RMSNorm (ar.cpp:268-275) */
} yuear_model_config;

/* Sampling, native/include/lyra/types.hpp:29-38. */
typedef struct yuear_sampling {
  double temperature, top_p;
  int32_t top_k;
  double repetition_penalty;
  int32_t penalty_window, min_tokens, max_tokens;
} yuear_sampling;

/* One named host tensor, names as in the reference checkpoint
 * (ar.cpp:216-233): model.embed_tokens.weight, model.norm.weight,
 * lm_head.weight, model.layers.{i}.{input_layernorm,post_attention_layernorm,
 * self_attn.{q,k,v,o}_proj,self_attn.{q,k}_norm,mlp.{gate,up,down}_proj}.weight.
 * With affine-quantized linears (ar.cpp:209-214) every *_proj and the
 * lm_head come as <name>.weight (YUEAR_DTYPE_U32 codes [rows][k * bits / 32])
 * plus <name>.scales and <name>.biases (bf16 [rows][k / 64]). numel counts
 * elements of `dtype`. */
enum { YUEAR_DTYPE_BF16 = 0, YUEAR_DTYPE_U32 = 1 };
typedef struct yuear_tensor {
  const char *name;
  const void *data;
  int64_t numel;
  int32_t dtype;
} yuear_tensor;

enum { YUEAR_WEIGHTS_RANDOM = 0, YUEAR_WEIGHTS_HOST = 1 };
typedef struct yuear_weight_source {
  int32_t kind;
  /* RANDOM: linear/embedding weights N(0, std); norm gains 1 + N(0, norm_std);
   * with bits 8 / 4 the linears are then quantized by yuear_quantize_affine */
  uint64_t seed;
  float std, norm_std;
  /* HOST: every tensor of the model exactly once */
  const yuear_tensor *tensors;
  int32_t count;
  /* 0: bf16 linears; 8 or 4: affine group-64 quantized linears (the
   * "8bit" / "4bit" precisions, conversion.cpp:470-532) */
  int32_t bits;
} yuear_weight_source;

typedef struct yuear_engine yuear_engine;
typedef struct yuear_session yuear_session;

/* Per-token callback (types.hpp:27 TokenCallback): phase and native id.
 * Runs synchronously on the calling thread; must not re-enter. */
typedef void (*yuear_token_callback)(void *user_data, const char *phase, int32_t token);

/* Cancellation poll (types.hpp:26 Cancelled): nonzero cancels the call.
 * Runs synchronously on the calling thread, like the token callback. */
typedef int32_t (*yuear_cancel_poll)(void *user_data);

/* Borrowed build identity (lyra.h:29). */
const char *yuear_build_identifier(void);
void yuear_string_free(char *s); /* lyra.h:54 */

/* ---- engine (replaces ARModel construction, ar.cpp:133-245) ---- */
yuear_status yuear_engine_create(const yuear_model_config *config,
                                 const yuear_weight_source *weights,
                                 yuear_engine **out, char **error_json);
void yuear_engine_destroy(yuear_engine *engine);
/* Checkpoint directory (replaces ARModel(directory, precision, verify=false),
 * ar.cpp:133-238): conversion.json (schema 1; precisions[precision].ar =
 * "ar-<precision>.safetensors", bf16 with dtype "bfloat16"), config.json
 * (ar.cpp:161-192 checks; strict != 0 also requires the YuE2 dimensions of
 * ar.cpp:164-178, otherwise any architecture this build implements), then
 * the safetensors file: every tensor of ar.cpp:216-233 with its shape and
 * dtype and nothing else, with the reference's error messages: BF16, or
 * for precision "8bit"/"4bit" (manifest bits, group_size 64, mode affine,
 * linear_only) U32 codes plus BF16 scales and biases for every linear.
 * Errors: FileNotFoundError (status 1) for missing files or
 * precisions, ValueError (status 2) otherwise. inspect reads and checks the
 * directory without touching the GPU and returns the architecture. */
yuear_status yuear_checkpoint_inspect(const char *directory, const char *precision,
                                      int32_t strict, yuear_model_config *config_out,
                                      char **error_json);
yuear_status yuear_engine_load(const char *directory, const char *precision, int32_t strict,
                               yuear_engine **out, char **error_json);
/* 0 for bf16 linears, else the quantization bits of the engine's linears. */
int32_t yuear_engine_bits(const yuear_engine *engine);
/* Host: affine group-64 quantization of bf16 rows w [rows][k] (k a multiple
 * of 64) into codes [rows][k * bits / 32] and bf16 scales / biases
 * [rows][k / 64], as mx::quantize(w, 64, bits, "affine") at
 * conversion.cpp:508 (restated from MLX's published algorithm: the edge of
 * larger magnitude is kept exactly as the bias). */
void yuear_quantize_affine(const uint16_t *w, int64_t rows, int32_t k, int32_t bits,
                           uint32_t *codes, uint16_t *scales, uint16_t *biases);
/* Thread-safe cooperative cancellation of the running call (lyra.h:40). */
void yuear_engine_cancel(yuear_engine *engine);
/* Deterministic weight generator (host): the bytes RANDOM sources upload. */
int32_t yuear_tensor_id(const char *name);
void yuear_random_tensor(uint64_t seed, int32_t tensor_id, float mean, float std,
                         int64_t numel, uint16_t *out);

/* ---- generate_tokens (sampling.cpp:185-288, ar.hpp:43-48) ----
 * phase: "full" (identity map, no end token), "abc" or "semantic".
 * tokens_out receives up to sampling->max_tokens native ids; *n_out the
 * count, *truncated 1 when no end token was drawn; *timing_json the timing
 * keys of sampling.cpp:274-284. Draws use the shared Philox uniforms
 * u(seed, step, index).
 * `cancelled` (may be NULL) and yuear_engine_cancel are checked where the
 * reference polls its Cancelled predicate, with its messages (status 130,
 * InterruptedError): after validation and at the start of each branch's
 * prefill, "Cancelled before prefill" (sampling.cpp:156, 206); between
 * prefill chunks, "Cancelled during prefill" (sampling.cpp:164); before each
 * token is emitted, "Cancelled during <phase>" (sampling.cpp:243). A decode
 * step runs as one graph, so the reference's per-layer poll inside a forward
 * (ar.cpp:261-262) becomes the next per-token poll. Both callbacks receive
 * `user_data`. */
yuear_status yuear_generate_tokens(
    yuear_engine *engine, const int32_t *prefix, int32_t n_prefix,
    const yuear_sampling *sampling, uint64_t seed, const char *phase,
    const int32_t *negative, int32_t n_negative, double cfg_scale,
    int32_t legacy_off, yuear_cancel_poll cancelled, yuear_token_callback on_token,
    void *user_data, int32_t *tokens_out, int32_t *n_out, int32_t *truncated,
    char **timing_json, char **error_json);

/* ---- decode-step session (GraphAR, cuda_graph.py:43-240; KVCache,
 * ar.cpp:98-132) ----
 * branches in [1, 8] (1 request, 2 = CFG pair, up to 8 independent
 * sequences); capacity in [1, min(24576, max_position_embeddings)]. */
yuear_status yuear_session_begin(yuear_engine *engine, int32_t branches,
                                 int32_t capacity, const char *phase,
                                 yuear_session **out, char **error_json);
void yuear_session_end(yuear_session *session);
/* Appends n ids to one branch (chunked causal prefill, sampling.cpp:152-183);
 * logits_out (nullable) receives that branch's last-token logits. Fails
 * without mutation when the capacity would be exceeded (ar.cpp:109-112). */
yuear_status yuear_session_prefill(yuear_session *session, int32_t branch,
                                   const int32_t *ids, int32_t n,
                                   uint16_t *logits_out, char **error_json);
/* One decode step for every branch (tokens[branches]); captured as one
 * hipGraph on first use. logits_out (nullable) is [branches][phase size]. */
yuear_status yuear_session_step(yuear_session *session, const int32_t *tokens,
                                uint16_t *logits_out, char **error_json);
/* Runs the device sampler once on the current logits of the session:
 * CFG merge (cfg_scale != 1 with 2 branches), distribution() with the given
 * step and history (native ids), then the draw. */
yuear_status yuear_session_sample(yuear_session *session,
                                  const yuear_sampling *sampling, uint64_t seed,
                                  double cfg_scale, int32_t legacy_off,
                                  int32_t step, const int32_t *history,
                                  int32_t history_len, int32_t *token_out,
                                  char **error_json);
int32_t yuear_session_position(const yuear_session *session, int32_t branch);
int32_t yuear_session_phase_size(const yuear_session *session);
/* Cache access for tests/tools: copies slots [0, n) of one layer/branch
 * (k, v: [Hkv][n][D] bf16). write sets the branch position to n. */
yuear_status yuear_session_write_kv(yuear_session *session, int32_t layer,
                                    int32_t branch, const uint16_t *k,
                                    const uint16_t *v, int32_t n,
                                    char **error_json);
yuear_status yuear_session_read_kv(yuear_session *session, int32_t layer,
                                   int32_t branch, uint16_t *k, uint16_t *v,
                                   int32_t n, char **error_json);
/* Test hooks: overwrite the session logits ([branches][phase size]) that the
 * next yuear_session_sample reads; set one branch's position (the next
 * slot; stale slots beyond it stay invisible, ar.cpp:124-126). */
yuear_status yuear_session_write_logits(yuear_session *session,
                                        const uint16_t *logits, char **error_json);
yuear_status yuear_session_set_position(yuear_session *session, int32_t branch,
                                        int32_t position, char **error_json);
/* One decoder layer decode step (ar.cpp:265-298) on explicit hidden rows
 * x_in [branches][H], appending at each branch's position (advanced by 1). */
yuear_status yuear_session_layer_step(yuear_session *session, int32_t layer,
                                      const uint16_t *x_in, uint16_t *x_out,
                                      char **error_json);
/* Mean device time of the last `yuear_session_time_steps` call, and a timed
 * loop of `steps` graph replays (no host sync between replays) with hipEvents
 * recorded on the session stream; returns milliseconds per step. */
yuear_status yuear_session_time_steps(yuear_session *session, int32_t steps,
                                      double *ms_per_step, char **error_json);

/* Timed device-side greedy/sampled decode loop for benchmarks: `steps`
 * graph replays of (sampler -> decode step) with no host synchronisation in
 * between, timed with hipEvents on the session stream. The sampler state
 * (step counter, history) restarts when reset != 0. tokens_out (nullable)
 * receives the emitted native ids of this call (branch 0). With more than
 * two branches every branch is an independent sequence (its own draw,
 * history and seed + branch); with one or two, one draw feeds all branches
 * (a request, or its CFG pair with cfg_scale 1). */
yuear_status yuear_session_time_generate(yuear_session *session,
                                         const yuear_sampling *sampling,
                                         uint64_t seed, int32_t steps,
                                         int32_t reset, double *ms_per_step,
                                         int32_t *tokens_out, char **error_json);
/* Average device time of one kernel of the decode step, launched `launches`
 * times back to back on the session stream (GEMVs cycle through the layers
 * so weights stream from HBM). kernel: "qkv", "attention", "o_proj",
 * "gate_up", "down" or "lm_head". */
yuear_status yuear_session_time_kernel(yuear_session *session,
                                       const char *kernel, int32_t launches,
                                       double *ms_per_launch, char **error_json);

/* ---- op-level entry points (model_ops, ar.hpp:8-19), device pointers,
 * `stream` is a hipStream_t (NULL = default stream). Scratch memory (the
 * batched GEMV's staging rows, the decode attention's split partials and
 * arrival counters, the split-K GEMM's partials) is per (device, stream):
 * calls on different streams never share it. The first call on a stream (or
 * one needing a larger buffer) allocates, so make it outside graph capture;
 * yuear_op_gemm and yuear_op_gemm_tile use no scratch. The first SwiGLU
 * GEMM (residual 2) on a device fills a 128 KiB silu table (one launch and a
 * stream synchronisation): make it outside graph capture too, where it
 * returns hipErrorStreamCaptureUnsupported. ---- */
/* y[b][r] = bf16(x[b] . W[row(r)]) with optional RMSNorm prologue
 * (norm_w != NULL) and epilogue 0 store / 1 residual add / 2 SwiGLU pairs. */
int32_t yuear_op_gemv(const uint16_t *dev_w, int32_t n, int32_t k,
                      int32_t batch, const uint16_t *dev_x, int32_t x_stride,
                      const uint16_t *dev_norm_w, float eps, uint16_t *dev_y,
                      int32_t y_stride, int32_t epilogue, void *stream);
/* Fused decode attention of one layer (see yuear_session_begin layout):
 * qkv [batch][(Hq+2Hkv)*128], caches [batch][Hkv] x cap slots (cap a
 * multiple of 32; K row-major [cap][128], V in 32-slot blocks stored
 * dim-major, element (t, d) at (t/32)*4096 + d*32 + t%32), pos [batch],
 * rope tables [positions][64] with a row for every position a branch is
 * at (pos < capacity; a branch whose pos is outside [0, capacity) is left
 * untouched), out [batch][Hq*128]; null q/k norm gains skip the RMSNorm. */
int32_t yuear_op_attention_decode(
    const uint16_t *dev_qkv, const uint16_t *dev_q_norm,
    const uint16_t *dev_k_norm, float eps, const uint16_t *dev_rope_cos,
    const uint16_t *dev_rope_sin, uint16_t *dev_k_cache, uint16_t *dev_v_cache,
    const int32_t *dev_pos, int32_t heads, int32_t kv_heads, int32_t capacity,
    int32_t batch, int32_t max_splits, uint16_t *dev_out, void *stream);
/* yuear_op_attention_decode without any allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * split partials and arrival counters live in a fixed 4 MiB device array per
 * GPU (YUEAR_NOALLOC_SCRATCH_BYTES), held until the process ends; a call
 * whose layout needs more -- 128 KiB of counters plus
 * batch * kv_heads * max_splits * (heads / kv_heads) * 130 floats -- returns
 * hipErrorOutOfMemory (2) and launches nothing. The first call on a device
 * looks up the array's address and clears its counters on `stream`. Calls
 * on one GPU share the array: calls that overlap in time on one GPU race.
 * Same arguments, kernels and results as yuear_op_attention_decode. */
#define YUEAR_NOALLOC_SCRATCH_BYTES (4 << 20)
int32_t yuear_op_attention_decode_noalloc(
    const uint16_t *dev_qkv, const uint16_t *dev_q_norm,
    const uint16_t *dev_k_norm, float eps, const uint16_t *dev_rope_cos,
    const uint16_t *dev_rope_sin, uint16_t *dev_k_cache, uint16_t *dev_v_cache,
    const int32_t *dev_pos, int32_t heads, int32_t kv_heads, int32_t capacity,
    int32_t batch, int32_t max_splits, uint16_t *dev_out, void *stream);
/* Affine group-64 quantized form of yuear_op_gemv for batch 1-2
 * (mx::quantized_matmul, ar.cpp:22-24): codes [n][k * bits / 32] uint32,
 * groups [n][k / 64] uint32 words scale | bias << 16 (bf16 halves). */
int32_t yuear_op_qgemv(const uint32_t *dev_codes, const uint32_t *dev_groups, int32_t bits,
                       int32_t n, int32_t k, int32_t batch, const uint16_t *dev_x,
                       int32_t x_stride, const uint16_t *dev_norm_w, float eps,
                       uint16_t *dev_y, int32_t y_stride, int32_t epilogue, void *stream);
/* out [n][k] = bf16(s q + b) of quantized rows (layout of yuear_op_qgemv). */
int32_t yuear_op_dequantize(const uint32_t *dev_codes, const uint32_t *dev_groups,
                            int32_t bits, int32_t n, int32_t k, uint16_t *dev_out,
                            void *stream);
/* C[m][n] = bf16(A[m] . W[n]) (residual 0), C = bf16(C + bf16(A[m] . W[n]))
 * (residual 1), or, on interleaved gate/up rows W[2i] / W[2i+1], the SwiGLU
 * pairs C[m][i] = bf16(bf16(silu(g)) * u), g / u = bf16(A[m] . W[2i] / [2i+1])
 * (residual 2, n even, C [m][n / 2]) -- the prefill projections, mx::matmul
 * and the mlp of ar.cpp:36-51, 258-298 -- with fp32 accumulation on MFMA.
 * k a multiple of 64, lda a multiple of 8, lda >= k, ldc >= n (n / 2 for
 * SwiGLU); otherwise hipErrorInvalidValue (1) and nothing is launched. */
int32_t yuear_op_gemm(const uint16_t *dev_a, int32_t lda, const uint16_t *dev_w,
                      int32_t m, int32_t n, int32_t k, uint16_t *dev_c,
                      int32_t ldc, int32_t residual, void *stream);
/* Test hook (no counterpart in the reference): yuear_op_gemm with its tile
 * shape forced instead of chosen, shape 0..5 = 256x256, 256x128, 128x256,
 * 256x192, 128x128, 192x192; other values return hipErrorInvalidValue (1). */
int32_t yuear_op_gemm_tile(const uint16_t *dev_a, int32_t lda, const uint16_t *dev_w,
                           int32_t m, int32_t n, int32_t k, uint16_t *dev_c,
                           int32_t ldc, int32_t residual, int32_t shape, void *stream);
/* Test hook (no counterpart in the reference): yuear_op_gemm_tile with K
 * split over `splits` workgroups per tile (1..16; k / 64 a multiple of
 * splits), each summing its K range into fp32 partials (splits * m * n
 * floats, in a per-(device, stream) buffer that the first such call on a
 * stream allocates, so make it outside graph capture) that a second kernel
 * adds in split order before the epilogue: the form the engine's prefill
 * GEMMs take where a time model of tile shape and split count picks it
 * (short prompts; the down projection up to ~2048 tokens at the 3B shape). */
int32_t yuear_op_gemm_split(const uint16_t *dev_a, int32_t lda, const uint16_t *dev_w,
                            int32_t m, int32_t n, int32_t k, uint16_t *dev_c,
                            int32_t ldc, int32_t residual, int32_t shape,
                            int32_t splits, void *stream);
/* Causal fp32-opmath attention for T queries at positions pos0 + t over one
 * branch's caches ([Hkv] x cap slots, the layout of
 * yuear_op_attention_decode). */
int32_t yuear_op_attention_prefill(const uint16_t *dev_q,
                                   const uint16_t *dev_k_cache,
                                   const uint16_t *dev_v_cache, int32_t tokens,
                                   int32_t pos0, int32_t heads,
                                   int32_t kv_heads, int32_t capacity,
                                   uint16_t *dev_out, void *stream);
/* Acoustic-model attention: the drop-in for nar_attention(query, key, value,
 * causal, query_chunk_size) (nar_attention.cpp:224-270) and its Metal kernel
 * lyra_nar_precise_attention (nar_attention.cpp:63-218). q [batch][heads]
 * [q_len][head_dim], k / v [batch][kv_heads][kv_len][head_dim], out like q,
 * all bf16; query head h reads kv head h / (heads / kv_heads). fp32 scores
 * times scale * log2(e), exp2 softmax, fp32 P.V, bf16(o / l); causal hides
 * the keys after each query (q_len == kv_len). query_chunk_size is validated
 * as in the reference and does not change the result (every query sees the
 * same keys in one pass). The reference runs its Metal kernel only for
 * non-causal calls with q_len > 8 and query_chunk_size >= 64; its other
 * calls go to MLX's sdpa (bf16 operands for chunks of <= 8 queries, fp32
 * otherwise, nar_attention.cpp:245-268). This entry point computes those
 * with the same precise kernel too: their parity with the reference is
 * unpinned. workspace: yuear_nar_attention_workspace_bytes()
 * of device memory. A non-causal launch too small to fill the GPU splits
 * its keys over workgroups; the split partials come from a library pool
 * per (device, stream). So the first such call on a stream, or one that
 * needs a larger pool, allocates: make it outside graph capture. Runs on
 * `stream` (a hipStream_t, NULL = default); the reference's ValueError
 * messages for invalid shapes. */
int64_t yuear_nar_attention_workspace_bytes(int32_t batch, int32_t kv_heads, int32_t kv_len);
/* The acoustic stage's conditioning prefill (CachedNAR, nar.cpp:139-190):
 * the AR layers over `tokens` with causal attention (the engine's prefill;
 * nar.cpp:80-99 keeps ar.cpp's RoPE and rounding points), then each layer's
 * keys and values of positions [0, visible), visible = visible_end ?
 * min(visible_end, n) : n, written to device memory dev_k / dev_v
 * [layers][kv_heads][visible][head_dim] bf16 (per layer the [1, heads,
 * tokens, dim] tensors yuear_nar_attention takes). *visible_out receives
 * visible. Errors as nar.cpp:142-154 (ValueError); engines with quantized
 * linears cannot condition (nar.cpp:303-307). */
yuear_status yuear_nar_condition(yuear_engine *engine, const int32_t *tokens, int32_t n,
                                 int32_t visible_end, uint16_t *dev_k, uint16_t *dev_v,
                                 int32_t *visible_out, char **error_json);
yuear_status yuear_nar_attention(const uint16_t *dev_q, const uint16_t *dev_k,
                                 const uint16_t *dev_v, int32_t batch, int32_t heads,
                                 int32_t kv_heads, int32_t q_len, int32_t kv_len,
                                 int32_t head_dim, int32_t causal, int32_t query_chunk_size,
                                 void *dev_workspace, uint16_t *dev_out, void *stream,
                                 char **error_json);
/* RoPE cos/sin tables exactly as the engine builds them (host). */
void yuear_rope_table(int32_t positions, int32_t head_dim, double theta,
                      uint16_t *cos_out, uint16_t *sin_out);

/* ---- text side of a request (host only): the prompt prefixes the decode
 * loop is given (protocol.hpp:5-24, protocol.mm:123-357, 428-591) ---- */
typedef struct yuear_tokenizer yuear_tokenizer;
/* lyra::Tokenizer(vocabulary) (protocol.mm:438-485): a checkpoint-native
 * qwen.tiktoken, one "base64-piece rank" line per ordinary token, exactly
 * 151643 of them (ranks [0, 151643)); the special and <extra_i> pieces
 * follow. Errors: FileNotFoundError / PermissionError / OSError, ValueError
 * with the reference's messages. */
yuear_status yuear_tokenizer_load(const char *vocabulary, yuear_tokenizer **out,
                                  char **error_json);
void yuear_tokenizer_destroy(yuear_tokenizer *tokenizer);
/* Tokenizer::encode (protocol.mm:558-579): `len` bytes of UTF-8 (NUL bytes
 * allowed) -> NFC -> the reference's pre-tokenizer pattern -> byte pair
 * merges. *ids is allocated by the library (free with yuear_ids_free), *n
 * its length. Invalid UTF-8: UnicodeDecodeError "Invalid UTF-8 text". */
yuear_status yuear_tokenizer_encode(const yuear_tokenizer *tokenizer, const char *text,
                                    int64_t len, int32_t **ids, int64_t *n, char **error_json);
/* Tokenizer::decode (protocol.mm:580-591): ids outside the text vocabulary
 * are skipped, invalid UTF-8 becomes U+FFFD per maximal subpart. *text is
 * NUL-terminated (free with yuear_string_free), *len its byte length
 * (len may be NULL). */
yuear_status yuear_tokenizer_decode(const yuear_tokenizer *tokenizer, const int32_t *ids,
                                    int64_t n, char **text, int64_t *len, char **error_json);
void yuear_ids_free(int32_t *ids);
/* Test hooks (no counterpart in the reference) for the two stages inside
 * encode: the NFC form of UTF-8 text (as yuear_tokenizer_decode returns
 * text), and the pre-tokenizer's pieces of that NFC text as the byte offset
 * where each ends (as yuear_tokenizer_encode returns ids). */
yuear_status yuear_text_nfc(const char *text, int64_t len, char **out, int64_t *out_len,
                            char **error_json);
yuear_status yuear_text_pieces(const char *text, int64_t len, int32_t **ends, int64_t *n,
                               char **error_json);
/* The SongRequest fields the prompt layout reads (protocol.hpp SongRequest):
 * NUL-terminated UTF-8; abc NULL when absent; has_cfg_scale 0 when absent. */
typedef struct yuear_song_request {
  const char *style, *lyrics, *cot, *abc, *id;
  uint64_t seed;
  double cfg_scale;
  int32_t has_cfg_scale;
} yuear_song_request;
/* SongRequest::validate (protocol.mm:212-237), same ValueError messages. */
yuear_status yuear_song_request_validate(const yuear_song_request *request, char **error_json);
/* SongRequest::guidance (protocol.mm:238-240): cfg_scale, else 1.01 for
 * cot "off" and 1 otherwise (1 for a NULL request). */
double yuear_song_request_guidance(const yuear_song_request *request);
/* token_prefixes(request, tokenizer, abc_ids) (protocol.mm:321-340):
 * [EOD] + encode(text) + [ABC_START], then for cot "off" [ABC_END,
 * MUSIC_START]; otherwise, when abc_ids are given (has_abc_ids) or the
 * request carries abc text, the ABC ids + [ABC_END, MUSIC_START]. Output as
 * yuear_tokenizer_encode. */
yuear_status yuear_token_prefixes(const yuear_tokenizer *tokenizer,
                                  const yuear_song_request *request, const int32_t *abc_ids,
                                  int64_t n_abc, int32_t has_abc_ids, int32_t **ids, int64_t *n,
                                  char **error_json);
/* negative_prefix(request, tokenizer, abc_ids) (protocol.mm:341-357): the
 * unconditional CFG branch, [EOD] + encode(instruction) + the same tail
 * (cot "off": [MUSIC_START]; otherwise abc_ids are required). */
yuear_status yuear_negative_prefix(const yuear_tokenizer *tokenizer,
                                   const yuear_song_request *request, const int32_t *abc_ids,
                                   int64_t n_abc, int32_t has_abc_ids, int32_t **ids, int64_t *n,
                                   char **error_json);
/* chunk_ranges(frames, prefix_tokens, context) (protocol.mm:358-369): the
 * acoustic stage's frame chunks [a, b) of min((context - prefix - 3) / 2,
 * 24576) frames each; *bounds receives n pairs (a, b) as 2 n ints (free
 * with yuear_ids_free). ValueError "Empty codec or prefix leaves no
 * acoustic context" when frames < 1 or context - prefix - 3 < 2. */
yuear_status yuear_chunk_ranges(int32_t frames, int32_t prefix_tokens, int32_t context,
                                int32_t **bounds, int64_t *n, char **error_json);

#ifdef __cplusplus
}
#endif
#endif /* YUEAR_H */
