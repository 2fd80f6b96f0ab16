// Host runtime of the gfx950 AR decode library: weights, sessions, hipGraph
// decode step, the device-side generate loop and the C ABI of include/yuear.h.
//
// Reference behaviour mirrored here:
//   native/src/ar.cpp:133-238        model construction and tensor validation
//   native/src/ar.cpp:98-132         fixed-capacity KV cache, overflow errors
//   native/src/sampling.cpp:139-288  request validation, prefill, decode loop,
//                                    EOS handling, timing keys
//   native/src/protocol.mm:123-134   Sampling::validate
//   native/src/bridge.mm:108-159     error JSON, status codes, no exceptions
//                                    across the ABI
//   vendor/yue/src/yue2/cuda_graph.py:43-240  device-side positions, one
//                                    graph replay per decode step
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/yuear.h"
#include "abi_util.h"
#include "attn_core.h"
#include "common.h"
#include "kernels.h"

namespace yuear {
namespace {

// ---------------------------------------------------------------------------
// deterministic weight generator (host): Philox4x32-10 -> Box-Muller (double)
// -> mean + std * z -> fp32 -> bf16 RNE. Element i uses block i/4 of the
// counter stream (ctr = {block lo, block hi, tensor id, 'WEIG'}).
void random_tensor(uint64_t seed, int32_t id, float mean, float sd, int64_t n, uint16_t *out) {
  const int64_t blocks = (n + 3) / 4;
  unsigned workers = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
  if (n < (1 << 16))
    workers = 1;
  const int64_t per = (blocks + workers - 1) / workers;
  auto work = [&](int64_t b0, int64_t b1) {
    for (int64_t blk = b0; blk < b1; ++blk) {
      const Philox4 r = philox4x32_10(uint32_t(blk), uint32_t(uint64_t(blk) >> 32), uint32_t(id),
                                      0x57454947u, uint32_t(seed), uint32_t(seed >> 32));
      double z[4];
      for (int h = 0; h < 2; ++h) {
        const double u1 = (double(r.v[2 * h]) + 1.0) * 2.3283064365386963e-10;  // (0,1]
        const double u2 = double(r.v[2 * h + 1]) * 2.3283064365386963e-10;      // [0,1)
        const double rad = std::sqrt(-2.0 * std::log(u1));
        const double ang = 6.283185307179586 * u2;
        z[2 * h] = rad * std::cos(ang);
        z[2 * h + 1] = rad * std::sin(ang);
      }
      for (int e = 0; e < 4; ++e) {
        const int64_t i = blk * 4 + e;
        if (i < n)
          out[i] = f2bf(float(double(mean) + double(sd) * z[e]));
      }
    }
  };
  if (workers == 1) {
    work(0, blocks);
    return;
  }
  std::vector<std::thread> pool;
  for (unsigned w = 0; w < workers; ++w) {
    const int64_t b0 = std::min(blocks, int64_t(w) * per), b1 = std::min(blocks, b0 + per);
    if (b0 < b1)
      pool.emplace_back(work, b0, b1);
  }
  for (auto &t : pool)
    t.join();
}

// Tensor ids of the generator: 0 embed, 1 final norm, 2 lm_head,
// 16 + 16 i + j for layer i with j in kLayerNames order.
const char *const kLayerNames[] = {"input_layernorm",  "post_attention_layernorm",
                                   "self_attn.q_norm", "self_attn.k_norm",
                                   "self_attn.q_proj", "self_attn.k_proj",
                                   "self_attn.v_proj", "self_attn.o_proj",
                                   "mlp.gate_proj",    "mlp.up_proj",
                                   "mlp.down_proj"};
constexpr int kNumLayerTensors = 11;
// Split-K workspace of a session's prefill GEMMs (fp32 partials, splits x
// tokens x features): the largest split the plan picks at the 3B shape is
// the down projection at 1024 tokens, 4 x 1024 x 3072 floats (48 MiB); a
// split that does not fit is not considered.
constexpr size_t kSplitBytes = size_t(64) << 20;

int32_t tensor_id(const std::string &name) {
  if (name == "model.embed_tokens.weight") return 0;
  if (name == "model.norm.weight") return 1;
  if (name == "lm_head.weight") return 2;
  const std::string pre = "model.layers.", suf = ".weight";
  if (name.rfind(pre, 0) != 0 || name.size() <= pre.size() + suf.size() ||
      name.compare(name.size() - suf.size(), suf.size(), suf) != 0)
    return -1;
  const size_t dot = name.find('.', pre.size());
  if (dot == std::string::npos) return -1;
  const std::string idx = name.substr(pre.size(), dot - pre.size());
  if (idx.empty() || idx.size() > 6 || idx.find_first_not_of("0123456789") != std::string::npos)
    return -1;
  const std::string rest = name.substr(dot + 1, name.size() - suf.size() - dot - 1);
  for (int j = 0; j < kNumLayerTensors; ++j)
    if (rest == kLayerNames[j])
      return 16 + 16 * std::stoi(idx) + j;
  return -1;
}

// RoPE tables, ar.cpp:62-74 (fp32 inverse frequencies and angles, bf16
// cos/sin), built on the host with the C library's single-precision math.
void rope_table(int positions, int d, double theta, uint16_t *c, uint16_t *s) {
  const int half = d / 2;
  std::vector<float> inv(half);
  for (int j = 0; j < half; ++j)
    inv[j] = 1.0f / std::pow(float(theta), float(2 * j) / float(d));
  for (int p = 0; p < positions; ++p)
    for (int j = 0; j < half; ++j) {
      const float a = float(p) * inv[j];
      c[size_t(p) * half + j] = f2bf(std::cos(a));
      s[size_t(p) * half + j] = f2bf(std::sin(a));
    }
}

// ---------------------------------------------------------------------------
struct Config {
  int H, F, layers, Hq, Hkv, D, V, max_pos;
  float eps;
  double theta;
  bool qk_norm;
  int qkv() const { return (Hq + 2 * Hkv) * D; }
};

Config validate_config(const yuear_model_config *c) {
  if (!c)
    invalid("config is required");
  Config k{c->hidden_size, c->intermediate_size, c->num_hidden_layers, c->num_attention_heads,
           c->num_key_value_heads, c->head_dim, c->vocab_size, c->max_position_embeddings,
           c->rms_norm_eps, c->rope_theta, c->qk_norm != 0};
  if (k.H < 1 || k.F < 1 || k.layers < 1 || k.Hq < 1 || k.Hkv < 1 || k.D < 1 || k.V < 1 ||
      k.max_pos < 1)
    invalid("Generator config fields must be positive integers");
  if (k.Hq % k.Hkv)
    invalid("num_attention_heads must be divisible by num_key_value_heads");
  if (!(std::isfinite(k.eps) && k.eps > 0))
    invalid("rms_norm_eps must be finite and positive");
  if (!(std::isfinite(k.theta) && k.theta > 0))
    invalid("rope_theta must be finite and positive");
  if (k.D != 128)
    invalid("the gfx950 kernels implement head_dim 128");
  if (k.H % 64 || k.F % 64 || k.H > 8192 || k.F > 8192 || k.Hq * k.D > 8192)
    invalid("hidden/intermediate sizes must be multiples of 64 and at most 8192");
  const int g = k.Hq / k.Hkv;
  if (g != 1 && g != 2 && g != 3 && g != 4 && g != 6 && g != 8)
    invalid("query heads per kv head must be 1, 2, 3, 4, 6 or 8");
  return k;
}

size_t align_elems(size_t n) { return (n + 127) & ~size_t(127); }  // 256 B

struct LayerW {
  uint16_t *input_ln, *post_ln, *q_norm, *k_norm, *qkv, *o, *gu, *down;
  // quantized linears: codes and group words (scale | bias << 16) of the
  // same rows; qkv / o / gu / down then hold their dequantized rows
  const uint32_t *qqkv = nullptr, *gqkv = nullptr, *qo = nullptr, *go = nullptr;
  const uint32_t *qgu = nullptr, *ggu = nullptr, *qdown = nullptr, *gdown = nullptr;
  // MFMA-tiled copies of the projections for batched decode (launch_tile_rows)
  uint16_t *qkv_t = nullptr, *o_t = nullptr, *gu_t = nullptr, *down_t = nullptr;
};

struct PhaseInfo {
  int kind, size, end, seg0_start, seg0_len, seg1_start;
  int stride() const { return (size + 7) & ~7; }  // logits row stride (16-byte rows)
};
PhaseInfo phase_info(const std::string &name, int vocab) {
  if (name == "full")
    return {kPhaseFull, vocab, -1, 0, vocab, 0};
  if (name == "abc") {
    if (vocab <= kAbcEnd)
      invalid("AR vocabulary does not contain the ABC end row");
    return {kPhaseAbc, kEOD + 1, kEOD, 0, kEOD, kAbcEnd};
  }
  if (name == "semantic") {
    if (vocab < kCodecOffset + kCodecSize)
      invalid("AR vocabulary does not contain all semantic rows");
    return {kPhaseSemantic, kCodecSize + 1, 0, kMusicEnd, kCodecSize + 1, 0};
  }
  invalid("phase must be 'full', 'abc' or 'semantic'");
}

int native_to_local(int token, const PhaseInfo &ph, int vocab) {
  switch (ph.kind) {
  case kPhaseAbc:
    if (token >= 0 && token < kEOD) return token;
    return token == kAbcEnd ? kEOD : -1;
  case kPhaseSemantic:
    if (token == kMusicEnd) return 0;
    if (token >= kCodecOffset && token < kCodecOffset + kCodecSize) return token - kMusicEnd;
    return -1;
  }
  return token >= 0 && token < vocab ? token : -1;
}

// protocol.mm:123-134
void validate_sampling(const yuear_sampling &s) {
  if (!std::isfinite(s.temperature) || !std::isfinite(s.top_p) ||
      !std::isfinite(s.repetition_penalty))
    invalid("Sampling numbers must be finite");
  if (!(s.temperature >= 0 && s.temperature <= 5 && s.top_p > 0 && s.top_p <= 1 && s.top_k >= 1))
    invalid("Invalid sampling temperature/top_p/top_k");
  if (s.repetition_penalty <= 0 || s.penalty_window < 1 || s.penalty_window > 100)
    invalid("Invalid repetition penalty/window");
  if (s.min_tokens < 0 || s.min_tokens > s.max_tokens || s.max_tokens < 1)
    invalid("Require 0 <= min_tokens <= max_tokens");
}

}  // namespace
}  // namespace yuear

using namespace yuear;

struct yuear_engine {
  Config cfg{};
  int device = 0;
  uint16_t *weights = nullptr;
  size_t weight_bytes = 0;
  uint16_t *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
  std::vector<LayerW> layers;
  uint16_t *rope_cos = nullptr, *rope_sin = nullptr;
  int bits = 0;                  // 0: bf16 linears; 8 / 4: affine group-64 quantized
  uint32_t *qweights = nullptr;  // codes and group words of every quantized linear
  const uint32_t *lm_q = nullptr, *lm_g = nullptr;
  // MFMA-tiled projection copies, built by the first session of 3+ branches
  // (6.15 GB more at the 3B shape: HBM is plentiful, the batched GEMVs read
  // 1 KiB contiguous per wave-load from them)
  uint16_t *tiled = nullptr, *lm_head_t = nullptr;
  std::mutex tiled_mu;
  std::atomic<bool> cancelled{false};
  std::mutex busy;

  ~yuear_engine() {
    if (weights) (void)hipFree(weights);
    if (qweights) (void)hipFree(qweights);
    if (rope_cos) (void)hipFree(rope_cos);
    if (tiled) (void)hipFree(tiled);
  }
  // Throws InterruptedError(message) when yuear_engine_cancel was called or
  // the caller's poll (sampling.cpp:135-137 cancelled_at) says so.
  void cancelled_at(const char *message, yuear_cancel_poll poll = nullptr,
                    void *user = nullptr) {
    if (cancelled.load(std::memory_order_relaxed) || (poll && poll(user) != 0))
      throw Error("InterruptedError", message);
  }
};

struct yuear_session {
  yuear_engine *e = nullptr;
  int B = 1, cap = 0, max_splits = 1;
  int kv_stride = 0;  // slots per (layer, branch, kv head): cap rounded up to a V block
  PhaseInfo phase{};
  hipStream_t stream = nullptr;
  // device state
  // [layers][B][Hkv] x kv_stride slots; K row-major, V in 32-slot dim-major
  // blocks (attn::v_index)
  uint16_t *kc = nullptr, *vc = nullptr;
  int32_t *pos = nullptr, *tok = nullptr;
  uint16_t *x = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
  uint16_t *stage = nullptr;  // [B][H] prepared (gathered / normalised) rows, batched GEMVs
  float *part_o = nullptr, *part_ml = nullptr;
  int32_t *counters = nullptr;
  float *scratch = nullptr, *alphas = nullptr;
  uint32_t *scratch_u = nullptr;
  int32_t *sstate = nullptr, *history = nullptr;
  int32_t *sampler_sync = nullptr;  // split sampler arrival counter, zero between launches
  int history_cap = 0;       // history entries per branch set
  int scratch_u_stride = 0;
  // prefill scratch
  int chunk = 0;
  uint16_t *px = nullptr, *ph = nullptr, *pqkv = nullptr, *pq = nullptr, *pattn = nullptr,
           *pact = nullptr;
  float *psplit = nullptr;  // split-K partials of the prefill GEMMs (kSplitBytes)
  // a split residual GEMM's reduce and the following RMSNorm in one kernel
  // (YUEAR_PREFILL_FUSE_NORM=0: two kernels, the same results)
  bool fuse_norm = true;
  int32_t *pids = nullptr;
  // host mirrors / pinned
  std::vector<int> host_pos;
  int32_t *pin_tok = nullptr;
  uint16_t *pin_logits = nullptr;
  std::vector<void *> allocations;
  hipGraphExec_t step_exec = nullptr;
  hipGraph_t step_graph = nullptr;
  hipGraphExec_t gen_exec = nullptr;  // sampler + step, for timed loops
  hipGraph_t gen_graph = nullptr;
  std::string gen_key;

  ~yuear_session() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (step_exec) (void)hipGraphExecDestroy(step_exec);
    if (step_graph) (void)hipGraphDestroy(step_graph);
    if (gen_exec) (void)hipGraphExecDestroy(gen_exec);
    if (gen_graph) (void)hipGraphDestroy(gen_graph);
    for (void *p : allocations) (void)hipFree(p);
    if (pin_tok) (void)hipHostFree(pin_tok);
    if (pin_logits) (void)hipHostFree(pin_logits);
    if (stream) (void)hipStreamDestroy(stream);
  }
  template <class T> T *alloc(size_t n) {
    void *p = nullptr;
    HIPC(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    allocations.push_back(p);
    return static_cast<T *>(p);
  }
  size_t layer_kv_offset(int layer, int branch) const {
    const Config &c = e->cfg;
    return (size_t(layer) * B + branch) * c.Hkv * size_t(kv_stride) * c.D;
  }
};

namespace yuear {
namespace {

// ---------------------------------------------------------------------------
// engine construction
void build_engine(yuear_engine &E, const yuear_weight_source *src) {
  const Config &c = E.cfg;
  HIPC(hipGetDevice(&E.device));
  if (!src)
    invalid("a weight source is required");
  const int bits = src->bits;
  if (bits != 0 && bits != 8 && bits != 4)
    invalid("weight bits must be 0 (bf16), 8 or 4");
  if (bits && !(qgemv_supported(bits, c.H, 1) && qgemv_supported(bits, c.Hq * c.D, 1) &&
                qgemv_supported(bits, c.F, 1)))
    invalid("quantized linears need input widths that the quantized GEMV implements");
  E.bits = bits;
  auto layer_name = [](int i, int j) {
    return "model.layers." + std::to_string(i) + "." + kLayerNames[j] + ".weight";
  };
  auto base_of = [](const std::string &weight) { return weight.substr(0, weight.size() - 7); };
  const size_t Hs = c.H, Fs = c.F, Vs = c.V, QD = size_t(c.Hq) * c.D, KD = size_t(c.Hkv) * c.D;
  // device layout: bf16 tensors (with quantized linears, their dequantized
  // rows, read by prefill and the batched GEMVs)
  size_t total = align_elems(Vs * Hs) * 2 + align_elems(Hs);
  const size_t per_layer = align_elems(Hs) * 2 + align_elems(c.D) * 2 +
                           align_elems((QD + 2 * KD) * Hs) + align_elems(Hs * QD) +
                           align_elems(2 * Fs * Hs) + align_elems(Hs * Fs);
  total += per_layer * c.layers;
  E.weight_bytes = total * 2;
  HIPC(hipMalloc(&E.weights, E.weight_bytes));
  uint16_t *cur = E.weights;
  auto take = [&](size_t n) {
    uint16_t *p = cur;
    cur += align_elems(n);
    return p;
  };
  E.embed = take(Vs * Hs);
  E.lm_head = take(Vs * Hs);
  E.final_norm = take(Hs);
  E.layers.resize(c.layers);
  for (auto &L : E.layers) {
    L.input_ln = take(Hs);
    L.post_ln = take(Hs);
    L.q_norm = take(c.D);
    L.k_norm = take(c.D);
    L.qkv = take((QD + 2 * KD) * Hs);
    L.o = take(Hs * QD);
    L.gu = take(2 * Fs * Hs);
    L.down = take(Hs * Fs);
  }
  // quantized linears: codes [rows][k * bits / 32] and group words [rows][k / 64]
  auto qwords = [&](size_t rows, size_t k) {
    return align_elems(rows * k * bits / 32) + align_elems(rows * k / 64);
  };
  if (bits) {
    size_t words = qwords(Vs, Hs);
    words += c.layers * (qwords(QD + 2 * KD, Hs) + qwords(Hs, QD) + qwords(2 * Fs, Hs) +
                         qwords(Hs, Fs));
    HIPC(hipMalloc(&E.qweights, words * 4));
    E.weight_bytes += words * 4;
    uint32_t *qc = E.qweights;
    auto qtake = [&](size_t rows, size_t k, const uint32_t *&codes, const uint32_t *&groups) {
      codes = qc;
      qc += align_elems(rows * k * bits / 32);
      groups = qc;
      qc += align_elems(rows * k / 64);
    };
    qtake(Vs, Hs, E.lm_q, E.lm_g);
    for (auto &L : E.layers) {
      qtake(QD + 2 * KD, Hs, L.qqkv, L.gqkv);
      qtake(Hs, QD, L.qo, L.go);
      qtake(2 * Fs, Hs, L.qgu, L.ggu);
      qtake(Hs, Fs, L.qdown, L.gdown);
    }
  }

  // expected tensors (ar.cpp:209-233)
  struct Spec {
    size_t numel;
    int dtype;
  };
  std::map<std::string, Spec> expected;
  auto linear = [&](const std::string &weight, size_t rows, size_t k) {
    if (!bits) {
      expected[weight] = {rows * k, YUEAR_DTYPE_BF16};
      return;
    }
    expected[weight] = {rows * k * bits / 32, YUEAR_DTYPE_U32};
    expected[base_of(weight) + ".scales"] = {rows * k / 64, YUEAR_DTYPE_BF16};
    expected[base_of(weight) + ".biases"] = {rows * k / 64, YUEAR_DTYPE_BF16};
  };
  expected["model.embed_tokens.weight"] = {Vs * Hs, YUEAR_DTYPE_BF16};
  expected["model.norm.weight"] = {Hs, YUEAR_DTYPE_BF16};
  linear("lm_head.weight", Vs, Hs);
  const size_t rows[kNumLayerTensors] = {Hs, Hs, size_t(c.D), size_t(c.D), QD, KD, KD, Hs, Fs, Fs,
                                         Hs};
  const size_t cols[kNumLayerTensors] = {1, 1, 1, 1, Hs, Hs, Hs, QD, Hs, Hs, Fs};
  for (int i = 0; i < c.layers; ++i)
    for (int j = 0; j < kNumLayerTensors; ++j) {
      if (j < 4)
        expected[layer_name(i, j)] = {rows[j], YUEAR_DTYPE_BF16};
      else
        linear(layer_name(i, j), rows[j], cols[j]);
    }

  std::map<std::string, const void *> host;
  if (src->kind == YUEAR_WEIGHTS_HOST) {
    if (!src->tensors || src->count < 0)
      invalid("host weight source needs a tensor table");
    for (int t = 0; t < src->count; ++t) {
      const yuear_tensor &tt = src->tensors[t];
      if (!tt.name || !tt.data)
        invalid("tensor entries need a name and data");
      auto it = expected.find(tt.name);
      if (it == expected.end())
        invalid(std::string("Unexpected AR tensor: ") + tt.name);
      if (size_t(tt.numel) != it->second.numel || tt.dtype != it->second.dtype)
        invalid(std::string("Incompatible AR tensor shape/dtype: ") + tt.name);
      if (!host.emplace(tt.name, tt.data).second)
        invalid(std::string("Duplicate AR tensor: ") + tt.name);
    }
    for (auto &kv : expected)
      if (!host.count(kv.first))
        invalid("Missing AR tensor: " + kv.first);
  } else if (src->kind != YUEAR_WEIGHTS_RANDOM) {
    invalid("unknown weight source kind");
  }

  // one bf16 tensor as host bytes (borrowed, or generated into `buf`; the
  // generator makes the bf16 values of a linear's `.weight` either way)
  std::vector<uint16_t> tmp, tmp2;
  auto fetch = [&](const std::string &name, size_t n,
                   std::vector<uint16_t> &buf) -> const uint16_t * {
    if (src->kind == YUEAR_WEIGHTS_HOST)
      return static_cast<const uint16_t *>(host.at(name));
    buf.resize(n);
    const bool gain = name.find("norm") != std::string::npos;
    random_tensor(src->seed, tensor_id(name), gain ? 1.0f : 0.0f,
                  gain ? src->norm_std : src->std, int64_t(n), buf.data());
    return buf.data();
  };
  auto upload = [&](void *dst, const void *h, size_t bytes) {
    HIPC(hipMemcpy(dst, h, bytes, hipMemcpyHostToDevice));
  };
  auto upload_bf16 = [&](uint16_t *dst, const std::string &name, size_t n) {
    upload(dst, fetch(name, n, tmp), n * 2);
  };
  upload_bf16(E.embed, "model.embed_tokens.weight", Vs * Hs);
  upload_bf16(E.final_norm, "model.norm.weight", Hs);

  // A projection of `rows` x `k` built from parts: part p's source rows go
  // to destination rows row0 + r * step (fused q|k|v rows; gate/up
  // interleaved by row, 2r = gate_r, 2r + 1 = up_r, cuda_graph.py:100-108).
  struct Part {
    std::string weight;
    size_t rows, row0, step;
  };
  std::vector<uint16_t> stage16;
  std::vector<uint32_t> qstage, gstage, qgen;
  std::vector<uint16_t> sgen, bgen;
  auto put_linear = [&](const std::vector<Part> &parts, size_t total_rows, size_t k,
                        uint16_t *dst, const uint32_t *dcodes, const uint32_t *dgroups) {
    if (!bits) {
      if (parts.size() == 1) {
        upload(dst, fetch(parts[0].weight, total_rows * k, tmp), total_rows * k * 2);
        return;
      }
      stage16.resize(total_rows * k);
      for (const Part &pt : parts) {
        const uint16_t *h = fetch(pt.weight, pt.rows * k, tmp);
        for (size_t r = 0; r < pt.rows; ++r)
          std::memcpy(&stage16[(pt.row0 + r * pt.step) * k], h + r * k, k * 2);
      }
      upload(dst, stage16.data(), stage16.size() * 2);
      return;
    }
    const size_t wpr = k * bits / 32, gpr = k / 64;
    qstage.resize(total_rows * wpr);
    gstage.resize(total_rows * gpr);
    for (const Part &pt : parts) {
      const uint32_t *codes;
      const uint16_t *scales, *biases;
      const std::string base = base_of(pt.weight);
      if (src->kind == YUEAR_WEIGHTS_HOST) {
        codes = static_cast<const uint32_t *>(host.at(pt.weight));
        scales = static_cast<const uint16_t *>(host.at(base + ".scales"));
        biases = static_cast<const uint16_t *>(host.at(base + ".biases"));
      } else {
        const uint16_t *w = fetch(pt.weight, pt.rows * k, tmp);
        qgen.resize(pt.rows * wpr);
        sgen.resize(pt.rows * gpr);
        bgen.resize(pt.rows * gpr);
        quantize_affine(w, int64_t(pt.rows), int(k), bits, qgen.data(), sgen.data(), bgen.data());
        codes = qgen.data();
        scales = sgen.data();
        biases = bgen.data();
      }
      for (size_t r = 0; r < pt.rows; ++r) {
        const size_t d = pt.row0 + r * pt.step;
        std::memcpy(&qstage[d * wpr], codes + r * wpr, wpr * 4);
        for (size_t g = 0; g < gpr; ++g)
          gstage[d * gpr + g] =
              uint32_t(scales[r * gpr + g]) | (uint32_t(biases[r * gpr + g]) << 16);
      }
    }
    upload(const_cast<uint32_t *>(dcodes), qstage.data(), qstage.size() * 4);
    upload(const_cast<uint32_t *>(dgroups), gstage.data(), gstage.size() * 4);
    HIPC(launch_dequantize(dcodes, dgroups, bits, int(total_rows), int(k), dst, nullptr));
    HIPC(hipDeviceSynchronize());  // the staging buffers are reused
  };
  put_linear({{"lm_head.weight", Vs, 0, 1}}, Vs, Hs, E.lm_head, E.lm_q, E.lm_g);
  for (int i = 0; i < c.layers; ++i) {
    LayerW &L = E.layers[i];
    upload_bf16(L.input_ln, layer_name(i, 0), Hs);
    upload_bf16(L.post_ln, layer_name(i, 1), Hs);
    upload_bf16(L.q_norm, layer_name(i, 2), c.D);
    upload_bf16(L.k_norm, layer_name(i, 3), c.D);
    put_linear({{layer_name(i, 4), QD, 0, 1},
                {layer_name(i, 5), KD, QD, 1},
                {layer_name(i, 6), KD, QD + KD, 1}},
               QD + 2 * KD, Hs, L.qkv, L.qqkv, L.gqkv);
    put_linear({{layer_name(i, 7), Hs, 0, 1}}, Hs, QD, L.o, L.qo, L.go);
    put_linear({{layer_name(i, 8), Fs, 0, 2}, {layer_name(i, 9), Fs, 1, 2}}, 2 * Fs, Hs, L.gu,
               L.qgu, L.ggu);
    put_linear({{layer_name(i, 10), Hs, 0, 1}}, Hs, Fs, L.down, L.qdown, L.gdown);
  }
  // RoPE tables for every position the model admits
  const int positions = std::min(c.max_pos, kContext);
  std::vector<uint16_t> cs(size_t(positions) * c.D / 2), sn(cs.size());
  rope_table(positions, c.D, c.theta, cs.data(), sn.data());
  HIPC(hipMalloc(&E.rope_cos, cs.size() * 4));
  E.rope_sin = E.rope_cos + cs.size();
  upload(E.rope_cos, cs.data(), cs.size() * 2);
  upload(E.rope_sin, sn.data(), sn.size() * 2);
}

// MFMA-tiled copies of every projection and the lm_head, for the batched
// (3..8 sequence) GEMVs; only for the K values that form has instances.
bool mfma_shapes(const Config &c) {
  auto ok = [](int k) { return k == 2048 || k == 3072 || k == 6144 || k == 8192; };
  return ok(c.H) && ok(c.Hq * c.D) && ok(c.F);
}
void build_tiled(yuear_engine &E, hipStream_t st) {
  std::lock_guard<std::mutex> lock(E.tiled_mu);
  const Config &c = E.cfg;
  if (E.tiled || !mfma_shapes(c))
    return;
  auto tiled_elems = [](size_t n, size_t k) { return align_elems((n + 15) / 16 * 16 * k); };
  const size_t H = c.H, F = c.F, QD = size_t(c.Hq) * c.D, KD = size_t(c.Hkv) * c.D;
  const size_t per_layer = tiled_elems(QD + 2 * KD, H) + tiled_elems(H, QD) +
                           tiled_elems(2 * F, H) + tiled_elems(H, F);
  const size_t total = per_layer * c.layers + tiled_elems(c.V, H);
  uint16_t *base = nullptr;
  HIPC(hipMalloc(&base, total * 2));
  uint16_t *cur = base;
  auto tile = [&](const uint16_t *w, size_t n, size_t k) {
    uint16_t *out = cur;
    cur += tiled_elems(n, k);
    HIPC(launch_tile_rows(w, int(n), int(k), out, st));
    return out;
  };
  for (auto &L : E.layers) {
    L.qkv_t = tile(L.qkv, QD + 2 * KD, H);
    L.o_t = tile(L.o, H, QD);
    L.gu_t = tile(L.gu, 2 * F, H);
    L.down_t = tile(L.down, H, F);
  }
  E.lm_head_t = tile(E.lm_head, c.V, H);
  HIPC(hipStreamSynchronize(st));
  E.tiled = base;
}

// ---------------------------------------------------------------------------
// session
void begin_session(yuear_session &S, yuear_engine *E, int branches, int capacity,
                   const std::string &phase) {
  const Config &c = E->cfg;
  if (branches < 1 || branches > 8)
    invalid("branches must be in [1, 8]");
  const int limit = std::min(kContext, c.max_pos);
  if (capacity < 1 || capacity > limit)
    invalid("KV cache capacity must be in [1, " + std::to_string(limit) + "]");
  S.e = E;
  S.B = branches;
  S.cap = capacity;
  S.kv_stride = (capacity + attn::kBlock - 1) / attn::kBlock * attn::kBlock;
  S.phase = phase_info(phase, c.V);
  HIPC(hipSetDevice(E->device));
  HIPC(hipStreamCreateWithFlags(&S.stream, hipStreamNonBlocking));
  if (branches >= 3)
    build_tiled(*E, S.stream);
  const size_t kv = size_t(c.layers) * branches * c.Hkv * size_t(S.kv_stride) * c.D;
  S.kc = S.alloc<uint16_t>(kv);
  S.vc = S.alloc<uint16_t>(kv);
  // zero-filled like mx::zeros (ar.cpp:113-118); done once at allocation
  HIPC(hipMemsetAsync(S.kc, 0, kv * 2, S.stream));
  HIPC(hipMemsetAsync(S.vc, 0, kv * 2, S.stream));
  S.pos = S.alloc<int32_t>(branches);
  S.tok = S.alloc<int32_t>(branches);
  HIPC(hipMemsetAsync(S.pos, 0, branches * 4, S.stream));
  HIPC(hipMemsetAsync(S.tok, 0, branches * 4, S.stream));
  S.x = S.alloc<uint16_t>(size_t(branches) * c.H);
  S.stage = S.alloc<uint16_t>(size_t(branches) * c.H);
  S.qkv = S.alloc<uint16_t>(size_t(branches) * c.qkv());
  S.attn = S.alloc<uint16_t>(size_t(branches) * c.Hq * c.D);
  S.act = S.alloc<uint16_t>(size_t(branches) * c.F);
  S.logits = S.alloc<uint16_t>(size_t(branches) * S.phase.stride());
  // split-K: one 128-key pass per workgroup at the session's capacity, at
  // most one workgroup per CU for one sequence and ~512 workgroups for more
  // branches (attn_decode_splits); YUEAR_ATTN_SPLITS overrides.
  {
    int splits = attn_decode_splits(branches, c.Hkv, S.kv_stride);
    if (const char *env = std::getenv("YUEAR_ATTN_SPLITS"))
      splits = std::atoi(env);
    if (const char *env = std::getenv("YUEAR_PREFILL_FUSE_NORM"))
      S.fuse_norm = std::atoi(env) != 0;
    S.max_splits = std::max(1, std::min({64, splits, S.kv_stride / attn::kBlock}));
  }
  const int G = c.Hq / c.Hkv;
  S.part_o = S.alloc<float>(size_t(branches) * c.Hkv * S.max_splits * G * c.D);
  S.part_ml = S.alloc<float>(size_t(branches) * c.Hkv * S.max_splits * G * 2);
  S.counters = S.alloc<int32_t>(size_t(branches) * c.Hkv * kCounterStride);
  HIPC(hipMemsetAsync(S.counters, 0, size_t(branches) * c.Hkv * kCounterStride * 4, S.stream));
  int pow2 = 1;
  while (pow2 < S.phase.size) pow2 <<= 1;
  // sampler buffers: one set per branch when more than two branches sample
  // independently (batched sequences), one shared set otherwise
  const int sets = branches > 2 ? branches : 1;
  S.scratch_u_stride = S.phase.size + 2 * pow2;
  S.scratch = S.alloc<float>(size_t(S.phase.size) * sets);
  S.scratch_u = S.alloc<uint32_t>(size_t(S.scratch_u_stride) * sets);
  S.alphas = S.alloc<float>(128);
  S.sampler_sync = S.alloc<int32_t>(1);
  HIPC(hipMemsetAsync(S.sampler_sync, 0, sizeof(int32_t), S.stream));
  S.sstate = S.alloc<int32_t>(2 * sets);
  S.history_cap = kContext;
  S.history = S.alloc<int32_t>(size_t(S.history_cap) * sets);
  // prefill in chunks of up to 4096 tokens (~210 MB of scratch at the 3B
  // shape, plus the GEMMs' split-K partials): larger GEMMs fill the GPU
  // better (M = 3000: 590 TFLOP/s against ~400 at M = 1024). A chunked
  // prefill equals the one-pass prefill bit for bit when their GEMMs take the
  // same tile shape and split count (shapes are chosen per M)
  S.chunk = std::min(capacity, 4096);
  const size_t T = S.chunk;
  S.px = S.alloc<uint16_t>(T * c.H);
  S.ph = S.alloc<uint16_t>(T * c.H);
  S.pqkv = S.alloc<uint16_t>(T * c.qkv());
  S.pq = S.alloc<uint16_t>(T * c.Hq * c.D);
  S.pattn = S.alloc<uint16_t>(T * c.Hq * c.D);
  S.pact = S.alloc<uint16_t>(T * c.F);
  S.psplit = S.alloc<float>(kSplitBytes / 4);
  S.pids = S.alloc<int32_t>(T);
  S.host_pos.assign(branches, 0);
  HIPC(hipHostMalloc(reinterpret_cast<void **>(&S.pin_tok), size_t(kContext + 16) * 4));
  HIPC(hipHostMalloc(reinterpret_cast<void **>(&S.pin_logits),
                     size_t(branches) * S.phase.stride() * 2));
  HIPC(hipStreamSynchronize(S.stream));
}

void set_device_pos(yuear_session &S) {
  for (int b = 0; b < S.B; ++b)
    S.pin_tok[b] = S.host_pos[b];
  HIPC(hipMemcpyAsync(S.pos, S.pin_tok, S.B * 4, hipMemcpyHostToDevice, S.stream));
  HIPC(hipStreamSynchronize(S.stream));
}

// Quantized codes of a projection: the 1-2 branch GEMVs read them instead
// of the dequantized rows in `w`.
void set_quant(GemvParams &g, int bits, const uint32_t *codes, const uint32_t *groups) {
  if (bits && codes) {
    g.bits = bits;
    g.qw = codes;
    g.qsb = groups;
  }
}

// decode kernels of one layer on S.x (all branches)
void enqueue_ffn(yuear_session &S, int l);

void enqueue_layer(yuear_session &S, int l, bool embed_first) {
  yuear_engine &E = *S.e;
  const Config &c = E.cfg;
  const LayerW &L = E.layers[l];
  hipStream_t st = S.stream;
  GemvParams q;
  q.w = L.qkv;
  set_quant(q, E.bits, L.qqkv, L.gqkv);
  q.n = c.qkv();
  q.k = c.H;
  q.batch = S.B;
  q.x = S.x;
  q.x_stride = c.H;
  if (embed_first) {
    q.embed = E.embed;
    q.tokens = S.tok;
    q.embed_rows = c.V;
    q.x_out = S.x;
  }
  q.norm_w = L.input_ln;
  q.eps = c.eps;
  q.stage = S.stage;
  q.w_tiled = L.qkv_t;
  q.y = S.qkv;
  q.y_stride = c.qkv();
  HIPC(launch_gemv(q, st));

  AttnDecodeParams a;
  a.qkv = S.qkv;
  a.qkv_stride = c.qkv();
  a.q_norm = c.qk_norm ? L.q_norm : nullptr;
  a.k_norm = c.qk_norm ? L.k_norm : nullptr;
  a.eps = c.eps;
  a.rope_cos = E.rope_cos;
  a.rope_sin = E.rope_sin;
  a.k_cache = S.kc + S.layer_kv_offset(l, 0);
  a.v_cache = S.vc + S.layer_kv_offset(l, 0);
  a.pos = S.pos;
  a.heads = c.Hq;
  a.kv_heads = c.Hkv;
  a.head_dim = c.D;
  a.capacity = S.kv_stride;
  a.batch = S.B;
  a.max_splits = S.max_splits;
  a.part_o = S.part_o;
  a.part_ml = S.part_ml;
  a.counters = S.counters;
  a.out = S.attn;
  a.out_stride = c.Hq * c.D;
  HIPC(launch_attn_decode(a, st));

  GemvParams o;
  o.w = L.o;
  set_quant(o, E.bits, L.qo, L.go);
  o.n = c.H;
  o.k = c.Hq * c.D;
  o.batch = S.B;
  o.x = S.attn;
  o.x_stride = c.Hq * c.D;
  o.y = S.x;
  o.y_stride = c.H;
  o.epilogue = kEpiResidual;
  o.w_tiled = L.o_t;
  HIPC(launch_gemv(o, st));

  enqueue_ffn(S, l);
}

// post-attention RMSNorm + gate/up + SwiGLU, down + residual (ar.cpp:295-298)
void enqueue_ffn(yuear_session &S, int l) {
  yuear_engine &E = *S.e;
  const Config &c = E.cfg;
  const LayerW &L = E.layers[l];
  hipStream_t st = S.stream;
  GemvParams g;
  g.w = L.gu;
  set_quant(g, E.bits, L.qgu, L.ggu);
  g.n = 2 * c.F;
  g.k = c.H;
  g.batch = S.B;
  g.x = S.x;
  g.x_stride = c.H;
  g.norm_w = L.post_ln;
  g.eps = c.eps;
  g.stage = S.stage;
  g.w_tiled = L.gu_t;
  g.y = S.act;
  g.y_stride = c.F;
  g.epilogue = kEpiSwiGLU;
  HIPC(launch_gemv(g, st));

  GemvParams d;
  d.w = L.down;
  set_quant(d, E.bits, L.qdown, L.gdown);
  d.n = c.H;
  d.k = c.F;
  d.batch = S.B;
  d.x = S.act;
  d.x_stride = c.F;
  d.y = S.x;
  d.y_stride = c.H;
  d.epilogue = kEpiResidual;
  d.w_tiled = L.down_t;
  HIPC(launch_gemv(d, st));
}

void enqueue_one(yuear_session &S, const std::string &which, int l);

void enqueue_head(yuear_session &S, const uint16_t *x, int batch, int x_stride, uint16_t *out,
                  int32_t *advance) {
  yuear_engine &E = *S.e;
  const Config &c = E.cfg;
  GemvParams h;
  h.w = E.lm_head;
  set_quant(h, E.bits, E.lm_q, E.lm_g);
  h.n = S.phase.size;
  h.k = c.H;
  h.batch = batch;
  h.x = x;
  h.x_stride = x_stride;
  h.norm_w = E.final_norm;
  h.eps = c.eps;
  h.stage = batch <= S.B ? S.stage : nullptr;
  h.w_tiled = E.lm_head_t;
  h.y = out;
  h.y_stride = S.phase.stride();
  h.seg0_start = S.phase.seg0_start;
  h.seg0_len = S.phase.seg0_len;
  h.seg1_start = S.phase.seg1_start;
  h.advance = advance;
  HIPC(launch_gemv(h, S.stream));
}

// One kernel of the decode step for layer l (timing only; same parameters
// as in enqueue_layer / enqueue_head).
void enqueue_one(yuear_session &S, const std::string &which, int l) {
  yuear_engine &E = *S.e;
  const Config &c = E.cfg;
  const LayerW &L = E.layers[l];
  GemvParams g;
  g.batch = S.B;
  g.eps = c.eps;
  if (which == "qkv") {
    g.w = L.qkv; g.n = c.qkv(); g.k = c.H; g.x = S.x; g.x_stride = c.H;
    set_quant(g, E.bits, L.qqkv, L.gqkv);
    g.norm_w = L.input_ln; g.y = S.qkv; g.y_stride = c.qkv(); g.stage = S.stage;
    g.w_tiled = L.qkv_t;
  } else if (which == "o_proj") {
    g.w = L.o; g.n = c.H; g.k = c.Hq * c.D; g.x = S.attn; g.x_stride = c.Hq * c.D;
    set_quant(g, E.bits, L.qo, L.go);
    g.y = S.x; g.y_stride = c.H; g.epilogue = kEpiResidual; g.w_tiled = L.o_t;
  } else if (which == "gate_up") {
    g.w = L.gu; g.n = 2 * c.F; g.k = c.H; g.x = S.x; g.x_stride = c.H;
    set_quant(g, E.bits, L.qgu, L.ggu);
    g.norm_w = L.post_ln; g.y = S.act; g.y_stride = c.F; g.epilogue = kEpiSwiGLU;
    g.stage = S.stage; g.w_tiled = L.gu_t;
  } else if (which == "down") {
    g.w = L.down; g.n = c.H; g.k = c.F; g.x = S.act; g.x_stride = c.F;
    set_quant(g, E.bits, L.qdown, L.gdown);
    g.y = S.x; g.y_stride = c.H; g.epilogue = kEpiResidual; g.w_tiled = L.down_t;
  } else if (which == "lm_head") {
    enqueue_head(S, S.x, S.B, c.H, S.logits, nullptr);
    return;
  } else if (which == "attention") {
    AttnDecodeParams a;
    a.qkv = S.qkv; a.qkv_stride = c.qkv();
    a.q_norm = c.qk_norm ? L.q_norm : nullptr; a.k_norm = c.qk_norm ? L.k_norm : nullptr;
    a.eps = c.eps; a.rope_cos = E.rope_cos; a.rope_sin = E.rope_sin;
    a.k_cache = S.kc + S.layer_kv_offset(l, 0); a.v_cache = S.vc + S.layer_kv_offset(l, 0);
    a.pos = S.pos; a.heads = c.Hq; a.kv_heads = c.Hkv; a.head_dim = c.D; a.capacity = S.kv_stride;
    a.batch = S.B; a.max_splits = S.max_splits; a.part_o = S.part_o; a.part_ml = S.part_ml;
    a.counters = S.counters; a.out = S.attn; a.out_stride = c.Hq * c.D;
    HIPC(launch_attn_decode(a, S.stream));
    return;
  } else {
    invalid("unknown kernel name: " + which);
  }
  HIPC(launch_gemv(g, S.stream));
}

// whole decode step: tok -> logits, pos += 1
void enqueue_step(yuear_session &S) {
  for (int l = 0; l < S.e->cfg.layers; ++l)
    enqueue_layer(S, l, l == 0);
  enqueue_head(S, S.x, S.B, S.e->cfg.H, S.logits, S.pos);
}

void ensure_step_graph(yuear_session &S) {
  if (S.step_exec)
    return;
  HIPC(hipStreamBeginCapture(S.stream, hipStreamCaptureModeThreadLocal));
  try {
    enqueue_step(S);
  } catch (...) {
    hipGraph_t g;
    (void)hipStreamEndCapture(S.stream, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  HIPC(hipStreamEndCapture(S.stream, &S.step_graph));
  HIPC(hipGraphInstantiate(&S.step_exec, S.step_graph, nullptr, nullptr, 0));
}

void drop_graphs(yuear_session &S) {
  HIPC(hipStreamSynchronize(S.stream));
  if (S.step_exec) (void)hipGraphExecDestroy(S.step_exec);
  if (S.step_graph) (void)hipGraphDestroy(S.step_graph);
  if (S.gen_exec) (void)hipGraphExecDestroy(S.gen_exec);
  if (S.gen_graph) (void)hipGraphDestroy(S.gen_graph);
  S.step_exec = nullptr;
  S.step_graph = nullptr;
  S.gen_exec = nullptr;
  S.gen_graph = nullptr;
  S.gen_key.clear();
}

void check_tokens(const int32_t *ids, int n, int vocab) {  // sampling.cpp:139-146
  if (!ids || n < 1)
    invalid("AR prefix must contain at least one token");
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= vocab)
      invalid("Token IDs must be in [0, " + std::to_string(vocab) + ")");
}

// prefill of one branch (sampling.cpp:152-183; ar.cpp:246-301 with T > 1).
// Cancellation is polled before any work and between chunks (each chunk ends
// in a stream synchronisation, so a poll falls between two chunks' work).
void prefill(yuear_session &S, int b, const int32_t *ids, int n, uint16_t *logits_out,
             yuear_cancel_poll poll = nullptr, void *poll_user = nullptr) {
  yuear_engine &E = *S.e;
  const Config &c = E.cfg;
  if (b < 0 || b >= S.B)
    invalid("branch out of range");
  check_tokens(ids, n, c.V);
  if (S.host_pos[b] + n > S.cap)
    invalid("KV cache capacity exceeded; generation was not shortened");
  E.cancelled_at("Cancelled before prefill", poll, poll_user);  // sampling.cpp:156
  hipStream_t st = S.stream;
  for (int start = 0; start < n; start += S.chunk) {
    E.cancelled_at("Cancelled during prefill", poll, poll_user);  // sampling.cpp:164
    const int T = std::min(S.chunk, n - start);
    const int pos0 = S.host_pos[b];
    std::memcpy(S.pin_tok, ids + start, size_t(T) * 4);
    HIPC(hipMemcpyAsync(S.pids, S.pin_tok, size_t(T) * 4, hipMemcpyHostToDevice, st));
    HIPC(launch_embed_rows(E.embed, S.pids, T, c.H, S.px, st));
    // a residual projection into x, then (norm_w set) the RMSNorm of the
    // updated rows into h: a split GEMM's reduce and the norm run as one
    // kernel (bit-identical to the reduce kernel followed by the norm)
    auto residual_then_norm = [&](GemmParams g, const uint16_t *norm_w) -> hipError_t {
      int shape = 0, splits = 1;
      gemm_plan(g.m, g.n, g.k, gemm_cus(), g.part_bytes, &shape, &splits);
      const bool fuse = norm_w && splits > 1 && S.fuse_norm;
      g.defer_reduce = fuse;
      hipError_t e = launch_gemm_tile(g, shape, st, splits);
      if (e != hipSuccess || !norm_w)
        return e;
      return fuse ? launch_gemm_reduce_norm(g, splits, norm_w, c.eps, S.ph, st)
                  : launch_rms_norm_rows(S.px, T, c.H, norm_w, c.eps, S.ph, st);
    };
    HIPC(launch_rms_norm_rows(S.px, T, c.H, E.layers[0].input_ln, c.eps, S.ph, st));
    for (int l = 0; l < c.layers; ++l) {
      const LayerW &L = E.layers[l];
      GemmParams g{S.ph, c.H, L.qkv, T, c.qkv(), c.H, S.pqkv, c.qkv(), 0, S.psplit, kSplitBytes};
      HIPC(launch_gemm(g, st));
      QkPrepParams qp;
      qp.qkv = S.pqkv;
      qp.qkv_stride = c.qkv();
      qp.tokens = T;
      qp.q_norm = c.qk_norm ? L.q_norm : nullptr;
      qp.k_norm = c.qk_norm ? L.k_norm : nullptr;
      qp.eps = c.eps;
      qp.rope_cos = E.rope_cos;
      qp.rope_sin = E.rope_sin;
      qp.pos0 = pos0;
      qp.heads = c.Hq;
      qp.kv_heads = c.Hkv;
      qp.head_dim = c.D;
      qp.capacity = S.kv_stride;
      qp.q_out = S.pq;
      qp.k_cache = S.kc + S.layer_kv_offset(l, b);
      qp.v_cache = S.vc + S.layer_kv_offset(l, b);
      HIPC(launch_qk_prep(qp, st));
      AttnPrefillParams ap;
      ap.q = S.pq;
      ap.k_cache = qp.k_cache;
      ap.v_cache = qp.v_cache;
      ap.tokens = T;
      ap.pos0 = pos0;
      ap.heads = c.Hq;
      ap.kv_heads = c.Hkv;
      ap.head_dim = c.D;
      ap.capacity = S.kv_stride;
      ap.out = S.pattn;
      HIPC(launch_attn_prefill(ap, st));
      GemmParams og{S.pattn, c.Hq * c.D, L.o, T, c.H, c.Hq * c.D, S.px, c.H, 1, S.psplit,
                    kSplitBytes};
      HIPC(residual_then_norm(og, L.post_ln));
      GemmParams gu{S.ph, c.H, L.gu, T, 2 * c.F, c.H, S.pact, c.F, 2, S.psplit,
                    kSplitBytes};  // SwiGLU epilogue
      HIPC(launch_gemm(gu, st));
      // down + residual, then the next layer's input norm (the last layer's
      // rows go to the final norm of the head)
      GemmParams dg{S.pact, c.F, L.down, T, c.H, c.F, S.px, c.H, 1, S.psplit, kSplitBytes};
      HIPC(residual_then_norm(dg, l + 1 < c.layers ? E.layers[l + 1].input_ln : nullptr));
    }
    S.host_pos[b] += T;
    if (start + T >= n)  // final norm + projection of the last hidden row
      enqueue_head(S, S.px + size_t(T - 1) * c.H, 1, c.H,
                   S.logits + size_t(b) * S.phase.stride(), nullptr);
    HIPC(hipStreamSynchronize(st));
  }
  set_device_pos(S);
  if (logits_out) {
    HIPC(hipMemcpyAsync(S.pin_logits, S.logits + size_t(b) * S.phase.stride(),
                        size_t(S.phase.size) * 2, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    std::memcpy(logits_out, S.pin_logits, size_t(S.phase.size) * 2);
  }
}

void step(yuear_session &S, const int32_t *tokens, uint16_t *logits_out) {
  const Config &c = S.e->cfg;
  if (!tokens)
    invalid("step needs one token per branch");
  for (int b = 0; b < S.B; ++b) {
    if (tokens[b] < 0 || tokens[b] >= c.V)
      invalid("Token is outside the model vocabulary");
    if (S.host_pos[b] + 1 > S.cap)
      invalid("Requested generation budget is exhausted");
  }
  ensure_step_graph(S);
  std::memcpy(S.pin_tok, tokens, size_t(S.B) * 4);
  HIPC(hipMemcpyAsync(S.tok, S.pin_tok, size_t(S.B) * 4, hipMemcpyHostToDevice, S.stream));
  HIPC(hipGraphLaunch(S.step_exec, S.stream));
  for (int b = 0; b < S.B; ++b)
    S.host_pos[b] += 1;
  if (logits_out) {
    const size_t ls = S.phase.stride(), n = S.phase.size;
    HIPC(hipMemcpyAsync(S.pin_logits, S.logits, size_t(S.B) * ls * 2, hipMemcpyDeviceToHost,
                        S.stream));
    HIPC(hipStreamSynchronize(S.stream));
    for (int b = 0; b < S.B; ++b)
      std::memcpy(logits_out + b * n, S.pin_logits + b * ls, n * 2);
  } else {
    HIPC(hipStreamSynchronize(S.stream));
  }
}

SamplerParams sampler_params(yuear_session &S, const yuear_sampling &s, uint64_t seed,
                             double cfg_scale, int legacy_off, int hist_len) {
  SamplerParams p;
  p.logits = S.logits;
  p.n = S.phase.size;
  p.ls = S.phase.stride();
  p.branches = S.B;
  p.cfg_scale = float(cfg_scale);
  p.temperature = float(s.temperature);
  p.top_p = float(s.top_p);
  p.top_k = s.top_k;
  p.min_tokens = s.min_tokens;
  p.penalty_window = s.penalty_window;
  p.alphas = s.repetition_penalty != 1.0 ? S.alphas : nullptr;
  p.phase = S.phase.kind;
  p.vocab = S.e->cfg.V;
  p.seed = seed;
  p.legacy_off = legacy_off;
  p.state = S.sstate;
  p.history = S.history;
  p.hist_len = hist_len;
  p.max_tokens = S.history_cap;
  p.tokens_out = S.tok;
  p.scratch = S.scratch;
  p.scratch_u = S.scratch_u;
  p.sync = S.sampler_sync;  // the shared-draw case may spread over workgroups
  if (S.B > 2) {  // batched sequences: each branch is its own request
    p.independent = 1;
    p.history_stride = S.history_cap;
    p.scratch_stride = S.phase.size;
    p.scratch_u_stride = S.scratch_u_stride;
  }
  return p;
}

void upload_alphas(yuear_session &S, const yuear_sampling &s) {
  // alpha[count] = pow(f32 penalty, f32 count) (sampling.cpp:67-70), as a
  // table indexed by the window count (vendor fast.py:123-136 lookup form)
  std::vector<float> a(128, 1.0f);
  for (int cnt = 0; cnt <= s.penalty_window && cnt < 128; ++cnt)
    a[cnt] = std::pow(float(s.repetition_penalty), float(cnt));
  HIPC(hipMemcpyAsync(S.alphas, a.data(), a.size() * 4, hipMemcpyHostToDevice, S.stream));
  HIPC(hipStreamSynchronize(S.stream));
}

void check_sampler_phase(yuear_session &S, double cfg_scale) {
  if (cfg_scale != 1.0 && S.B != 2)
    invalid("CFG needs a session with exactly two branches");
}

}  // namespace
}  // namespace yuear

// ===========================================================================
// C ABI
namespace {
// Scratch of the op-level entry points, one buffer per (device, stream):
// calls on one stream are ordered and may share it, calls on different
// streams or devices never do. Grown on demand (the stream is synchronised
// before the smaller buffer is freed), kept until the process ends.
// Scratch of the op-level entry points, one buffer per (device, stream). A
// buffer handed out is never freed: a launch still in flight, or a graph
// captured on that stream, may hold its address. A request larger than the
// current buffer retires it (kept until the process ends) and allocates
// max(request, 2 x current) rounded to a power of two, so a growing caller
// retires O(log size) buffers and never synchronises. Growth while the
// stream is being captured is refused (hipErrorStreamCaptureUnsupported):
// make the largest call once before capturing.
struct OpPool {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> bufs;
  std::vector<void *> retired;
  hipError_t get(hipStream_t s, size_t bytes, void **out, bool *fresh) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
      return e;
    std::lock_guard<std::mutex> lock(mu);
    auto &b = bufs[{dev, s}];
    *fresh = false;
    if (bytes > b.second) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if ((e = hipStreamIsCapturing(s, &cs)) != hipSuccess)
        return e;
      if (cs != hipStreamCaptureStatusNone)
        return hipErrorStreamCaptureUnsupported;
      size_t size = 256;
      while (size < std::max(bytes, 2 * b.second))
        size <<= 1;
      void *p = nullptr;
      if ((e = hipMalloc(&p, size)) != hipSuccess)
        return e;
      if (b.first)
        retired.push_back(b.first);
      b = {p, size};
      *fresh = true;
    }
    *out = b.first;
    return hipSuccess;
  }
};
}  // namespace

extern "C" {

const char *yuear_build_identifier(void) {
  return "yuear-gfx950 0.1";
}

void yuear_string_free(char *s) { std::free(s); }

int32_t yuear_tensor_id(const char *name) { return name ? tensor_id(name) : -1; }

void yuear_random_tensor(uint64_t seed, int32_t id, float mean, float sd, int64_t n,
                         uint16_t *out) {
  if (out && n > 0)
    random_tensor(seed, id, mean, sd, n, out);
}

void yuear_rope_table(int32_t positions, int32_t head_dim, double theta, uint16_t *c,
                      uint16_t *s) {
  if (positions > 0 && head_dim > 0 && c && s)
    rope_table(positions, head_dim, theta, c, s);
}

yuear_status yuear_engine_create(const yuear_model_config *config,
                                 const yuear_weight_source *weights, yuear_engine **out,
                                 char **error_json) {
  if (out)
    *out = nullptr;
  return guarded(error_json, [&] {
    if (!out)
      invalid("output pointer is required");
    auto E = std::make_unique<yuear_engine>();
    E->cfg = validate_config(config);
    build_engine(*E, weights);
    *out = E.release();
  });
}

void yuear_engine_destroy(yuear_engine *engine) { delete engine; }

int32_t yuear_engine_bits(const yuear_engine *engine) { return engine ? engine->bits : -1; }

void yuear_quantize_affine(const uint16_t *w, int64_t rows, int32_t k, int32_t bits,
                           uint32_t *codes, uint16_t *scales, uint16_t *biases) {
  if (!w || !codes || !scales || !biases || rows < 0 || k <= 0 || k % 64 ||
      (bits != 4 && bits != 8))
    return;
  quantize_affine(w, rows, k, bits, codes, scales, biases);
}

void yuear_engine_cancel(yuear_engine *engine) {
  if (engine)
    engine->cancelled.store(true, std::memory_order_relaxed);
}

yuear_status yuear_session_begin(yuear_engine *engine, int32_t branches, int32_t capacity,
                                 const char *phase, yuear_session **out, char **error_json) {
  if (out)
    *out = nullptr;
  return guarded(error_json, [&] {
    if (!engine || !out)
      invalid("engine and output pointer are required");
    auto S = std::make_unique<yuear_session>();
    begin_session(*S, engine, branches, capacity, phase ? phase : "full");
    *out = S.release();
  });
}

void yuear_session_end(yuear_session *session) { delete session; }

yuear_status yuear_session_prefill(yuear_session *S, int32_t branch, const int32_t *ids,
                                   int32_t n, uint16_t *logits_out, char **error_json) {
  return guarded(error_json, [&] {
    if (!S)
      invalid("session is required");
    prefill(*S, branch, ids, n, logits_out);
  });
}

yuear_status yuear_session_step(yuear_session *S, const int32_t *tokens, uint16_t *logits_out,
                                char **error_json) {
  return guarded(error_json, [&] {
    if (!S)
      invalid("session is required");
    step(*S, tokens, logits_out);
  });
}

yuear_status yuear_session_sample(yuear_session *S, const yuear_sampling *sampling,
                                  uint64_t seed, double cfg_scale, int32_t legacy_off,
                                  int32_t step_index, const int32_t *history,
                                  int32_t history_len, int32_t *token_out, char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !sampling || !token_out)
      invalid("session, sampling and output are required");
    validate_sampling(*sampling);
    check_sampler_phase(*S, cfg_scale);
    if (S->B > 2)
      invalid("sessions of more than two branches sample each branch independently "
              "(yuear_session_time_generate); sample one token per request session");
    if (seed >= (uint64_t(1) << 63))
      invalid("seed must be an integer in [0, 2**63)");
    if (history_len < 0 || history_len > S->history_cap || (history_len && !history))
      invalid("invalid history");
    upload_alphas(*S, *sampling);
    if (history_len) {
      std::memcpy(S->pin_tok, history, size_t(history_len) * 4);
      HIPC(hipMemcpyAsync(S->history, S->pin_tok, size_t(history_len) * 4,
                          hipMemcpyHostToDevice, S->stream));
      HIPC(hipStreamSynchronize(S->stream));
    }
    int32_t st[2] = {step_index, 0};
    HIPC(hipMemcpyAsync(S->sstate, st, 8, hipMemcpyHostToDevice, S->stream));
    SamplerParams p = sampler_params(*S, *sampling, seed, cfg_scale, legacy_off, history_len);
    p.max_tokens = 0;  // do not append to the uploaded history
    HIPC(launch_sampler(p, S->stream));
    HIPC(hipMemcpyAsync(S->pin_tok, S->tok, 4, hipMemcpyDeviceToHost, S->stream));
    HIPC(hipStreamSynchronize(S->stream));
    *token_out = S->pin_tok[0];
  });
}

int32_t yuear_session_position(const yuear_session *S, int32_t branch) {
  return S && branch >= 0 && branch < S->B ? S->host_pos[branch] : -1;
}

int32_t yuear_session_phase_size(const yuear_session *S) { return S ? S->phase.size : -1; }

yuear_status yuear_session_write_kv(yuear_session *S, int32_t layer, int32_t branch,
                                    const uint16_t *k, const uint16_t *v, int32_t n,
                                    char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !k || !v)
      invalid("session and data are required");
    const Config &c = S->e->cfg;
    if (layer < 0 || layer >= c.layers || branch < 0 || branch >= S->B || n < 0 || n > S->cap)
      invalid("layer/branch/length out of range");
    // V goes into the cache's block layout: whole blocks covering [0, n),
    // slots past n zero (invisible: the position becomes n)
    const int nb = (n + attn::kBlock - 1) / attn::kBlock * attn::kBlock;
    std::vector<uint16_t> vb(size_t(nb) * c.D);
    HIPC(hipStreamSynchronize(S->stream));
    for (int h = 0; h < c.Hkv; ++h) {
      const size_t off = S->layer_kv_offset(layer, branch) + size_t(h) * S->kv_stride * c.D;
      HIPC(hipMemcpy(S->kc + off, k + size_t(h) * n * c.D, size_t(n) * c.D * 2,
                     hipMemcpyHostToDevice));
      std::fill(vb.begin(), vb.end(), uint16_t(0));
      for (int t = 0; t < n; ++t)
        for (int d = 0; d < c.D; ++d)
          vb[attn::v_index(t, d)] = v[(size_t(h) * n + t) * c.D + d];
      HIPC(hipMemcpy(S->vc + off, vb.data(), vb.size() * 2, hipMemcpyHostToDevice));
    }
    S->host_pos[branch] = n;
    set_device_pos(*S);
  });
}

yuear_status yuear_session_read_kv(yuear_session *S, int32_t layer, int32_t branch, uint16_t *k,
                                   uint16_t *v, int32_t n, char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !k || !v)
      invalid("session and data are required");
    const Config &c = S->e->cfg;
    if (layer < 0 || layer >= c.layers || branch < 0 || branch >= S->B || n < 0 || n > S->cap)
      invalid("layer/branch/length out of range");
    HIPC(hipStreamSynchronize(S->stream));
    const int nb = (n + attn::kBlock - 1) / attn::kBlock * attn::kBlock;
    std::vector<uint16_t> vb(size_t(nb) * c.D);
    for (int h = 0; h < c.Hkv; ++h) {
      const size_t off = S->layer_kv_offset(layer, branch) + size_t(h) * S->kv_stride * c.D;
      HIPC(hipMemcpy(k + size_t(h) * n * c.D, S->kc + off, size_t(n) * c.D * 2,
                     hipMemcpyDeviceToHost));
      HIPC(hipMemcpy(vb.data(), S->vc + off, vb.size() * 2, hipMemcpyDeviceToHost));
      for (int t = 0; t < n; ++t)
        for (int d = 0; d < c.D; ++d)
          v[(size_t(h) * n + t) * c.D + d] = vb[attn::v_index(t, d)];
    }
  });
}

yuear_status yuear_session_write_logits(yuear_session *S, const uint16_t *logits,
                                        char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !logits)
      invalid("session and logits are required");
    HIPC(hipStreamSynchronize(S->stream));
    HIPC(hipMemcpy2D(S->logits, size_t(S->phase.stride()) * 2, logits, size_t(S->phase.size) * 2,
                     size_t(S->phase.size) * 2, S->B, hipMemcpyHostToDevice));
  });
}

yuear_status yuear_session_set_position(yuear_session *S, int32_t branch, int32_t position,
                                        char **error_json) {
  return guarded(error_json, [&] {
    if (!S || branch < 0 || branch >= S->B || position < 0 || position > S->cap)
      invalid("branch/position out of range");
    S->host_pos[branch] = position;
    set_device_pos(*S);
  });
}

yuear_status yuear_session_layer_step(yuear_session *S, int32_t layer, const uint16_t *x_in,
                                      uint16_t *x_out, char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !x_in || !x_out)
      invalid("session and data are required");
    const Config &c = S->e->cfg;
    if (layer < 0 || layer >= c.layers)
      invalid("layer out of range");
    for (int b = 0; b < S->B; ++b)
      if (S->host_pos[b] + 1 > S->cap)
        invalid("KV cache capacity exceeded; generation was not shortened");
    const size_t bytes = size_t(S->B) * c.H * 2;
    HIPC(hipMemcpy(S->x, x_in, bytes, hipMemcpyHostToDevice));
    enqueue_layer(*S, layer, false);
    HIPC(hipStreamSynchronize(S->stream));
    HIPC(hipMemcpy(x_out, S->x, bytes, hipMemcpyDeviceToHost));
    for (int b = 0; b < S->B; ++b)
      S->host_pos[b] += 1;
    set_device_pos(*S);
  });
}

yuear_status yuear_session_time_steps(yuear_session *S, int32_t steps, double *ms_per_step,
                                      char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !ms_per_step || steps < 1)
      invalid("session, steps >= 1 and output are required");
    for (int b = 0; b < S->B; ++b)
      if (S->host_pos[b] + steps > S->cap)
        invalid("KV cache capacity exceeded; generation was not shortened");
    ensure_step_graph(*S);
    hipEvent_t e0, e1;
    HIPC(hipEventCreate(&e0));
    HIPC(hipEventCreate(&e1));
    HIPC(hipEventRecord(e0, S->stream));
    for (int i = 0; i < steps; ++i)
      HIPC(hipGraphLaunch(S->step_exec, S->stream));
    HIPC(hipEventRecord(e1, S->stream));
    HIPC(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPC(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    for (int b = 0; b < S->B; ++b)
      S->host_pos[b] += steps;
    *ms_per_step = double(ms) / steps;
  });
}

yuear_status yuear_session_time_generate(yuear_session *S, const yuear_sampling *sampling,
                                         uint64_t seed, int32_t steps, int32_t reset,
                                         double *ms_per_step, int32_t *tokens_out,
                                         char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !sampling || !ms_per_step || steps < 1)
      invalid("session, sampling, steps >= 1 and output are required");
    validate_sampling(*sampling);
    for (int b = 0; b < S->B; ++b)
      if (S->host_pos[b] + steps > S->cap)
        invalid("KV cache capacity exceeded; generation was not shortened");
    const yuear_sampling &s = *sampling;
    char key[256];
    std::snprintf(key, sizeof key, "%a %a %d %a %d %d %llu", s.temperature, s.top_p, s.top_k,
                  s.repetition_penalty, s.penalty_window, s.min_tokens,
                  (unsigned long long)seed);
    if (S->gen_key != key) {
      if (S->gen_exec) (void)hipGraphExecDestroy(S->gen_exec);
      if (S->gen_graph) (void)hipGraphDestroy(S->gen_graph);
      S->gen_exec = nullptr;
      S->gen_graph = nullptr;
      S->gen_key.clear();
      upload_alphas(*S, s);
      SamplerParams sp = sampler_params(*S, s, seed, 1.0, 0, -1);
      HIPC(hipStreamBeginCapture(S->stream, hipStreamCaptureModeThreadLocal));
      try {
        HIPC(launch_sampler(sp, S->stream));
        enqueue_step(*S);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(S->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HIPC(hipStreamEndCapture(S->stream, &S->gen_graph));
      HIPC(hipGraphInstantiate(&S->gen_exec, S->gen_graph, nullptr, nullptr, 0));
      S->gen_key = key;
      reset = 1;
    }
    const int sets = S->B > 2 ? S->B : 1;
    std::vector<int32_t> st(2 * sets, 0);
    if (!reset)
      HIPC(hipMemcpy(st.data(), S->sstate, st.size() * 4, hipMemcpyDeviceToHost));
    else
      HIPC(hipMemcpy(S->sstate, st.data(), st.size() * 4, hipMemcpyHostToDevice));
    const int32_t st0[2] = {st[0], st[1]};
    const int first = st0[0];
    if (first + steps > S->history_cap)
      invalid("generation history exceeds the context");
    hipEvent_t e0, e1;
    HIPC(hipEventCreate(&e0));
    HIPC(hipEventCreate(&e1));
    HIPC(hipEventRecord(e0, S->stream));
    for (int i = 0; i < steps; ++i)
      HIPC(hipGraphLaunch(S->gen_exec, S->stream));
    HIPC(hipEventRecord(e1, S->stream));
    HIPC(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPC(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    for (int b = 0; b < S->B; ++b)
      S->host_pos[b] += steps;
    *ms_per_step = double(ms) / steps;
    if (tokens_out)
      HIPC(hipMemcpy(tokens_out, S->history + first, size_t(steps) * 4, hipMemcpyDeviceToHost));
  });
}

yuear_status yuear_session_time_kernel(yuear_session *S, const char *kernel, int32_t launches,
                                       double *ms_per_launch, char **error_json) {
  return guarded(error_json, [&] {
    if (!S || !kernel || !ms_per_launch || launches < 1)
      invalid("session, kernel, launches >= 1 and output are required");
    const std::string which = kernel;
    for (int b = 0; b < S->B; ++b)
      if (which == "attention" && S->host_pos[b] >= S->cap)
        invalid("attention timing needs a free slot");
    enqueue_one(*S, which, 0);  // validates the name, warms the code object
    HIPC(hipStreamSynchronize(S->stream));
    hipEvent_t e0, e1;
    HIPC(hipEventCreate(&e0));
    HIPC(hipEventCreate(&e1));
    HIPC(hipEventRecord(e0, S->stream));
    for (int i = 0; i < launches; ++i)
      enqueue_one(*S, which, i % S->e->cfg.layers);
    HIPC(hipEventRecord(e1, S->stream));
    HIPC(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPC(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms_per_launch = double(ms) / launches;
  });
}

// sampling.cpp:185-288
yuear_status yuear_generate_tokens(yuear_engine *E, const int32_t *prefix, int32_t n_prefix,
                                   const yuear_sampling *sampling, uint64_t seed,
                                   const char *phase_name, const int32_t *negative,
                                   int32_t n_negative, double cfg_scale, int32_t legacy_off,
                                   yuear_cancel_poll cancel_poll, yuear_token_callback on_token,
                                   void *user_data, int32_t *tokens_out, int32_t *n_out,
                                   int32_t *truncated, char **timing_json, char **error_json) {
  if (n_out) *n_out = 0;
  if (timing_json) *timing_json = nullptr;
  return guarded(error_json, [&] {
    if (!E || !sampling || !tokens_out || !n_out)
      invalid("engine, sampling and outputs are required");
    std::unique_lock<std::mutex> lock(E->busy, std::try_to_lock);
    if (!lock.owns_lock())
      throw Error("RuntimeError", "This engine is already executing an operation");
    E->cancelled.store(false, std::memory_order_relaxed);
    const std::string phase = phase_name ? phase_name : "full";
    const Config &c = E->cfg;
    const PhaseInfo ph = phase_info(phase, c.V);
    const yuear_sampling &s = *sampling;
    validate_sampling(s);
    check_tokens(prefix, n_prefix, c.V);
    if (n_prefix + int64_t(s.max_tokens) > kContext)
      invalid("Prefix + requested generation budget exceeds 24576; no implicit truncation");
    if (cfg_scale != 1 && n_negative < 1)
      invalid("CFG requires a negative prefix");
    if (n_negative > 0) {
      check_tokens(negative, n_negative, c.V);
      if (n_negative + int64_t(s.max_tokens) > kContext)
        invalid("Negative prefix + generation budget exceeds context");
    }
    if (seed >= (uint64_t(1) << 63))
      invalid("seed must be an integer in [0, 2**63)");
    E->cancelled_at("Cancelled before prefill", cancel_poll, user_data);  // sampling.cpp:206
    const int branches = cfg_scale != 1 ? 2 : 1;
    const int capacity =
        std::max(n_prefix, branches == 2 ? n_negative : 0) + s.max_tokens;
    auto S = std::make_unique<yuear_session>();
    begin_session(*S, E, branches, std::min(capacity, std::min(kContext, c.max_pos)), phase);
    using clock = std::chrono::steady_clock;
    const auto t0 = clock::now();
    auto since = [&](clock::time_point t) {
      return std::chrono::duration<double>(clock::now() - t).count();
    };
    prefill(*S, 0, prefix, n_prefix, nullptr, cancel_poll, user_data);
    if (branches == 2)
      prefill(*S, 1, negative, n_negative, nullptr, cancel_poll, user_data);
    HIPC(hipStreamSynchronize(S->stream));
    const double prefill_seconds = since(t0);

    // device sampler state: step 0, no end token yet, penalty table
    upload_alphas(*S, s);
    int32_t st0[2] = {0, 0};
    HIPC(hipMemcpyAsync(S->sstate, st0, 8, hipMemcpyHostToDevice, S->stream));
    SamplerParams sp = sampler_params(*S, s, seed, cfg_scale, legacy_off, -1);
    sp.max_tokens = S->history_cap;
    // one graph per token: sample from the current logits, then decode it
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    HIPC(hipStreamBeginCapture(S->stream, hipStreamCaptureModeThreadLocal));
    try {
      HIPC(launch_sampler(sp, S->stream));
      enqueue_step(*S);
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(S->stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    HIPC(hipStreamEndCapture(S->stream, &graph));
    HIPC(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    struct GraphGuard {
      hipGraph_t g;
      hipGraphExec_t x;
      ~GraphGuard() {
        if (x) (void)hipGraphExecDestroy(x);
        if (g) (void)hipGraphDestroy(g);
      }
    } guard{graph, exec};

    constexpr int kDepth = 3;
    hipEvent_t ev[kDepth];
    for (auto &e : ev)
      HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    struct EventGuard {
      hipEvent_t *e;
      ~EventGuard() {
        for (int i = 0; i < kDepth; ++i) (void)hipEventDestroy(e[i]);
      }
    } eguard{ev};
    double ttft = -1.0;
    bool eos = false, cancelled = false;
    int count = 0, launched = 0, consumed = 0;
    // The reference polls at the start of every step, before that step's
    // token is drawn and reported (sampling.cpp:243): here token i is
    // reported only after a poll that follows token i - 1's report, and
    // nothing is launched or reported once a poll has seen the cancel.
    auto poll = [&]() {
      if (!cancelled && (E->cancelled.load(std::memory_order_relaxed) ||
                         (cancel_poll && cancel_poll(user_data) != 0)))
        cancelled = true;
      return cancelled;
    };
    auto consume = [&]() {
      if (poll())
        return;
      HIPC(hipEventSynchronize(ev[consumed % kDepth]));
      const int token = S->pin_tok[consumed];
      ++consumed;
      if (ttft < 0)
        ttft = since(t0);
      if (on_token)
        on_token(user_data, phase.c_str(), token);
      if (native_to_local(token, ph, c.V) == ph.end && ph.end >= 0) {
        eos = true;
        return;
      }
      tokens_out[count++] = token;
    };
    while (launched < s.max_tokens && !eos) {
      if (poll())
        break;
      if (launched + 1 < s.max_tokens)
        HIPC(hipGraphLaunch(exec, S->stream));  // sample + forward
      else
        HIPC(launch_sampler(sp, S->stream));  // last token: no forward
      HIPC(hipMemcpyAsync(S->pin_tok + launched, S->tok, 4, hipMemcpyDeviceToHost, S->stream));
      HIPC(hipEventRecord(ev[launched % kDepth], S->stream));
      ++launched;
      if (launched - consumed >= kDepth - 1)
        consume();
      if (cancelled)
        break;
    }
    while (consumed < launched && !eos && !cancelled)
      consume();
    HIPC(hipStreamSynchronize(S->stream));
    if (cancelled)
      throw Error("InterruptedError", "Cancelled during " + phase);
    const double seconds = since(t0);
    const int out_count = count + (eos ? 1 : 0);
    *n_out = count;
    if (truncated)
      *truncated = eos ? 0 : 1;
    if (timing_json) {
      char buf[1024];
      std::snprintf(buf, sizeof buf,
                    "{\"seconds\":%.9g,\"prefill_seconds\":%.9g,\"ttft_seconds\":%s,"
                    "\"output_tokens\":%d,\"content_tokens\":%d,\"output_tps\":%.9g,"
                    "\"prefix_tokens\":%d,\"cfg_branches\":%d,\"execution\":\"hip_graph\","
                    "\"attention\":\"split_k_flash_decode\",\"backend\":\"hip-gfx950\"}",
                    seconds, prefill_seconds,
                    ttft < 0 ? "null" : std::to_string(ttft).c_str(), out_count, count,
                    out_count / seconds, n_prefix, branches);
      *timing_json = dup_string(buf);
    }
  });
}

// ---- op-level entry points ----
int32_t yuear_op_gemv(const uint16_t *w, int32_t n, int32_t k, int32_t batch, const uint16_t *x,
                      int32_t x_stride, const uint16_t *norm_w, float eps, uint16_t *y,
                      int32_t y_stride, int32_t epilogue, void *stream) {
  GemvParams p;
  p.w = w;
  p.n = n;
  p.k = k;
  p.batch = batch;
  p.x = x;
  p.x_stride = x_stride;
  p.norm_w = norm_w;
  p.eps = eps;
  p.y = y;
  p.y_stride = y_stride;
  p.epilogue = epilogue;
  if (batch >= 3 && norm_w && k > 0) {
    // the batched form normalises the rows once into a scratch buffer
    static OpPool pool;
    void *stage = nullptr;
    bool fresh = false;
    const hipError_t e = pool.get(static_cast<hipStream_t>(stream), size_t(batch) * k * 2, &stage,
                                  &fresh);
    if (e != hipSuccess)
      return int32_t(e);
    p.stage = static_cast<uint16_t *>(stage);
    return int32_t(launch_gemv(p, static_cast<hipStream_t>(stream)));
  }
  return int32_t(launch_gemv(p, static_cast<hipStream_t>(stream)));
}

int32_t yuear_op_qgemv(const uint32_t *codes, const uint32_t *groups, int32_t bits, int32_t n,
                       int32_t k, int32_t batch, const uint16_t *x, int32_t x_stride,
                       const uint16_t *norm_w, float eps, uint16_t *y, int32_t y_stride,
                       int32_t epilogue, void *stream) {
  GemvParams p;
  p.qw = codes;
  p.qsb = groups;
  p.bits = bits;
  p.n = n;
  p.k = k;
  p.batch = batch;
  p.x = x;
  p.x_stride = x_stride;
  p.norm_w = norm_w;
  p.eps = eps;
  p.y = y;
  p.y_stride = y_stride;
  p.epilogue = epilogue;
  return int32_t(launch_qgemv(p, static_cast<hipStream_t>(stream)));
}

int32_t yuear_op_dequantize(const uint32_t *codes, const uint32_t *groups, int32_t bits, int32_t n,
                            int32_t k, uint16_t *out, void *stream) {
  return int32_t(launch_dequantize(codes, groups, bits, n, k, out, static_cast<hipStream_t>(stream)));
}

yuear_status yuear_nar_condition(yuear_engine *E, const int32_t *tokens, int32_t n,
                                 int32_t visible_end, uint16_t *dev_k, uint16_t *dev_v,
                                 int32_t *visible_out, char **error_json) {
  if (visible_out)
    *visible_out = 0;
  return guarded(error_json, [&] {
    if (!E || !dev_k || !dev_v)
      invalid("engine and output buffers are required");
    std::unique_lock<std::mutex> lock(E->busy, std::try_to_lock);
    if (!lock.owns_lock())
      throw Error("RuntimeError", "This engine is already executing an operation");
    E->cancelled.store(false, std::memory_order_relaxed);
    const Config &c = E->cfg;
    // nar.cpp:142-154, 303-307
    if (E->bits)
      invalid("Shared AR tensors must be BF16; quantized AR cannot condition NAR");
    if (!tokens || n < 1)
      invalid("AR conditioning tokens are outside the model vocabulary");
    for (int i = 0; i < n; ++i)
      if (tokens[i] < 0 || tokens[i] >= c.V)
        invalid("AR conditioning tokens are outside the model vocabulary");
    if (visible_end < 0)
      invalid("nar_cond_end must be a nonnegative integer");
    if (n > std::min(kContext, c.max_pos))
      invalid("AR conditioning tokens exceed the model context");
    const int visible = visible_end ? std::min(visible_end, n) : n;
    auto S = std::make_unique<yuear_session>();
    begin_session(*S, E, 1, n, "full");
    prefill(*S, 0, tokens, n, nullptr);
    // per layer: keys / values of positions [0, visible), [Hkv][visible][D]
    const size_t per_layer = size_t(c.Hkv) * visible * c.D;
    for (int l = 0; l < c.layers; ++l) {
      const size_t off = S->layer_kv_offset(l, 0);
      HIPC(hipMemcpy2DAsync(dev_k + l * per_layer, size_t(visible) * c.D * 2, S->kc + off,
                            size_t(S->kv_stride) * c.D * 2, size_t(visible) * c.D * 2, c.Hkv,
                            hipMemcpyDeviceToDevice, S->stream));
      HIPC(launch_v_rows(S->vc + off, S->kv_stride, c.Hkv, visible, dev_v + l * per_layer,
                         S->stream));
    }
    HIPC(hipStreamSynchronize(S->stream));
    if (visible_out)
      *visible_out = visible;
  });
}

int64_t yuear_nar_attention_workspace_bytes(int32_t batch, int32_t kv_heads, int32_t kv_len) {
  if (batch < 1 || kv_heads < 1 || kv_len < 1)
    return 0;
  return int64_t(nar_attention_workspace_elems(batch, kv_heads, kv_len) * 2);
}

yuear_status yuear_nar_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                 int32_t batch, int32_t heads, int32_t kv_heads, int32_t q_len,
                                 int32_t kv_len, int32_t head_dim, int32_t causal,
                                 int32_t query_chunk_size, void *workspace, uint16_t *out,
                                 void *stream, char **error_json) {
  return guarded(error_json, [&] {
    // nar_attention.cpp:227-243
    if (batch < 1 || head_dim < 1)
      invalid("Expected attention Q/K/V shaped [batch,heads,tokens,dim]");
    if (kv_heads < 1 || heads < 1 || heads % kv_heads)
      invalid("Invalid grouped-query head count");
    if (q_len < 1 || kv_len < 1)
      invalid("Attention sequences must be nonempty");
    if (causal && q_len != kv_len)
      invalid("Causal prefill requires equal query and key lengths");
    if (query_chunk_size < 1)
      invalid("query_chunk_size must be a positive integer");
    if (head_dim != 128)
      invalid("the gfx950 kernels implement head_dim 128");
    if (!q || !k || !v || !workspace || !out)
      invalid("device buffers are required");
    NarAttnParams p;
    p.q = q;
    p.k = k;
    p.v = v;
    p.vb = static_cast<uint16_t *>(workspace);
    // split-key partials for launches too small to fill the GPU, from a
    // per-(device, stream) pool
    const size_t pf = nar_attention_part_floats(batch, heads, q_len, kv_len, causal != 0);
    if (pf) {
      static OpPool pool;
      void *buf = nullptr;
      bool fresh = false;
      HIPC(pool.get(static_cast<hipStream_t>(stream), pf * 4, &buf, &fresh));
      p.part = static_cast<float *>(buf);
      p.part_floats = pf;
    }
    p.out = out;
    p.batch = batch;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.q_len = q_len;
    p.kv_len = kv_len;
    p.causal = causal != 0;
    HIPC(launch_nar_attention(p, static_cast<hipStream_t>(stream)));
  });
}

int32_t yuear_op_attention_decode(const uint16_t *qkv, const uint16_t *q_norm,
                                  const uint16_t *k_norm, float eps, const uint16_t *rope_cos,
                                  const uint16_t *rope_sin, uint16_t *k_cache, uint16_t *v_cache,
                                  const int32_t *pos, int32_t heads, int32_t kv_heads,
                                  int32_t capacity, int32_t batch, int32_t max_splits,
                                  uint16_t *out, void *stream) {
  // split partials and arrival counters (zero between launches: the merging
  // workgroup resets its counter) from a per-(device, stream) pool
  if (batch < 1 || kv_heads < 1 || max_splits < 1 || size_t(batch) * kv_heads > 64 * 8)
    return int32_t(hipErrorInvalidValue);
  const int G = heads / kv_heads;
  const size_t need = size_t(batch) * kv_heads * max_splits * std::max(G, 1) * (128 + 2);
  static OpPool pool;
  void *buf = nullptr;
  bool fresh = false;
  const size_t counter_bytes = size_t(64) * 8 * kCounterStride * 4;
  hipError_t e = pool.get(static_cast<hipStream_t>(stream), counter_bytes + need * 4, &buf, &fresh);
  if (e != hipSuccess)
    return int32_t(e);
  int32_t *counters = static_cast<int32_t *>(buf);
  float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(buf) + counter_bytes);
  if (fresh && (e = hipMemsetAsync(counters, 0, counter_bytes, static_cast<hipStream_t>(stream))) !=
                   hipSuccess)
    return int32_t(e);
  AttnDecodeParams p;
  p.qkv = qkv;
  p.qkv_stride = (heads + 2 * kv_heads) * 128;
  p.q_norm = q_norm;
  p.k_norm = k_norm;
  p.eps = eps;
  p.rope_cos = rope_cos;
  p.rope_sin = rope_sin;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.pos = pos;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.head_dim = 128;
  p.capacity = capacity;
  p.batch = batch;
  p.max_splits = max_splits;
  p.part_o = part;
  p.part_ml = part + size_t(batch) * kv_heads * max_splits * G * 128;
  p.counters = counters;
  p.out = out;
  p.out_stride = heads * 128;
  return int32_t(launch_attn_decode(p, static_cast<hipStream_t>(stream)));
}

int32_t yuear_op_gemm(const uint16_t *a, int32_t lda, const uint16_t *w, int32_t m, int32_t n,
                      int32_t k, uint16_t *c, int32_t ldc, int32_t residual, void *stream) {
  GemmParams p{a, lda, w, m, n, k, c, ldc, residual};
  return int32_t(launch_gemm(p, static_cast<hipStream_t>(stream)));
}

int32_t yuear_op_gemm_tile(const uint16_t *a, int32_t lda, const uint16_t *w, int32_t m,
                           int32_t n, int32_t k, uint16_t *c, int32_t ldc, int32_t residual,
                           int32_t shape, void *stream) {
  GemmParams p{a, lda, w, m, n, k, c, ldc, residual};
  return int32_t(launch_gemm_tile(p, shape, static_cast<hipStream_t>(stream)));
}
int32_t yuear_op_gemm_split(const uint16_t *a, int32_t lda, const uint16_t *w, int32_t m,
                            int32_t n, int32_t k, uint16_t *c, int32_t ldc, int32_t residual,
                            int32_t shape, int32_t splits, void *stream) {
  GemmParams p{a, lda, w, m, n, k, c, ldc, residual};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (splits > 1) {
    // the checks launch_gemm_tile repeats, before anything is allocated
    // (m * n below 2^58 keeps the workspace size within size_t)
    if (m < 1 || n < 1 || splits > 16 || k < 64 || k % 64 || (k / 64) % splits ||
        size_t(m) * size_t(n) > (SIZE_MAX >> 6))
      return int32_t(hipErrorInvalidValue);
    static OpPool pool;
    void *buf = nullptr;
    bool fresh = false;
    const size_t bytes = size_t(splits) * size_t(m) * size_t(n) * 4;
    const hipError_t e = pool.get(st, bytes, &buf, &fresh);
    if (e != hipSuccess)
      return int32_t(e);
    p.part = static_cast<float *>(buf);
    p.part_bytes = bytes;
  }
  return int32_t(launch_gemm_tile(p, shape, st, splits));
}

int32_t yuear_op_attention_prefill(const uint16_t *q, const uint16_t *k_cache,
                                   const uint16_t *v_cache, int32_t tokens, int32_t pos0,
                                   int32_t heads, int32_t kv_heads, int32_t capacity,
                                   uint16_t *out, void *stream) {
  AttnPrefillParams p;
  p.q = q;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.tokens = tokens;
  p.pos0 = pos0;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.head_dim = 128;
  p.capacity = capacity;
  p.out = out;
  return int32_t(launch_attn_prefill(p, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
