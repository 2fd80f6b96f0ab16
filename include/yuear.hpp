// C++20 facade over the C ABI of yuear.h: the engine and generate_tokens with
// the reference's signatures, for a native caller that held an ARModel.
//
//   lyra::ARModel(directory, precision, verify)  -> yuear::Engine(directory,
//                                                   precision)  (ar.hpp:31-38)
//   lyra::generate_tokens(model, prefix, sampling, seed, phase, negative,
//                         cfg_scale, legacy_off, cancelled, on_token,
//                         progress)                -> yuear::generate_tokens
//                                                   (ar.hpp:43-48)
//   lyra::Error{type, message}                    -> yuear::Error (types.hpp:20-24)
//   lyra::Sampling defaults                       -> yuear::Sampling (types.hpp:29-38)
//   lyra::Tokenizer, token_prefixes, negative_prefix, chunk_ranges,
//   SongRequest                                   -> yuear::Tokenizer, ... (protocol.hpp:5-26,
//                                                   types.hpp:50-62)
//   Pipeline::generate_phase / plan / generate_semantic
//                                                 -> yuear::Pipeline (pipeline.cpp:186-263)
//
// Header-only; link with -lyuear. Errors reported by the library (JSON
// {"type", "message"}) become yuear::Error with the same type name
// ("ValueError", "FileNotFoundError", "InterruptedError", "RuntimeError").
// An exception thrown by on_token or cancelled cancels the running call and
// is rethrown once the library has returned (no exception crosses the C
// ABI). Timing comes back as the library's JSON text (the keys of
// sampling.cpp:274-284); this header carries no JSON library.
#pragma once

#include <cstdint>
#include <exception>
#include <filesystem>
#include <functional>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "yuear.h"

namespace yuear {

struct Error : std::runtime_error {
  std::string type;
  Error(std::string kind, const std::string &message)
      : std::runtime_error(message), type(std::move(kind)) {}
};

using Cancelled = std::function<bool()>;
using TokenCallback = std::function<void(std::string_view, int)>;

struct Sampling {
  double temperature = 1, top_p = .95;
  int top_k = 100;
  double repetition_penalty = 1.2;
  int penalty_window = 50, min_tokens = 200, max_tokens = 9000;
};

struct TokenGeneration {
  std::vector<int> tokens;
  std::string timing_json;
  bool truncated = false;
};

namespace detail {

// Value of a top-level string field of the library's error JSON (escapes
// \" \\ \/ \n \t \r \b \f and \u00XX, the ones the library writes).
inline std::string json_string(const std::string &json, const std::string &key) {
  const std::string pat = "\"" + key + "\":\"";
  const size_t at = json.find(pat);
  if (at == std::string::npos)
    return {};
  std::string out;
  for (size_t i = at + pat.size(); i < json.size() && json[i] != '"'; ++i) {
    char c = json[i];
    if (c == '\\' && i + 1 < json.size()) {
      const char e = json[++i];
      switch (e) {
      case 'n': c = '\n'; break;
      case 't': c = '\t'; break;
      case 'r': c = '\r'; break;
      case 'b': c = '\b'; break;
      case 'f': c = '\f'; break;
      case 'u':
        if (i + 4 < json.size()) {
          c = char(std::stoi(json.substr(i + 1, 4), nullptr, 16));
          i += 4;
        }
        break;
      default: c = e;
      }
    }
    out += c;
  }
  return out;
}

inline std::string take(char *s) {
  std::string out = s ? s : "";
  yuear_string_free(s);
  return out;
}

// error_json is taken by reference: in check(call(&error), error) the call
// may run after a by-value copy of `error` had been taken.
inline void check(yuear_status st, char *const &error_json) {
  if (st == YUEAR_SUCCESS) {
    yuear_string_free(error_json);
    return;
  }
  const std::string json = take(error_json);
  std::string type = json_string(json, "type");
  throw Error(type.empty() ? "RuntimeError" : type, json_string(json, "message"));
}

}  // namespace detail

class Engine {
 public:
  // Checkpoint directory: conversion.json, config.json and
  // ar-<precision>.safetensors, checked as ar.cpp:133-238 does.
  explicit Engine(const std::filesystem::path &directory, const std::string &precision = "bf16",
                  bool strict = true) {
    char *error = nullptr;
    detail::check(yuear_engine_load(directory.c_str(), precision.c_str(), strict ? 1 : 0,
                                    &engine_, &error),
                  error);
  }
  // Architecture plus host tensors or the deterministic generator.
  Engine(const yuear_model_config &config, const yuear_weight_source &weights) {
    char *error = nullptr;
    detail::check(yuear_engine_create(&config, &weights, &engine_, &error), error);
  }
  Engine(const Engine &) = delete;
  Engine &operator=(const Engine &) = delete;
  Engine(Engine &&o) noexcept : engine_(std::exchange(o.engine_, nullptr)) {}
  Engine &operator=(Engine &&o) noexcept {
    std::swap(engine_, o.engine_);
    return *this;
  }
  ~Engine() { yuear_engine_destroy(engine_); }

  yuear_engine *get() const { return engine_; }
  int bits() const { return yuear_engine_bits(engine_); }
  void cancel() { yuear_engine_cancel(engine_); }

 private:
  yuear_engine *engine_ = nullptr;
};

inline TokenGeneration generate_tokens(Engine &engine, const std::vector<int> &prefix,
                                       const Sampling &s, uint64_t seed, std::string_view phase,
                                       const std::vector<int> &negative = {},
                                       double cfg_scale = 1, bool legacy_off = false,
                                       const Cancelled &cancelled = {},
                                       const TokenCallback &on_token = {},
                                       bool /*progress*/ = false) {
  const yuear_sampling ys{s.temperature, s.top_p,          s.top_k,     s.repetition_penalty,
                          s.penalty_window, s.min_tokens, s.max_tokens};
  struct Ctx {
    const TokenCallback *cb;
    const Cancelled *cancel;
    Engine *engine;
    std::exception_ptr thrown;
  } ctx{&on_token, &cancelled, &engine, nullptr};
  auto trampoline = [](void *user, const char *ph, int32_t token) {
    auto *c = static_cast<Ctx *>(user);
    if (c->thrown)
      return;
    try {
      if (*c->cb)
        (*c->cb)(ph, int(token));
    } catch (...) {
      c->thrown = std::current_exception();
      c->engine->cancel();
    }
  };
  // polled by the library where the reference calls cancelled_at
  // (sampling.cpp:156, 164, 206, 243); a throwing predicate cancels the call
  // and its exception reaches the caller
  auto poll = [](void *user) -> int32_t {
    auto *c = static_cast<Ctx *>(user);
    if (c->thrown)
      return 1;
    try {
      return *c->cancel && (*c->cancel)() ? 1 : 0;
    } catch (...) {
      c->thrown = std::current_exception();
      return 1;
    }
  };
  const std::vector<int32_t> pre(prefix.begin(), prefix.end());
  const std::vector<int32_t> neg(negative.begin(), negative.end());
  std::vector<int32_t> out(s.max_tokens > 0 ? size_t(s.max_tokens) : 1);
  int32_t n = 0, truncated = 0;
  char *timing = nullptr, *error = nullptr;
  const std::string ph(phase);
  const yuear_status st = yuear_generate_tokens(
      engine.get(), pre.data(), int32_t(pre.size()), &ys, seed, ph.c_str(), neg.data(),
      int32_t(neg.size()), cfg_scale, legacy_off ? 1 : 0, poll, trampoline, &ctx, out.data(), &n,
      &truncated, &timing, &error);
  if (ctx.thrown) {
    yuear_string_free(timing);
    yuear_string_free(error);
    std::rethrow_exception(ctx.thrown);
  }
  TokenGeneration g;
  g.timing_json = detail::take(timing);
  detail::check(st, error);  // status 130: Error("InterruptedError", ...), sampling.cpp:243
  g.tokens.assign(out.begin(), out.begin() + n);
  g.truncated = truncated != 0;
  return g;
}

// ---- text side and the phase glue ----

inline constexpr int kEOD = 151643, kCodecOffset = 151853;

namespace detail {
inline std::vector<int> take_ids(int32_t *ids, int64_t n) {
  std::vector<int> out(ids, ids + n);
  yuear_ids_free(ids);
  return out;
}
}  // namespace detail

// lyra::Tokenizer (protocol.hpp:5-16) over a checkpoint-native qwen.tiktoken.
class Tokenizer {
 public:
  explicit Tokenizer(const std::filesystem::path &vocabulary) {
    char *error = nullptr;
    detail::check(yuear_tokenizer_load(vocabulary.c_str(), &tok_, &error), error);
  }
  Tokenizer(const Tokenizer &) = delete;
  Tokenizer &operator=(const Tokenizer &) = delete;
  Tokenizer(Tokenizer &&o) noexcept : tok_(std::exchange(o.tok_, nullptr)) {}
  Tokenizer &operator=(Tokenizer &&o) noexcept {
    std::swap(tok_, o.tok_);
    return *this;
  }
  ~Tokenizer() { yuear_tokenizer_destroy(tok_); }

  std::vector<int> encode(std::string_view text) const {
    int32_t *ids = nullptr;
    int64_t n = 0;
    char *error = nullptr;
    detail::check(yuear_tokenizer_encode(tok_, text.data(), int64_t(text.size()), &ids, &n,
                                         &error),
                  error);
    return detail::take_ids(ids, n);
  }
  std::string decode(const std::vector<int> &tokens) const {
    const std::vector<int32_t> ids(tokens.begin(), tokens.end());
    char *text = nullptr, *error = nullptr;
    int64_t len = 0;
    detail::check(yuear_tokenizer_decode(tok_, ids.data(), int64_t(ids.size()), &text, &len,
                                         &error),
                  error);
    std::string out(text, size_t(len));
    yuear_string_free(text);
    return out;
  }
  const yuear_tokenizer *get() const { return tok_; }

 private:
  yuear_tokenizer *tok_ = nullptr;
};

// lyra::SongRequest (types.hpp:50-62): the fields the prompt layout reads.
struct SongRequest {
  std::string style, lyrics, cot = "full";
  uint64_t seed = 831001;
  std::optional<std::string> abc;
  std::optional<double> cfg_scale;
  std::string id = "song";

  yuear_song_request c() const {
    return {style.c_str(), lyrics.c_str(), cot.c_str(), abc ? abc->c_str() : nullptr,
            id.c_str(),    seed,           cfg_scale.value_or(0.0), cfg_scale ? 1 : 0};
  }
  void validate() const {  // protocol.mm:212-237
    const auto r = c();
    char *error = nullptr;
    detail::check(yuear_song_request_validate(&r, &error), error);
  }
  double guidance() const {  // protocol.mm:238-240
    const auto r = c();
    return yuear_song_request_guidance(&r);
  }
};

namespace detail {
template <class F>
std::vector<int> prefix(F fn, const SongRequest &r, const Tokenizer &t,
                        const std::optional<std::vector<int>> &abc_ids) {
  const auto req = r.c();
  std::vector<int32_t> ids;
  if (abc_ids)
    ids.assign(abc_ids->begin(), abc_ids->end());
  int32_t *out = nullptr;
  int64_t n = 0;
  char *error = nullptr;
  check(fn(t.get(), &req, ids.data(), int64_t(ids.size()), abc_ids ? 1 : 0, &out, &n, &error),
        error);
  return take_ids(out, n);
}
}  // namespace detail

// token_prefixes / negative_prefix (protocol.hpp:19-24, protocol.mm:321-357)
inline std::vector<int> token_prefixes(const SongRequest &r, const Tokenizer &t,
                                       const std::optional<std::vector<int>> &abc_ids = {}) {
  return detail::prefix(yuear_token_prefixes, r, t, abc_ids);
}
inline std::vector<int> negative_prefix(const SongRequest &r, const Tokenizer &t,
                                        const std::optional<std::vector<int>> &abc_ids = {}) {
  return detail::prefix(yuear_negative_prefix, r, t, abc_ids);
}

// chunk_ranges (protocol.hpp:25-26, protocol.mm:358-369)
inline std::vector<std::pair<int, int>> chunk_ranges(int frames, int prefix_tokens,
                                                     int context = 24576) {
  int32_t *bounds = nullptr;
  int64_t n = 0;
  char *error = nullptr;
  detail::check(yuear_chunk_ranges(frames, prefix_tokens, context, &bounds, &n, &error), error);
  std::vector<std::pair<int, int>> out;
  for (int64_t i = 0; i < n; ++i)
    out.emplace_back(bounds[2 * i], bounds[2 * i + 1]);
  yuear_ids_free(bounds);
  return out;
}

// GenerationConfig's per-phase sampling defaults (vendor protocol.py:44-47;
// vendor test_protocol.py:18-19).
struct GenerationConfig {
  Sampling abc{.7, .9, 30, 1.005, 100, 32, 4096};
  Sampling semantic{1., .95, 100, 1.2, 50, 200, 9000};
};

struct SymbolicPlan {
  SongRequest request;
  std::vector<int> prefix;
  std::optional<std::string> abc;
  std::vector<int> abc_ids;
  std::string timing_json;  // the abc phase's timing; external ABC: zero seconds
  bool truncated = false;
};

struct SemanticResult {
  SymbolicPlan plan;
  std::vector<int> codes;  // codec frames: semantic tokens - CODEC_OFFSET
  std::string timing_json;
  bool truncated = false;
};

// The phase glue of lyra::Pipeline (pipeline.cpp:186-263) over one engine
// and tokenizer. Per-phase sampling overrides are whole Sampling values
// (the reference merges a JSON object over the defaults).
class Pipeline {
 public:
  Pipeline(Engine &engine, const Tokenizer &tokenizer, GenerationConfig config = {})
      : engine_(engine), tokenizer_(tokenizer), config_(config) {}

  // generate_phase (pipeline.cpp:186-211): the library checks the sampling
  // and the 24576-token context budget with the reference's messages.
  TokenGeneration generate_phase(const std::vector<int> &prefix, const Sampling &sampling,
                                 uint64_t seed, std::string_view phase,
                                 const std::vector<int> &negative = {}, double guidance = 1,
                                 bool legacy_off = false, const Cancelled &cancelled = {},
                                 const TokenCallback &on_token = {}) {
    return generate_tokens(engine_, prefix, sampling, seed, phase, negative, guidance, legacy_off,
                           cancelled, on_token);
  }

  // plan (pipeline.cpp:213-241): the ABC phase, or the request's own score
  SymbolicPlan plan(const SongRequest &request,
                    const std::optional<Sampling> &abc_sampling = std::nullopt,
                    const Cancelled &cancelled = {}, const TokenCallback &on_token = {}) {
    request.validate();
    SymbolicPlan out;
    out.request = request;
    if (request.cot == "off") {
      out.prefix = token_prefixes(request, tokenizer_);
    } else if (request.abc) {
      out.abc = request.abc;
      out.abc_ids = tokenizer_.encode(*request.abc);
      out.prefix = token_prefixes(request, tokenizer_, out.abc_ids);
      out.timing_json = "{\"seconds\":0.0,\"output_tokens\":0,\"external_prefix_tokens\":" +
                        std::to_string(out.abc_ids.size()) + "}";
    } else {
      auto g = generate_phase(token_prefixes(request, tokenizer_),
                              abc_sampling.value_or(config_.abc), request.seed, "abc", {}, 1,
                              false, cancelled, on_token);
      out.abc_ids = std::move(g.tokens);
      out.abc = tokenizer_.decode(out.abc_ids);
      out.prefix = token_prefixes(request, tokenizer_, out.abc_ids);
      out.timing_json = std::move(g.timing_json);
      out.truncated = g.truncated;
    }
    return out;
  }

  // generate_semantic (pipeline.cpp:243-263)
  SemanticResult generate_semantic(const SymbolicPlan &plan,
                                   const std::optional<Sampling> &overrides = std::nullopt,
                                   const Cancelled &cancelled = {},
                                   const TokenCallback &on_token = {}) {
    if (token_prefixes(plan.request, tokenizer_, plan.abc_ids) != plan.prefix)
      throw Error("ValueError", "Plan prefix disagrees with request/exact ABC IDs");
    std::vector<int> negative;
    const double guidance = plan.request.guidance();
    if (guidance != 1)
      negative = negative_prefix(plan.request, tokenizer_, plan.abc_ids);
    auto g = generate_phase(plan.prefix, overrides.value_or(config_.semantic), plan.request.seed,
                            "semantic", negative, guidance, plan.request.cot == "off", cancelled,
                            on_token);
    if (g.tokens.empty())
      throw Error("RuntimeError", "Semantic generation produced no codec frames");
    for (int &t : g.tokens)
      t -= kCodecOffset;
    return {plan, std::move(g.tokens), std::move(g.timing_json), g.truncated};
  }

 private:
  Engine &engine_;
  const Tokenizer &tokenizer_;
  GenerationConfig config_;
};

}  // namespace yuear
