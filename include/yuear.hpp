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

inline void check(yuear_status st, char *error_json) {
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
      if (*c->cancel && (*c->cancel)())
        c->engine->cancel();  // polled once per token
    } catch (...) {
      c->thrown = std::current_exception();
      c->engine->cancel();
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
      int32_t(neg.size()), cfg_scale, legacy_off ? 1 : 0, trampoline, &ctx, out.data(), &n,
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

}  // namespace yuear
