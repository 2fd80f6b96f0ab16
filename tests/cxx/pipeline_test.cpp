// Drives the phase glue of include/yuear.hpp (yuear::Pipeline, the
// reference's Pipeline::plan / generate_semantic, pipeline.cpp:186-263) over
// a 2-layer model with the YuE2 vocabulary (deterministic generator, seed
// 13) and the tokenizer whose qwen.tiktoken path is argv[1]; prints one JSON
// line per case for tests/test_gpu_facade.py.
#include <cstdio>
#include <string>
#include <vector>

#include "yuear.hpp"

namespace {

std::string ints(const std::vector<int> &v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i)
    s += (i ? "," : "") + std::to_string(v[i]);
  return s + "]";
}

std::string quote(const std::string &t) {
  std::string o = "\"";
  for (unsigned char c : t) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += char(c);
    } else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof buf, "\\u%04x", c);
      o += buf;
    } else {
      o += char(c);
    }
  }
  return o + "\"";
}

void line(const std::string &name, const std::string &body) {
  std::printf("{\"case\":\"%s\",%s}\n", name.c_str(), body.c_str());
  std::fflush(stdout);
}

std::string plan_json(const yuear::SymbolicPlan &p) {
  return "\"prefix\":" + ints(p.prefix) + ",\"abc_ids\":" + ints(p.abc_ids) +
         ",\"abc\":" + (p.abc ? quote(*p.abc) : "null") + ",\"truncated\":" +
         (p.truncated ? "true" : "false") + ",\"timing\":" +
         (p.timing_json.empty() ? "null" : p.timing_json);
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s qwen.tiktoken\n", argv[0]);
    return 2;
  }
  const yuear_model_config cfg{256, 512, 2, 4, 2, 128, 184704, 1024, 1e-5f, 500000.0, 1};
  const yuear_weight_source src{YUEAR_WEIGHTS_RANDOM, 13, 0.02f, 0.1f, nullptr, 0, 0};
  yuear::Engine engine(cfg, src);
  const yuear::Tokenizer tokenizer(argv[1]);
  yuear::Pipeline pipeline(engine, tokenizer);
  const yuear::Sampling abc{0.7, 0.9, 30, 1.005, 100, 4, 16};
  const yuear::Sampling semantic{1.0, 0.95, 100, 1.2, 50, 4, 12};

  // generated score, classifier-free guidance 1.5 in the semantic phase
  yuear::SongRequest full;
  full.style = "female vocal, pop, piano";
  full.lyrics = "[verse]\nI've been walking down this road tonight\n";
  full.cfg_scale = 1.5;
  full.seed = 21;
  const auto p1 = pipeline.plan(full, abc);
  line("plan_full", plan_json(p1));
  const auto s1 = pipeline.generate_semantic(p1, semantic);
  line("semantic_full", "\"codes\":" + ints(s1.codes) + ",\"truncated\":" +
                            (s1.truncated ? "true" : "false"));

  // no score (cot off): default guidance 1.01 and the legacy-off sampler
  yuear::SongRequest off = full;
  off.cot = "off";
  off.cfg_scale.reset();
  const auto p2 = pipeline.plan(off, abc);
  line("plan_off", plan_json(p2));
  const auto s2 = pipeline.generate_semantic(p2, semantic);
  line("semantic_off", "\"codes\":" + ints(s2.codes));

  // the request's own score: encoded, no ABC phase
  yuear::SongRequest given = full;
  given.cot = "melody";
  given.abc = "X:1\nK:C\n\"C\"CDEF|GABc|\n";
  given.cfg_scale.reset();
  const auto p3 = pipeline.plan(given, abc);
  line("plan_external", plan_json(p3));
  const auto s3 = pipeline.generate_semantic(p3, semantic);
  line("semantic_external", "\"codes\":" + ints(s3.codes));

  try {
    auto bad = p1;
    bad.prefix.push_back(5);
    pipeline.generate_semantic(bad, semantic);
    line("tampered", "\"error\":null");
  } catch (const yuear::Error &e) {
    line("tampered", "\"error\":" + quote(e.type) + ",\"message\":" + quote(e.what()));
  }
  try {
    auto bad = full;
    bad.id = "../x";
    pipeline.plan(bad, abc);
    line("invalid_request", "\"error\":null");
  } catch (const yuear::Error &e) {
    line("invalid_request", "\"error\":" + quote(e.type) + ",\"message\":" + quote(e.what()));
  }
  try {
    auto big = semantic;
    big.max_tokens = 24576;
    pipeline.generate_semantic(p1, big);
    line("budget", "\"error\":null");
  } catch (const yuear::Error &e) {
    line("budget", "\"error\":" + quote(e.type) + ",\"message\":" + quote(e.what()));
  }
  return 0;
}
