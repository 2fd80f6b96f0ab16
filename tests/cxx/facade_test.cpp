// Drives libyuear through include/yuear.hpp the way a native caller of the
// reference's generate_tokens (ar.hpp:43-48; caller pipeline.cpp:186-211)
// would, and prints one JSON line per case for tests/test_gpu_facade.py:
// tokens of greedy, sampled and CFG runs on a 2-layer model of the
// deterministic generator (seed 11), the per-token callback stream, the
// error type of invalid sampling, of a cancelled run and of a throwing
// callback, and that the engine still generates after each of them.
#include <cstdio>
#include <stdexcept>
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

void line(const std::string &name, const std::string &body) {
  std::printf("{\"case\":\"%s\",%s}\n", name.c_str(), body.c_str());
  std::fflush(stdout);
}

}  // namespace

int main() {
  const yuear_model_config cfg{256, 512, 2, 4, 2, 128, 512, 64, 1e-5f, 500000.0, 1};
  const yuear_weight_source src{YUEAR_WEIGHTS_RANDOM, 11, 0.02f, 0.1f, nullptr, 0, 0};
  yuear::Engine engine(cfg, src);
  const std::vector<int> prefix{3, 17, 255, 1, 98};

  yuear::Sampling greedy{0.0, 1.0, 1, 1.0, 50, 0, 24};
  auto g = yuear::generate_tokens(engine, prefix, greedy, 0, "full");
  line("greedy", "\"tokens\":" + ints(g.tokens) + ",\"truncated\":" +
                     (g.truncated ? "true" : "false") + ",\"timing\":" + g.timing_json);

  yuear::Sampling sampled{1.0, 0.9, 40, 1.1, 50, 0, 24};
  std::vector<int> seen;
  std::string phases;
  auto s = yuear::generate_tokens(engine, prefix, sampled, 77, "full", {}, 1.0, false, {},
                                  [&](std::string_view ph, int tok) {
                                    seen.push_back(tok);
                                    phases = std::string(ph);
                                  });
  line("sampled", "\"tokens\":" + ints(s.tokens) + ",\"callback\":" + ints(seen) +
                      ",\"phase\":\"" + phases + "\"");

  auto c = yuear::generate_tokens(engine, prefix, sampled, 78, "full", {9, 8, 7}, 1.5);
  line("cfg", "\"tokens\":" + ints(c.tokens));

  try {
    yuear::Sampling bad = sampled;
    bad.top_p = 1.5;
    yuear::generate_tokens(engine, prefix, bad, 1, "full");
    line("invalid", "\"error\":null");
  } catch (const yuear::Error &e) {
    line("invalid", "\"error\":\"" + e.type + "\"");
  }

  // Cancellation where the reference polls (sampling.cpp:156, 164, 206,
  // 243): `cancel_after` polls answer false, the rest true. With a CFG pair
  // the polls come: after validation, before branch 0's prefill, its chunk,
  // before branch 1's prefill, its chunk, then before each token.
  struct Cancel {
    const char *name;
    int cancel_after, stop_after_calls;
  };
  for (const Cancel &k : {Cancel{"cancel_before", 0, -1}, Cancel{"cancel_branch1", 3, -1},
                          Cancel{"cancel_prefill", 4, -1}, Cancel{"cancelled", -1, 3}}) {
    int calls = 0, polls = 0;
    try {
      yuear::generate_tokens(
          engine, prefix, sampled, 5, "full", {9, 8, 7}, 1.5, false,
          [&] {
            ++polls;
            return k.cancel_after >= 0 ? polls > k.cancel_after : calls >= k.stop_after_calls;
          },
          [&](std::string_view, int) { ++calls; });
      line(k.name, "\"error\":null");
    } catch (const yuear::Error &e) {
      line(k.name, "\"error\":\"" + e.type + "\",\"message\":\"" + e.what() +
                       "\",\"calls\":" + std::to_string(calls) +
                       ",\"polls\":" + std::to_string(polls));
    }
  }

  try {
    yuear::generate_tokens(engine, prefix, sampled, 5, "full", {}, 1.0, false, {},
                           [](std::string_view, int) { throw std::out_of_range("boom"); });
    line("throwing", "\"error\":null");
  } catch (const std::out_of_range &e) {
    line("throwing", std::string("\"error\":\"out_of_range\",\"what\":\"") + e.what() + "\"");
  }

  auto again = yuear::generate_tokens(engine, prefix, greedy, 0, "full");
  line("again", "\"tokens\":" + ints(again.tokens));
  return 0;
}
