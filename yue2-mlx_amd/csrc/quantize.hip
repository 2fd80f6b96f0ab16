// Host-side affine group-64 quantizer: the step the reference's converter
// applies to every AR linear before the decode loop sees it
// (native/src/conversion.cpp:470-532, mx::quantize(w, 64, bits, "affine")).
// This build uses it only to make quantized weights for the RANDOM weight
// source; checkpoints arrive already quantized.
//
// Per group of 64 weights (restated from MLX's published affine quantize):
// the edge of larger magnitude (w_min if |w_min| > |w_max|, else w_max) is
// kept exactly as the bias; the scale (w_max - w_min) / (2^bits - 1), at
// least 1e-7, takes the sign that maps the group onto codes >= 0 from that
// edge, and is refined to edge / round(edge / scale) when that quotient is
// nonzero (bias then 0 when it is zero); scale and bias are stored as bf16
// and the codes are clip(round((w - bias) / scale), 0, 2^bits - 1) with the
// stored values, rounded half to even. Codes are packed 32 / bits per
// uint32, code j of a word at bits [bits * j, bits * j + bits).
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace yuear {

void quantize_affine(const uint16_t *w, int64_t rows, int k, int bits, uint32_t *codes,
                     uint16_t *scales, uint16_t *biases) {
  const int groups = k / 64, per = 32 / bits, words = k / per;
  const float levels = float((1 << bits) - 1);
  auto work = [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      const uint16_t *wr = w + r * k;
      uint32_t *cr = codes + r * words;
      std::fill(cr, cr + words, 0u);
      for (int g = 0; g < groups; ++g) {
        float lo = bf2f(wr[g * 64]), hi = lo;
        for (int i = 1; i < 64; ++i) {
          const float v = bf2f(wr[g * 64 + i]);
          lo = std::min(lo, v);
          hi = std::max(hi, v);
        }
        const bool low_edge = std::fabs(lo) > std::fabs(hi);
        float scale = std::max((hi - lo) / levels, 1e-7f);
        if (!low_edge)
          scale = -scale;
        const float edge = low_edge ? lo : hi;
        const float q0 = std::nearbyint(edge / scale);
        if (q0 != 0.f)
          scale = edge / q0;
        const float bias = q0 == 0.f ? 0.f : edge;
        const uint16_t sb = f2bf(scale), bb = f2bf(bias);
        scales[r * groups + g] = sb;
        biases[r * groups + g] = bb;
        const float s = bf2f(sb), b = bf2f(bb);
        for (int i = 0; i < 64; ++i) {
          const float q = std::nearbyint((bf2f(wr[g * 64 + i]) - b) / s);
          const uint32_t code = uint32_t(std::min(std::max(q, 0.f), levels));
          const int j = g * 64 + i;
          cr[j / per] |= code << ((j % per) * bits);
        }
      }
    }
  };
  const unsigned workers = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (workers == 1 || rows < 64) {
    work(0, rows);
    return;
  }
  const int64_t per_worker = (rows + workers - 1) / workers;
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < workers; ++t) {
    const int64_t r0 = std::min(rows, int64_t(t) * per_worker), r1 = std::min(rows, r0 + per_worker);
    if (r0 < r1)
      pool.emplace_back(work, r0, r1);
  }
  for (auto &t : pool)
    t.join();
}

}  // namespace yuear
