// Split-K flash-decode attention for one layer on gfx950 (head_dim 128),
// one kernel per layer: a one-dimensional grid of max_splits * batch * Hkv
// workgroups of 256 threads, block = split * (batch * Hkv) + bh (the splits
// of one (branch, kv head) spread over the XCDs). The workgroup body is
// attn_block.h. The chunk length is derived on device from pos[b], so one
// captured graph serves every KV length up to capacity.
#include <cmath>

#include "attn_block.h"
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int D = attn::D;
constexpr int kWaves = 4;  // 128 keys per pass (8 waves measured no faster on MI355X)

template <int G, int W>
__global__ __launch_bounds__(64 * W) void attn_decode_kernel(AttnDecodeParams p, float scale) {
  __shared__ AttnShared<G, W> sm;
  const int nbh = p.batch * p.kv_heads;
  attn_block<G, W>(p, scale, int(blockIdx.x) / nbh, int(blockIdx.x) % nbh, p.max_splits, sm);
}

template <int G>
hipError_t launch_g(const AttnDecodeParams &p, hipStream_t s) {
  const float scale = float(std::pow(double(D), -0.5));  // ar.cpp:283
  hipLaunchKernelGGL((attn_decode_kernel<G, kWaves>),
                     dim3(p.max_splits * p.batch * p.kv_heads), dim3(64 * kWaves), 0, s, p,
                     scale);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_decode(const AttnDecodeParams &p, hipStream_t s) {
  if (p.head_dim != D || p.kv_heads < 1 || p.heads % p.kv_heads || p.max_splits < 1 ||
      p.max_splits > kAttnMaxSplits || p.batch < 1 || p.capacity < 1 ||
      p.capacity % attn::kBlock)
    return hipErrorInvalidValue;
  switch (p.heads / p.kv_heads) {
  case 1: return launch_g<1>(p, s);
  case 2: return launch_g<2>(p, s);
  case 3: return launch_g<3>(p, s);
  case 4: return launch_g<4>(p, s);
  case 6: return launch_g<6>(p, s);
  case 8: return launch_g<8>(p, s);
  }
  return hipErrorInvalidValue;
}

int attn_decode_splits(int batch, int kv_heads, int kv_stride) {
  // One 128-key pass per workgroup at the session's capacity (every K/V
  // operand of a split in flight at once), capped so that a launch stays
  // within about 512 workgroups; never more splits than 32-key blocks.
  const int nbh = batch * kv_heads;
  const int passes = (kv_stride + 32 * kWaves - 1) / (32 * kWaves);
  const int cap = std::max(2, 512 / nbh);
  return std::max(1, std::min({kAttnMaxSplits, cap, passes, kv_stride / attn::kBlock}));
}

}  // namespace yuear
