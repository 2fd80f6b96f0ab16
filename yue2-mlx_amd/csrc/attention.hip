// Split-K flash-decode attention for one layer on gfx950 (head_dim 128),
// one kernel per layer: a one-dimensional grid of max_splits * batch * Hkv
// workgroups of 256 threads, block = split * (batch * Hkv) + bh (with
// batch * Hkv a multiple of 8, round-robin dispatch puts the splits of one
// (branch, kv head) on one XCD; the partial hand-off does not rely on it and
// uses device-scope stores and loads). The workgroup body is
// attn_block.h. The chunk length is derived on device from pos[b], so one
// captured graph serves every KV length up to capacity.
#include <cmath>
#include <map>
#include <mutex>

#include "../../include/yuear.h"
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
  // operand of a split in flight at once), capped at one workgroup per CU
  // for a single sequence and at about 512 workgroups for several branches;
  // never more splits than 32-key blocks. Measured on MI355X (3B, 8 kv
  // heads, whole decode steps): one sequence at KV 4096 / 8000 / 16000 /
  // 24000 steps 0.4 / 3.4 / 1.4 / 2.0% faster with 256 workgroups than with
  // 264-512, and slower with 240 or 384; two branches gain at KV 4000 but
  // lose at 16000 with 256 instead of 512, so they keep the 512 cap.
  const int nbh = batch * kv_heads;
  const int passes = (kv_stride + 32 * kWaves - 1) / (32 * kWaves);
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  const int cap = std::max(2, (batch == 1 ? cus : 512) / nbh);
  return std::max(1, std::min({kAttnMaxSplits, cap, passes, kv_stride / attn::kBlock}));
}

}  // namespace yuear

// ---------------------------------------------------------------------------
// yuear_op_attention_decode_noalloc: the decode attention with its scratch in
// a fixed device array instead of library-allocated memory.
//
// `scratch` holds the arrival counters (kNoallocCounterBytes: 512 (branch,
// kv head) pairs, kCounterStride ints apart) and then the split partials. In
// host code the array's name is only a stand-in: its device address, which
// differs per GPU, is looked up once per device with hipGetSymbolAddress and
// used for every kernel argument. Calls on one GPU share the array: calls
// that overlap in time on one GPU race. The counters are cleared by a fill
// kernel the first time a device is used (the attention's merging workgroup
// returns each counter to zero after every launch).
namespace yuear {
namespace {

constexpr size_t kNoallocBytes = size_t(4) << 20;
constexpr size_t kNoallocCounterBytes = size_t(512) * kCounterStride * 4;
static __device__ __align__(256) uint8_t scratch[kNoallocBytes];

__global__ void zero_words_kernel(uint32_t *p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

struct NoallocScratch {
  std::mutex mu;
  std::map<int, uint8_t *> ptr;  // device -> address of `scratch` on it
};
NoallocScratch &noalloc_scratch() {
  static NoallocScratch s;
  return s;
}

// Address of this device's `scratch`; set up (symbol lookup, counters
// cleared on `stream`) on the first call for the device.
hipError_t noalloc_base(hipStream_t stream, uint8_t **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return e;
  NoallocScratch &s = noalloc_scratch();
  std::lock_guard<std::mutex> lock(s.mu);
  auto it = s.ptr.find(dev);
  if (it != s.ptr.end()) {
    *out = it->second;
    return hipSuccess;
  }
  void *p = nullptr;
  if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess)
    return e;
  hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, stream,
                     static_cast<uint32_t *>(p), int(kNoallocCounterBytes / 4));
  if ((e = hipGetLastError()) != hipSuccess)
    return e;
  s.ptr[dev] = static_cast<uint8_t *>(p);
  *out = static_cast<uint8_t *>(p);
  return hipSuccess;
}

}  // namespace

}  // namespace yuear

extern "C" int32_t yuear_op_attention_decode_noalloc(
    const uint16_t *qkv, const uint16_t *q_norm, const uint16_t *k_norm, float eps,
    const uint16_t *rope_cos, const uint16_t *rope_sin, uint16_t *k_cache, uint16_t *v_cache,
    const int32_t *pos, int32_t heads, int32_t kv_heads, int32_t capacity, int32_t batch,
    int32_t max_splits, uint16_t *out, void *stream) {
  using namespace yuear;
  if (batch < 1 || kv_heads < 1 || heads < kv_heads || heads % kv_heads || max_splits < 1 ||
      size_t(batch) * kv_heads > 512)
    return int32_t(hipErrorInvalidValue);
  const int G = heads / kv_heads;
  const size_t part_floats = size_t(batch) * kv_heads * max_splits * G * (128 + 2);
  if (kNoallocCounterBytes + part_floats * 4 > kNoallocBytes)
    return int32_t(hipErrorOutOfMemory);  // beyond the fixed scratch
  const hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t *base = nullptr;
  hipError_t e = noalloc_base(st, &base);
  if (e != hipSuccess)
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
  p.counters = reinterpret_cast<int32_t *>(base);
  p.part_o = reinterpret_cast<float *>(base + kNoallocCounterBytes);
  p.part_ml = p.part_o + size_t(batch) * kv_heads * max_splits * G * 128;
  p.out = out;
  p.out_stride = heads * 128;
  return int32_t(launch_attn_decode(p, st));
}
