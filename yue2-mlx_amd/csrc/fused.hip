// Fused decode-layer kernel for 1-2 branches: the QKV projection (input
// RMSNorm; the embedding gather in the first layer), the split-K attention
// (q/k RMSNorm, RoPE, KV append, merge) and the o_proj + residual of one
// layer in one launch on gfx950.
//
// Reference: native/src/ar.cpp:266-294 (input_layernorm, q/k/v projections,
// q_norm/k_norm, RoPE, cache update, SDPA, o_proj, residual).
//
// Why: as three kernels, attention cannot start streaming its K/V until the
// QKV kernel has drained, and o_proj cannot start streaming its weights until
// the attention's merge has finished; both waits are latency-bound (launch,
// first-load latency, the merge's counter round trip) while HBM idles. Here
// the grid is [QKV workgroups][attention workgroups][o_proj workgroups]:
// attention workgroups issue the first pass of their K/V and o_proj
// workgroups their whole weight slice before waiting for their inputs, so
// those streams run under the QKV projection and the attention chain.
//
// Inputs produced in the same launch travel as activation words (tag << 16 |
// bf16, gemv_core.h): the producer stores them with agent-scope write-through
// stores and moves on; the consumer re-reads them past the caches until every
// word carries this launch's tag. The tag comes from a step counter that the
// lm_head advances once per step, so a word left by an earlier step is never
// taken for a fresh one. Word buffers are per layer. The attention's split
// partials are tagged the same way (32-bit tags of step and layer, one buffer
// for all layers) and merged by the workgroup of split 0 without a counter
// (attn_block.h).
//
// Progress: workgroups are dispatched in index order on each XCD and every
// wait is on a lower-indexed workgroup, so a waiting workgroup never holds a
// slot that a producer it waits for still needs. Every wait is bounded in
// time (max_ticks of the 100 MHz clock); an expired wait sets the sticky
// error word and the workgroup proceeds, so the grid always drains and the
// host raises.
//
// The arithmetic is gemv_core.h and attn_block.h, the same functions as the
// per-op kernels: both paths produce the same bits.
#include <algorithm>
#include <cmath>

#include "attn_block.h"
#include "common.h"
#include "gemv_core.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int kAttnWaves = 4;

// Rows per wave of the two GEMV roles: two (one row per wave, the per-op
// choice at batch 1, measured 4% slower here: the launch's register budget,
// set by the attention role, limits residency, and more workgroups queue).
template <int B>
constexpr int fused_rows() { return 2; }

template <int B, int G, int KC>
__global__ __launch_bounds__(256) void fused_layer_kernel(FusedLayerParams fp) {
  extern __shared__ u32x4 xs[];  // [B][k / 8] GEMV activation chunks
  __shared__ float red[B][4];
  __shared__ AttnShared<G, kAttnWaves> sm;
  const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
  WordIO io;
  const uint32_t epoch = uint32_t(*fp.epoch);
  io.tag = (epoch % 65535u) + 1u;
  io.tag32 = 0x80000000u | ((epoch & 0x7fffffu) << 8) | (uint32_t(fp.layer) & 0xffu);
  io.part = fp.part;
  io.err = fp.err;
  io.max_ticks = fp.max_ticks;
  // trace stamps are kept in LDS until the end: a global store per stamp
  // would make later register reuse wait for its completion
  __shared__ unsigned long long lst[8];
  unsigned long long *tr = fp.trace ? fp.trace + size_t(blockIdx.x) * 16 : nullptr;
  io.ready = tr ? lst : nullptr;
  if (tr && threadIdx.x == 0)
    for (int i = 0; i < 8; ++i)
      lst[i] = 0;
  int blk = blockIdx.x, role;
  if (blk < fp.qkv_blocks) {
    role = 0;
    io.out = fp.qkv_words;
    io.out_stride = fp.q.y_stride;
    gemv_block<B, KC, fused_rows<B>(), kEpiStore, kGemvProduce>(fp.q, blk, xs, red, io);
  } else if ((blk -= fp.qkv_blocks) < fp.attn_blocks) {
    role = 1;
    const int splits = fp.a.max_splits, hkv = fp.a.kv_heads;
    io.in = fp.qkv_words;
    io.in_stride = fp.q.y_stride;
    io.out = fp.attn_words;
    io.out_stride = fp.o.x_stride;
    attn_block<G, kAttnWaves, true>(fp.a, fp.scale, blk % splits, (blk / splits) % hkv,
                                    blk / (splits * hkv), splits, sm, io);
  } else {
    role = 2;
    blk -= fp.attn_blocks;
    io.late_weights = fp.o_late != 0;
    io.in = fp.attn_words;
    io.in_stride = fp.o.x_stride;
    gemv_block<B, KC, fused_rows<B>(), kEpiResidual, kGemvConsume>(fp.o, blk, xs, red, io);
  }
  if (tr && threadIdx.x == 0) {
    uint32_t xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    tr[0] = t_start;
    tr[1] = lst[0];
    tr[2] = __builtin_amdgcn_s_memrealtime();
    for (int i = 1; i < 7; ++i)
      tr[i + 3] = lst[i];
    tr[3] = uint32_t(role) | ((xcc & 0xffu) << 8) | (static_cast<unsigned long long>(hw) << 32);
  }
}

template <int B, int G, int KC>
hipError_t launch_bgk(const FusedLayerParams &p, hipStream_t s) {
  const size_t lds = size_t(B) * (std::max(p.q.k, p.o.k) >> 3) * sizeof(u32x4);
  hipLaunchKernelGGL((fused_layer_kernel<B, G, KC>),
                     dim3(p.qkv_blocks + p.attn_blocks + p.o_blocks), dim3(256), lds, s, p);
  return hipGetLastError();
}

template <int B, int G>
hipError_t launch_bg(const FusedLayerParams &p, hipStream_t s) {
  switch ((p.q.k + 511) / 512) {
  case 1: return launch_bgk<B, G, 1>(p, s);
  case 4: return launch_bgk<B, G, 4>(p, s);
  case 6: return launch_bgk<B, G, 6>(p, s);
  }
  return hipErrorInvalidValue;
}

template <int B>
hipError_t launch_b(const FusedLayerParams &p, hipStream_t s) {
  switch (p.a.heads / p.a.kv_heads) {
  case 2: return launch_bg<B, 2>(p, s);
  case 3: return launch_bg<B, 3>(p, s);
  case 4: return launch_bg<B, 4>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool fused_layer_supported(int hidden, int heads, int kv_heads, int head_dim, int batch) {
  if (batch < 1 || batch > 2 || head_dim != attn::D || kv_heads < 1 || heads % kv_heads)
    return false;
  const int g = heads / kv_heads;
  if (g != 2 && g != 3 && g != 4)
    return false;
  const int kc = (hidden + 511) / 512, kco = (heads * head_dim + 511) / 512;
  return hidden % 8 == 0 && kc == kco && (kc == 1 || kc == 4 || kc == 6);
}

hipError_t launch_fused_layer(FusedLayerParams p, hipStream_t s) {
  if (!fused_layer_supported(p.q.k, p.a.heads, p.a.kv_heads, p.a.head_dim, p.q.batch) ||
      p.o.k != p.a.heads * p.a.head_dim || p.q.n % 8 || p.o.n % 8 || p.a.max_splits < 1 ||
      p.a.max_splits > kAttnMaxSplits || p.a.capacity % attn::kBlock || !p.epoch || !p.err ||
      !p.qkv_words || !p.attn_words || !p.part || p.o.batch != p.q.batch ||
      p.a.batch != p.q.batch)
    return hipErrorInvalidValue;
  const int rows = 4 * (p.q.batch == 1 ? fused_rows<1>() : fused_rows<2>());  // per workgroup
  p.qkv_blocks = p.q.n / rows;
  p.attn_blocks = p.a.max_splits * p.a.kv_heads * p.a.batch;
  p.o_blocks = p.o.n / rows;
  p.scale = float(std::pow(double(attn::D), -0.5));  // ar.cpp:283
  if (p.q.batch == 1) return launch_b<1>(p, s);
  return launch_b<2>(p, s);
}

}  // namespace yuear
