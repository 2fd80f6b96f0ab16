// Device sampler: CFG merge + distribution() + draw, one workgroup.
//
// Reference: native/src/sampling.cpp:38-134 (distribution, guided_logits,
// RequestRNG) and sampling.cpp:242-260 (loop body). One launch produces the
// next token entirely on the GPU, so the decode loop never waits on the host.
//
//  1. scores[i] = f32(logit) (bf16 when legacy_off), CFG-merged with the
//     reference's three bf16 rounding points, end row masked before
//     min_tokens; scores live in a global fp32 scratch (L2 resident).
//  2. windowed repetition penalty on the distinct local ids of the last
//     `penalty_window` emitted tokens, alpha = pow(p, count) from a host-built
//     table (the lookup form of vendor fast.py:123-136).
//  3. temperature 0: argmax (lowest index on ties).
//  4. otherwise: temperature; exact k-th largest threshold by a 3-pass radix
//     select on order-preserving keys (ties at the cut survive); ordered
//     compaction of the survivors; for top_p < 1 a bitonic sort by (value
//     desc, index asc), portable-exp softmax and the shifted-cumsum cut
//     evaluated sequentially in that order; Gumbel-max draw with Philox
//     uniforms u(seed, step, index).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int kT = 1024;        // threads
constexpr int kWaves = kT / 64;
constexpr int kSortLds = 4096;  // survivors sorted in LDS up to this count

struct Shared {
  union {
    struct {
      uint32_t key[kSortLds];
      uint32_t idx[kSortLds];
    } sort;
    uint32_t bits[2 * kSortLds];  // special-index bitmap (up to 262144 rows)
  } u;
  uint32_t hist[2048];
  int wave_tmp[kWaves];
  float wave_val[kWaves];
  int wave_idx[kWaves];
  int pen_loc[128];
  int bcast[4];
  int count;
  float prob[kSortLds];
  uint8_t keep[kSortLds];
};

__device__ __forceinline__ int local_of(int token, int phase, int vocab) {
  switch (phase) {  // sampling.cpp:19-32
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

__device__ __forceinline__ int native_of(int local, int phase) {
  switch (phase) {  // sampling.cpp:33-37
  case kPhaseAbc: return local < kEOD ? local : kAbcEnd;
  case kPhaseSemantic: return kMusicEnd + local;
  }
  return local;
}

// Inclusive block scan of one int per thread; returns inclusive prefix and
// writes the block total to *total.
__device__ int block_scan(int x, Shared &sh, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int v = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (lane == 63) sh.wave_tmp[wave] = v;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int t = sh.wave_tmp[w];
    if (w < wave) before += t;
    all += t;
  }
  __syncthreads();
  *total = all;
  return v + before;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Block argmax with the lowest index winning ties; result broadcast.
__device__ void block_argmax(float val, int idx, Shared &sh, float *out_val, int *out_idx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(val, o, 64);
    const int i2 = __shfl_xor(idx, o, 64);
    if (better(v2, i2, val, idx)) {
      val = v2;
      idx = i2;
    }
  }
  if (lane == 0) {
    sh.wave_val[wave] = val;
    sh.wave_idx[wave] = idx;
  }
  __syncthreads();
  float bv = sh.wave_val[0];
  int bi = sh.wave_idx[0];
  for (int w = 1; w < kWaves; ++w) {
    if (better(sh.wave_val[w], sh.wave_idx[w], bv, bi)) {
      bv = sh.wave_val[w];
      bi = sh.wave_idx[w];
    }
  }
  __syncthreads();
  *out_val = bv;
  *out_idx = bi;
}

// Ascending bitonic sort of (key, idx) pairs of power-of-two length (flat
// pointers: LDS or global).
__device__ void bitonic(uint32_t *key, uint32_t *idx, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n / 2; t += kT) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint32_t ka = key[lo], kb = key[hi], ia = idx[lo], ib = idx[hi];
        const bool greater = ka > kb || (ka == kb && ia > ib);
        if (greater == up) {
          key[lo] = kb;
          key[hi] = ka;
          idx[lo] = ib;
          idx[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
}

struct Ctx {
  const SamplerParams &p;
  bool legacy, cfg;
  float ninf;
  __device__ float cast(float v) const { return legacy ? rbf(v) : v; }
  // Score of the 8 logits of chunk c (sampling.cpp:44 and the CFG merge of
  // sampling.cpp:100-115), before penalty and temperature.
  __device__ void chunk(int c, float *out) const {
    const u32x4 a = reinterpret_cast<const u32x4 *>(p.logits)[c];
    const uint32_t av[4] = {a.x, a.y, a.z, a.w};
    if (!cfg) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        out[2 * q] = bflo(av[q]);
        out[2 * q + 1] = bfhi(av[q]);
      }
      return;
    }
    const u32x4 u = reinterpret_cast<const u32x4 *>(p.logits + p.ls)[c];
    const uint32_t uv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      out[2 * q] = guided(bflo(av[q]), bflo(uv[q]));
      out[2 * q + 1] = guided(bfhi(av[q]), bfhi(uv[q]));
    }
  }
  __device__ float one(int i) const {
    if (!cfg) return bf2f(p.logits[i]);
    return guided(bf2f(p.logits[i]), bf2f(p.logits[p.ls + i]));
  }
  __device__ float guided(float c, float u) const {
    const float delta = rbf(c - u);
    const float scaled = rbf(delta * p.cfg_scale);
    return rbf(u + scaled);
  }
  __device__ float temp(float v) const {
    return p.temperature != 0.f && p.temperature != 1.0f ? cast(v / p.temperature) : v;
  }
};

__device__ __forceinline__ bool special(const Shared &sh, int i) {
  return (sh.u.bits[i >> 5] >> (i & 31)) & 1u;
}

__global__ __launch_bounds__(kT) void sampler_kernel(SamplerParams p0) {
  __shared__ Shared sh;
  SamplerParams p = p0;
  if (p0.independent) {  // workgroup b: branch b on its own, as a 1-branch request
    const int b = blockIdx.x;
    p.logits += size_t(b) * p0.ls;
    p.branches = 1;
    p.state += 2 * b;
    p.history += size_t(b) * p0.history_stride;
    p.tokens_out += b;
    p.scratch += size_t(b) * p0.scratch_stride;
    p.scratch_u += size_t(b) * p0.scratch_u_stride;
    p.seed += uint64_t(b);
  }
  const int tid = threadIdx.x;
  const int n = p.n;
  if (p.state[1])
    return;  // the end token was already drawn
  const int step = p.state[0];
  const bool greedy = p.temperature == 0.f;
  const Ctx cx{p, p.legacy_off != 0, p.branches == 2 && p.cfg_scale != 1.0f, -__builtin_inff()};
  const float ninf = cx.ninf;
  const int end = p.phase == kPhaseAbc ? kEOD : p.phase == kPhaseSemantic ? 0 : -1;
  const bool end_masked = end >= 0 && end < n && step < p.min_tokens;  // sampling.cpp:47-50

  // Greedy without CFG: this thread's logit chunks are loaded first, so
  // their latency overlaps the special-row set-up below (kPre chunks per
  // thread cover 90112 logits in one round).
  constexpr int kPre = 11;
  const int n8 = n >> 3;
  const bool prefetch = greedy && !cx.cfg;
  u32x4 pre[kPre];
  if (prefetch) {
#pragma unroll
    for (int u = 0; u < kPre; ++u)
      pre[u] = reinterpret_cast<const u32x4 *>(p.logits)[min(tid + u * kT, max(n8 - 1, 0))];
  }

  // Special rows: the end row while masked and the distinct local ids of the
  // penalty window (sampling.cpp:51-75); everything else is a plain score.
  const int nw = (n + 31) >> 5;
  for (int i = tid; i < nw; i += kT)
    sh.u.bits[i] = 0;
  const int hlen = p.hist_len < 0 ? step : p.hist_len;
  const int wlen = p.alphas && p.penalty_window > 0 ? min(hlen, p.penalty_window) : 0;
  if (tid < wlen)
    sh.pen_loc[tid] = local_of(p.history[hlen - wlen + tid], p.phase, p.vocab);
  __syncthreads();
  int pen_count = 0;  // > 0: this thread owns a distinct penalised row
  if (tid < wlen) {
    const int loc = sh.pen_loc[tid];
    bool first = loc >= 0 && loc < n;
    for (int t = 0; t < wlen; ++t)
      if (sh.pen_loc[t] == loc) {
        ++pen_count;
        if (t < tid) first = false;
      }
    if (first)
      atomicOr(&sh.u.bits[loc >> 5], 1u << (loc & 31));
    else
      pen_count = 0;
  }
  if (tid == 0 && end_masked)
    atomicOr(&sh.u.bits[end >> 5], 1u << (end & 31));
  __syncthreads();
  // full score of a special row: mask, then penalty (a masked -inf stays -inf)
  auto special_score = [&](int loc, int count) {
    float v = cx.one(loc);
    if (loc == end && end_masked)
      v = ninf;
    if (count > 0) {
      const float a = p.alphas[count];
      v = v < 0.f ? cx.cast(v * a) : cx.cast(v / a);
    }
    return v;
  };

  int local = 0;
  if (greedy) {  // sampling.cpp:247: argmax, lowest index on ties
    // Scan of this thread's logits; with kCheck the special rows (an LDS
    // bitmap) are skipped. The special rows are few, so the first scan takes
    // every row's plain score without the per-element bitmap look-up: when
    // its winner is not special it is the best of the non-special rows, and
    // only the penalised rows (rescored below) can still beat it. A special
    // winner falls back to the checked scan.
    auto scan = [&](auto check_tag, float &bv, int &bi) {
      constexpr bool kCheck = decltype(check_tag)::value;
      bv = ninf;
      bi = 0x7fffffff;
      int c_from = tid;
      if (prefetch) {
#pragma unroll
        for (int u = 0; u < kPre; ++u) {
          const int c = tid + u * kT;
          if (c >= n8)
            break;
          const uint32_t w[4] = {pre[u].x, pre[u].y, pre[u].z, pre[u].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float v = e & 1 ? bfhi(w[e >> 1]) : bflo(w[e >> 1]);
            if ((!kCheck || !special(sh, 8 * c + e)) && better(v, 8 * c + e, bv, bi)) {
              bv = v;
              bi = 8 * c + e;
            }
          }
        }
        c_from = tid + kPre * kT;
      }
      for (int c0 = c_from; c0 < n8; c0 += 2 * kT) {
        float v[2][8];
        const int c1 = min(c0 + kT, n8 - 1);
        cx.chunk(c0, v[0]);
        cx.chunk(c1, v[1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h == 1 && c0 + kT >= n8) break;
          const int base = 8 * (h ? c1 : c0);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if ((!kCheck || !special(sh, base + e)) && better(v[h][e], base + e, bv, bi)) {
              bv = v[h][e];
              bi = base + e;
            }
        }
      }
      for (int i = 8 * n8 + tid; i < n; i += kT)
        if ((!kCheck || !special(sh, i)) && better(cx.one(i), i, bv, bi)) {
          bv = cx.one(i);
          bi = i;
        }
    };
    float bv, rv;
    int bi, raw;
    scan(std::integral_constant<bool, false>{}, bv, bi);
    block_argmax(bv, bi, sh, &rv, &raw);
    if (raw != 0x7fffffff && special(sh, raw)) {  // uniform: every thread holds raw
      scan(std::integral_constant<bool, true>{}, bv, bi);
    } else {
      bv = rv;
      bi = raw;
    }
    if (pen_count > 0) {
      const int loc = sh.pen_loc[tid];
      const float v = special_score(loc, pen_count);
      if (better(v, loc, bv, bi)) {
        bv = v;
        bi = loc;
      }
    }
    block_argmax(bv, bi, sh, &rv, &local);
    if (local == 0x7fffffff) local = 0;
  } else {
    float *sc = p.scratch;
    // 4a. scores with penalty and temperature (sampling.cpp:44-81)
    for (int c = tid; c < n8; c += kT) {
      float v[8];
      cx.chunk(c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = cx.temp(v[e]);
      reinterpret_cast<float4 *>(sc)[2 * c] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4 *>(sc)[2 * c + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    for (int i = 8 * n8 + tid; i < n; i += kT)
      sc[i] = cx.temp(cx.one(i));
    __syncthreads();
    if (pen_count > 0) {
      const int loc = sh.pen_loc[tid];
      sc[loc] = cx.temp(special_score(loc, pen_count));
    }
    if (tid == 0 && end_masked)
      sc[end] = ninf;
    __syncthreads();
    // 4b. k-th largest threshold (sampling.cpp:82-84): 3-pass radix select
    const int k = min(p.top_k, n);
    const int n4 = n >> 2;
    uint32_t thr_key = 0;
    if (k < n) {
      uint32_t prefix = 0, pmask = 0;
      int krem = k;
      const int shifts[3] = {21, 10, 0};
      const int widths[3] = {11, 11, 10};
      for (int pass = 0; pass < 3; ++pass) {
        const int shift = shifts[pass];
        const uint32_t dmask = (1u << widths[pass]) - 1u;
        for (int i = tid; i < 2048; i += kT)
          sh.hist[i] = 0;
        __syncthreads();
        for (int c = tid; c < n4; c += kT) {
          const float4 f = reinterpret_cast<const float4 *>(sc)[c];
          const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t key = order_key(fv[e]);
            if ((key & pmask) == prefix)
              atomicAdd(&sh.hist[(key >> shift) & dmask], 1u);
          }
        }
        for (int i = 4 * n4 + tid; i < n; i += kT) {
          const uint32_t key = order_key(sc[i]);
          if ((key & pmask) == prefix)
            atomicAdd(&sh.hist[(key >> shift) & dmask], 1u);
        }
        __syncthreads();
        // thread t owns bins 2t (low) and 2t+1 (high); count strictly above
        const int h0 = int(sh.hist[2 * tid]), h1 = int(sh.hist[2 * tid + 1]);
        int total;
        const int incl = block_scan(h0 + h1, sh, &total);
        const int above = total - incl;  // bins > 2t+1
        if (above < krem && krem <= above + h1) {
          sh.bcast[0] = 2 * tid + 1;
          sh.bcast[1] = krem - above;
        } else if (above + h1 < krem && krem <= above + h1 + h0) {
          sh.bcast[0] = 2 * tid;
          sh.bcast[1] = krem - above - h1;
        }
        __syncthreads();
        prefix |= uint32_t(sh.bcast[0]) << shift;
        pmask |= dmask << shift;
        krem = sh.bcast[1];
        __syncthreads();
      }
      thr_key = prefix;
    }
    // 4c. survivors (score >= threshold, ties kept), compacted in any order:
    // the nucleus sort and the draw's index tie-break restore determinism
    if (tid == 0) sh.count = 0;
    __syncthreads();
    uint32_t *surv = p.scratch_u;  // [n] survivor indices
    for (int c = tid; c < n4; c += kT) {
      const float4 f = reinterpret_cast<const float4 *>(sc)[c];
      const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (order_key(fv[e]) >= thr_key)
          surv[atomicAdd(&sh.count, 1)] = uint32_t(4 * c + e);
    }
    for (int i = 4 * n4 + tid; i < n; i += kT)
      if (order_key(sc[i]) >= thr_key)
        surv[atomicAdd(&sh.count, 1)] = uint32_t(i);
    __syncthreads();
    const int n_s = sh.count;

    float bv = ninf;
    int bi = 0x7fffffff;
    if (p.top_p >= 1.0f) {
      // 4e. draw over the survivors (Gumbel-max)
      for (int r = tid; r < n_s; r += kT) {
        const int i = int(surv[r]);
        const float v = sc[i];
        if (!(v > ninf)) continue;
        const float key = v + gumbel(draw_uniform(p.seed, step, i));
        if (better(key, i, bv, bi)) {
          bv = key;
          bi = i;
        }
      }
    } else {
      // 4d. nucleus over survivors sorted by (value desc, index asc)
      int P = 1;
      while (P < n_s) P <<= 1;
      const bool in_lds = P <= kSortLds;
      uint32_t *key = in_lds ? sh.u.sort.key : p.scratch_u + n;
      uint32_t *idx = in_lds ? sh.u.sort.idx : p.scratch_u + n + P;
      __syncthreads();  // the bitmap shares storage with the LDS sort arrays
      for (int r = tid; r < P; r += kT) {
        if (r < n_s) {
          const int i = int(surv[r]);
          key[r] = ~order_key(sc[i]);
          idx[r] = uint32_t(i);
        } else {
          key[r] = 0xffffffffu;
          idx[r] = 0x7fffffffu;
        }
      }
      __syncthreads();
      bitonic(key, idx, P);
      float *prob = in_lds ? sh.prob : reinterpret_cast<float *>(surv);
      uint8_t *keep = in_lds ? sh.keep : nullptr;
      const float m = sc[idx[0]];
      for (int r = tid; r < n_s; r += kT)
        prob[r] = m == ninf ? 0.f : portable_exp(sc[idx[r]] - m);
      __syncthreads();
      if (tid == 0) {
        float total = 0.f;  // sequential sum in sorted order
        for (int r = 0; r < n_s; ++r)
          total += prob[r];
        const int minimum = cx.legacy ? 3 : 1;
        float cum = 0.f;
        for (int r = 0; r < n_s; ++r) {
          const float pr = cx.legacy ? rbf(prob[r] / total) : prob[r] / total;
          cum = cx.cast(cum + pr);
          const float pre = cx.cast(cum - pr);
          const bool removed = pre > p.top_p && r >= minimum;
          if (keep)
            keep[r] = !removed;
          else
            prob[r] = removed ? 0.f : 1.f;
        }
      }
      __syncthreads();
      for (int r = tid; r < n_s; r += kT) {
        const bool kept = keep ? keep[r] != 0 : prob[r] != 0.f;
        if (!kept) continue;
        const int i = int(idx[r]);
        const float v = sc[i];
        if (!(v > ninf)) continue;
        const float gk = v + gumbel(draw_uniform(p.seed, step, i));
        if (better(gk, i, bv, bi)) {
          bv = gk;
          bi = i;
        }
      }
    }
    float rv;
    block_argmax(bv, bi, sh, &rv, &local);
    if (local == 0x7fffffff) local = 0;
  }

  if (tid == 0) {  // sampling.cpp:249-260
    const int native = native_of(local, p.phase);
    for (int b = 0; b < p.branches; ++b)
      p.tokens_out[b] = native;
    if (local == end)
      p.state[1] = 1;
    else if (step < p.max_tokens)
      p.history[step] = native;
    p.state[0] = step + 1;
  }
}

}  // namespace

hipError_t launch_sampler(const SamplerParams &p, hipStream_t s) {
  if (p.n < 1 || p.n > 64 * kSortLds || p.ls < p.n || p.ls % 8 || p.branches < 1 ||
      p.branches > 8 || p.penalty_window > 128 || !p.scratch || !p.scratch_u || !p.state ||
      !p.tokens_out ||
      (p.independent && (p.history_stride < p.max_tokens || p.scratch_stride < p.n ||
                         p.scratch_u_stride < p.n)))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(sampler_kernel, dim3(p.independent ? p.branches : 1), dim3(kT), 0, s, p);
  return hipGetLastError();
}

}  // namespace yuear
