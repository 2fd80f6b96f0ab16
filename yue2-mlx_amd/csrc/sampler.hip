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
#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int kT = 1024;        // threads
constexpr int kWaves = kT / 64;
constexpr int kSortLds = 4096;  // survivors sorted in LDS up to this count

struct Shared {
  uint32_t hist[2048];
  int wave_tmp[kWaves];
  float wave_val[kWaves];
  int wave_idx[kWaves];
  int pen_loc[128];
  int bcast[4];
  uint32_t sort_key[kSortLds];
  uint32_t sort_idx[kSortLds];
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

// Block argmax with the lowest index winning ties; result broadcast.
__device__ void block_argmax(float val, int idx, Shared &sh, float *out_val, int *out_idx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(val, o, 64);
    const int i2 = __shfl_xor(idx, o, 64);
    if (v2 > val || (v2 == val && i2 < idx)) {
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
    const float v2 = sh.wave_val[w];
    const int i2 = sh.wave_idx[w];
    if (v2 > bv || (v2 == bv && i2 < bi)) {
      bv = v2;
      bi = i2;
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

__global__ __launch_bounds__(kT) void sampler_kernel(SamplerParams p) {
  __shared__ Shared sh;
  const int tid = threadIdx.x;
  const int n = p.n;
  if (p.state[1])
    return;  // the end token was already drawn
  const int step = p.state[0];
  const bool greedy = p.temperature == 0.f;
  const bool legacy = p.legacy_off != 0;
  const float ninf = -__builtin_inff();
  const int end = p.phase == kPhaseAbc ? kEOD : p.phase == kPhaseSemantic ? 0 : -1;
  float *sc = p.scratch;
  auto cast = [&](float v) { return legacy ? rbf(v) : v; };

  // 1. scores (sampling.cpp:44-50, 100-115)
  const bool cfg = p.branches == 2 && p.cfg_scale != 1.0f;
  for (int i = tid; i < n; i += kT) {
    float s;
    if (cfg) {
      const float c = bf2f(p.logits[i]), u = bf2f(p.logits[n + i]);
      const float delta = rbf(c - u);
      const float scaled = rbf(delta * p.cfg_scale);
      s = rbf(u + scaled);
    } else {
      s = bf2f(p.logits[i]);
    }
    if (i == end && step < p.min_tokens)
      s = ninf;
    sc[i] = s;
  }
  __syncthreads();

  // 2. windowed repetition penalty (sampling.cpp:51-75)
  const int hlen = p.hist_len < 0 ? step : p.hist_len;
  if (p.alphas && p.penalty_window > 0 && hlen > 0) {
    const int wlen = min(hlen, p.penalty_window);
    if (tid < wlen)
      sh.pen_loc[tid] = local_of(p.history[hlen - wlen + tid], p.phase, p.vocab);
    __syncthreads();
    if (tid < wlen) {
      const int loc = sh.pen_loc[tid];
      bool first = loc >= 0 && loc < n;
      int count = 0;
      for (int t = 0; t < wlen; ++t) {
        if (sh.pen_loc[t] == loc) {
          ++count;
          if (t < tid) first = false;
        }
      }
      if (first) {
        const float a = p.alphas[count];
        const float v = sc[loc];
        sc[loc] = v < 0.f ? cast(v * a) : cast(v / a);
      }
    }
    __syncthreads();
  }

  int local = 0;
  if (greedy) {  // 3. argmax (sampling.cpp:247)
    float bv = ninf;
    int bi = 0x7fffffff;
    for (int i = tid; i < n; i += kT) {
      const float v = sc[i];
      if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
    float rv;
    block_argmax(bv, bi, sh, &rv, &local);
  } else {
    // 4a. temperature (sampling.cpp:78-81)
    if (p.temperature != 1.0f) {
      for (int i = tid; i < n; i += kT)
        sc[i] = cast(sc[i] / p.temperature);
      __syncthreads();
    }
    // 4b. k-th largest threshold (sampling.cpp:82-84)
    const int k = min(p.top_k, n);
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
        for (int i = tid; i < n; i += kT) {
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
    // 4c. ordered compaction of survivors (score >= threshold)
    const int per = (n + kT - 1) / kT;
    const int lo = min(n, tid * per), hi = min(n, lo + per);
    int cnt = 0;
    for (int i = lo; i < hi; ++i)
      cnt += order_key(sc[i]) >= thr_key;
    int n_s;
    const int incl = block_scan(cnt, sh, &n_s);
    uint32_t *surv = p.scratch_u;  // [n] survivor indices, index order
    {
      int o = incl - cnt;
      for (int i = lo; i < hi; ++i)
        if (order_key(sc[i]) >= thr_key)
          surv[o++] = uint32_t(i);
    }
    __syncthreads();

    float bv = ninf;
    int bi = 0x7fffffff;
    if (p.top_p >= 1.0f) {
      // 4e. draw over the survivors (Gumbel-max)
      for (int r = tid; r < n_s; r += kT) {
        const int i = int(surv[r]);
        const float v = sc[i];
        if (!(v > ninf)) continue;
        const float key = v + gumbel(draw_uniform(p.seed, step, i));
        if (key > bv || (key == bv && i < bi)) {
          bv = key;
          bi = i;
        }
      }
    } else {
      // 4d. nucleus over survivors sorted by (value desc, index asc)
      int P = 1;
      while (P < n_s) P <<= 1;
      const bool in_lds = P <= kSortLds;
      uint32_t *key = in_lds ? sh.sort_key : p.scratch_u + n;
      uint32_t *idx = in_lds ? sh.sort_idx : p.scratch_u + n + P;
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
        const int minimum = legacy ? 3 : 1;
        float cum = 0.f;
        for (int r = 0; r < n_s; ++r) {
          const float pr = legacy ? rbf(prob[r] / total) : prob[r] / total;
          cum = cast(cum + pr);
          const float pre = cast(cum - pr);
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
        if (gk > bv || (gk == bv && i < bi)) {
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
  if (p.n < 1 || p.branches < 1 || p.branches > 8 || p.penalty_window > 128 || !p.scratch ||
      !p.scratch_u || !p.state || !p.tokens_out)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(sampler_kernel, dim3(1), dim3(kT), 0, s, p);
  return hipGetLastError();
}

}  // namespace yuear
