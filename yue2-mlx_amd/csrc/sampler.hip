// Device sampler: CFG merge + distribution() + draw.
//
// Reference: native/src/sampling.cpp:38-134 (distribution, guided_logits,
// RequestRNG) and sampling.cpp:242-260 (loop body). One launch produces the
// next token entirely on the GPU, so the decode loop never waits on the host.
// Two forms with the same arithmetic: sampler_split_kernel (a shared draw
// over more than 8192 rows, greedy or top k up to 128: one workgroup per
// ~8192 rows, the last to arrive finishing) and sampler_kernel (one
// workgroup per request, or per sequence for batched sequences).
//
//  1. scores[i] = f32(logit) (bf16 when legacy_off), CFG-merged with the
//     reference's three bf16 rounding points, end row masked before
//     min_tokens (one workgroup: in a global fp32 scratch; split: as order
//     keys in each workgroup's LDS).
//  2. windowed repetition penalty on the distinct local ids of the last
//     `penalty_window` emitted tokens, alpha = pow(p, count) from a host-built
//     table (the lookup form of vendor fast.py:123-136).
//  3. temperature 0: argmax (lowest index on ties).
//  4. otherwise: temperature; exact k-th largest threshold by a radix select
//     on order-preserving keys (ties at the cut survive): the first digit
//     (13 bits) is counted while the scores are written and the rows at or
//     above its cut are gathered into LDS; up to 256 of them are ordered by
//     rank counting and the threshold read off that order, more go through
//     the other two digits (11, 8 bits); for top_p < 1 the survivors sorted
//     by (value desc, index asc) (rank counting, or a bitonic network beyond
//     256), portable-exp softmax and the shifted-cumsum cut evaluated
//     sequentially in that order (one wave stepping through lanes);
//     Gumbel-max draw with Philox uniforms u(seed, step, index).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int kT = 1024;        // threads
constexpr int kWaves = kT / 64;
constexpr int kSortLds = 4096;  // survivors sorted in LDS up to this count
// Radix digits of the order keys: the top 13 bits (counted while the scores
// are written), then 11, then 8; kBins covers the widest.
constexpr int kShift0 = 19, kShift1 = 8;
constexpr int kBins = 8192;
// Rows whose first digit is at or above the cut digit, held in LDS for the
// remaining digits when they fit (otherwise those passes read the scores).
constexpr int kList = 4096;
// Up to this many rows are ordered by rank counting instead of a network.
constexpr int kRankSort = 256;
// The split kernel samples top k up to this (greedy at any k), with at
// most kMaxGroups workgroups (rows up to 262144 in groups of 8192).
constexpr int kSplitMaxTopK = 128;
constexpr int kMaxGroups = 32;
static_assert(4 * kRankSort <= kT, "rank_sort counts with four threads per row");

// A row as one sortable word: ascending order is (score desc, index asc).
__device__ __forceinline__ uint64_t row_word(uint32_t key, uint32_t index) {
  return (uint64_t(~key) << 32) | index;
}

struct Shared {
  union {
    struct {
      uint32_t key[kSortLds];  // ~order key: ascending = score descending
      uint32_t idx[kSortLds];
    } sort;
    uint32_t bits[2 * kSortLds];  // special-index bitmap (up to 262144 rows)
  } u;
  union {
    uint64_t list[kList];  // row words of the rows gathered after the first digit
    uint32_t slice[2 * kList];  // order keys of a split workgroup's rows
  };
  union {
    uint32_t hist[kBins];
    uint64_t stage[kBins / 2];  // survivors' row words, once the digits are done
  };
  int wave_tmp[kWaves];
  float wave_val[kWaves];
  int wave_idx[kWaves];
  int pen_loc[128];
  int bcast[4];
  int count;
  int n_surv;
  int end_penalised;  // the masked end row is also a penalised row
  int is_last;        // split kernel: this workgroup arrived last
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

// The bin of sh.hist that holds the krem-th largest counted key (1-based,
// krem >= 1 and at most the number counted), the rank left inside that bin
// and the bin's count; every thread receives all three. One wave: lane l
// sums bins [128 l, 128 l + 128) (reading its 32 16-byte pieces in a
// lane-rotated order, so a wave's reads spread over the LDS banks), a
// suffix scan over lanes finds the 128-bin group, then the group's bins,
// two per lane, the bin. Callers separate consecutive calls by a barrier
// (the result goes through sh.bcast).
__device__ void find_cut(Shared &sh, int krem, int *bin, int *rem, int *in_bin) {
  static_assert(kBins == 64 * 128, "one wave, 128 bins per lane");
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const u32x4 *h4 = reinterpret_cast<const u32x4 *>(sh.hist);
    int s = 0;
#pragma unroll 8
    for (int j = 0; j < 32; ++j) {
      const u32x4 v = h4[lane * 32 + ((j + lane) & 31)];
      s += int(v.x + v.y + v.z + v.w);
    }
    int suf = s;  // keys in this lane's group and the groups above it
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_down(suf, o, 64);
      if (lane + o < 64) suf += t;
    }
    const uint64_t hit = __ballot(suf - s < krem && krem <= suf);
    const int g = hit ? __ffsll((unsigned long long)hit) - 1 : 0;  // one lane holds krem
    const int kg = krem - __builtin_amdgcn_readlane(suf - s, g);
    const int b0 = g * 128 + 2 * lane;
    const int c0 = int(sh.hist[b0]), c1 = int(sh.hist[b0 + 1]);
    int suf2 = c0 + c1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_down(suf2, o, 64);
      if (lane + o < 64) suf2 += t;
    }
    const int above = suf2 - c0 - c1;  // keys in the group's bins above b0 + 1
    if (lane == 0) {  // overwritten below by the lane holding the bin
      sh.bcast[0] = 0;
      sh.bcast[1] = 1;
      sh.bcast[2] = 0;
    }
    if (above < kg && kg <= above + c1) {
      sh.bcast[0] = b0 + 1;
      sh.bcast[1] = kg - above;
      sh.bcast[2] = c1;
    } else if (above + c1 < kg && kg <= above + c1 + c0) {
      sh.bcast[0] = b0;
      sh.bcast[1] = kg - above - c1;
      sh.bcast[2] = c0;
    }
  }
  __syncthreads();
  *bin = sh.bcast[0];
  *rem = sh.bcast[1];
  *in_bin = sh.bcast[2];
}

// Slot of this lane in a list grown by whole waves: the lanes whose `pred`
// holds take consecutive slots from *counter (one LDS atomic per wave);
// -1 for the others. Lanes of a wave may have left the loop around it.
__device__ __forceinline__ int wave_append(bool pred, int *counter) {
  const uint64_t m = __ballot(pred);
  if (m == 0)
    return -1;
  const int leader = __ffsll((unsigned long long)m) - 1;
  int base = 0;
  if ((threadIdx.x & 63) == leader)
    base = atomicAdd(counter, __popcll(m));
  base = __builtin_amdgcn_readlane(base, leader);
  const int below =
      __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u));
  return pred ? base + below : -1;
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Ascending sort of m <= kRankSort distinct row words by rank counting:
// four threads count the words below each one (LDS broadcast reads, no
// barriers between steps) and the word goes to that position of key/idx.
__device__ void rank_sort(const uint64_t *src, int m, uint32_t *key, uint32_t *idx) {
  const int e = threadIdx.x >> 2, q = threadIdx.x & 3;
  const uint64_t mine = e < m ? src[e] : 0;
  int below = 0;
  if (e < m) {
    int u = q;
    for (; u + 12 < m; u += 16)  // four independent reads in flight
      below += int(src[u] < mine) + int(src[u + 4] < mine) + int(src[u + 8] < mine) +
               int(src[u + 12] < mine);
    for (; u < m; u += 4)
      below += src[u] < mine;
  }
  below += __shfl_xor(below, 1, 64);
  below += __shfl_xor(below, 2, 64);
  if (e < m && q == 0) {
    key[below] = uint32_t(mine >> 32);
    idx[below] = uint32_t(mine);
  }
  __syncthreads();
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
    merge(a, cfg ? reinterpret_cast<const u32x4 *>(p.logits + p.ls)[c] : a, out);
  }
  // The same from the chunk's loaded words (u: the unconditional branch's).
  __device__ void merge(const u32x4 a, const u32x4 u, float *out) const {
    const uint32_t av[4] = {a.x, a.y, a.z, a.w};
    if (!cfg) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        out[2 * q] = bflo(av[q]);
        out[2 * q + 1] = bfhi(av[q]);
      }
      return;
    }
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

// Special rows among [lo, lo + span): the end row while masked and the
// distinct local ids of the penalty window (sampling.cpp:51-75), marked in
// the LDS bitmap at bit (row - lo). Returns, for the thread that holds the
// first occurrence of a penalised row in the window (sh.pen_loc[tid]), the
// row's count in the window, else 0. Also clears the histogram (when asked),
// the list counters and end_penalised.
__device__ __forceinline__ int mark_specials(const SamplerParams &p, Shared &sh, int step,
                                             int end, bool end_masked, int lo, int span,
                                             bool clear_hist) {
  const int tid = threadIdx.x;
  for (int i = tid; i < (span + 31) >> 5; i += kT)
    sh.u.bits[i] = 0;
  if (clear_hist)
    for (int i = tid; i < kBins; i += kT)
      sh.hist[i] = 0;
  if (tid == 0) {
    sh.count = 0;
    sh.n_surv = 0;
    sh.end_penalised = 0;
  }
  const int hlen = p.hist_len < 0 ? step : p.hist_len;
  const int wlen = p.alphas && p.penalty_window > 0 ? min(hlen, p.penalty_window) : 0;
  if (tid < wlen)
    sh.pen_loc[tid] = local_of(p.history[hlen - wlen + tid], p.phase, p.vocab);
  __syncthreads();
  int pen_count = 0;
  if (tid < wlen) {
    const int loc = sh.pen_loc[tid];
    bool first = loc >= 0 && loc < p.n;
    for (int t = 0; t < wlen; ++t)
      if (sh.pen_loc[t] == loc) {
        ++pen_count;
        if (t < tid) first = false;
      }
    if (!first)
      pen_count = 0;
    if (pen_count > 0 && loc >= lo && loc < lo + span)
      atomicOr(&sh.u.bits[(loc - lo) >> 5], 1u << ((loc - lo) & 31));
    if (pen_count > 0 && loc == end && end_masked)
      sh.end_penalised = 1;
  }
  if (tid == 0 && end_masked && end >= lo && end < lo + span)
    atomicOr(&sh.u.bits[(end - lo) >> 5], 1u << ((end - lo) & 31));
  __syncthreads();
  return pen_count;
}

// Full score of a special row: mask, then penalty (a masked -inf stays
// -inf); before temperature.
__device__ __forceinline__ float special_score(const SamplerParams &p, const Ctx &cx, int loc,
                                               int count, int end, bool end_masked) {
  float v = cx.one(loc);
  if (loc == end && end_masked)
    v = cx.ninf;
  if (count > 0) {
    // alpha in the scores' dtype (sampling.cpp:67-70): bf16 in legacy-off mode
    const float a = cx.cast(p.alphas[count]);
    v = v < 0.f ? cx.cast(v * a) : cx.cast(v / a);
  }
  return v;
}

// Survivors from rows held in sh.list[0, L): every row of the top k is
// there, `top` of the rows have their first digit at or above the cut
// (prefix under pmask) and the k-th largest score is the krem-th largest of
// that digit. Up to kRankSort such rows are ordered at once (the list
// itself when top == L, else gathered into sh.stage) and the survivors are
// the sorted prefix down to the k-th largest with its ties: returns true,
// survivors in key/idx. More rows go through the other two digits and the
// survivors are left unsorted in sh.stage: returns false. sh.n_surv holds the
// count after a barrier. sh.count must be 0.
__device__ __forceinline__ bool select_in_list(Shared &sh, int L, int top, int k,
                                               uint32_t prefix, uint32_t pmask, int krem) {
  const int tid = threadIdx.x;
  uint32_t *key = sh.u.sort.key, *idx = sh.u.sort.idx;
  if (top <= kRankSort) {
    const uint64_t *src = sh.list;
    if (top < L) {
      for (int i = tid; i < L; i += kT) {
        const uint64_t w = sh.list[i];
        const int slot = wave_append(~uint32_t(w >> 32) >= prefix, &sh.count);
        if (slot >= 0 && slot < kRankSort)
          sh.stage[slot] = w;
      }
      __syncthreads();
      src = sh.stage;
    }
    rank_sort(src, top, key, idx);
    const uint32_t cut = key[k - 1];
    for (int r = tid; r < top; r += kT)
      if (key[r] <= cut)
        atomicMax(&sh.n_surv, r + 1);
    return true;
  }
  for (int pass = 1; pass < 3; ++pass) {
    const int shift = pass == 1 ? kShift1 : 0;
    const uint32_t dmask = pass == 1 ? 0x7ffu : 0xffu;
    for (int i = tid; i < kBins; i += kT)
      sh.hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < L; i += kT) {
      const uint32_t key_i = ~uint32_t(sh.list[i] >> 32);
      if ((key_i & pmask) == prefix)
        atomicAdd(&sh.hist[(key_i >> shift) & dmask], 1u);
    }
    __syncthreads();
    int d, in_d;
    find_cut(sh, krem, &d, &krem, &in_d);
    prefix |= uint32_t(d) << shift;
    pmask |= dmask << shift;
  }
  // survivors (key >= prefix, ties at the cut kept), in any order: the
  // nucleus sort and the draw's index tie-break restore determinism
  for (int i = tid; i < L; i += kT) {
    const uint64_t w = sh.list[i];
    const int slot = wave_append(~uint32_t(w >> 32) >= prefix, &sh.n_surv);
    if (slot >= 0 && slot < kBins / 2)
      sh.stage[slot] = w;
  }
  return false;
}

// 4d/4e. The draw among the n_s survivors: sorted in the LDS key/idx
// arrays (sorted), unsorted in sh.stage (in_stage), or unsorted in
// surv = p.scratch_u with their scores in p.scratch.
__device__ __forceinline__ int draw_survivors(const SamplerParams &p, Shared &sh, const Ctx &cx,
                                              int step, int n_s, bool sorted, bool in_stage) {
  const int tid = threadIdx.x, n = p.n;
  const float ninf = cx.ninf;
  const float *sc = p.scratch;
  uint32_t *surv = p.scratch_u;
  uint32_t *key = sh.u.sort.key, *idx = sh.u.sort.idx;
  float bv = ninf;
  int bi = 0x7fffffff;
  if (p.top_p >= 1.0f) {
    // 4e. draw over the survivors (Gumbel-max)
    for (int r = tid; r < n_s; r += kT) {
      int i;
      float v;
      if (sorted) {
        i = int(idx[r]);
        v = key_value(~key[r]);
      } else if (in_stage) {
        const uint64_t w = sh.stage[r];
        i = int(uint32_t(w));
        v = key_value(~uint32_t(w >> 32));
      } else {
        i = int(surv[r]);
        v = sc[i];
      }
      if (!(v > ninf)) continue;
      const float gk = v + gumbel(draw_uniform(p.seed, step, i));
      if (better(gk, i, bv, bi)) {
        bv = gk;
        bi = i;
      }
    }
  } else {
    // 4d. nucleus over survivors sorted by (value desc, index asc)
    bool in_lds = true;
    if (!sorted && n_s <= kRankSort) {
      if (!in_stage) {
        for (int r = tid; r < n_s; r += kT) {
          const uint32_t i = surv[r];
          sh.stage[r] = row_word(order_key(sc[i]), i);
        }
        __syncthreads();
      }
      rank_sort(sh.stage, n_s, key, idx);
    } else if (!sorted) {
      int P = 1;
      while (P < n_s) P <<= 1;
      in_lds = P <= kSortLds;
      if (!in_lds) {
        key = p.scratch_u + n;
        idx = p.scratch_u + n + P;
      }
      for (int r = tid; r < P; r += kT) {
        if (r >= n_s) {
          key[r] = 0xffffffffu;
          idx[r] = 0x7fffffffu;
        } else if (in_stage) {
          const uint64_t w = sh.stage[r];
          key[r] = uint32_t(w >> 32);
          idx[r] = uint32_t(w);
        } else {
          const uint32_t i = surv[r];
          key[r] = ~order_key(sc[i]);
          idx[r] = i;
        }
      }
      __syncthreads();
      bitonic(key, idx, P);
    }
    float *prob = in_lds ? sh.prob : reinterpret_cast<float *>(surv);
    uint8_t *keep = in_lds ? sh.keep : nullptr;
    const float m = key_value(~key[0]);
    // the draw's Gumbel keys are formed here too, beside the exponentials
    // (in sh.slice, when the survivors fit); the wave that runs the
    // sequential sums below then takes the best kept key as it goes
    const bool keyed = n_s <= 2 * kList;
    for (int r = tid; r < n_s; r += kT) {
      const float v = key_value(~key[r]);
      prob[r] = m == ninf ? 0.f : portable_exp(v - m);
      if (keyed)
        sh.slice[r] =
            __builtin_bit_cast(uint32_t, v + gumbel(draw_uniform(p.seed, step, int(idx[r]))));
    }
    __syncthreads();
    // sequential sums in sorted order, on one wave: 64 values at a time
    // are loaded and divided in parallel and the running sums step through
    // them lane by lane. Zeros after the last survivor leave both sums as
    // they are.
    if (tid < 64) {
      const int lane = tid;
      float total = 0.f;
      for (int r0 = 0; r0 < n_s; r0 += 64) {
        const float pv = r0 + lane < n_s ? prob[r0 + lane] : 0.f;
#pragma unroll
        for (int j = 0; j < 64; ++j)
          total += lane_value(pv, j);
      }
      const int minimum = cx.legacy ? 3 : 1;
      float cum = 0.f;
      for (int r0 = 0; r0 < n_s; r0 += 64) {
        const int r = r0 + lane;
        const float pv = r < n_s ? prob[r] : 0.f;
        const float pr = cx.legacy ? rbf(pv / total) : pv / total;
        float cum_r = 0.f;
        if (cx.legacy) {  // uniform: the bf16 rounding stays out of the plain chain
#pragma unroll
          for (int j = 0; j < 64; ++j) {
            cum = rbf(cum + lane_value(pr, j));
            cum_r = lane == j ? cum : cum_r;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 64; ++j) {
            cum = cum + lane_value(pr, j);
            cum_r = lane == j ? cum : cum_r;
          }
        }
        if (r < n_s) {
          const float pre = cx.cast(cum_r - pr);
          const bool removed = pre > p.top_p && r >= minimum;
          if (keyed) {  // the draw on this wave: the best key of the kept rows
            const float v = key_value(~key[r]);
            const int i = int(idx[r]);
            const float gk = __builtin_bit_cast(float, sh.slice[r]);
            if (!removed && v > ninf && better(gk, i, bv, bi)) {
              bv = gk;
              bi = i;
            }
          } else if (keep) {
            keep[r] = !removed;
          } else {
            prob[r] = removed ? 0.f : 1.f;
          }
        }
      }
      if (keyed) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float v2 = __shfl_xor(bv, o, 64);
          const int i2 = __shfl_xor(bi, o, 64);
          if (better(v2, i2, bv, bi)) {
            bv = v2;
            bi = i2;
          }
        }
        if (lane == 0)
          sh.bcast[3] = bi;
      }
    }
    __syncthreads();
    if (keyed) {
      const int b = sh.bcast[3];
      return b == 0x7fffffff ? 0 : b;
    }
    for (int r = tid; r < n_s; r += kT) {
      const bool kept = keep ? keep[r] != 0 : prob[r] != 0.f;
      if (!kept) continue;
      const int i = int(idx[r]);
      const float v = key_value(~key[r]);
      if (!(v > ninf)) continue;
      const float gk = keyed ? __builtin_bit_cast(float, sh.slice[r])
                             : v + gumbel(draw_uniform(p.seed, step, i));
      if (better(gk, i, bv, bi)) {
        bv = gk;
        bi = i;
      }
    }
  }
  float rv;
  int local;
  block_argmax(bv, bi, sh, &rv, &local);
  return local == 0x7fffffff ? 0 : local;
}

// The whole draw by one workgroup (kGreedy: with the temperature-0 path).
template <bool kGreedy>
__device__ __forceinline__ int sample_block(const SamplerParams &p, Shared &sh, int step) {
  const int tid = threadIdx.x;
  const int n = p.n;
  const bool greedy = kGreedy && p.temperature == 0.f;
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
  // > 0: this thread owns a distinct penalised row; everything else is a
  // plain score
  const int pen_count = mark_specials(p, sh, step, end, end_masked, 0, n, !greedy);
  auto special_score = [&](int loc, int count) {
    return ::yuear::special_score(p, cx, loc, count, end, end_masked);
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
    uint32_t *surv = p.scratch_u;  // [n] survivor indices outside LDS
    const int k = min(p.top_k, n);
    const bool select = k < n;  // otherwise every row survives
    // 4a. scores with penalty and temperature (sampling.cpp:44-81), counted
    // by their first radix digit in the same pass (k-th largest below)
    constexpr int kU = 4;  // chunks in flight per thread
    for (int c0 = tid; c0 < n8; c0 += kU * kT) {
      float v[kU][8];
#pragma unroll
      for (int u = 0; u < kU; ++u)
        cx.chunk(min(c0 + u * kT, n8 - 1), v[u]);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = c0 + u * kT;
        if (c < n8) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            v[u][e] = cx.temp(v[u][e]);
            if (select)
              atomicAdd(&sh.hist[order_key(v[u][e]) >> kShift0], 1u);
          }
          reinterpret_cast<float4 *>(sc)[2 * c] =
              make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
          reinterpret_cast<float4 *>(sc)[2 * c + 1] =
              make_float4(v[u][4], v[u][5], v[u][6], v[u][7]);
        }
      }
    }
    for (int i = 8 * n8 + tid; i < n; i += kT) {
      const float v = cx.temp(cx.one(i));
      sc[i] = v;
      if (select)
        atomicAdd(&sh.hist[order_key(v) >> kShift0], 1u);
    }
    __syncthreads();
    // special rows: the final score replaces the plain one, in the scores
    // and in the count
    auto patch = [&](int loc, float s) {
      if (select) {
        atomicSub(&sh.hist[order_key(cx.temp(cx.one(loc))) >> kShift0], 1u);
        atomicAdd(&sh.hist[order_key(s) >> kShift0], 1u);
      }
      sc[loc] = s;
    };
    if (pen_count > 0) {
      const int loc = sh.pen_loc[tid];
      patch(loc, cx.temp(special_score(loc, pen_count)));
    }
    if (tid == 0 && end_masked && !sh.end_penalised)
      patch(end, ninf);
    __syncthreads();

    // 4b. k-th largest threshold (sampling.cpp:82-84) on order-preserving
    // keys. The rows at or above the cut first digit (all of the top k) are
    // gathered into LDS when they fit; up to kRankSort of them are ordered at
    // once and the k-th largest read off that order, more go through the
    // other two digits (11, 8 bits), and without room every pass reads the
    // scores instead.
    const int n4 = n >> 2;
    bool in_list = false;  // the rows at or above the cut first digit are in sh.list
    bool sorted = false;   // survivors sorted into the LDS key/idx arrays
    if (select) {
      int digit, krem, in_digit;
      find_cut(sh, k, &digit, &krem, &in_digit);
      uint32_t prefix = uint32_t(digit) << kShift0, pmask = ~0u << kShift0;
      const int L = k - krem + in_digit;  // rows above the cut digit, and in it
      in_list = L <= kList;
      if (in_list) {
        for (int c0 = tid; c0 < n4; c0 += kU * kT) {
          float4 f[kU];
#pragma unroll
          for (int u = 0; u < kU; ++u)
            f[u] = reinterpret_cast<const float4 *>(sc)[min(c0 + u * kT, n4 - 1)];
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            const int c = c0 + u * kT;
            const float fv[4] = {f[u].x, f[u].y, f[u].z, f[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t key_e = order_key(fv[e]);
              const int slot = wave_append(c < n4 && key_e >= prefix, &sh.count);
              if (slot >= 0 && slot < kList)
                sh.list[slot] = row_word(key_e, uint32_t(4 * c + e));
            }
          }
        }
        for (int i = 4 * n4 + tid; i < n; i += kT) {
          const uint32_t key_i = order_key(sc[i]);
          const int slot = wave_append(key_i >= prefix, &sh.count);
          if (slot >= 0 && slot < kList)
            sh.list[slot] = row_word(key_i, uint32_t(i));
        }
        __syncthreads();
        sorted = select_in_list(sh, L, L, k, prefix, pmask, krem);
      } else {
        for (int pass = 1; pass < 3; ++pass) {
          const int shift = pass == 1 ? kShift1 : 0;
          const uint32_t dmask = pass == 1 ? 0x7ffu : 0xffu;
          for (int i = tid; i < kBins; i += kT)
            sh.hist[i] = 0;
          __syncthreads();
          for (int c = tid; c < n4; c += kT) {
            const float4 f = reinterpret_cast<const float4 *>(sc)[c];
            const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t key_e = order_key(fv[e]);
              if ((key_e & pmask) == prefix)
                atomicAdd(&sh.hist[(key_e >> shift) & dmask], 1u);
            }
          }
          for (int i = 4 * n4 + tid; i < n; i += kT) {
            const uint32_t key_i = order_key(sc[i]);
            if ((key_i & pmask) == prefix)
              atomicAdd(&sh.hist[(key_i >> shift) & dmask], 1u);
          }
          __syncthreads();
          int d, in_d;
          find_cut(sh, krem, &d, &krem, &in_d);
          prefix |= uint32_t(d) << shift;
          pmask |= dmask << shift;
        }
        // 4c. survivors (key >= prefix, ties at the cut kept), in any order
        for (int c = tid; c < n4; c += kT) {
          const float4 f = reinterpret_cast<const float4 *>(sc)[c];
          const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (order_key(fv[e]) >= prefix)
              surv[atomicAdd(&sh.n_surv, 1)] = uint32_t(4 * c + e);
        }
        for (int i = 4 * n4 + tid; i < n; i += kT)
          if (order_key(sc[i]) >= prefix)
            surv[atomicAdd(&sh.n_surv, 1)] = uint32_t(i);
      }
    } else {  // every row survives
      for (int i = tid; i < n; i += kT)
        surv[i] = uint32_t(i);
      if (tid == 0)
        sh.n_surv = n;
    }
    __syncthreads();
    local = draw_survivors(p, sh, cx, step, sh.n_surv, sorted, in_list);
  }

  return local;
}

// The chosen local row becomes the next input token of every branch, the
// history entry and the step counter (sampling.cpp:249-260).
__device__ void emit_token(const SamplerParams &p, int local, int step) {
  if (threadIdx.x != 0)
    return;
  const int end = p.phase == kPhaseAbc ? kEOD : p.phase == kPhaseSemantic ? 0 : -1;
  const int native = native_of(local, p.phase);
  for (int b = 0; b < p.branches; ++b)
    p.tokens_out[b] = native;
  if (local == end)
    p.state[1] = 1;
  else if (step < p.max_tokens)
    p.history[step] = native;
  p.state[0] = step + 1;
}

// One workgroup per request (or per sequence with `independent`).
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
  if (p.state[1])
    return;  // the end token was already drawn
  const int step = p.state[0];
  emit_token(p, sample_block<true>(p, sh, step), step);
}

// One request over gridDim.x workgroups, workgroup w on rows
// [w * split_rows, (w + 1) * split_rows) (split_rows a multiple of 8, at
// most 2 * kList, so one 8-row chunk per thread):
//  - greedy: each wave's best (score, row) with the single-workgroup rules
//    (special rows skipped, penalised rows rescored);
//  - sampling: the scores' order keys in LDS, counted by first digit; the
//    rows at or above the digit of the workgroup's own k-th largest (a
//    superset of its share of the global top k, ties included) go to its
//    region of a global array of row words (p.scratch_u), their count to
//    p.scratch (as int).
// Results go out with write-through stores; after they complete each
// workgroup counts its arrival (device-scope counter p.sync[0]), and the
// last one reads them back past the per-XCD L2 (agent-scope loads), finishes
// the selection and the draw, emits the token and returns the counter to
// zero. A list longer than kList sends the last workgroup through the
// single-workgroup algorithm instead.
__global__ __launch_bounds__(kT) void sampler_split_kernel(SamplerParams p) {
  __shared__ Shared sh;
  if (p.state[1])
    return;  // the end token was already drawn (the same for every workgroup)
  const int step = p.state[0];
  const int tid = threadIdx.x, n = p.n, G = gridDim.x;
  const bool greedy = p.temperature == 0.f;
  const Ctx cx{p, p.legacy_off != 0, p.branches == 2 && p.cfg_scale != 1.0f, -__builtin_inff()};
  const float ninf = cx.ninf;
  const int end = p.phase == kPhaseAbc ? kEOD : p.phase == kPhaseSemantic ? 0 : -1;
  const bool end_masked = end >= 0 && end < n && step < p.min_tokens;  // sampling.cpp:47-50
  const int lo = int(blockIdx.x) * p.split_rows, hi = min(n, lo + p.split_rows);
  const int n8 = n >> 3;
  const int c_lo = lo >> 3, c_hi = min(hi >> 3, n8);  // whole 8-row chunks of the slice
  // this thread's chunk of logits (both branches) is loaded first, so its
  // latency overlaps the special-row set-up
  const int c = c_lo + int(tid);
  const int cc = min(c, max(n8 - 1, 0));
  const u32x4 la = reinterpret_cast<const u32x4 *>(p.logits)[cc];
  const u32x4 lu = cx.cfg ? reinterpret_cast<const u32x4 *>(p.logits + p.ls)[cc] : la;
  // greedy with no special row (no penalty window, end row not masked)
  // needs no set-up at all
  const int hlen = p.hist_len < 0 ? step : p.hist_len;
  const bool specials = end_masked || (p.alphas && p.penalty_window > 0 && hlen > 0);
  const int pen_count = greedy && !specials
                            ? 0
                            : mark_specials(p, sh, step, end, end_masked, lo, hi - lo, !greedy);
  auto penalised_here = [&](int &loc) {
    loc = pen_count > 0 ? sh.pen_loc[tid] : -1;
    return loc >= lo && loc < hi;
  };
  uint64_t *cand = reinterpret_cast<uint64_t *>(p.scratch_u);  // [n] candidate row words
  int32_t *counts = reinterpret_cast<int32_t *>(p.scratch);  // [G] candidates per workgroup
  int32_t *sync = p.sync;

  if (greedy) {  // sampling.cpp:247: argmax, lowest index on ties
    float bv = ninf;
    int bi = 0x7fffffff;
    if (c < c_hi) {
      float v[8];
      cx.merge(la, lu, v);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!(specials && special(sh, 8 * c + e - lo)) && better(v[e], 8 * c + e, bv, bi)) {
          bv = v[e];
          bi = 8 * c + e;
        }
    }
    for (int i = max(lo, 8 * n8) + tid; i < hi; i += kT)
      if (!(specials && special(sh, i - lo)) && better(cx.one(i), i, bv, bi)) {
        bv = cx.one(i);
        bi = i;
      }
    int loc;
    if (penalised_here(loc)) {
      const float v = special_score(p, cx, loc, pen_count, end, end_masked);
      if (better(v, loc, bv, bi)) {
        bv = v;
        bi = loc;
      }
    }
    // each wave's best goes out on its own (no workgroup barrier)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(bv, o, 64);
      const int i2 = __shfl_xor(bi, o, 64);
      if (better(v2, i2, bv, bi)) {
        bv = v2;
        bi = i2;
      }
    }
    if ((tid & 63) == 0) {
      const int slot = int(blockIdx.x) * kWaves + (tid >> 6);
      __hip_atomic_store(&p.scratch[slot], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&p.scratch_u[slot], uint32_t(bi), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    const int k = min(p.top_k, n);
    // 4a. scores of the slice (sampling.cpp:44-81) as order keys, counted by
    // their first digit
    if (c < c_hi) {
      float v[8];
      cx.merge(la, lu, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = order_key(cx.temp(v[e]));
        sh.slice[8 * c + e - lo] = key;
        atomicAdd(&sh.hist[key >> kShift0], 1u);
      }
    }
    for (int i = max(lo, 8 * n8) + tid; i < hi; i += kT) {
      const uint32_t key = order_key(cx.temp(cx.one(i)));
      sh.slice[i - lo] = key;
      atomicAdd(&sh.hist[key >> kShift0], 1u);
    }
    __syncthreads();
    // special rows of the slice: the final score replaces the plain one
    auto patch = [&](int loc, float s) {
      const uint32_t key = order_key(s);
      atomicSub(&sh.hist[sh.slice[loc - lo] >> kShift0], 1u);
      atomicAdd(&sh.hist[key >> kShift0], 1u);
      sh.slice[loc - lo] = key;
    };
    int loc;
    if (penalised_here(loc))
      patch(loc, cx.temp(special_score(p, cx, loc, pen_count, end, end_masked)));
    if (tid == 0 && end_masked && !sh.end_penalised && end >= lo && end < hi)
      patch(end, ninf);
    __syncthreads();
    // 4b, first part: the candidates of this slice, compacted in LDS and
    // written to the workgroup's own region cand[lo, lo + count); the count
    // goes out beside them (a count above kBins / 2 leaves the region empty:
    // the total then exceeds kList and the last workgroup takes the
    // single-workgroup path)
    int digit, krem, in_digit;
    const int kw = min(k, hi - lo);
    find_cut(sh, kw, &digit, &krem, &in_digit);
    const uint32_t prefix = uint32_t(digit) << kShift0;
    const int count = kw - krem + in_digit;
    if (count <= kBins / 2) {
      for (int r = tid; r < hi - lo; r += kT) {
        const uint32_t key = sh.slice[r];
        const int slot = wave_append(key >= prefix, &sh.count);
        if (slot >= 0 && slot < kBins / 2)
          sh.stage[slot] = row_word(key, uint32_t(lo + r));
      }
      __syncthreads();
      for (int j = tid; j < count; j += kT)
        __hip_atomic_store(&cand[lo + j], sh.stage[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0)
      __hip_atomic_store(&counts[blockIdx.x], count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- arrival: every wave waits for its write-through stores to complete
  // (a barrier alone does not wait for memory), then one count per
  // workgroup; the last one to arrive finishes ----
  wait_vmem();
  __syncthreads();
  if (tid == 0)
    sh.is_last = __hip_atomic_fetch_add(&sync[0], 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == G - 1;
  __syncthreads();
  if (!sh.is_last)
    return;

  int local = 0;
  if (greedy) {  // the waves' bests (at most kMaxGroups * kWaves) on wave 0
    if (tid < 64) {
      constexpr int kPer = kMaxGroups * kWaves / 64;
      const int total = G * kWaves;
      float vs[kPer];
      int is[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {  // one round of loads
        const int e = min(int(tid) + 64 * j, total - 1);
        vs[j] = __hip_atomic_load(&p.scratch[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is[j] = int(__hip_atomic_load(&p.scratch_u[e], __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT));
      }
      float bv = ninf;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (int(tid) + 64 * j < total && better(vs[j], is[j], bv, bi)) {
          bv = vs[j];
          bi = is[j];
        }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o, 64);
        const int i2 = __shfl_xor(bi, o, 64);
        if (better(v2, i2, bv, bi)) {
          bv = v2;
          bi = i2;
        }
      }
      local = bi == 0x7fffffff ? 0 : bi;
    }
  } else {
    const int k = min(p.top_k, n);
    // offsets of the workgroups' candidates in the gathered list (wave 0)
    if (tid < 64) {
      const int c = tid < G ? __hip_atomic_load(&counts[tid], __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0;
      int incl = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (tid >= o) incl += t;
      }
      if (tid < kMaxGroups)  // first list slot of workgroup tid (past the end: unused)
        sh.pen_loc[tid] = tid < G ? incl - c : 0x7fffffff;
      if (tid == 63)
        sh.bcast[3] = incl;
    }
    __syncthreads();
    const int C = sh.bcast[3];
    if (C <= kList) {
      // 4b, second part: every candidate into LDS, its first digit counted
      int first[kMaxGroups];
#pragma unroll
      for (int v = 0; v < kMaxGroups; ++v)
        first[v] = sh.pen_loc[v];
      for (int i = tid; i < C; i += kT) {
        int w = 0;  // the workgroup whose candidates hold list slot i
#pragma unroll
        for (int v = 1; v < kMaxGroups; ++v)
          w += first[v] <= i;
        int base = 0;
#pragma unroll
        for (int v = 0; v < kMaxGroups; ++v)
          base = v == w ? first[v] : base;
        sh.list[i] = __hip_atomic_load(&cand[w * p.split_rows + (i - base)], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
      }
      for (int i = tid; i < kBins; i += kT)
        sh.hist[i] = 0;
      if (tid == 0) {
        sh.count = 0;
        sh.n_surv = 0;
      }
      __syncthreads();
      for (int i = tid; i < C; i += kT)
        atomicAdd(&sh.hist[~uint32_t(sh.list[i] >> 32) >> kShift0], 1u);
      __syncthreads();
      int digit, krem, in_digit;
      find_cut(sh, k, &digit, &krem, &in_digit);
      const uint32_t prefix = uint32_t(digit) << kShift0;
      const bool sorted =
          select_in_list(sh, C, k - krem + in_digit, k, prefix, ~0u << kShift0, krem);
      __syncthreads();
      local = draw_survivors(p, sh, cx, step, sh.n_surv, sorted, true);
    } else {
      __syncthreads();
      local = sample_block<false>(p, sh, step);
    }
  }
  emit_token(p, local, step);
  if (tid == 0)
    __hip_atomic_store(&sync[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

static int sampler_split_rows(const SamplerParams &p) {
  // One 8-row chunk per thread in workgroups of about 8192 rows; greedy, or
  // a shared draw whose top k leaves the candidate list (about k plus the
  // cut digit's rows per workgroup) well inside LDS.
  const int k = std::min(p.top_k, p.n);
  if (p.independent || !p.sync || p.n <= 2 * kList ||
      !(p.temperature == 0.f || (k < p.n && k <= kSplitMaxTopK)))
    return 0;
  const int groups = (p.n + 2 * kList - 1) / (2 * kList);
  if (groups > kMaxGroups)
    return 0;
  return ((p.n + groups - 1) / groups + 7) / 8 * 8;
}

hipError_t launch_sampler(const SamplerParams &p, hipStream_t s) {
  if (p.n < 1 || p.n > 64 * kSortLds || p.ls < p.n || p.ls % 8 || p.branches < 1 ||
      p.branches > 8 || p.penalty_window > 128 || !p.scratch || !p.scratch_u || !p.state ||
      !p.tokens_out ||
      (p.independent && (p.history_stride < p.max_tokens || p.scratch_stride < p.n ||
                         p.scratch_u_stride < p.n)))
    return hipErrorInvalidValue;
  const int rows = sampler_split_rows(p);
  if (rows > 0) {
    SamplerParams q = p;
    q.split_rows = rows;
    hipLaunchKernelGGL(sampler_split_kernel, dim3((p.n + rows - 1) / rows), dim3(kT), 0, s, q);
  } else {
    hipLaunchKernelGGL(sampler_kernel, dim3(p.independent ? p.branches : 1), dim3(kT), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace yuear
