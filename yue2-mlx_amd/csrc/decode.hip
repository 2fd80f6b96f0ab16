// Persistent decode step: the whole AR decode step for one token (all layers
// and the lm_head) in one launch on gfx950.
//
// Reference: native/src/ar.cpp:246-323 (hidden(), project()) for one token.
// Every phase repeats the arithmetic of the per-op kernels (gemv.hip,
// attention.hip) operation for operation, so both decode paths produce the
// same bits.
//
// Why: with one kernel per op, every launch pays a ramp (workgroup dispatch,
// first-load latency) and a tail during which HBM idles, and the attention
// kernel is a chain of dependent memory round trips. Here the grid stays
// resident for the whole step and every wave issues the weight loads of its
// tasks of a phase BEFORE it waits for that phase's input, so the weight
// stream runs through the dependency waits.
//
// Structure. Grid: 2 co-resident 256-thread workgroups per CU (the host
// sizes it from the occupancy query), 2048 waves on 256 CUs, up to 256 VGPRs
// each. Per layer, six phases, each a task list spread over the grid:
//   QKV    wave tasks of 4 rows of the fused q|k|v weight, input RMSNorm
//          (layer 0 gathers the embedding row; workgroup 0 stores it as x_0)
//   ATTN   workgroup tasks (branch, kv head, key split): split-K attention
//          with the q/k RMSNorm + RoPE prologue and the KV append
//   MERGE  workgroup tasks (branch, q head): exact merge of the partials
//   O      wave tasks of 4 rows of o_proj, residual add
//   GU     wave tasks of one interleaved (gate, up) row pair, post-attention
//          RMSNorm, SwiGLU (four tasks per wave, two in flight)
//   DOWN   wave tasks of 2 rows of down_proj, residual add
// then LM: wave tasks of 2 rows of the phase-mapped lm_head, final RMSNorm,
// double-buffered over ~20 tasks per wave.
//
// Dependencies. A workgroup that finished its tasks of a phase adds their
// count to the phase's counter (8 slots on separate lines, summed by the
// reader); a phase waits until the producing phase's count is complete.
// Activations never need a store-completion wait or a cache flush: every
// activation is a 32-bit word (tag << 16) | payload, tag unique to the
// launch (from an epoch counter), written with agent-scope write-through
// stores. A reader loads words past the caches (sc1 buffer loads) and
// accepts them only with the current tag, re-reading stale words; a counter
// that arrives before the data it covers therefore costs a re-read, never a
// wrong value. Weights, gains, rope tables, the embedding and the KV cache
// of earlier positions are read-only in a launch (plain, cached loads); the
// KV append of this token and the logits are read by the next launch only.
//
// Termination. Every wait and re-read loop is bounded: after max_spins polls
// the waiter sets the sticky error word and proceeds, later waits give up at
// once when it is set, so the grid always drains and the host reports the
// error. All loads of activation words are buffer loads with a range: a word
// outside it reads as 0 (stale), never as a fault. The last workgroup to
// finish resets the counters, stores the epoch and advances pos.
#include <cmath>

#include "attn_core.h"
#include "common.h"
#include "decode.h"
#include "kernels.h"

namespace yuear {

namespace {

constexpr int D = 128;
constexpr int kMaxSplitsP = 64;

// Weight and gain pointers read from the layer table are generic to the
// compiler, which would emit flat loads; flat loads also count against the
// LDS counter, so every LDS wait would drain the weight stream too. They are
// used through global address space types instead.
#define GLB __attribute__((address_space(1)))

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ---- activation words ----
struct Ctx {
  uint32_t tag;      // 1..65535
  int32_t *err;      // sticky error word
  int max_spins;
};

__device__ __forceinline__ uint32_t word(uint32_t tag, uint32_t v16) { return (tag << 16) | v16; }
__device__ __forceinline__ bool fresh(uint32_t w, uint32_t tag) { return (w >> 16) == tag; }
__device__ __forceinline__ bool fresh4(u32x4 v, uint32_t tag) {
  return fresh(v.x, tag) & fresh(v.y, tag) & fresh(v.z, tag) & fresh(v.w, tag);
}

// Buffer resource over [base, base + bytes): loads outside read as 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
// Loads past the caches (sc1): a stale line can never be served or kept.
__device__ __forceinline__ u32x4 ld_w4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);
}
__device__ __forceinline__ u32x2 ld_w2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 16);
}
__device__ __forceinline__ uint32_t ld_w1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 16);
}
// Agent-scope write-through stores.
__device__ __forceinline__ void st_w1(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_w2(uint32_t *p, uint32_t lo, uint32_t hi) {
  __hip_atomic_store(reinterpret_cast<unsigned long long *>(p),
                     (static_cast<unsigned long long>(hi) << 32) | lo, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_w4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, 16);
}

// ---- sync ----
__device__ __forceinline__ int ld_ctr(const int32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_error(const Ctx &cx) {
  __hip_atomic_store(cx.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase trace stamp (thread 0; 100 MHz constant clock shared by all CUs).
__device__ __forceinline__ void stamp(unsigned long long *tr, int which) {
  if (tr && threadIdx.x == 0)
    __hip_atomic_store(tr + which, __builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of a phase's counter slots.
__device__ __forceinline__ int phase_count(const int32_t *ctr) {
  int v[kSlots];
#pragma unroll
  for (int i = 0; i < kSlots; ++i)
    v[i] = ld_ctr(ctr + i * kSlotStride);
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kSlots; ++i)
    sum += v[i];
  return sum;
}

// Bounded wait of the workgroup until the phase count reaches target.
__device__ void wg_wait(const int32_t *ctr, int target, const Ctx &cx) {
  if (threadIdx.x == 0) {
    int spins = 0;
    while (phase_count(ctr) < target) {
      if (ld_ctr(cx.err) != 0)
        break;
      if (++spins > cx.max_spins) {
        raise_error(cx);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

// The workgroup adds its finished task count (uniform call: a barrier, so
// every wave has issued its stores; their completion is not awaited).
__device__ __forceinline__ void wg_signal(int32_t *ctr, int done) {
  __syncthreads();
  if (threadIdx.x == 0 && done > 0)
    __hip_atomic_fetch_add(ctr + (blockIdx.x % kSlots) * kSlotStride, done, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup-uniform end of a re-read loop: true when every thread's words
// are fresh; gives up (error word) after max_spins rounds or when the error
// word is already set.
__device__ __forceinline__ bool wg_settled(bool ok, int spin, const Ctx &cx) {
  if (__syncthreads_and(ok))
    return true;
  const bool give = spin >= cx.max_spins || (threadIdx.x == 0 && ld_ctr(cx.err) != 0);
  if (__syncthreads_or(give)) {
    if (threadIdx.x == 0)
      raise_error(cx);
    return true;
  }
  __builtin_amdgcn_s_sleep(1);
  return false;
}
// Wave-uniform variant.
__device__ __forceinline__ bool wave_settled(bool ok, int spin, const Ctx &cx) {
  if (__all(ok))
    return true;
  if (__any(spin >= cx.max_spins || ld_ctr(cx.err) != 0)) {
    raise_error(cx);
    return true;
  }
  __builtin_amdgcn_s_sleep(1);
  return false;
}

// 8 activation words -> 8 packed bf16 (4 dwords).
__device__ __forceinline__ u32x4 pack8(u32x4 a, u32x4 b) {
  return u32x4{(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
               (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16)};
}

// LDS of one workgroup; the phases use it one at a time.
template <int B, int G, int KCMAX>
union Shared {
  u32x4 xs[B * KCMAX * 64];  // GEMV input rows, bf16 x 8 per chunk
  attn::Lds<G> at;            // attention phase
  struct {
    float o[kMaxSplitsP][D];  // partial outputs of one q head
    float m[kMaxSplitsP], w[kMaxSplitsP];
  } mg;
};

// Stage B input rows of K = KC * 512 values into LDS (xs[b * KC * 64 + c],
// 8 bf16 per chunk), then RMS-normalise them with `gain` when given
// (ar.cpp:30-35 with the rounding points and summation order of gemv.hip).
// Rows come from activation words at `in` (row stride in_stride words) or,
// with `embed`, from the embedding rows of p.tok; with write_x the gathered
// rows are also stored as words at x0.
template <int KC, int B, class SH>
__device__ void stage_input(SH &sh, float (*red)[4], const DecodeParams &p, const Ctx &cx,
                            const uint32_t *in, int in_stride, const uint16_t *gain,
                            const uint16_t *embed, uint32_t *x0, bool write_x) {
  constexpr int NCH = KC * 64;
  constexpr int XPT = (NCH + 255) / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (embed) {
    const auto xr = rsrc(x0, uint32_t(B) * NCH * 32);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const GLB u32x4 *row =
          (const GLB u32x4 *)embed + size_t(min(max(p.tok[b], 0), p.vocab - 1)) * NCH;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c < NCH) {
          const u32x4 v = row[c];
          sh.xs[b * NCH + c] = v;
          if (write_x) {
            const uint32_t off = uint32_t(b * NCH + c) * 32;
            st_w4(xr, off, u32x4{word(cx.tag, v.x & 0xffffu), word(cx.tag, v.x >> 16),
                                 word(cx.tag, v.y & 0xffffu), word(cx.tag, v.y >> 16)});
            st_w4(xr, off + 16, u32x4{word(cx.tag, v.z & 0xffffu), word(cx.tag, v.z >> 16),
                                      word(cx.tag, v.w & 0xffffu), word(cx.tag, v.w >> 16)});
          }
        }
      }
    }
  } else {
    // all-or-nothing rounds: stale words are rare, a round re-reads all
    const auto r = rsrc(in, uint32_t((B - 1) * in_stride + NCH * 8) * 4);
    for (int spin = 0;; ++spin) {
      bool ok = true;
#pragma unroll
      for (int b = 0; b < B; ++b)
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          if (c < NCH) {
            const uint32_t off = uint32_t(b * in_stride + c * 8) * 4;
            const u32x4 a = ld_w4(r, off), bb = ld_w4(r, off + 16);
            ok &= fresh4(a, cx.tag) & fresh4(bb, cx.tag);
            sh.xs[b * NCH + c] = pack8(a, bb);
          }
        }
      if (wg_settled(ok, spin, cx))
        break;
    }
  }
  if (gain) {
    __syncthreads();
    float ss[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      ss[b] = 0.f;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c < NCH) {
          const u32x4 v = sh.xs[b * NCH + c];
          const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float lo = bflo(w4[q]), hi = bfhi(w4[q]);
            ss[b] += lo * lo;
            ss[b] += hi * hi;
          }
        }
      }
      const float t = wave_sum(ss[b]);
      if (lane == 0)
        red[b][wave] = t;
    }
    __syncthreads();
    const GLB u32x4 *g4 = (const GLB u32x4 *)gain;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float total = (red[b][0] + red[b][1]) + (red[b][2] + red[b][3]);
      const float scale = rbf(1.0f / __builtin_sqrtf(total / float(KC * 512) + p.eps));
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c < NCH) {
          const u32x4 v = sh.xs[b * NCH + c], g = g4[c];
          const uint32_t vi[4] = {v.x, v.y, v.z, v.w}, gi[4] = {g.x, g.y, g.z, g.w};
          uint32_t o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t lo = f2bf(rbf(bflo(vi[q]) * scale) * bflo(gi[q]));
            const uint32_t hi = f2bf(rbf(bfhi(vi[q]) * scale) * bfhi(gi[q]));
            o[q] = lo | (hi << 16);
          }
          sh.xs[b * NCH + c] = u32x4{o[0], o[1], o[2], o[3]};
        }
      }
    }
  }
  __syncthreads();
}

struct RowMap {
  int seg0_start, seg0_len, seg1_start;
  bool mapped;
};

// Issue the weight loads of R rows starting at row0 (non-temporal: read once).
template <int R, int KC>
__device__ __forceinline__ void load_rows(const GLB uint16_t *w, int row0, int nrows, RowMap m,
                                          int lane, u32x4 (&wv)[R][KC]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int row = min(row0 + r, nrows - 1);  // a ragged last task re-reads a valid row
    if (m.mapped)
      row = row < m.seg0_len ? m.seg0_start + row : m.seg1_start + (row - m.seg0_len);
    const GLB u32x4 *wrow = (const GLB u32x4 *)w + size_t(row) * (KC * 64);
#pragma unroll
    for (int j = 0; j < KC; ++j)
      wv[r][j] = __builtin_nontemporal_load(wrow + j * 64 + lane);
  }
}

// Residual words of rows [task * R, task * R + R) (issued early; checked at use).
template <int B, int R>
__device__ __forceinline__ void load_resid(__amdgpu_buffer_rsrc_t r, int stride, int task,
                                           int nrows, uint32_t (&rw)[B][R]) {
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int q = 0; q < R; ++q)
      rw[b][q] = ld_w1(r, uint32_t(b * stride + min(task * R + q, nrows - 1)) * 4);
}

// Rows [task * R, task * R + R) against the staged inputs, then the epilogue
// (gemv.hip's operation order: dot8 over j, butterfly sum, lane-0 store).
// Outputs are activation words, or plain bf16 for the logits.
template <int B, int KC, int R, int EPI, bool LOGITS>
__device__ __forceinline__ void row_task(const u32x4 *xs, const u32x4 (&wv)[R][KC], int task,
                                         int nrows, __amdgpu_buffer_rsrc_t rr,
                                         uint32_t (&rw)[B][R], void *out, int out_stride,
                                         int lane, const Ctx &cx) {
  float acc[B][R];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[b][r] = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const u32x4 xv = xs[b * (KC * 64) + j * 64 + lane];
#pragma unroll
      for (int r = 0; r < R; ++r)
        acc[b][r] = dot8(wv[r][j], xv, acc[b][r]);
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[b][r] = wave_sum(acc[b][r]);
  if constexpr (EPI == kEpiResidual) {
    for (int spin = 0;; ++spin) {  // residual words: their producer phase has completed
      bool ok = true;
#pragma unroll
      for (int b = 0; b < B; ++b)
#pragma unroll
        for (int r = 0; r < R; ++r)
          ok &= fresh(rw[b][r], cx.tag);
      if (wave_settled(ok, spin, cx))
        break;
      load_resid<B, R>(rr, out_stride, task, nrows, rw);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if constexpr (LOGITS) {
        uint16_t *yb = static_cast<uint16_t *>(out) + size_t(b) * out_stride;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (task * R + r < nrows)
            yb[task * R + r] = f2bf(acc[b][r]);
      } else {
        uint32_t *yb = static_cast<uint32_t *>(out) + size_t(b) * out_stride;
        if constexpr (EPI == kEpiSwiGLU) {
          uint32_t v[R / 2];
#pragma unroll
          for (int r = 0; r < R; r += 2) {
            const float g = rbf(acc[b][r]), u = rbf(acc[b][r + 1]);
            const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
            v[r / 2] = word(cx.tag, f2bf(act * u));
          }
          if constexpr (R == 4)
            st_w2(yb + task * 2, v[0], v[1]);
          else
            st_w1(yb + task, v[0]);
        } else {
          uint32_t v[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float y = acc[b][r];
            if constexpr (EPI == kEpiResidual)
              y = bf2f(uint16_t(rw[b][r])) + rbf(y);
            v[r] = word(cx.tag, f2bf(y));
          }
          // activation rows are never ragged (row counts are multiples of R)
#pragma unroll
          for (int r = 0; r < R; r += 2)
            st_w2(yb + task * R + r, v[r], v[r + 1]);
        }
      }
    }
  }
}

// GEMV phase over rows [0, nrows) in wave tasks of R rows; task t belongs to
// global wave t mod NW (NW = 4 * gridDim.x). Before the dependency wait a
// wave issues the weights of its first task (DOUBLE: of its first two);
// afterwards task t + NW (DOUBLE: t + 2 NW) is issued before task t is
// computed. A prefetch past the last task re-reads the wave's own rows.
template <int B, int KC, int R, int EPI, bool DOUBLE, bool LOGITS, class SH>
__device__ void gemv_phase(SH &sh, float (*red)[4], const DecodeParams &p, const Ctx &cx,
                           const uint16_t *wgen, int nrows, RowMap map, const int32_t *wait_ctr,
                           int wait_target, const uint32_t *in, int in_stride,
                           const uint16_t *gain, const uint16_t *embed, bool write_x,
                           const uint32_t *res, void *out, int out_stride, int32_t *signal,
                           unsigned long long *tr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NW = gridDim.x * 4;
  const int ntasks = (nrows + R - 1) / R;  // the SwiGLU phase has an even row count
  if (int(blockIdx.x) * 4 >= ntasks && !write_x)
    return;  // no task in this workgroup (uniform)
  int task = blockIdx.x * 4 + wave;
  const GLB uint16_t *w = (const GLB uint16_t *)wgen;
  u32x4 wa[R][KC], wb[DOUBLE ? R : 1][DOUBLE ? KC : 1];
  const auto next = [&](int t) { return t < ntasks ? t : task; };
  load_rows<R, KC>(w, min(task, ntasks - 1) * R, nrows, map, lane, wa);
  if constexpr (DOUBLE)
    load_rows<R, KC>(w, min(next(task + NW), ntasks - 1) * R, nrows, map, lane, wb);
  if (wait_ctr)
    wg_wait(wait_ctr, wait_target, cx);
  stamp(tr, 0);
  const auto rr = rsrc(res, EPI == kEpiResidual ? uint32_t((B - 1) * out_stride + nrows) * 4 : 0);
  uint32_t rw[B][R];
  if constexpr (EPI == kEpiResidual)
    load_resid<B, R>(rr, out_stride, min(task, ntasks - 1), nrows, rw);
  stage_input<KC, B>(sh, red, p, cx, in, in_stride, gain, embed, p.xs, write_x);
  if (task < ntasks) {
    for (;;) {
      row_task<B, KC, R, EPI, LOGITS>(sh.xs, wa, task, nrows, rr, rw, out, out_stride, lane, cx);
      task += NW;
      if (task >= ntasks)
        break;
      if constexpr (EPI == kEpiResidual)
        load_resid<B, R>(rr, out_stride, task, nrows, rw);
      if constexpr (DOUBLE) {
        load_rows<R, KC>(w, next(task + NW) * R, nrows, map, lane, wa);
        row_task<B, KC, R, EPI, LOGITS>(sh.xs, wb, task, nrows, rr, rw, out, out_stride, lane,
                                        cx);
        task += NW;
        if (task >= ntasks)
          break;
        if constexpr (EPI == kEpiResidual)
          load_resid<B, R>(rr, out_stride, task, nrows, rw);
        load_rows<R, KC>(w, next(task + NW) * R, nrows, map, lane, wb);
      } else {
        load_rows<R, KC>(w, task * R, nrows, map, lane, wa);
      }
    }
  }
  if (signal) {
    // tasks of this workgroup's 4 waves: wave gw owns tasks gw, gw + NW, ...
    int wg_tasks = 0;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int gw = blockIdx.x * 4 + v;
      wg_tasks += gw < ntasks ? (ntasks - gw + NW - 1) / NW : 0;
    }
    wg_signal(signal, wg_tasks);  // its barrier also frees the staged input
  } else {
    __syncthreads();  // the staged input is overwritten by the next phase
  }
  stamp(tr, 1);
}

// Split-K attention phase of layer l: workgroup tasks (b, kv head, split)
// on the shared core (attn_core.h). The split's first K/V pass is issued
// before the dependency wait; q/k/v come from activation words. Partials are
// fp32 values stored as two activation words (high half, low half).
template <int B, int G, class SH>
__device__ void attn_phase(SH &sh, const DecodeParams &p, const Ctx &cx, int l,
                           const DecodeLayer &Lw, const uint32_t *qkv, uint32_t *part_o,
                           uint32_t *part_ml, const int32_t *wait_ctr, int wait_target,
                           int32_t *signal, unsigned long long *tr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int Hkv = p.Hkv, S = p.max_splits;
  const int ntasks = B * Hkv * S;
  const float qscale = p.attn_scale * attn::kLog2e;
  const auto qr = rsrc(qkv, uint32_t(B * p.qkv_stride) * 4);
  bool waited = false;
  int done = 0;
  for (int task = blockIdx.x; task < ntasks; task += gridDim.x) {
    const int s = task % S, kvh = (task / S) % Hkv, b = task / (S * Hkv);
    const int pos = p.pos[b];
    const bool valid = pos >= 0 && pos < p.cap;
    const int L = pos + 1;
    const int per = (L + S - 1) / S;
    const int chunk = (per + attn::kBlock - 1) & ~(attn::kBlock - 1);
    const int s0 = s * chunk, s1 = min(L, s0 + chunk);
    const bool active = valid && s0 < s1;
    const size_t head_base = ((size_t(l) * B + b) * Hkv + kvh) * p.cap;
    const u32x4 *kc = reinterpret_cast<const u32x4 *>(p.kc) + head_base * (D / 8);
    const u32x4 *vc = reinterpret_cast<const u32x4 *>(p.vc) + head_base * (D / 8);
    const int last_cached = active && pos > 0 ? pos - 1 : 0;
    u32x4 kr[8], vr[8];  // first pass: cached keys only, no dependency
    attn::load_k(kc, s0, wave, lane, last_cached, kr);
    attn::load_v(vc, s0, wave, lane, last_cached, vr);
    if (!waited) {
      wg_wait(wait_ctr, wait_target, cx);
      waited = true;
      stamp(tr, 0);
    }
    if (active) {
      const uint32_t row = uint32_t(b) * p.qkv_stride;
      const uint16_t *cs = p.rope_cos + size_t(pos) * (D / 2);
      const uint16_t *sn = p.rope_sin + size_t(pos) * (D / 2);
      for (int h = wave; h < G + 2; h += 4) {
        const uint32_t col = h < G ? uint32_t(kvh * G + h) * D
                                   : uint32_t(p.Hq + (h - G) * Hkv + kvh) * D;
        u32x2 pr{};
        for (int spin = 0;; ++spin) {
          pr = ld_w2(qr, (row + col + 2 * lane) * 4);
          if (wave_settled(fresh(pr.x, cx.tag) & fresh(pr.y, cx.tag), spin, cx))
            break;
        }
        const GLB uint16_t *gain = (const GLB uint16_t *)(h < G ? Lw.q_norm : Lw.k_norm);
        NormRope nr;
        load_rope(nr, cs, sn, lane);
        if (gain)
          load_gain(nr, gain, lane);
        attn::prologue_head<G>(sh.at, h, (pr.x & 0xffffu) | (pr.y << 16), gain != nullptr,
                               p.eps, nr, lane);
      }
      __syncthreads();
      if (pos >= s0 && pos < s1 && threadIdx.x < D / 8 + D) {  // append (ar.cpp:119-123)
        if (threadIdx.x < D / 8) {
          reinterpret_cast<u32x4 *>(p.kc)[(head_base + pos) * (D / 8) + threadIdx.x] =
              sh.at.kv_new[0][threadIdx.x];
        } else {
          const int d = threadIdx.x - D / 8;
          p.vc[head_base * D + attn::v_index(pos, d)] =
              reinterpret_cast<const uint16_t *>(&sh.at.kv_new[1][0])[d];
        }
      }
      attn::split<G>(sh.at, kc, vc, s0, s1, pos, last_cached, lane, wave, qscale, kr, vr);
      __syncthreads();
      const size_t part = (size_t(b) * Hkv + kvh) * S + s;
      for (int e = threadIdx.x; e < G * D; e += 256) {
        float o, M, lsum;
        attn::combine<G>(sh.at, e, o, M, lsum);
        const uint32_t ob = __builtin_bit_cast(uint32_t, o);
        st_w2(part_o + (part * (G * D) + e) * 2, word(cx.tag, ob >> 16),
              word(cx.tag, ob & 0xffffu));
        if (e % D == 0) {
          const int h = e / D;
          const uint32_t mb = __builtin_bit_cast(uint32_t, M);
          const uint32_t lb = __builtin_bit_cast(uint32_t, lsum);
          st_w2(part_ml + (part * G + h) * 4, word(cx.tag, mb >> 16), word(cx.tag, mb & 0xffffu));
          st_w2(part_ml + (part * G + h) * 4 + 2, word(cx.tag, lb >> 16),
                word(cx.tag, lb & 0xffffu));
        }
      }
    }
    ++done;
    __syncthreads();  // this task's LDS use ends before the next task's begins
  }
  if (int(blockIdx.x) < ntasks) {
    wg_signal(signal, done);
    stamp(tr, 1);
  }
}

// Two activation words (high half, low half) -> fp32.
__device__ __forceinline__ float join(uint32_t hi, uint32_t lo) {
  return __builtin_bit_cast(float, (hi << 16) | (lo & 0xffffu));
}

// Merge phase: workgroup tasks (b, q head); the merge arithmetic of
// attention.hip's last-arriving workgroup (merge_weight, then a sequential
// sum over splits per output), one head per task.
template <int B, int G, class SH>
__device__ void merge_phase(SH &sh, const DecodeParams &p, const Ctx &cx,
                            const uint32_t *part_o, const uint32_t *part_ml, uint32_t *attn,
                            const int32_t *wait_ctr, int wait_target, int32_t *signal,
                            unsigned long long *tr) {
  const int Hkv = p.Hkv, S = p.max_splits;
  const int ntasks = B * p.Hq;
  const auto ro = rsrc(part_o, uint32_t(B * Hkv * S * G * D) * 8);
  const auto rm = rsrc(part_ml, uint32_t(B * Hkv * S * G) * 16);
  bool waited = false;
  int done = 0;
  for (int task = blockIdx.x; task < ntasks; task += gridDim.x) {
    const int b = task / p.Hq, head = task % p.Hq;
    const int kvh = head / G, h = head % G;
    const int pos = p.pos[b];
    const bool valid = pos >= 0 && pos < p.cap;
    const int L = pos + 1;
    const int per = (L + S - 1) / S;
    const int chunk = (per + attn::kBlock - 1) & ~(attn::kBlock - 1);
    const int n_active = valid ? min(max((L + chunk - 1) / chunk, 1), S) : 1;
    const size_t part0 = (size_t(b) * Hkv + kvh) * S;
    if (!waited) {
      wg_wait(wait_ctr, wait_target, cx);
      waited = true;
      stamp(tr, 0);
    }
    if (valid) {
      // partial o words of this head: split t, dims 2c, 2c + 1 in one 16-byte
      // load; thread x takes split x / 64 + 4 i, chunk x % 64
      const int c = threadIdx.x & 63, t_off = threadIdx.x >> 6;
      for (int half = 0; half < 2; ++half) {  // all-or-nothing rounds per half
        for (int spin = 0;; ++spin) {
          bool ok = true;
#pragma unroll
          for (int i = 0; i < kMaxSplitsP / 8; ++i) {
            const int t = t_off + 4 * (i + half * (kMaxSplitsP / 8));
            if (t < n_active) {
              const u32x4 v = ld_w4(ro, uint32_t(((part0 + t) * G + h) * D + 2 * c) * 8);
              ok &= fresh4(v, cx.tag);
              sh.mg.o[t][2 * c] = join(v.x, v.y);
              sh.mg.o[t][2 * c + 1] = join(v.z, v.w);
            }
          }
          if (half == 0 && int(threadIdx.x) < n_active) {
            const int t = threadIdx.x;
            const u32x4 v = ld_w4(rm, uint32_t((part0 + t) * G + h) * 16);
            ok &= fresh4(v, cx.tag);
            sh.mg.m[t] = join(v.x, v.y);
            sh.mg.w[t] = join(v.z, v.w);  // l; made a weight below
          }
          if (wg_settled(ok, spin, cx))
            break;
        }
      }
      if (threadIdx.x < 64) {  // wave 0, lane t: merge weight of split t
        const int t = threadIdx.x;
        const bool act = t < n_active;
        const float w = merge_weight(act ? sh.mg.m[t] : 0.f, act ? sh.mg.w[t] : 0.f, act);
        if (act)
          sh.mg.w[t] = w;
      }
      __syncthreads();
      if (threadIdx.x < D) {
        const int d = threadIdx.x;
        float acc = 0.f;
        for (int t = 0; t < n_active; ++t)
          acc = fmaf(sh.mg.w[t], sh.mg.o[t][d], acc);
        st_w1(attn + size_t(b) * p.Hq * D + size_t(head) * D + d, word(cx.tag, f2bf(acc)));
      }
    }
    ++done;
    __syncthreads();  // this task's LDS use ends before the next task's begins
  }
  if (int(blockIdx.x) < ntasks) {
    wg_signal(signal, done);
    stamp(tr, 1);
  }
}

template <int B, int G, int KCH, int KCF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void decode_step_kernel(
    DecodeParams p) {
  __shared__ Shared<B, G, (KCF > KCH ? KCF : KCH)> sh;
  __shared__ float red[B][4];
  __shared__ int last;
  constexpr int H = KCH * 512, F = KCF * 512;
  const uint32_t epoch = uint32_t(ld_ctr(p.sync + kSyncEpoch)) + 1u;
  const Ctx cx{epoch % 65535u + 1u, p.sync + kSyncError, p.max_spins};
  const int qkv_rows = (p.Hq + 2 * p.Hkv) * D;
  const int n_attn = B * p.Hkv * p.max_splits;
  const size_t part_len = size_t(B) * p.Hkv * p.max_splits * G;
  const RowMap plain{0, 1 << 30, 0, false};
  int32_t *ctr = p.sync + kSyncBase;
  auto phase_ctr = [&](int l, int ph) {
    return ctr + size_t(l * kPhases + ph) * kSlots * kSlotStride;
  };
  auto trace_at = [&](int l, int ph) -> unsigned long long * {
    return p.trace ? p.trace + (size_t(l * kPhases + ph) * gridDim.x + blockIdx.x) * 2 : nullptr;
  };
  // rows per wave task of each GEMV phase; a phase's task count (its
  // counter's target) is ceil(rows / R)
  constexpr int R_QKV = 4, R_O = 4, R_GU = 2, R_DOWN = 2, R_LM = 2;
  const int t_qkv = qkv_rows / R_QKV, t_o = H / R_O, t_gu = 2 * F / R_GU, t_down = H / R_DOWN;
  for (int l = 0; l < p.n_layers; ++l) {
    const DecodeLayer Lw = p.layers[l];
    const uint32_t *x_in = p.xs + size_t(2 * l) * B * H;
    uint32_t *x_mid = p.xs + size_t(2 * l + 1) * B * H;
    uint32_t *x_out = p.xs + size_t(2 * l + 2) * B * H;
    uint32_t *qkv = p.qkv + size_t(l) * B * p.qkv_stride;
    uint32_t *attn = p.attn + size_t(l) * B * H;
    uint32_t *act = p.act + size_t(l) * B * F;
    uint32_t *part_o = p.part_o + size_t(l) * part_len * D * 2;
    uint32_t *part_ml = p.part_ml + size_t(l) * part_len * 4;
    const int32_t *prev_down = l ? phase_ctr(l - 1, kPhDown) : nullptr;
    gemv_phase<B, KCH, R_QKV, kEpiStore, false, false>(
        sh, red, p, cx, Lw.qkv, qkv_rows, plain, prev_down, t_down, x_in, H, Lw.input_ln,
        l == 0 ? p.embed : nullptr, l == 0 && blockIdx.x == 0, nullptr, qkv, p.qkv_stride,
        phase_ctr(l, kPhQkv), trace_at(l, kPhQkv));
    attn_phase<B, G>(sh, p, cx, l, Lw, qkv, part_o, part_ml, phase_ctr(l, kPhQkv), t_qkv,
                     phase_ctr(l, kPhAttn), trace_at(l, kPhAttn));
    merge_phase<B, G>(sh, p, cx, part_o, part_ml, attn, phase_ctr(l, kPhAttn), n_attn,
                      phase_ctr(l, kPhMerge), trace_at(l, kPhMerge));
    gemv_phase<B, KCH, R_O, kEpiResidual, false, false>(
        sh, red, p, cx, Lw.o, H, plain, phase_ctr(l, kPhMerge), B * p.Hq, attn, H, nullptr,
        nullptr, false, x_in, x_mid, H, phase_ctr(l, kPhO), trace_at(l, kPhO));
    gemv_phase<B, KCH, R_GU, kEpiSwiGLU, true, false>(
        sh, red, p, cx, Lw.gu, 2 * F, plain, phase_ctr(l, kPhO), t_o, x_mid, H, Lw.post_ln,
        nullptr, false, nullptr, act, F, phase_ctr(l, kPhGu), trace_at(l, kPhGu));
    gemv_phase<B, KCF, R_DOWN, kEpiResidual, false, false>(
        sh, red, p, cx, Lw.down, H, plain, phase_ctr(l, kPhGu), t_gu, act, F, nullptr, nullptr,
        false, x_mid, x_out, H, phase_ctr(l, kPhDown), trace_at(l, kPhDown));
  }
  const RowMap head_map{p.seg0_start, p.seg0_len, p.seg1_start, true};
  gemv_phase<B, KCH, R_LM, kEpiStore, true, true>(
      sh, red, p, cx, p.lm_head, p.n_logits, head_map, phase_ctr(p.n_layers - 1, kPhDown), t_down,
      p.xs + size_t(2 * p.n_layers) * B * H, H, p.final_norm, nullptr, false, nullptr, p.logits,
      p.ls, nullptr, trace_at(p.n_layers, 0));
  // exit: the last workgroup out resets the counters, stores the epoch and
  // advances pos (read by the next launch)
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(p.sync + kSyncExit, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    last = prev == int(gridDim.x) - 1;
  }
  __syncthreads();
  if (last) {
    for (int i = threadIdx.x; i < p.n_layers * kPhases * kSlots; i += 256)
      __hip_atomic_store(ctr + size_t(i) * kSlotStride, 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < B)
      p.pos[threadIdx.x] += 1;
    if (threadIdx.x == 0) {
      __hip_atomic_store(p.sync + kSyncEpoch, int32_t(epoch), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.sync + kSyncExit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int B, int G, int KCH, int KCF>
hipError_t launch_t(const DecodeParams &p, hipStream_t s) {
  hipLaunchKernelGGL((decode_step_kernel<B, G, KCH, KCF>), dim3(p.grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int B, int G, int KCH, int KCF>
int occupancy_t() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &blocks, reinterpret_cast<const void *>(decode_step_kernel<B, G, KCH, KCF>), 256, 0) !=
      hipSuccess)
    return 0;
  return blocks;
}

}  // namespace

bool decode_supported(int H, int F, int Hq, int Hkv, int B) {
  return (B == 1 || B == 2) && Hkv == 8 &&
         ((H == 3072 && F == 8192 && Hq == 24) || (H == 2048 && F == 6144 && Hq == 16));
}

int decode_occupancy(int H, int F, int Hq, int Hkv, int B) {
  if (!decode_supported(H, F, Hq, Hkv, B))
    return 0;
  if (H == 3072)
    return B == 1 ? occupancy_t<1, 3, 6, 16>() : occupancy_t<2, 3, 6, 16>();
  return B == 1 ? occupancy_t<1, 2, 4, 12>() : occupancy_t<2, 2, 4, 12>();
}

hipError_t launch_decode_step(const DecodeParams &p, hipStream_t s) {
  if (!decode_supported(p.H, p.F, p.Hq, p.Hkv, p.B) || p.max_splits < 1 ||
      p.max_splits > kMaxSplitsP || p.grid < 1 || p.n_layers < 1 || !p.layers || !p.sync ||
      p.Hq * D != p.H)
    return hipErrorInvalidValue;
  if (p.H == 3072)
    return p.B == 1 ? launch_t<1, 3, 6, 16>(p, s) : launch_t<2, 3, 6, 16>(p, s);
  return p.B == 1 ? launch_t<1, 2, 4, 12>(p, s) : launch_t<2, 2, 4, 12>(p, s);
}

}  // namespace yuear
