// Prefill projections on gfx950 MFMA: C[m][n] = bf16(sum_k A[m][k] W[n][k])
// (A: token rows, W: row-major weights, both K-contiguous), fp32 accumulation
// with one rounding, the residual form C = bf16(C + bf16(acc)) with both of
// the reference's rounding points (native/src/ar.cpp:20-29, 292-298), or the
// SwiGLU form C[m][i] = swiglu(acc[m][2 i], acc[m][2 i + 1]) on interleaved
// gate/up rows (ar.cpp:36-51).
//
// Tiling: a workgroup of WM x WN waves computes a BM x BN tile of C; each
// wave owns (BM / WM) token rows x (BN / WN) features as 32 x 32
// v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators) with the weights as the
// MFMA's first operand, so a lane ends up holding 4 consecutive features of
// one token row (8-byte stores). K advances 64 at a time through a two-stage
// LDS ring filled by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds):
// each load instruction moves 8 rows x 128 bytes into one contiguous KiB
// without passing through registers; the workgroup's (BM + BN) / 8 blocks per
// step are spread evenly over its waves. Rows past M or N read as zero
// (buffer range). One barrier per K step; the next step's loads are in flight
// while the current one computes.
//
// LDS stage: A rows [BM][128 B] then W rows [BN][128 B]. The 16-byte chunk
// kc (k = 8 kc .. 8 kc + 7) of row R is stored at slot kc ^ f(R),
// f(R) = (R >> 1) & 7. On gfx950 a ds_read_b128 is served in four groups of
// 16 lanes, lane l in group (bit 5 of l, bit 3 ^ bit 4 of l), and two lanes
// of a group reading different addresses in the same 16-byte slot of a
// 256-byte line conflict (inferred from SQ_LDS_BANK_CONFLICT over lane
// patterns on MI355X). With this f every fragment read below, of both MFMA
// forms, is conflict-free (the previous f(R) = (R & 7) ^ ((R >> 3) & 1) left
// the 16 x 16 x 32 form's reads two-way conflicted: half of the LDS cycles of
// the 256 x 256 tile were conflict stalls). Fragment of a 16-wide K sub-step
// s: lane l reads row l % 32, chunk 2 s + l / 32.
//
// Tile shapes (launch_gemm picks the one with the least estimated time for
// the shape and the CU count): 256 x 256 (8 waves of 128 x 64), 256 x 128 and
// 128 x 256 (8 waves of 64 x 64), 256 x 192 (8 waves of 64 x 96), 192 x 192
// (8 waves of 96 x 48) and 128 x 128 (4 waves of 64 x 64, two workgroups per
// CU); all but the last on 16 x 16 x 32 MFMAs (gemm_tile16 below), that one
// on 32 x 32 x 16. At the 3B prefill shapes (M = 3000) QKV and gate/up take
// 256 x 256 tiles, the output and down projections (N = 3072) 192 x 192:
// 256 tiles for 256 CUs where 256 x 192 leaves 64 CUs idle (down 148 -> 131
// us, o_proj 61 -> 52).
#include <algorithm>
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace yuear {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void *lds_ptr_t;

constexpr int kBK = 64;  // K per step; one LDS row = 128 bytes
constexpr int kMaxSplits = 16;  // split-K: at most this many K ranges per tile

// The kernel's only LDS object (dynamic size: 2 stages of (BM + BN) rows).
// With a second __shared__ variable the compiler no longer tells the
// direct-to-LDS writes of one stage from the reads of the other and waits for
// every load in flight (vmcnt(0)) before each step's first LDS read.
extern __shared__ __attribute__((aligned(1024))) char gemm_lds[];

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           uint32_t(bytes > 0xffffffffu ? 0xffffffffu : bytes),
                                           0x00020000);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return uint32_t(f2bf(a)) | uint32_t(f2bf(b)) << 16;
}

// SwiGLU epilogue (ar.cpp:36-51) on interleaved (gate_i, up_i) columns: the
// lane's features n .. n + 3 (n a multiple of 4) are two pairs, written as
// outputs n / 2 and n / 2 + 1 of the row with the rounding points of the
// decode GEMV's epilogue: g, u rounded to bf16, silu(g) rounded, then g * u.
__device__ __forceinline__ uint16_t swiglu_one(float gate, float up) {
  const float g = rbf(gate), u = rbf(up);
  const float act = rbf(g * (1.0f / (1.0f + expf(-g))));
  return f2bf(act * u);
}
__device__ __forceinline__ void swiglu_store(const GemmParams &p, int m, int n, const float *v) {
  uint16_t *c = p.c + size_t(m) * p.ldc + (n >> 1);
  if (n + 3 < p.n && (p.ldc & 1) == 0) {
    *reinterpret_cast<uint32_t *>(c) =
        uint32_t(swiglu_one(v[0], v[1])) | uint32_t(swiglu_one(v[2], v[3])) << 16;
  } else {
    if (n + 1 < p.n)
      c[0] = swiglu_one(v[0], v[1]);
    if (n + 3 < p.n)
      c[1] = swiglu_one(v[2], v[3]);
  }
}

// silu(g) rounded to bf16 for every bf16 value g (index = g's bits), by the
// expression swiglu_one evaluates: filled once per device (silu_table_kernel)
// before the first SwiGLU launch that reads it.
__device__ uint16_t g_silu_table[65536];
constexpr int kSiluTableBytes = 65536 * 2;

__global__ __launch_bounds__(256) void silu_table_kernel() {
  const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
  const float g = bf2f(uint16_t(i));
  g_silu_table[i] = f2bf(g * (1.0f / (1.0f + expf(-g))));
}

// swiglu_store with silu read from the table copy in LDS (`tab`): the same
// bits as swiglu_one.
__device__ __forceinline__ uint16_t swiglu_tab(const uint16_t *tab, float gate, float up) {
  const float act = bf2f(tab[f2bf(gate)]);
  return f2bf(act * rbf(up));
}
__device__ __forceinline__ void swiglu_store_tab(const GemmParams &p, const uint16_t *tab, int m,
                                                 int n, const float *v) {
  uint16_t *c = p.c + size_t(m) * p.ldc + (n >> 1);
  if (n + 3 < p.n && (p.ldc & 1) == 0) {
    *reinterpret_cast<uint32_t *>(c) =
        uint32_t(swiglu_tab(tab, v[0], v[1])) | uint32_t(swiglu_tab(tab, v[2], v[3])) << 16;
  } else {
    if (n + 1 < p.n)
      c[0] = swiglu_tab(tab, v[0], v[1]);
    if (n + 3 < p.n)
      c[1] = swiglu_tab(tab, v[2], v[3]);
  }
}

// Epilogue of a lane's 4 consecutive features n .. n + 3 (n a multiple of 4)
// of token row m < p.m: the 8-byte form when all four are in range and rows
// stay 8-byte aligned, else element by element.
__device__ __forceinline__ void epilogue4(const GemmParams &p, int m, int n, const float *v) {
  if (p.residual == 2) {
    swiglu_store(p, m, n, v);
    return;
  }
  uint16_t *c = p.c + size_t(m) * p.ldc + n;
  if (n + 3 < p.n && (p.ldc & 3) == 0) {
    uint2 o;
    if (p.residual) {
      const uint2 old = *reinterpret_cast<const uint2 *>(c);
      o.x = pack_bf16x2(bf2f(uint16_t(old.x)) + rbf(v[0]), bf2f(uint16_t(old.x >> 16)) + rbf(v[1]));
      o.y = pack_bf16x2(bf2f(uint16_t(old.y)) + rbf(v[2]), bf2f(uint16_t(old.y >> 16)) + rbf(v[3]));
    } else {
      o.x = pack_bf16x2(v[0], v[1]);
      o.y = pack_bf16x2(v[2], v[3]);
    }
    *reinterpret_cast<uint2 *>(c) = o;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < p.n)
        c[e] = p.residual ? f2bf(bf2f(c[e]) + rbf(v[e])) : f2bf(v[e]);
  }
}

// Split-K: split s of a workgroup's K range stores its fp32 sums of the
// 4 features at p.part[s][m][n .. n + 3]; gemm_reduce_kernel adds the splits
// in split order and applies the epilogue.
__device__ __forceinline__ void partial4(const GemmParams &p, int m, int n, const float *v) {
  float *dst = p.part + (size_t(blockIdx.y) * p.m + m) * p.n + n;
  if (n + 3 < p.n && (p.n & 3) == 0) {
    *reinterpret_cast<float4 *>(dst) = float4{v[0], v[1], v[2], v[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < p.n)
        dst[e] = v[e];
  }
}

// Tile of workgroup b. Workgroups are dispatched to the 8 XCDs round-robin
// (b % 8), each XCD with its own L2: XCD x takes the contiguous range
// [x T / 8, (x + 1) T / 8) of a grouped order (columns of 4 tile rows), so
// the tiles sharing an L2 form a compact block of A rows and W rows (QKV at
// M = 3000: 4 x 7.5 tiles per XCD instead of ~12 x 5). Any other dispatch
// order only changes the cache traffic, not the result.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int &tm, int &tn) {
  constexpr int kXcds = 8, kGroup = 4;
  const int total = tiles_m * tiles_n;
  int t = b;
  if (total % kXcds == 0)
    t = (b % kXcds) * (total / kXcds) + b / kXcds;
  const int per_group = kGroup * tiles_n;
  const int first = (t / per_group) * kGroup;
  const int rows = min(tiles_m - first, kGroup);
  const int r = t % per_group;
  tm = first + r % rows;
  tn = r / rows;
}

// SPLIT: the workgroup takes K range blockIdx.y of `splits` and stores fp32
// partial sums (a separate instantiation, so the one-pass kernels keep their
// compile-time K range and direct epilogue).
template <int BM, int BN, int WM, int WN, bool SPLIT>
__device__ __forceinline__ void gemm_tile(const GemmParams &p, int tiles_n, int splits) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // 32 x 32 MFMA tiles per wave
  constexpr int ABLK = BM / 8, BLK = (BM + BN) / 8;   // 1 KiB load blocks per stage
  constexpr int BPW = BLK / NW;                        // per wave
  constexpr int STAGE = (BM + BN) * 128;
  static_assert(TM * WM * 32 == BM && TN * WN * 32 == BN && BPW * NW == BLK, "tile shape");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int h = lane >> 5;
  int tm, tn;
  tile_of(int(blockIdx.x), (p.m + BM - 1) / BM, tiles_n, tm, tn);
  // split blockIdx.y of `splits` takes K [kbeg, kbeg + k / splits)
  const int kspan = SPLIT ? p.k / splits : p.k, kbeg = SPLIT ? int(blockIdx.y) * kspan : 0;
  const int m0 = tm * BM, n0 = tn * BN;
  const auto ra = rows_rsrc(p.a + size_t(m0) * p.lda, size_t(p.m - m0) * p.lda * 2);
  const auto rw = rows_rsrc(p.w + size_t(n0) * p.k, size_t(p.n - n0) * p.k * 2);

  // this wave's blocks q = wave BPW + i of the stage's A | W block list:
  // lane l loads row 8 q' + l / 8, chunk (l % 8) ^ f(row), into LDS slot l % 8
  uint32_t goff[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int q = wave * BPW + i;
    const bool is_a = q < ABLK;
    const int row = 8 * (is_a ? q : q - ABLK) + (lane >> 3);
    const int kc = (lane & 7) ^ (lane >> 4) ^ (4 * (q & 1));  // f(row), BM / 8 even
    goff[i] = uint32_t(row * (is_a ? p.lda : p.k) + kc * 8 + kbeg) * 2;
  }
  auto dma = [&](int st, int k0) {
    char *stage = gemm_lds + st * STAGE;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int q = wave * BPW + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(q < ABLK ? ra : rw, (lds_ptr_t)(stage + q * 1024),
                                               16, goff[i] + k0 * 2, 0, 0, 0);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  // fragment addresses: row (l % 32) of the wave's slice, chunk (2 s + h) ^ f
  const int f = (lane >> 1) & 7;  // f(row): row % 16 = lane % 16
  const int a_row = (wm * (BM / WM) + (lane & 31)) * 128;
  const int w_row = BM * 128 + (wn * (BN / WN) + (lane & 31)) * 128;
  const int steps = kspan / kBK;
  bf16x8_t af[2][TM], wf[2][TN];
  // fragments of sub-step s of the stage at `stage`, W and A tiles in the
  // order the MFMAs use them, so the first MFMA waits for two reads only
  auto rd = [&](const char *stage, int buf, int s) {
    const int co = ((2 * s + h) ^ f) * 16;
#pragma unroll
    for (int x = 0; x < (TM > TN ? TM : TN); ++x) {
      if (x < TN)
        wf[buf][x] = *reinterpret_cast<const bf16x8_t *>(stage + w_row + x * 4096 + co);
      if (x < TM)
        af[buf][x] = *reinterpret_cast<const bf16x8_t *>(stage + a_row + x * 4096 + co);
    }
  };
  auto mfma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[buf][j], af[buf][i], acc[i][j],
                                                            0, 0, 0);
  };
  // Step kt reads stage kt & 1. Its barrier sits before the last sub-step's
  // MFMAs, whose fragments are already in registers: past it, every wave has
  // finished reading stage kt & 1 (it is refilled with step kt + 2) and every
  // wave's part of step kt + 1 has landed (the first fragments of step kt + 1
  // are read), both under those MFMAs. Loads past K (the last two steps'
  // refills) read zeros or other rows into a stage nobody reads again.
  dma(0, 0);
  __builtin_amdgcn_s_waitcnt(0);  // (a barrier waits for no global load)
  if (steps > 1)
    dma(1, kBK);
  __syncthreads();
  rd(gemm_lds, 0, 0);
  for (int kt = 0; kt < steps; ++kt) {
    const char *stage = gemm_lds + (kt & 1) * STAGE;
#pragma unroll
    for (int s = 0; s + 1 < kBK / 16; ++s) {
      rd(stage, (s + 1) & 1, s + 1);
      mfma(s & 1);
    }
    // each sub-step: the next sub-step's reads one per MFMA
#pragma unroll
    for (int s = 0; s + 1 < kBK / 16; ++s) {
#pragma unroll
      for (int q = 0; q < TM + TN; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of step kt + 1, its LDS reads
    __syncthreads();
    dma(kt & 1, (kt + 2) * kBK);
    rd(gemm_lds + ((kt + 1) & 1) * STAGE, 0, 0);  // stale past the last step, unused
    mfma((kBK / 16 - 1) & 1);
    // refill loads and next reads spread over the last sub-step's MFMAs
#pragma unroll
    for (int q = 0; q < TM * TN; ++q) {
      if (q < BPW)
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (q < TM + TN)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // refills past K still in flight

  // epilogue: lane holds token row i 32 + l % 32 of the wave's slice, and
  // features j 32 + 8 q + 4 h + [0, 4) of its slice
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * (BM / WM) + i * 32 + (lane & 31);
    if (m >= p.m)
      continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * (BN / WN) + j * 32 + 8 * q + 4 * h;
        const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                            acc[i][j][4 * q + 3]};
        if (SPLIT)
          partial4(p, m, n, v);
        else
          epilogue4(p, m, n, v);
      }
    }
  }
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

// The same tile on v_mfma_f32_16x16x32_bf16: 16-row fragments (lane l: row
// l % 16, chunk 4 s + l / 16 of a 32-wide K sub-step s, two sub-steps per
// step), 16 x 16 accumulators (lane l: token row l % 16, features
// 4 (l / 16) + [0, 4)). Twice the MFMAs of half the length: measured 6-7 %
// faster than the 32 x 32 form for 256 x 256 tiles at M = 1024-3000.
template <int BM, int BN, int WM, int WN, bool SPLIT>
__device__ __forceinline__ void gemm_tile16(const GemmParams &p, int tiles_n, int splits) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int ABLK = BM / 8, BLK = (BM + BN) / 8;
  constexpr int BPW = BLK / NW;
  constexpr int STAGE = (BM + BN) * 128;
  static_assert(BPW * NW == BLK && TM * WM * 16 == BM && TN * WN * 16 == BN, "tile shape");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int q4 = lane >> 4;
  int tm, tn;
  tile_of(int(blockIdx.x), (p.m + BM - 1) / BM, tiles_n, tm, tn);
  // split blockIdx.y of `splits` takes K [kbeg, kbeg + k / splits)
  const int kspan = SPLIT ? p.k / splits : p.k, kbeg = SPLIT ? int(blockIdx.y) * kspan : 0;
  const int m0 = tm * BM, n0 = tn * BN;
  const auto ra = rows_rsrc(p.a + size_t(m0) * p.lda, size_t(p.m - m0) * p.lda * 2);
  const auto rw = rows_rsrc(p.w + size_t(n0) * p.k, size_t(p.n - n0) * p.k * 2);
  uint32_t goff[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int q = wave * BPW + i;
    const bool is_a = q < ABLK;
    const int row = 8 * (is_a ? q : q - ABLK) + (lane >> 3);
    const int kc = (lane & 7) ^ (lane >> 4) ^ (4 * (q & 1));  // f(row), BM / 8 even
    goff[i] = uint32_t(row * (is_a ? p.lda : p.k) + kc * 8 + kbeg) * 2;
  }
  auto dma = [&](int st, int k0) {
    char *stage = gemm_lds + st * STAGE;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int q = wave * BPW + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(q < ABLK ? ra : rw, (lds_ptr_t)(stage + q * 1024),
                                               16, goff[i] + k0 * 2, 0, 0, 0);
    }
  };
  f32x4v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const int f = (lane >> 1) & 7;  // f(row): row % 16 = lane % 16
  const int a_row = (wm * (BM / WM) + (lane & 15)) * 128;
  const int w_row = BM * 128 + (wn * (BN / WN) + (lane & 15)) * 128;
  const int steps = kspan / kBK;
  bf16x8_t af[2][TM], wf[2][TN];
  auto rd = [&](const char *stage, int buf, int s) {
    const int co = ((4 * s + q4) ^ f) * 16;
#pragma unroll
    for (int x = 0; x < (TM > TN ? TM : TN); ++x) {
      if (x < TN)
        wf[buf][x] = *reinterpret_cast<const bf16x8_t *>(stage + w_row + x * 2048 + co);
      if (x < TM)
        af[buf][x] = *reinterpret_cast<const bf16x8_t *>(stage + a_row + x * 2048 + co);
    }
  };
  auto mfma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  dma(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  if (steps > 1)
    dma(1, kBK);
  __syncthreads();
  rd(gemm_lds, 0, 0);
  for (int kt = 0; kt < steps; ++kt) {
    const char *stage = gemm_lds + (kt & 1) * STAGE;
    rd(stage, 1, 1);
    mfma(0);
    // the second sub-step's fragment reads among the first sub-step's MFMAs:
    // one per MFMA where a sub-step has 32 or more (256 x 256: QKV and gate/up
    // 1.5-2% faster on MI355X), else one per two (192 x 192: 2.5% faster so)
    constexpr int kPer = TM * TN >= 32 ? 1 : 2;
#pragma unroll
    for (int q = 0; q < TM + TN; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - kPer * (TM + TN), 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    dma(kt & 1, (kt + 2) * kBK);
    rd(gemm_lds + ((kt + 1) & 1) * STAGE, 0, 0);
    mfma(1);
#pragma unroll
    for (int q = 0; q < TM * TN; ++q) {
      if (q < BPW)
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (q < TM + TN)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (!SPLIT && p.residual == 2) {
    // SwiGLU: the ring is free once every wave is past its last fragment
    // reads; it takes the 128 KiB silu table (direct-to-LDS loads from the
    // L2-resident global copy), and each pair's silu becomes one LDS read
    // instead of an accurate exp and a division
    __syncthreads();
    const auto rt = rows_rsrc(g_silu_table, kSiluTableBytes);
#pragma unroll
    for (int i = 0; i < kSiluTableBytes / (NW * 1024); ++i) {
      const int blk = i * NW + wave;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_ptr_t)(gemm_lds + blk * 1024), 16,
                                               uint32_t(blk * 1024 + lane * 16), 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): a barrier waits for no global load
    __syncthreads();
    const uint16_t *tab = reinterpret_cast<const uint16_t *>(gemm_lds);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * (BM / WM) + i * 16 + (lane & 15);
      if (m >= p.m)
        continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * (BN / WN) + j * 16 + 4 * q4;
        const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        swiglu_store_tab(p, tab, m, n, v);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * (BM / WM) + i * 16 + (lane & 15);
    if (m >= p.m)
      continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + j * 16 + 4 * q4;
      const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      if (SPLIT)
        partial4(p, m, n, v);
      else
        epilogue4(p, m, n, v);
    }
  }
}

// One kernel per tile shape. The kernels are not templates: this clang emits
// no host launch stub for these kernel bodies when the kernel itself is a
// template instantiated from host code.
#define YUEAR_GEMM_KERNEL(NAME, BODY, BM, BN, WM, WN)                                        \
  __global__ __launch_bounds__(WM * WN * 64) void NAME(GemmParams p, int tiles_n, int splits) { \
    BODY<BM, BN, WM, WN, false>(p, tiles_n, splits);                                         \
  }                                                                                          \
  __global__ __launch_bounds__(WM * WN * 64) void NAME##_split(GemmParams p, int tiles_n,     \
                                                               int splits) {                 \
    BODY<BM, BN, WM, WN, true>(p, tiles_n, splits);                                          \
  }
// MFMA form per shape, as measured: 16 x 16 x 32 for all but 128 x 128
// (256 x 192 on it 2-4% faster than on 32 x 32 x 16 once its fragment reads
// were conflict-free; 128 x 128 6-10% slower).
YUEAR_GEMM_KERNEL(gemm_256x256, gemm_tile16, 256, 256, 2, 4)
YUEAR_GEMM_KERNEL(gemm_256x128, gemm_tile16, 256, 128, 4, 2)
YUEAR_GEMM_KERNEL(gemm_128x256, gemm_tile16, 128, 256, 2, 4)
YUEAR_GEMM_KERNEL(gemm_256x192, gemm_tile16, 256, 192, 4, 2)
YUEAR_GEMM_KERNEL(gemm_128x128, gemm_tile, 128, 128, 2, 2)
YUEAR_GEMM_KERNEL(gemm_192x192, gemm_tile16, 192, 192, 2, 4)
#undef YUEAR_GEMM_KERNEL

// Time model of the tile shapes, in microseconds per 48 K steps measured on
// MI355X (K = 3072, 256 CUs): `alone` for a tile with a CU to itself on an
// otherwise idle chip, `busy` with every CU holding one such tile, `round` for
// a full round of per_cu workgroups on every CU.
struct TileShape {
  int bm, bn, per_cu;
  double alone, busy, round;
};
constexpr TileShape kShapes[] = {
    {256, 256, 1, 63.0, 85.0, 85.0}, {256, 128, 1, 43.5, 50.0, 50.0},
    {128, 256, 1, 44.3, 50.0, 50.0}, {256, 192, 1, 49.0, 58.0, 58.0},
    {128, 128, 2, 34.3, 40.0, 50.8}, {192, 192, 1, 41.0, 49.0, 49.0},
};

// Split-K: the sum over the splits in split order (a fixed order: the result
// does not depend on which split finished first), then the epilogue; one
// thread per 4 consecutive features of a row. All of a thread's partial loads
// are issued before the first add, so a thread waits for one memory latency
// rather than one per split.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p, int splits) {
  const int nq = (p.n + 3) / 4;
  const size_t total = size_t(p.m) * nq;
  const size_t plane = size_t(p.m) * p.n;
  for (size_t x = size_t(blockIdx.x) * 256 + threadIdx.x; x < total; x += size_t(gridDim.x) * 256) {
    const int m = int(x / nq), n = int(x % nq) * 4;
    const float *src = p.part + size_t(m) * p.n + n;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (n + 3 < p.n && (p.n & 3) == 0) {
      f32x4v t[kMaxSplits];
#pragma unroll
      for (int z = 0; z < kMaxSplits; ++z)
        if (z < splits)
          t[z] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(src + z * plane));
#pragma unroll
      for (int z = 0; z < kMaxSplits; ++z)
        if (z < splits) {
          v[0] += t[z].x;
          v[1] += t[z].y;
          v[2] += t[z].z;
          v[3] += t[z].w;
        }
    } else {
      for (int z = 0; z < splits; ++z)
        for (int e = 0; e < 4; ++e)
          if (n + e < p.n)
            v[e] += src[z * plane + e];
    }
    epilogue4(p, m, n, v);
  }
}

// gemm_reduce_kernel's sum and residual epilogue for one row per workgroup,
// then rms_norm_rows_kernel's RMSNorm of that row: the same 8-feature chunks
// per thread (c = thread, thread + 256, ...), the same order of the squares'
// sum, so x and y come out bit-identical to the two kernels. The row's new
// values stay in registers (at most kNormChunks chunks per thread).
constexpr int kNormChunks = 4;  // rows up to 8192 features
__global__ __launch_bounds__(256) void gemm_reduce_norm_kernel(GemmParams p, int splits,
                                                               const uint16_t *w, float eps,
                                                               uint16_t *y) {
  __shared__ float red[4];
  const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = p.n / 8;
  const size_t plane = size_t(p.m) * p.n;
  u32x4 *xr = reinterpret_cast<u32x4 *>(p.c + size_t(r) * p.ldc);
  uint32_t xn[kNormChunks][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = int(threadIdx.x) + 256 * i;
    if (c >= chunks)
      break;
    const float *src = p.part + size_t(r) * p.n + 8 * c;
    f32x4v a[kMaxSplits], b[kMaxSplits];
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < splits) {
        a[z] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(src + z * plane));
        b[z] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(src + z * plane + 4));
      }
    const u32x4 old = xr[c];
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < splits) {
        v[0] += a[z].x;
        v[1] += a[z].y;
        v[2] += a[z].z;
        v[3] += a[z].w;
        v[4] += b[z].x;
        v[5] += b[z].y;
        v[6] += b[z].z;
        v[7] += b[z].w;
      }
    const uint32_t oi[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xn[i][q] = pack_bf16x2(bflo(oi[q]) + rbf(v[2 * q]), bfhi(oi[q]) + rbf(v[2 * q + 1]));
      const float lo = bflo(xn[i][q]), hi = bfhi(xn[i][q]);
      ss += lo * lo;
      ss += hi * hi;
    }
    xr[c] = u32x4{xn[i][0], xn[i][1], xn[i][2], xn[i][3]};
  }
  ss = wave_sum(ss);
  if (lane == 0)
    red[wave] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = rbf(1.0f / __builtin_sqrtf(total / float(p.n) + eps));
  const u32x4 *g4 = reinterpret_cast<const u32x4 *>(w);
  u32x4 *dst = reinterpret_cast<u32x4 *>(y + size_t(r) * p.n);
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = int(threadIdx.x) + 256 * i;
    if (c >= chunks)
      break;
    const u32x4 g = g4[c];
    const uint32_t gi[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = f2bf(rbf(bflo(xn[i][q]) * scale) * bflo(gi[q]));
      const uint32_t hi = f2bf(rbf(bfhi(xn[i][q]) * scale) * bfhi(gi[q]));
      o[q] = lo | (hi << 16);
    }
    dst[c] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// The global silu table of this device, filled on first use (one launch and
// a synchronisation, so not inside a graph capture: refused there).
hipError_t ensure_silu_table(hipStream_t s) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static bool done[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return e;
  if (dev < 0 || dev >= kMaxDevices)
    return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (done[dev])
    return hipSuccess;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if ((e = hipStreamIsCapturing(s, &cs)) != hipSuccess)
    return e;
  if (cs != hipStreamCaptureStatusNone)
    return hipErrorStreamCaptureUnsupported;
  hipLaunchKernelGGL(silu_table_kernel, dim3(65536 / 256), dim3(256), 0, s);
  if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(s)) != hipSuccess)
    return e;
  done[dev] = true;
  return hipSuccess;
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_tile(void (*kern)(GemmParams, int, int), const GemmParams &p, int splits,
                       hipStream_t s) {
  // the 16 x 16 x 32 tile bodies (all shapes but 128 x 128) read silu from an
  // LDS table in a one-pass SwiGLU launch
  constexpr bool kTile16 = !(BM == 128 && BN == 128);
  const bool table = kTile16 && p.residual == 2 && splits == 1;
  const int ring = 2 * (BM + BN) * 128;
  const int lds = table ? std::max(ring, kSiluTableBytes) : ring;
  hipError_t e = table ? ensure_silu_table(s) : hipSuccess;
  if (e != hipSuccess)
    return e;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess)
    return e;
  const int tiles_n = (p.n + BN - 1) / BN;
  const unsigned tiles = unsigned((p.m + BM - 1) / BM) * unsigned(tiles_n);
  hipLaunchKernelGGL(kern, dim3(tiles, unsigned(splits)), dim3(WM * WN * 64), lds, s, p, tiles_n,
                     splits);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1 || p.defer_reduce)
    return e;
  const size_t quads = size_t(p.m) * ((p.n + 3) / 4);
  const unsigned blocks = unsigned(std::min<size_t>((quads + 255) / 256, 4096));
  hipLaunchKernelGGL(gemm_reduce_kernel, dim3(blocks), dim3(256), 0, s, p, splits);
  return hipGetLastError();
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  return cus;
}

}  // namespace

int gemm_tile_choice(int m, int n, int cus) {
  int best = 0;
  double best_t = 0;
  for (int i = 0; i < int(sizeof(kShapes) / sizeof(kShapes[0])); ++i) {
    const TileShape &t = kShapes[i];
    const long long tiles = (long long)((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
    const long long slots = (long long)cus * t.per_cu;
    const long long full = tiles / slots, rem = tiles % slots;
    // full rounds, then a last round that is cheaper the fewer CUs it loads
    double time = double(full) * t.round;
    if (rem > cus)
      time += t.round;
    else if (rem > 0)
      time += t.alone + (t.busy - t.alone) * double(rem) / cus;
    if (i == 0 || time < best_t * 0.999) {
      best = i;
      best_t = time;
    }
  }
  return best;
}

// Shape and split count together, by the tile model scaled to K / splits
// steps, plus, for a split, the reduce kernel: 4 us and 0.4 us per MB it
// moves (the splits' fp32 partials read, the bf16 result written) and 0.1 us
// per MB of partials the tiles write instead of bf16 results. Fitted to
// every (shape, splits) of the four 3B prefill projections at 128-2048
// tokens on MI355X: the pick is within 9% of the fastest measured (split or
// not) in all 28 cases; without a split it is gemm_tile_choice's shape.
void gemm_plan(int m, int n, int k, int cus, size_t part_bytes, int *shape, int *splits) {
  *shape = gemm_tile_choice(m, n, cus);
  *splits = 1;
  double best_t = 0;
  const double mn = double(m) * double(n);
  for (int i = 0; i < int(sizeof(kShapes) / sizeof(kShapes[0])); ++i) {
    const TileShape &t = kShapes[i];
    const long long tiles = (long long)((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
    const long long slots = (long long)cus * t.per_cu;
    for (int z = 1; z <= kMaxSplits; ++z) {
      // whole 64-wide steps, at least 4 per split, the partials in the workspace
      if ((k / kBK) % z || k / z < 4 * kBK ||
          (z > 1 && size_t(m) * size_t(n) > part_bytes / (size_t(z) * 4)))
        continue;
      const long long wgs = tiles * z, full = wgs / slots, rem = wgs % slots;
      double round = double(full) * t.round;
      if (rem > cus)
        round += t.round;
      else if (rem > 0)
        round += t.alone + (t.busy - t.alone) * double(rem) / cus;
      double time = round * (double(k) / z / kBK) / 48.0;
      if (z > 1)
        time += 4.0 + 0.4e-6 * (4.0 * z * mn + 2.0 * mn) + 0.1e-6 * 4.0 * z * mn;
      if ((i == 0 && z == 1) || time < best_t * 0.999) {
        *shape = i;
        *splits = z;
        best_t = time;
      }
    }
  }
}

hipError_t launch_gemm_tile(const GemmParams &p, int shape, hipStream_t s, int splits) {
  if (p.m < 1 || p.n < 1 || p.k < kBK || p.k % kBK || p.lda < p.k || p.lda % 8 || !p.a ||
      !p.w || !p.c || p.residual < 0 || p.residual > 2 || (p.residual == 2 && p.n % 2) ||
      p.ldc < (p.residual == 2 ? p.n / 2 : p.n) || splits < 1 || splits > kMaxSplits ||
      (p.k / kBK) % splits ||
      (splits > 1 && (!p.part || size_t(p.m) * size_t(p.n) > p.part_bytes / (size_t(splits) * 4))))
    return hipErrorInvalidValue;
  const bool sp = splits > 1;
  switch (shape) {
  case 0: return launch_tile<256, 256, 2, 4>(sp ? gemm_256x256_split : gemm_256x256, p, splits, s);
  case 1: return launch_tile<256, 128, 4, 2>(sp ? gemm_256x128_split : gemm_256x128, p, splits, s);
  case 2: return launch_tile<128, 256, 2, 4>(sp ? gemm_128x256_split : gemm_128x256, p, splits, s);
  case 3: return launch_tile<256, 192, 4, 2>(sp ? gemm_256x192_split : gemm_256x192, p, splits, s);
  case 4: return launch_tile<128, 128, 2, 2>(sp ? gemm_128x128_split : gemm_128x128, p, splits, s);
  case 5: return launch_tile<192, 192, 2, 4>(sp ? gemm_192x192_split : gemm_192x192, p, splits, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_reduce_norm(const GemmParams &p, int splits, const uint16_t *norm_w,
                                   float eps, uint16_t *y, hipStream_t s) {
  if (p.m < 1 || p.n < 8 || p.n % 8 || p.n > 8 * 256 * kNormChunks || p.ldc != p.n ||
      p.residual != 1 || !p.c || !p.part || !norm_w || !y || splits < 2 || splits > kMaxSplits ||
      size_t(p.m) * size_t(p.n) > p.part_bytes / (size_t(splits) * 4))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemm_reduce_norm_kernel, dim3(p.m), dim3(256), 0, s, p, splits, norm_w, eps,
                     y);
  return hipGetLastError();
}

int gemm_cus() { return device_cus(); }

hipError_t launch_gemm(const GemmParams &p, hipStream_t s) {
  const int cus = device_cus();
  int shape = gemm_tile_choice(p.m, p.n, cus), splits = 1;
  if (p.part)
    gemm_plan(p.m, p.n, p.k, cus, p.part_bytes, &shape, &splits);
  return launch_gemm_tile(p, shape, s, splits);
}

}  // namespace yuear
