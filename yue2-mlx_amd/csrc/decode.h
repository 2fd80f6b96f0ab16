// Persistent decode step (one launch per token): parameter block and launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yuear {

// Phases of one layer.
enum DecodePhase : int { kPhQkv = 0, kPhAttn, kPhMerge, kPhO, kPhGu, kPhDown, kPhases };
// Sync array (int32 words): [kSyncError] sticky error word (a bounded wait
// expired), [kSyncEpoch] launch counter (never reset: it tags activation
// words), [kSyncExit] exit counter, then per (layer, phase) kSlots
// completion counters kSlotStride words apart (one 128-byte line each); a
// workgroup adds its finished task count to slot blockIdx % kSlots and a
// waiter sums the slots.
constexpr int kSyncError = 0, kSyncEpoch = 16, kSyncExit = 32, kSyncBase = 64;
constexpr int kSlots = 8, kSlotStride = 32;
constexpr size_t decode_sync_words(int layers) {
  return kSyncBase + size_t(layers) * kPhases * kSlots * kSlotStride;
}

struct DecodeLayer {
  const uint16_t *input_ln, *post_ln, *q_norm, *k_norm;  // [H] / [D] gains
  const uint16_t *qkv, *o, *gu, *down;                   // weights, row-major [rows][k]
};

// Activation words: every activation of the step lives in 32-bit words
// (tag << 16) | payload16, tag = the launch's tag (1..65535, from the epoch),
// so a reader recognises a word written by this launch. A bf16 activation
// takes one word; an fp32 split partial takes two (high half, low half).
struct DecodeParams {
  int H = 0, F = 0, Hq = 0, Hkv = 0, B = 1, n_layers = 0, vocab = 0;
  float eps = 1e-6f, attn_scale = 0.f;
  const uint16_t *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
  const uint16_t *rope_cos = nullptr, *rope_sin = nullptr;  // [positions][64]
  const DecodeLayer *layers = nullptr;  // [n_layers], device memory
  uint16_t *kc = nullptr, *vc = nullptr;  // [layers][B][Hkv][cap][128]
  int cap = 0;
  int32_t *pos = nullptr;        // [B] slot of the current token; += 1 at exit
  const int32_t *tok = nullptr;  // [B] input token ids
  uint32_t *xs = nullptr;        // [2 * n_layers + 1][B][H] residual stream words
  uint32_t *qkv = nullptr;       // [n_layers][B][qkv_stride] words
  int qkv_stride = 0;
  uint32_t *attn = nullptr;      // [n_layers][B][Hq * 128] words
  uint32_t *act = nullptr;       // [n_layers][B][F] words
  uint32_t *part_o = nullptr;    // [n_layers][B][Hkv][max_splits][G][128][2] words
  uint32_t *part_ml = nullptr;   // [n_layers][B][Hkv][max_splits][G][2][2] words
  int max_splits = 1;
  uint16_t *logits = nullptr;    // [B][ls] phase-local rows (plain bf16)
  int ls = 0, n_logits = 0;
  int seg0_start = 0, seg0_len = 1 << 30, seg1_start = 0;  // lm_head row map
  int32_t *sync = nullptr;       // decode_sync_words(n_layers) words
  int grid = 0;                  // workgroups (all co-resident)
  int max_spins = 1 << 20;       // polls before a wait gives up and sets the error word
  // Optional phase trace (profiling): [(n_layers * kPhases + 1) * grid][2]
  // 100 MHz timestamps per phase and workgroup: input ready, tasks signalled
  // (0 when the workgroup had no task in that phase); the last phase is the
  // lm_head.
  unsigned long long *trace = nullptr;
};

// Shapes with a compiled persistent step.
bool decode_supported(int H, int F, int Hq, int Hkv, int B);
// Co-resident 256-thread workgroups per CU for that shape (0: unsupported).
int decode_occupancy(int H, int F, int Hq, int Hkv, int B);
hipError_t launch_decode_step(const DecodeParams &p, hipStream_t s);

}  // namespace yuear
