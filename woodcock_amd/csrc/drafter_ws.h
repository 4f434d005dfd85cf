// drafter_ws.h -- layout of the drafter workspace (wc_drafter_workspace_bytes),
// shared by the per-op drafter launches (drafter.hip) and the one-launch draft
// step (step.hip).  The caller zero-fills it once (wc_workspace_init); every
// counter in it is either self-resetting or monotone, so no call clears it.
#pragma once

#include "attention.h"
#include "gemv.h"
#include "gemvf.h"

namespace wc {

// One-launch draft step (step.hip): per-phase completion counters.  Each phase
// counter is kStepLeaves monotone 64-bit leaves, one 128-byte line each (the
// arrivals of a phase spread so that few of them meet on one line); every
// launch adds exactly kStepUnit to every phase counter (split over the phase's
// blocks), so the launch index is the final phase's sum / kStepUnit and a
// phase of launch L is complete when its sum reaches (L + 1) * kStepUnit.
enum StepPhase { kPhHead = 0, kPhQkv, kPhAttn, kPhO, kPhGateUp, kPhDown, kStepPhases };
constexpr int kStepLeaves = 128;
constexpr int kStepLeafStride = 16;  // uint64s per leaf
constexpr unsigned long long kStepUnit = 1ull << 20;
constexpr size_t kStepCtrBytes = 8ull * kStepPhases * kStepLeaves * kStepLeafStride;
constexpr size_t kStepSlotBytes = 8ull * 2 * kSlots * kSlotStride;  // two argmax slot sets (launch parity)

struct DrafterWs {
  unsigned int* head_ctr;  // tree counters (kTreeCounterBytes each)
  unsigned int* fin_ctr;
  unsigned int* attn_ctr;  // per kv head: splits done (decode attention's fused merge)
  unsigned long long* slots;
  float* qkv;
  float* attn;
  float* h1;
  float* act;
  float* partial;
  float* gs_part;        // k-split few-row GEMV: partial tiles per (tile, piece)
  unsigned int* gs_ctr;  // and one counter line per tile
  // one-launch draft step
  unsigned long long* step_ctr;    // [kStepPhases][kStepLeaves][kStepLeafStride] monotone
  unsigned long long* step_slots;  // [2][kSlots][kSlotStride] argmax keys, set = launch parity
  unsigned int* step_split;        // [kMaxKvHeads][kCounterStride] splits done per kv head (self-resetting)
  unsigned int* step_status;       // sticky: nonzero once a bounded wait gave up
  size_t bytes;
};

static inline size_t ws_align256(size_t x) { return (x + 255) / 256 * 256; }

static inline DrafterWs drafter_ws(const wc_drafter_dims& d, void* base) {
  DrafterWs w{};
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = ws_align256(off + bytes);
    return q;
  };
  const size_t R = WC_MAX_STEP_ROWS;
  const size_t nqkv = static_cast<size_t>(d.heads + 2 * d.kv_heads) * d.head_dim;
  w.head_ctr = reinterpret_cast<unsigned int*>(take(kTreeCounterBytes));
  w.fin_ctr = reinterpret_cast<unsigned int*>(take(kTreeCounterBytes));
  w.attn_ctr = reinterpret_cast<unsigned int*>(take(4 * kCounterStride * static_cast<size_t>(kMaxKvHeads)));
  w.slots = reinterpret_cast<unsigned long long*>(take(8 * R * kSlots * kSlotStride));
  w.qkv = reinterpret_cast<float*>(take(4 * R * nqkv));
  w.attn = reinterpret_cast<float*>(take(4 * R * d.heads * d.head_dim));
  w.h1 = reinterpret_cast<float*>(take(4 * R * d.hidden));
  w.act = reinterpret_cast<float*>(take(4 * R * d.inter));
  w.partial = reinterpret_cast<float*>(take(4 * static_cast<size_t>(d.kv_heads) * kMaxSplits * kMaxQV *
                                            (d.head_dim + 2)));
  w.gs_part = reinterpret_cast<float*>(take(4 * static_cast<size_t>(kGsMaxPieces) * kGsPieceFloats));
  w.gs_ctr = reinterpret_cast<unsigned int*>(take(4 * kCounterStride * static_cast<size_t>(kGsMaxPieces)));
  w.step_ctr = reinterpret_cast<unsigned long long*>(take(kStepCtrBytes));
  w.step_slots = reinterpret_cast<unsigned long long*>(take(kStepSlotBytes));
  w.step_split = reinterpret_cast<unsigned int*>(take(4 * kCounterStride * static_cast<size_t>(kMaxKvHeads)));
  w.step_status = reinterpret_cast<unsigned int*>(take(256));
  w.bytes = off;
  return w;
}

// The one-launch path of wc_drafter_forward for one row (step.hip): false
// when the call is outside what it covers (the per-op launches run instead).
bool step_layer_fits(const wc_drafter_dims& d, const wc_drafter_weights& w, int rows, const int32_t* n_rows_dev,
                     const uint8_t* mask_dev, int kv_dtype, const float* out_out, const int32_t* advance_dev);
bool step_layer_grid_ok(const wc_drafter_dims& d, const wc_drafter_weights& w, int kv_dtype, int capacity);
int step_layer_launch(const wc_drafter_dims& d, const wc_drafter_weights& w, int layer, const int32_t* tokens_dev,
                      const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add,
                      void* k_cache, void* v_cache, int kv_dtype, int capacity, const int32_t* offset_dev,
                      int offset_add, const int32_t* positions_dev, float* hidden_out, void* workspace,
                      hipStream_t s);

}  // namespace wc
