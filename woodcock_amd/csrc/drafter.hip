// drafter.hip -- the EAGLE-3 drafter step on gfx950.
//
// One decoder layer (python/woodcock/drafter.py:164-191; src/core/drafter.cpp:91-136)
// is six launches, all stream-ordered on the caller's stream:
//   1. QKV    : dual-input streaming GEMV  q,k,v = W.RMS(h) + W_aux.RMS(e(x))
//   2. attend : q/k RMSNorm + RoPE + KV append + split-KV GQA attention,
//               then a merge launch combines the splits
//   3. o_proj : GEMV with residual epilogue          h1 = h + W_o.o
//   4. gate/up: paired-row GEMV, SiLU(gate)*up epilogue
//   5. down   : GEMV with residual epilogue, last block applies the final
//               RMSNorm (out) and advances the cache offset
// plus the fc fusion (drafter.py:149-153) and the draft head with a fused
// argmax / Gumbel-max and d2t map (drafter.py:204-215, spec.py:346).
// Every round-varying integer (offset, row counts, gathered rows, tokens) is
// read from device memory.
#include <mutex>
#include <unordered_map>

#include "attention.h"
#include "gemv.h"
#include "gemvf.h"
#include "gemv1s.h"

namespace wc {

// ------------------------------------------------------------------ workspace


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
  size_t bytes;
};

static size_t align256(size_t x) { return (x + 255) / 256 * 256; }

static DrafterWs drafter_ws(const wc_drafter_dims& d, void* base) {
  DrafterWs w{};
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = align256(off + bytes);
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
  w.bytes = off;
  return w;
}

// ------------------------------------------------------------------ GEMV launch

// Weight registers per lane are 4 * R * P * NIN * S; variants above the budget
// are not instantiated (they would spill) and report false to the dispatcher.
constexpr int kGemv1Budget = 24;
constexpr size_t kCuLds = 160 * 1024 - 2048;       // LDS per CU on gfx950, less the kernels' static LDS
constexpr int kGemvxBudget = 32;                   // weight vectors per lane of the few-row kernel
constexpr size_t kGemvxMaxLds = 144 * 1024;        // dynamic LDS of the few-row GEMV, at most

template <int R, bool PAIR, int NIN, int S, int XB>
static bool launch_gemv1_s(const GemvArgs& a, hipStream_t s) {
  if constexpr (R * (PAIR ? 2 : 1) * NIN * S > kGemv1Budget) {
    return false;
  } else {
    int gb = 0;
    for (int i = 0; i < a.n_in; ++i)
      if (a.in[i].gain) gb |= 1 << i;
    const dim3 grid((a.N + kGemvWaves * R - 1) / (kGemvWaves * R)), block(kGemvThreads);
    constexpr int kAll = (1 << NIN) - 1;
    // a long gain-free input row (the down projection, K >= 6144) is staged
    // once per block (k_gemv1s): each wave would otherwise read twice its
    // weight bytes of x from L2 (2048 x 6144: 7.1 -> 6.2 us); for shorter or
    // normed rows the per-wave loads measured as fast or faster
    if constexpr (NIN == 1 && !PAIR && S >= 12) {
      if (gb == 0) {
        const size_t lds = static_cast<size_t>(a.in[0].K) * sizeof(float);
        hipLaunchKernelGGL((k_gemv1s<R, PAIR, NIN, S, XB, 0>), grid, block, lds, s, a);
        return true;
      }
    }
    // normed rows wider than 2048 (the Qwen3-4B shapes: the drafter's head,
    // dual-stream QKV and gate / up pair, the target's one-row layers and its
    // logits head): the per-wave kernel holds every segment's x slices, gains
    // and weights -- 116 VGPRs for one 2560-wide segment (four waves per SIMD;
    // the head's 8192 waves and the pair's 9728 run in two or more rounds of
    // resident waves), 210 for the dual-stream QKV (two per SIMD: 1.5 rounds
    // for its 6144 rows) -- while staging x * gain per block keeps 73-82 and
    // 146 (six, five and three per SIMD).  4B draft step 87.7 -> 84.4 us warm,
    // the 36-layer 4B target's one-row forward 2.345 -> 2.300 ms
    if constexpr (S >= 5 && NIN <= 2) {
      size_t lds = 0;
      for (int i = 0; i < NIN; ++i) lds += static_cast<size_t>(a.in[i].K) * sizeof(float);
      if (gb == kAll && lds <= 64 * 1024) {  // within the default dynamic LDS limit
        hipLaunchKernelGGL((k_gemv1s<R, PAIR, NIN, S, XB, kAll>), grid, block, lds, s, a);
        return true;
      }
    }
    // at 2048 only the draft head (argmax epilogue; 8192 waves at five per SIMD
    // on the per-wave kernel's 94 VGPRs, six per SIMD on the staged one's 73):
    // 1.7B draft step 53.25 -> 52.7 us warm, 65.9 -> 64.9 us cold, greedy round
    // 261.55 -> 260.4 us.  Four head rows per wave (4096 waves, all resident)
    // and the staged gate / up pair measured slower; the staged dual-stream QKV
    // (whose 2048 waves already fit one round) within noise (round 252.4
    // against 253.1 us, step 49.5 against 49.4 us)
    if constexpr (S == 4 && NIN == 1 && !PAIR) {
      if (gb == kAll && a.epi == kEpiArgmax) {
        hipLaunchKernelGGL((k_gemv1s<R, PAIR, NIN, S, XB, kAll>), grid, block, a.in[0].K * sizeof(float), s, a);
        return true;
      }
    }
    if (gb == kAll) {
      hipLaunchKernelGGL((k_gemv1<R, PAIR, NIN, S, XB, kAll>), grid, block, 0, s, a);
    } else if constexpr (NIN == 1) {
      hipLaunchKernelGGL((k_gemv1<R, PAIR, NIN, S, XB, 0>), grid, block, 0, s, a);  // no gain
    } else {
      return false;  // mixed gains on several segments: the general kernel
    }
    return true;
  }
}

// Step counts: 4 (K 2048), 5 (K 2560), 8, 12 (K 6144) and 20 (K up to 10240,
// e.g. 9728); a count between two variants runs the larger with its last steps
// masked, so the Qwen3-1.7B and -4B widths each get an exact variant.
template <int R, bool PAIR, int NIN, int XB>
static bool launch_gemv1(const GemvArgs& a, int steps, hipStream_t s) {
  if (steps <= 4) return launch_gemv1_s<R, PAIR, NIN, 4, XB>(a, s);
  if (steps <= 5) return launch_gemv1_s<R, PAIR, NIN, 5, XB>(a, s);
  if (steps <= 8) return launch_gemv1_s<R, PAIR, NIN, 8, XB>(a, s);
  if (steps <= 12) return launch_gemv1_s<R, PAIR, NIN, 12, XB>(a, s);
  if (steps <= 20) return launch_gemv1_s<R, PAIR, NIN, 20, XB>(a, s);
  return false;
}

// Largest rows-per-wave that keeps at least 512 blocks and fits the budget;
// the draft head (argmax epilogue) takes at most two and the gate/up pair one:
// more waves in flight measured faster (head 16384 x 2048: 14.3 against 15.6 us
// at four; the pair: 0.4 us of a 1.7B draft step, 0.9 us of a 4B one).
template <bool PAIR, int NIN, int XB>
static bool launch_gemv1_r(const GemvArgs& a, int steps, hipStream_t s) {
  if (a.N >= 4 * kGemvWaves * 512 && a.epi != kEpiArgmax && !PAIR && launch_gemv1<4, PAIR, NIN, XB>(a, steps, s))
    return true;
  if (a.N >= 2 * kGemvWaves * 512 && !PAIR && launch_gemv1<2, PAIR, NIN, XB>(a, steps, s)) return true;
  return launch_gemv1<1, PAIR, NIN, XB>(a, steps, s);
}

// Few-row kernel: x staged in LDS; same register budget for the weights.
template <int R, bool PAIR, int NIN, int S, int XB, int MM>
static bool launch_gemvx_s(const GemvArgs& a, size_t lds, hipStream_t s) {
  if constexpr (R * (PAIR ? 2 : 1) * NIN * S > kGemvxBudget) {
    return false;
  } else {
    const void* fn = reinterpret_cast<const void*>(&k_gemvx<R, PAIR, NIN, S, XB, MM>);
    static size_t attr_bytes = 64 * 1024;  // default dynamic-LDS limit
    if (lds > attr_bytes) {
      if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
        return false;
      attr_bytes = lds;
    }
    const dim3 grid((a.N + kGemvWaves * R - 1) / (kGemvWaves * R)), block(kGemvThreads);
    hipLaunchKernelGGL((k_gemvx<R, PAIR, NIN, S, XB, MM>), grid, block, lds, s, a);
    return true;
  }
}

template <int R, bool PAIR, int NIN, int XB, int MM>
static bool launch_gemvx_m(const GemvArgs& a, int steps, hipStream_t s) {
  const int S = steps <= 4 ? 4 : steps <= 8 ? 8 : 12;
  const size_t lds = static_cast<size_t>(NIN) * a.M * S * 512 * 4;
  if (lds > kGemvxMaxLds) return false;
  if (steps <= 4) return launch_gemvx_s<R, PAIR, NIN, 4, XB, MM>(a, lds, s);
  if (steps <= 8) return launch_gemvx_s<R, PAIR, NIN, 8, XB, MM>(a, lds, s);
  if (steps <= 12) return launch_gemvx_s<R, PAIR, NIN, 12, XB, MM>(a, lds, s);
  return false;
}

// Rows per wave: the fewest that keep every block resident at once (the LDS
// footprint sets how many blocks fit on a CU), within the register budget.
template <bool PAIR, int NIN, int XB, int MM>
static bool launch_gemvx_r(const GemvArgs& a, int steps, hipStream_t s) {
  const int S = steps <= 4 ? 4 : steps <= 8 ? 8 : 12;
  const size_t lds = static_cast<size_t>(NIN) * a.M * S * 512 * 4;
  const int per_cu = std::max<int>(1, static_cast<int>(kCuLds / std::max<size_t>(lds, 1)));
  const long resident = 256L * std::min(per_cu, 4);
  if ((a.N + kGemvWaves - 1) / kGemvWaves <= resident && launch_gemvx_m<1, PAIR, NIN, XB, MM>(a, steps, s))
    return true;
  if ((a.N + 2 * kGemvWaves - 1) / (2 * kGemvWaves) <= resident && launch_gemvx_m<2, PAIR, NIN, XB, MM>(a, steps, s))
    return true;
  if (launch_gemvx_m<4, PAIR, NIN, XB, MM>(a, steps, s)) return true;
  if (launch_gemvx_m<2, PAIR, NIN, XB, MM>(a, steps, s)) return true;
  return launch_gemvx_m<1, PAIR, NIN, XB, MM>(a, steps, s);
}

// Dynamic LDS of the staged few-row GEMV: a kernel takes `bytes` when its static
// LDS plus `bytes` fits the CU (its dynamic limit raised once per kernel).
constexpr size_t kGfStageMax = 136 * 1024;
static bool gf_stage_ok(const void* kern, size_t bytes) {
  static std::mutex mu;
  static std::unordered_map<const void*, size_t> room;  // kernel -> dynamic bytes it may take
  std::lock_guard<std::mutex> lock(mu);
  auto it = room.find(kern);
  if (it == room.end()) {
    hipFuncAttributes fa{};
    size_t r = 0;
    if (hipFuncGetAttributes(&fa, kern) == hipSuccess && fa.sharedSizeBytes + 1024 < kCuLds + 2048) {
      r = kCuLds + 2048 - 1024 - fa.sharedSizeBytes;
      if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(r)) != hipSuccess)
        r = 0;
    }
    (void)hipGetLastError();
    it = room.emplace(kern, r).first;
  }
  return bytes <= it->second;
}

// Staged few-row MFMA GEMV (k_gemvs): 8-wave blocks, one input segment each
// (several segments need the split workspace).  The weights stream at what one
// CU sustains (a 2048 x 6144 GEMV: 7.0 us on 128 blocks, 4.5 us on 256), so the
// time goes with the blocks the busiest CU runs: each segment's k steps are
// split into the part count P (1..8) that minimises ceil(blocks / 256) / blocks
// (ties: fewer parts), unless the launch reduces an argmax.  D = the smallest
// depth holding a wave's share of its part (chunks of the largest otherwise:
// 12 steps for one tile, 8 for two, beyond which the weights no longer fit
// the registers).
// Two-segment launches (the dual-stream QKV) on k_gemvs with eight waves per
// segment measured slower than k_gemvf (33.5 MB at M = 5: 17.1 against 14.2
// us), so they stay there.
constexpr bool kGsPairedQkv = false;

template <int TW, bool PAIR, int NIN, int XB, int GB>
static bool launch_gemvs(const GemvArgs& a, hipStream_t s) {
  constexpr int W = 8;
  constexpr int WG = 16;  // two-segment blocks: eight waves per segment
  constexpr int RB = PAIR ? 16 : 16 * TW;
  const bool split_ok = a.gs_part && a.gs_ctr && a.epi != kEpiArgmax;
  int kmax = 0, ksum = 0;
  for (int i = 0; i < a.n_in; ++i) {
    kmax = std::max(kmax, a.in[i].K);
    ksum += a.in[i].K + 4;
  }
  const int tiles = (a.N + RB - 1) / RB;
  // two segments and a grid that fills the GPU: one block takes both, eight
  // waves on each, so no piece hand-over is needed; otherwise the few-row
  // kernel k_gemvf (one launch, measured faster than pieces here)
  if constexpr (NIN == 2) {
    const size_t st2 = static_cast<size_t>(a.M) * ksum * sizeof(float);
    const int per2 = (kmax / 32 + WG / 2 - 1) / (WG / 2);
    if (kGsPairedQkv && TW == 1 && tiles >= 256 && st2 <= kGfStageMax && a.M * ((kmax + kGsUnit - 1) / kGsUnit) <= kGsMaxUnits / 2 &&
        a.epi != kEpiArgmax && per2 <= 12) {
      const size_t lds2 = std::max(st2, static_cast<size_t>(WG) * TW * 4 * kWave * sizeof(float));
      const dim3 grid2(tiles, 1), block2(WG * kWave);
#define WC_GS2(DD)                                                                                              \
  do {                                                                                                          \
    if (!gf_stage_ok(reinterpret_cast<const void*>(&k_gemvs<TW, WG, DD, PAIR, NIN, XB, GB, true>), lds2)) break; \
    hipLaunchKernelGGL((k_gemvs<TW, WG, DD, PAIR, NIN, XB, GB, true>), grid2, block2, lds2, s, a);             \
    return true;                                                                                                \
  } while (0)
      if constexpr (TW == 1) {
        if (per2 <= 4) WC_GS2(4);
        else if (per2 <= 8) WC_GS2(8);
        else WC_GS2(12);
      }
#undef WC_GS2
    }
    return false;
  }
  if (NIN > 1 && !split_ok) return false;
  int parts = 1;
  // fewer blocks than CUs, or pieces handed over anyway (several segments):
  // split the k steps for balance; a full one-segment grid stays whole
  if (split_ok && (tiles * NIN < 256 || NIN > 1)) {
    double best = 0.0;
    for (int pc = 1; pc <= 8; ++pc) {
      const long blocks = static_cast<long>(tiles) * NIN * pc;
      if (pc > 1 && (blocks > kGsMaxPieces || kmax / 32 / pc < W)) break;
      const double per_block = static_cast<double>((blocks + 255) / 256) / static_cast<double>(blocks);
      if (pc == 1 || per_block < best * (1.0 - 1e-9)) {
        best = per_block;
        parts = pc;
      }
    }
  }
  const int pp = (kmax / 32 + parts - 1) / parts;  // steps of the longest part
  const int per = (pp + W - 1) / W;
  const size_t stage = static_cast<size_t>(a.M) * (pp * 32 + 4) * sizeof(float);
  const size_t lds = std::max(stage, static_cast<size_t>(W) * TW * 4 * kWave * sizeof(float));
  if (stage > kGfStageMax || a.M * ((pp * 32 + kGsUnit - 1) / kGsUnit) > kGsMaxUnits) return false;
  if (NIN * parts > 1 && tiles * NIN * parts > kGsMaxPieces) return false;  // the split workspace's slots
  const dim3 grid(tiles, NIN * parts), block(W * kWave);
#define WC_GS(DD)                                                                                            \
  do {                                                                                                       \
    if (!gf_stage_ok(reinterpret_cast<const void*>(&k_gemvs<TW, W, DD, PAIR, NIN, XB, GB>), lds)) return false; \
    hipLaunchKernelGGL((k_gemvs<TW, W, DD, PAIR, NIN, XB, GB>), grid, block, lds, s, a);                      \
    return true;                                                                                             \
  } while (0)
  if (per <= 4) WC_GS(4);
  if constexpr (TW > 1) {
    WC_GS(8);
  } else {
    if (per <= 8) WC_GS(8);
    WC_GS(12);
  }
#undef WC_GS
}

// Few-row MFMA GEMV: 16 (TW = 1) or 32 (TW = 2, and the gate / up pair) rows
// per block, every K a multiple of 32, no last-block norm / normalised-input
// epilogues (those are the one-row kernel's; a bare offset advance is done).
template <bool PAIR, int NIN, int XB>
static bool launch_gemvf(const GemvArgs& a, hipStream_t s) {
  if (a.M < 2 || a.M > kMaxM || a.fin_gain || a.xn_out) return false;
  int gb = 0;
  for (int i = 0; i < a.n_in; ++i) {
    if (a.in[i].K % 32 != 0) return false;
    if (a.in[i].gain) gb |= 1 << i;
  }
  constexpr int kAll = (1 << NIN) - 1;
  const bool wide = PAIR || a.N >= 8192;
  const int rb = PAIR ? 16 : wide ? 32 : 16;
  const dim3 grid((a.N + rb - 1) / rb);
  // single-tile grids of at most one block per CU split each block's k steps
  // over 16 waves (4 steps in flight each) instead of 8 (6 in flight)
  const bool deep = !wide && grid.x <= 256;
  // the input rows staged once per block in LDS (x * gain, fp32) when they fit
  size_t stage = 0;
  int units = 0;
  for (int i = 0; i < a.n_in; ++i) {
    stage += static_cast<size_t>(a.M) * a.in[i].K * sizeof(float);
    units += a.M * ((a.in[i].K + kGfUnit - 1) / kGfUnit);
  }
  const bool stg = units <= 3 * 16 * 3 && stage <= kGfStageMax;
  // staged with every weight step in flight when a block's piece of the rows
  // fits the CU (inputs [M][piece K + 4] fp32)
  {
    bool ok = true;
    for (int i = 0; i < a.n_in; ++i) ok = ok && a.in[i].K <= 10240;
    // one-tile projections only: the gate / up pair and two-tile grids
    // measured faster on k_gemvf (50 MB gate / up at M = 5: 14.2 against 17 us)
    if (ok && !wide) {
      if constexpr (!PAIR) {
        if (gb == kAll) {
          if (launch_gemvs<1, PAIR, NIN, XB, kAll>(a, s)) return true;
        } else if constexpr (NIN == 1) {
          if (launch_gemvs<1, PAIR, NIN, XB, 0>(a, s)) return true;
        }
      }
    }
  }
  GemvArgs as = a;
  as.lds_floats = static_cast<int>(stage / sizeof(float));
  // the dynamic region also holds the waves' partial tiles after the main loop
#define WC_GF_DYN(TW, W) std::max(stage, static_cast<size_t>(W) * NIN * (TW) * 4 * kWave * sizeof(float))
#define WC_GF_L(TW, W, D, GBV)                                                                              \
  do {                                                                                                      \
    if (stg && gf_stage_ok(reinterpret_cast<const void*>(&k_gemvf<TW, W, D, PAIR, NIN, XB, GBV, true>),       \
                           WC_GF_DYN(TW, W)))                                                               \
      hipLaunchKernelGGL((k_gemvf<TW, W, D, PAIR, NIN, XB, GBV, true>), grid, dim3((W) * kWave),              \
                         WC_GF_DYN(TW, W), s, as);                                                          \
    else                                                                                                    \
      hipLaunchKernelGGL((k_gemvf<TW, W, D, PAIR, NIN, XB, GBV>), grid, dim3((W) * kWave), 0, s, a);        \
  } while (0)
#define WC_GF(TW, GBV)                          \
  do {                                          \
    if (TW == 2) WC_GF_L(2, 4, 4, GBV);         \
    else if (deep) WC_GF_L(1, 16, 4, GBV);      \
    else WC_GF_L(1, 8, 6, GBV);                 \
  } while (0)
  if constexpr (PAIR && NIN == 1) {
    if (a.wfrag) {
      if (gb != kAll) return false;
      // four waves of four k steps in flight: 15.1 us for the Qwen3-1.7B pair at
      // 5 rows (eight waves 14.8, sixteen 18.1; 17.0 on the row-major layout)
      if (stg && gf_stage_ok(reinterpret_cast<const void*>(&k_gemvf<2, 4, 4, PAIR, NIN, XB, kAll, true, true>),
                             WC_GF_DYN(2, 4)))
        hipLaunchKernelGGL((k_gemvf<2, 4, 4, PAIR, NIN, XB, kAll, true, true>), grid, dim3(4 * kWave),
                           WC_GF_DYN(2, 4), s, as);
      else
        hipLaunchKernelGGL((k_gemvf<2, 4, 4, PAIR, NIN, XB, kAll, false, true>), grid, dim3(4 * kWave), 0, s, a);
      return true;
    }
  }
  if (a.wfrag) return false;
  if (gb == kAll) {
    if (wide) WC_GF_L(2, 4, 4, kAll); else if constexpr (!PAIR) WC_GF(1, kAll);
  } else if constexpr (NIN == 1) {
    if (wide) WC_GF_L(2, 4, 4, 0); else if constexpr (!PAIR) WC_GF(1, 0);
  } else {
    return false;
  }
#undef WC_GF
#undef WC_GF_L
#undef WC_GF_DYN
  return true;
}

// Few-row VALU GEMV (k_gemvk, csrc/gemvk.hip): false when the launch does not fit it.
bool launch_gemvk_any(const GemvArgs& a, bool pair, int xb, hipStream_t s);

template <bool PAIR, int NIN, int XB>
static bool launch_gemvx(const GemvArgs& a, int steps, hipStream_t s) {
  if (a.M <= 2) return launch_gemvx_r<PAIR, NIN, XB, 2>(a, steps, s);
  if (a.M <= 4) return launch_gemvx_r<PAIR, NIN, XB, 4>(a, steps, s);
  if (a.M <= 8) return launch_gemvx_r<PAIR, NIN, XB, 8>(a, steps, s);
  return false;
}

template <bool PAIR>
static int launch_gemvm(GemvArgs a, int max_k, hipStream_t s) {
  const dim3 grid((a.N + kGemvWaves - 1) / kGemvWaves), block(kGemvThreads);
  const int kr = (max_k + 511) / 512 * 512;
  a.lds_floats = std::min(kGemvLdsBytes / 4, a.M * kr);
  const size_t lds = sizeof(float) * static_cast<size_t>(a.lds_floats);
#define WC_GM(MMV) hipLaunchKernelGGL((k_gemvm<1, MMV, PAIR, 4>), grid, block, lds, s, a)
  if (a.M <= 2)
    WC_GM(2);
  else if (a.M <= 4)
    WC_GM(4);
  else if (a.M <= 8)
    WC_GM(8);
  else
    WC_GM(16);
#undef WC_GM
  WC_LAUNCHED();
  return WC_OK;
}

// One row with every K a multiple of 512 (up to 10240) goes to the
// register-resident kernel; 2..16 rows to the MFMA few-row kernel (K multiple
// of 32), else 2..8 rows to the LDS-staged few-row kernel; anything else to the
// chunked LDS kernel.
static int launch_gemv(const GemvArgs& a, int /*R hint*/, hipStream_t s) {
  if (a.M < 1 || a.M > kMaxM) return set_error(WC_E_INVALID, "gemv: rows %d not in 1..%d", a.M, kMaxM);
  int max_k = 0;
  bool k512 = true;
  int xb = 0;
  for (int i = 0; i < a.n_in; ++i) {
    max_k = std::max(max_k, a.in[i].K);
    k512 = k512 && a.in[i].K % 512 == 0;
    if (a.in[i].dtype == WC_BF16) xb |= 1 << i;
  }
  const int steps = max_k / 512;
  const bool pair = a.epi == kEpiSiluPair;
  bool done = false;
  if (a.wfrag) {
    // fragment-major gate / up pair: the few-row MFMA kernel only
    if (pair && a.n_in == 1 && xb == 0 && a.M > 1) done = launch_gemvf<true, 1, 0>(a, s);
    if (!done) return set_error(WC_E_UNSUPPORTED, "gemv: fragment-major weights need the few-row gate / up pair");
    WC_LAUNCHED();
    return WC_OK;
  }
  if (a.M > 1 && a.M <= 8 && !a.few_mfma) done = launch_gemvk_any(a, pair, xb, s);
  if (!done && a.M > 1) {
    if (pair && a.n_in == 1 && xb == 0)
      done = launch_gemvf<true, 1, 0>(a, s);
    else if (!pair && a.n_in == 1 && xb == 0)
      done = launch_gemvf<false, 1, 0>(a, s);
    else if (!pair && a.n_in == 2 && xb == 2)
      done = launch_gemvf<false, 2, 2>(a, s);
    else if (!pair && a.n_in == 3 && xb == 0)
      done = launch_gemvf<false, 3, 0>(a, s);
    else if (!pair && a.n_in == 3 && xb == 7)
      done = launch_gemvf<false, 3, 7>(a, s);
  }
  if (!done && a.M > 1 && k512) {
    if (pair && a.n_in == 1 && xb == 0)
      done = launch_gemvx<true, 1, 0>(a, steps, s);
    else if (!pair && a.n_in == 1 && xb == 0)
      done = launch_gemvx<false, 1, 0>(a, steps, s);
    else if (!pair && a.n_in == 2 && xb == 2)
      done = launch_gemvx<false, 2, 2>(a, steps, s);
    else if (!pair && a.n_in == 3 && xb == 0)
      done = launch_gemvx<false, 3, 0>(a, steps, s);
    else if (!pair && a.n_in == 3 && xb == 7)
      done = launch_gemvx<false, 3, 7>(a, steps, s);
  }
  if (a.M == 1 && k512) {
    if (pair && a.n_in == 1 && xb == 0)
      done = launch_gemv1_r<true, 1, 0>(a, steps, s);
    else if (!pair && a.n_in == 1 && xb == 0)
      done = launch_gemv1_r<false, 1, 0>(a, steps, s);
    else if (!pair && a.n_in == 2 && xb == 2)
      done = launch_gemv1_r<false, 2, 2>(a, steps, s);
    else if (!pair && a.n_in == 3 && xb == 0)
      done = launch_gemv1_r<false, 3, 0>(a, steps, s);
    else if (!pair && a.n_in == 3 && xb == 7)
      done = launch_gemv1_r<false, 3, 7>(a, steps, s);
  }
  if (done) {
    WC_LAUNCHED();
    return WC_OK;
  }
  return pair ? launch_gemvm<true>(a, max_k, s) : launch_gemvm<false>(a, max_k, s);
}

static GemvArgs gemv_defaults() {
  GemvArgs g{};
  g.n_seg = 1;
  g.seg_start[0] = 0;
  return g;
}

static const uint16_t* u16(const void* p) { return static_cast<const uint16_t*>(p); }

static int check_dims(const wc_drafter_dims* d) {
  WC_REQUIRE(d != nullptr, "dims is NULL");
  WC_REQUIRE(d->hidden > 0 && d->hidden % 8 == 0, "hidden_size must be a positive multiple of 8");
  WC_REQUIRE(d->heads > 0 && d->kv_heads > 0 && d->heads % d->kv_heads == 0, "heads must be a multiple of kv_heads");
  WC_REQUIRE(d->kv_heads <= kMaxKvHeads, "at most %d kv heads", kMaxKvHeads);
  WC_REQUIRE(d->head_dim > 0 && d->head_dim % 8 == 0, "head_dim must be a positive multiple of 8");
  WC_REQUIRE(d->inter > 0 && d->inter % 8 == 0, "intermediate_size must be a positive multiple of 8");
  WC_REQUIRE(d->target_hidden > 0 && d->target_hidden % 8 == 0, "target_hidden_size must be a multiple of 8");
  WC_REQUIRE(d->num_features >= 1 && d->num_features <= WC_MAX_FEATURES, "num_features must be in 1..%d",
             WC_MAX_FEATURES);
  WC_REQUIRE(d->num_layers >= 1 && d->num_layers <= WC_MAX_DRAFTER_LAYERS, "num_layers must be in 1..%d",
             WC_MAX_DRAFTER_LAYERS);
  WC_REQUIRE(d->head_rows >= 1, "head_rows must be positive");
  WC_REQUIRE(d->vocab >= 1, "vocab must be positive");
  return WC_OK;
}

static bool al16(const void* p) { return aligned(p, 16); }

}  // namespace wc

using namespace wc;

namespace wc {

// One row's RMSNorm into y (one block): the general-shape path of the fused
// final norm + head, for hidden sizes the one-row GEMV does not fuse.
__global__ __launch_bounds__(256) void k_row_rmsnorm(const float* __restrict__ x, int64_t ld,
                                                     const int32_t* __restrict__ row_dev, int row_add, int K,
                                                     const uint16_t* __restrict__ gain, float eps,
                                                     float* __restrict__ y, int64_t ldy) {
  __shared__ float red[256 / kWave];
  const int64_t row = row_dev ? static_cast<int64_t>(*row_dev + row_add) : 0;
  const float* xr = x + row * ld;
  float ss = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) ss = fmaf(xr[k], xr[k], ss);
  ss = wave_sum_dpp(ss);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 256 / kWave; ++i) t += red[i];
  const float inv = 1.f / sqrtf(t / static_cast<float>(K) + eps);
  float* yr = y + row * ldy;
  for (int k = threadIdx.x; k < K; k += 256) yr[k] = xr[k] * bf16_to_float(gain[k]) * inv;
}

// Draft head over `rows` input rows; with `norm`, the rows are pre-norm hidden
// states and the final RMSNorm is applied on the fly (its normalised row is
// written to xn_out when not NULL; one row).
static int draft_head_impl(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* out_rows,
                           int64_t out_ld, const int32_t* out_row_dev, int out_row_add, int rows, float* xn_out,
                           int64_t ld_xn, float* logits_out, int64_t logits_ld, int32_t* token_out, int32_t* row_out,
                           const wc_gumbel* gumbel, void* workspace, wc_stream_t stream, bool norm,
                           bool pending = false) {
  if (int rc = check_dims(dims)) return rc;
  // no token output (and no pending keys): the logits alone, no argmax
  const bool logits_only = !token_out && !pending;
  WC_REQUIRE(w && w->head && out_rows && workspace && (!logits_only || (logits_out && !gumbel)),
             "wc_draft_head: NULL argument (the logits alone need logits_out and no Gumbel noise)");
  WC_REQUIRE(!pending || rows == 1, "wc_draft_head_norm_pending: one row");
  WC_REQUIRE(xn_out == nullptr || (rows == 1 && ld_xn >= dims->hidden && ld_xn % 4 == 0 && al16(xn_out)),
             "wc_draft_head_norm: the normalised row needs rows == 1 and a 16-byte aligned output, stride >= hidden");
  WC_REQUIRE(al16(w->head) && al16(workspace), "wc_draft_head: head weight / workspace must be 16-byte aligned");
  WC_REQUIRE(rows >= 1, "wc_draft_head: rows must be positive");
  WC_REQUIRE(out_row_dev == nullptr || rows == 1, "wc_draft_head: a gathered input row needs rows == 1");
  WC_REQUIRE(out_ld >= dims->hidden && out_ld % 4 == 0 && al16(out_rows),
             "wc_draft_head: input rows must be 16-byte aligned with a stride >= hidden_size, multiple of 4");
  WC_REQUIRE(logits_out == nullptr || logits_ld >= dims->head_rows, "wc_draft_head: logits row stride too small");
  WC_REQUIRE(gumbel == nullptr || (gumbel->round_dev && gumbel->temperature > 0.f),
             "wc_draft_head: gumbel needs a round counter and a positive temperature");
  const DrafterWs ws = drafter_ws(*dims, workspace);
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (norm && xn_out && dims->hidden % 512 != 0) {
    // the one-row GEMV fuses the norm for hidden % 512 == 0 only: normalise
    // into xn_out first and run the plain head on it
    WC_REQUIRE(w->final_norm, "wc_draft_head_norm: final norm weight is NULL");
    k_row_rmsnorm<<<1, 256, 0, s>>>(out_rows, out_ld, out_row_dev, out_row_add, dims->hidden, u16(w->final_norm),
                                    dims->eps, xn_out, ld_xn);
    WC_LAUNCHED();
    return draft_head_impl(dims, w, xn_out, ld_xn, out_row_dev, out_row_add, 1, nullptr, 0, logits_out, logits_ld,
                           token_out, row_out, gumbel, workspace, stream, false, pending);
  }
  for (int t0 = 0; t0 < rows; t0 += WC_MAX_STEP_ROWS) {
    const int tr = std::min(WC_MAX_STEP_ROWS, rows - t0);
    GemvArgs h = gemv_defaults();
    h.in[0].x = out_rows + (out_row_dev ? 0 : t0 * out_ld);
    h.in[0].ld = out_ld;
    h.in[0].dtype = WC_F32;
    h.in[0].row_idx = out_row_dev;
    h.in[0].row_add = out_row_dev ? out_row_add : 0;
    h.in[0].K = dims->hidden;
    h.in[0].gain = norm ? u16(w->final_norm) : nullptr;
    h.n_in = 1;
    h.xn_out = xn_out;
    h.ld_xn = ld_xn;
    h.ldw[0] = dims->hidden;
    h.w[0][0] = u16(w->head);
    h.N = dims->head_rows;
    h.seg_start[1] = h.N;
    h.M = tr;
    h.eps = dims->eps;
    h.y = logits_out ? logits_out + t0 * logits_ld : nullptr;
    h.ldy = logits_ld;
    if (logits_only) {
      h.epi = kEpiStore;
      h.few_mfma = 1;
    } else {
      h.epi = kEpiArgmax;
      h.slots = ws.slots;
      h.counter = pending ? nullptr : ws.head_ctr;  // pending: only the block maxima, resolved by the next forward
      h.d2t = w->d2t;
      h.tok_out = pending ? nullptr : token_out + t0;
      h.row_out = row_out && !pending ? row_out + t0 : nullptr;
    }
    if (gumbel) {
      h.use_gumbel = 1;
      h.gumbel.seed = gumbel->seed;
      h.gumbel.round_dev = gumbel->round_dev;
      h.gumbel.purpose = gumbel->purpose + t0;
      h.gumbel.inv_temperature = 1.f / gumbel->temperature;
    }
    if (int rc = launch_gemv(h, dims->head_rows >= 8192 ? 2 : 1, s)) return rc;
  }
  return WC_OK;
}


}  // namespace wc

extern "C" {

int wc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim, float base) {
  WC_REQUIRE(cos_out && sin_out, "wc_rope_table: NULL output");
  WC_REQUIRE(max_pos > 0 && head_dim > 0 && head_dim % 2 == 0, "wc_rope_table: bad sizes");
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float inv = powf(base, -2.f * static_cast<float>(i) / static_cast<float>(head_dim));
    for (int p = 0; p < max_pos; ++p) {
      const float ang = static_cast<float>(p) * inv;
      cos_out[static_cast<int64_t>(p) * half + i] = cosf(ang);
      sin_out[static_cast<int64_t>(p) * half + i] = sinf(ang);
    }
  }
  return WC_OK;
}

size_t wc_drafter_workspace_bytes(const wc_drafter_dims* dims) {
  if (!dims) return 0;
  return drafter_ws(*dims, nullptr).bytes;
}

}  // extern "C"

namespace wc {
// The fuse's GEMV arguments for rows 0..rows-1 of the taps (no gather, every
// row live, rows <= WC_MAX_STEP_ROWS): the launch that runs the greedy verify
// beside the fuse builds its GEMV part from these.
int fuse_gemv_args(const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps, int tap_dtype,
                   int64_t tap_ld, int rows, float* g_out, int64_t g_ld, GemvArgs* out) {
  if (int rc = check_dims(dims)) return rc;
  WC_REQUIRE(w && taps && g_out && out, "fuse: NULL argument");
  WC_REQUIRE(w->fc && al16(w->fc), "fuse: fc weight missing or not 16-byte aligned");
  WC_REQUIRE(tap_dtype == WC_F32 || tap_dtype == WC_BF16, "fuse: tap dtype must be f32 or bf16");
  WC_REQUIRE(tap_ld >= dims->target_hidden && g_ld >= dims->hidden && tap_ld % 8 == 0 && g_ld % 4 == 0,
             "fuse: bad row stride");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_STEP_ROWS, "fuse: rows must be in 1..%d", WC_MAX_STEP_ROWS);
  const int nf = dims->num_features, Dt = dims->target_hidden;
  GemvArgs g = gemv_defaults();
  g.n_in = nf;
  for (int f = 0; f < nf; ++f) {
    WC_REQUIRE(taps[f] != nullptr && al16(taps[f]), "fuse: tap %d is NULL or not 16-byte aligned", f);
    g.in[f].x = taps[f];
    g.in[f].ld = tap_ld;
    g.in[f].dtype = tap_dtype;
    g.in[f].gain = u16(w->feature_norm[f]);
    g.in[f].K = Dt;
    g.ldw[f] = static_cast<int64_t>(nf) * Dt;
    g.w[0][f] = u16(w->fc) + static_cast<int64_t>(f) * Dt;
  }
  g.N = dims->hidden;
  g.seg_start[1] = g.N;
  g.M = rows;
  g.eps = dims->eps;
  g.epi = kEpiStore;
  g.y = g_out;
  g.ldy = g_ld;
  *out = g;
  return WC_OK;
}
}  // namespace wc

extern "C" {

int wc_drafter_fuse(const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps, int tap_dtype,
                    int64_t tap_ld, const int32_t* tap_rows_dev, int tap_rows, int rows, const int32_t* n_rows_dev,
                    float* g_out, int64_t g_ld, void* workspace, wc_stream_t stream) {
  if (int rc = check_dims(dims)) return rc;
  WC_REQUIRE(w && taps && g_out, "wc_drafter_fuse: NULL argument");
  WC_REQUIRE(w->fc && al16(w->fc), "wc_drafter_fuse: fc weight missing or not 16-byte aligned");
  WC_REQUIRE(tap_dtype == WC_F32 || tap_dtype == WC_BF16, "wc_drafter_fuse: tap dtype must be f32 or bf16");
  WC_REQUIRE(tap_ld >= dims->target_hidden && g_ld >= dims->hidden, "wc_drafter_fuse: bad row stride");
  WC_REQUIRE(tap_ld % 8 == 0 && g_ld % 4 == 0, "wc_drafter_fuse: row strides must be multiples of 8 (taps) / 4");
  WC_REQUIRE(rows >= 1, "wc_drafter_fuse: rows must be positive");
  WC_REQUIRE(tap_rows_dev == nullptr || tap_rows >= 1,
             "wc_drafter_fuse: gathering tap rows needs the taps' row count (tap_rows >= 1)");
  WC_REQUIRE(n_rows_dev == nullptr || rows <= WC_MAX_STEP_ROWS,
             "wc_drafter_fuse: a device row count needs rows <= %d", WC_MAX_STEP_ROWS);
  auto s = reinterpret_cast<hipStream_t>(stream);
  const int nf = dims->num_features, Dt = dims->target_hidden;
  const DrafterWs ws = drafter_ws(*dims, workspace);  // NULL workspace: no k split
  for (int t0 = 0; t0 < rows; t0 += WC_MAX_STEP_ROWS) {
    const int tr = std::min(WC_MAX_STEP_ROWS, rows - t0);
    GemvArgs g = gemv_defaults();
    g.gs_part = ws.gs_part;
    g.gs_ctr = ws.gs_ctr;
    g.n_in = nf;
    for (int f = 0; f < nf; ++f) {
      WC_REQUIRE(taps[f] != nullptr && al16(taps[f]), "wc_drafter_fuse: tap %d is NULL or not 16-byte aligned", f);
      g.in[f].x = static_cast<const char*>(taps[f]) + (tap_rows_dev ? 0 : t0 * tap_ld * (tap_dtype ? 2 : 4));
      g.in[f].ld = tap_ld;
      g.in[f].dtype = tap_dtype;
      g.in[f].row_idx = tap_rows_dev ? tap_rows_dev + t0 : nullptr;
      // gathered rows are clamped into the taps: entries past the device row
      // count may be stale (an earlier round's longer keep list)
      g.in[f].max_row = tap_rows_dev ? tap_rows : 0;
      g.in[f].gain = u16(w->feature_norm[f]);  // NULL: feature_norm off (drafter.py:151-152)
      g.in[f].K = Dt;
      g.ldw[f] = static_cast<int64_t>(nf) * Dt;
      g.w[0][f] = u16(w->fc) + static_cast<int64_t>(f) * Dt;
    }
    g.N = dims->hidden;
    g.seg_start[1] = g.N;
    g.M = tr;
    g.m_dev = n_rows_dev;
    g.eps = dims->eps;
    g.epi = kEpiStore;
    g.y = g_out + t0 * g_ld;
    g.ldy = g_ld;
    if (int rc = launch_gemv(g, 1, s)) return rc;
  }
  return WC_OK;
}

}  // extern "C"

namespace wc {
// The token of the pending draft-head argmax (left in the workspace slots by
// the head launch before): where the forward writes it and its head row.
struct PendTok {
  int32_t* tok;
  int32_t* row;
};

static int drafter_forward_impl(const wc_drafter_dims* dims, const wc_drafter_weights* w, const int32_t* tokens_dev,
                                const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add,
                                int rows, const int32_t* n_rows_dev, void* const* k_cache, void* const* v_cache,
                                int kv_dtype, int capacity, const int32_t* offset_dev, int offset_add,
                                const int32_t* positions_dev, const uint8_t* mask_dev, int64_t mask_ld,
                                float* hidden_out, float* out_out, int32_t* advance_dev, void* workspace,
                                wc_stream_t stream, const PendTok* pend) {
  if (int rc = check_dims(dims)) return rc;
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(w && (tokens_dev || pend) && feat && hidden_out && workspace && offset_dev && k_cache && v_cache,
             "wc_drafter_forward: NULL argument");
  WC_REQUIRE(pend == nullptr || (rows == 1 && n_rows_dev == nullptr && mask_dev == nullptr && pend->tok &&
                                 w->layers[0].aux_norm),
             "wc_drafter_forward_pending: one row, no device row count or mask, a token output and a first layer "
             "with the token stream");
  WC_REQUIRE(pend == nullptr || (d.hidden % 512 == 0 && d.hidden <= 10240 && w->layers[0].in_norm),
             "wc_drafter_forward_pending: hidden_size must be a multiple of 512 (at most 10240)");
  WC_REQUIRE(al16(workspace), "wc_drafter_forward: workspace must be 16-byte aligned");
  WC_REQUIRE(rows >= 1, "wc_drafter_forward: rows must be positive");
  WC_REQUIRE(kv_dtype == WC_F32 || kv_dtype == WC_BF16, "wc_drafter_forward: kv dtype must be f32 or bf16");
  WC_REQUIRE(feat_ld >= d.hidden && feat_ld % 4 == 0,
             "wc_drafter_forward: feature row stride must be >= hidden_size and a multiple of 4");
  WC_REQUIRE(al16(feat) && al16(hidden_out) && (out_out == nullptr || al16(out_out)),
             "wc_drafter_forward: buffers must be 16-byte aligned");
  WC_REQUIRE(n_rows_dev == nullptr || rows <= WC_MAX_STEP_ROWS,
             "wc_drafter_forward: a device row count needs rows <= %d", WC_MAX_STEP_ROWS);
  WC_REQUIRE(mask_dev == nullptr || mask_ld >= rows, "wc_drafter_forward: mask row stride too small");
  WC_REQUIRE(w->embed && al16(w->embed) && w->final_norm && w->rope_cos && w->rope_sin && w->rope_max_pos > 0,
             "wc_drafter_forward: embedding / final norm / rope table missing");
  WC_REQUIRE(w->rope_max_pos >= capacity, "wc_drafter_forward: rope table (%d positions) shorter than capacity %d",
             w->rope_max_pos, capacity);
  const int H = d.heads, Hk = d.kv_heads, D = d.head_dim, rep = H / Hk;
  const int tile_rows = std::min(WC_MAX_STEP_ROWS, kMaxQV / rep);
  WC_REQUIRE(tile_rows >= 1, "wc_drafter_forward: GQA group of %d heads too large", rep);
  WC_REQUIRE(n_rows_dev == nullptr || rows <= tile_rows,
             "wc_drafter_forward: a device row count needs rows <= %d for this head grouping", tile_rows);
  for (int li = 0; li < d.num_layers; ++li) {
    const wc_layer_weights& L = w->layers[li];
    WC_REQUIRE(L.in_norm && L.post_norm && L.q && L.k && L.v && L.o && L.q_norm && L.k_norm && L.gate && L.up &&
                   L.down && k_cache[li] && v_cache[li],
               "wc_drafter_forward: layer %d has a NULL weight or cache", li);
    WC_REQUIRE(al16(L.q) && al16(L.k) && al16(L.v) && al16(L.o) && al16(L.gate) && al16(L.up) && al16(L.down),
               "wc_drafter_forward: layer %d weights must be 16-byte aligned", li);
    WC_REQUIRE(al16(k_cache[li]) && al16(v_cache[li]), "wc_drafter_forward: layer %d cache must be 16-byte aligned",
               li);
    if (L.aux_norm)
      WC_REQUIRE(L.aux_q && L.aux_k && L.aux_v && al16(L.aux_q) && al16(L.aux_k) && al16(L.aux_v),
                 "wc_drafter_forward: layer %d aux projections missing", li);
  }
  const DrafterWs ws = drafter_ws(d, workspace);
  auto s = reinterpret_cast<hipStream_t>(stream);
  const int nqkv = (H + 2 * Hk) * D;
  const int splits = std::max(1, std::min(kMaxSplits, (capacity + kAttnChunkMax - 1) / kAttnChunkMax));

  for (int t0 = 0; t0 < rows; t0 += tile_rows) {
    const int tr = std::min(tile_rows, rows - t0);
    const bool last_tile = t0 + tr >= rows;
    for (int li = 0; li < d.num_layers; ++li) {
      const wc_layer_weights& L = w->layers[li];
      const bool last_layer = li == d.num_layers - 1;
      // residual-stream input of this layer: the feature (layer 0) or the previous layer's output
      InSeg xin{};
      xin.dtype = WC_F32;
      xin.K = d.hidden;
      if (li == 0) {
        xin.x = feat + (feat_row_dev ? 0 : t0 * feat_ld);
        xin.ld = feat_ld;
        xin.row_idx = feat_row_dev ? feat_row_dev + t0 : nullptr;
        xin.row_add = feat_row_dev ? feat_row_add : 0;
      } else {
        xin.x = hidden_out + t0 * d.hidden;
        xin.ld = d.hidden;
      }

      // 1. QKV (dual stream on layers with the token embedding)
      GemvArgs q = gemv_defaults();
      q.gs_part = ws.gs_part;
      q.gs_ctr = ws.gs_ctr;
      q.in[0] = xin;
      q.in[0].gain = u16(L.in_norm);
      q.ldw[0] = d.hidden;
      q.w[0][0] = u16(L.q);
      q.w[1][0] = u16(L.k);
      q.w[2][0] = u16(L.v);
      q.n_in = 1;
      if (L.aux_norm) {
        InSeg e{};
        e.x = w->embed;
        e.ld = d.hidden;
        e.dtype = WC_BF16;
        if (pend && li == 0) {  // the token of the pending head argmax, published by block 0
          e.pend_slots = ws.slots;
          e.pend_d2t = w->d2t;
          q.pend_tok_out = pend->tok;
          q.pend_row_out = pend->row;
        } else {
          e.row_idx = pend ? pend->tok : tokens_dev + t0;  // later layers: the token layer 0 published
        }
        e.max_row = d.vocab;
        e.gain = u16(L.aux_norm);
        e.K = d.hidden;
        q.in[1] = e;
        q.ldw[1] = d.hidden;
        q.w[0][1] = u16(L.aux_q);
        q.w[1][1] = u16(L.aux_k);
        q.w[2][1] = u16(L.aux_v);
        q.n_in = 2;
      }
      q.n_seg = 3;
      q.seg_start[1] = H * D;
      q.seg_start[2] = (H + Hk) * D;
      q.seg_start[3] = nqkv;
      q.N = nqkv;
      q.M = tr;
      q.m_dev = n_rows_dev;
      q.eps = d.eps;
      q.epi = kEpiStore;
      q.y = ws.qkv;
      q.ldy = nqkv;
      if (int rc = launch_gemv(q, 1, s)) return rc;

      // 2. attention with q/k norm, RoPE and the KV append
      AttnArgs at{};
      at.qkv = ws.qkv;
      at.ld_qkv = nqkv;
      at.H = H;
      at.Hk = Hk;
      at.rows = tr;
      at.n_rows_dev = n_rows_dev;
      at.q_gain = u16(L.q_norm);
      at.k_gain = u16(L.k_norm);
      at.eps = d.eps;
      at.scale = 1.f / sqrtf(static_cast<float>(D));
      at.rope_cos = w->rope_cos;
      at.rope_sin = w->rope_sin;
      at.rope_max = w->rope_max_pos;
      at.positions = positions_dev ? positions_dev + t0 : nullptr;
      at.kc = k_cache[li];
      at.vc = v_cache[li];
      at.cap = capacity;
      at.offset_dev = offset_dev;
      at.offset_add = offset_add + t0;
      at.mask = mask_dev ? mask_dev + t0 * mask_ld : nullptr;
      at.mask_ld = mask_ld;
      at.window = d.window;
      at.partial = ws.partial;
      at.qv_ld = kMaxQV;
      at.ctr = ws.attn_ctr;
      at.out = ws.attn;
      at.ld_out = H * D;
      at.clear_slots = pend && li == 0 ? ws.slots : nullptr;  // the QKV launch above consumed them
      if (int rc = launch_attention(at, D, kv_dtype, splits, s)) return rc;

      // 3. o_proj with the residual: h1 = h + W_o . o
      GemvArgs o = gemv_defaults();
      o.gs_part = ws.gs_part;
      o.gs_ctr = ws.gs_ctr;
      o.in[0].x = ws.attn;
      o.in[0].ld = H * D;
      o.in[0].dtype = WC_F32;
      o.in[0].K = H * D;
      o.n_in = 1;
      o.ldw[0] = H * D;
      o.w[0][0] = u16(L.o);
      o.N = d.hidden;
      o.seg_start[1] = o.N;
      o.M = tr;
      o.m_dev = n_rows_dev;
      o.eps = d.eps;
      o.epi = kEpiResidual;
      o.res = static_cast<const float*>(xin.x);
      o.ldres = xin.ld;
      o.res_row_idx = xin.row_idx;
      o.res_row_add = xin.row_add;
      o.y = ws.h1;
      o.ldy = d.hidden;
      if (int rc = launch_gemv(o, 1, s)) return rc;

      // 4. gate / up with SiLU(gate) * up
      GemvArgs gu = gemv_defaults();
      gu.gs_part = ws.gs_part;
      gu.gs_ctr = ws.gs_ctr;
      gu.in[0].x = ws.h1;
      gu.in[0].ld = d.hidden;
      gu.in[0].dtype = WC_F32;
      gu.in[0].gain = u16(L.post_norm);
      gu.in[0].K = d.hidden;
      gu.n_in = 1;
      gu.ldw[0] = d.hidden;
      gu.w[0][0] = u16(L.gate);
      gu.w[1][0] = u16(L.up);
      if (L.gate_frag && L.up_frag && tr > 1) {
        // several rows: the MFMA pair kernel over the fragment-major copies,
        // one contiguous kilobyte per weight load instruction
        gu.w[0][0] = u16(L.gate_frag);
        gu.w[1][0] = u16(L.up_frag);
        gu.wfrag = 1;
      }
      gu.N = d.inter;
      gu.M = tr;
      gu.m_dev = n_rows_dev;
      gu.eps = d.eps;
      gu.epi = kEpiSiluPair;
      gu.y = ws.act;
      gu.ldy = d.inter;
      if (int rc = launch_gemv(gu, 1, s)) return rc;

      // 5. down with the residual; the last layer also writes out = RMSNorm(h)
      GemvArgs dn = gemv_defaults();
      dn.gs_part = ws.gs_part;
      dn.gs_ctr = ws.gs_ctr;
      dn.in[0].x = ws.act;
      dn.in[0].ld = d.inter;
      dn.in[0].dtype = WC_F32;
      dn.in[0].K = d.inter;
      dn.n_in = 1;
      dn.ldw[0] = d.inter;
      dn.w[0][0] = u16(L.down);
      dn.N = d.hidden;
      dn.seg_start[1] = dn.N;
      dn.M = tr;
      dn.m_dev = n_rows_dev;
      dn.eps = d.eps;
      dn.epi = kEpiResidual;
      dn.res = ws.h1;
      dn.ldres = d.hidden;
      dn.y = hidden_out + t0 * d.hidden;
      dn.ldy = d.hidden;
      // the last layer's last-block epilogue: the final RMSNorm (unless the
      // caller leaves it to the consumer: out_out == NULL) and the offset advance
      const bool fin = last_layer && out_out != nullptr;
      const bool adv = last_layer && advance_dev && last_tile;
      if (fin || adv) {
        dn.fin_counter = ws.fin_ctr;
        dn.ld_fin = d.hidden;
        if (fin) {
          dn.fin_gain = u16(w->final_norm);
          dn.fin_out = out_out + t0 * d.hidden;
        }
        if (adv) {
          dn.adv_dst = advance_dev;
          dn.adv_src = offset_dev;
          dn.adv_add = offset_add + t0;
        }
      }
      if (int rc = launch_gemv(dn, 1, s)) return rc;
    }
  }
  return WC_OK;
}
}  // namespace wc

extern "C" {

int wc_drafter_forward(const wc_drafter_dims* dims, const wc_drafter_weights* w, const int32_t* tokens_dev,
                       const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add, int rows,
                       const int32_t* n_rows_dev, void* const* k_cache, void* const* v_cache, int kv_dtype,
                       int capacity, const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                       const uint8_t* mask_dev, int64_t mask_ld, float* hidden_out, float* out_out,
                       int32_t* advance_dev, void* workspace, wc_stream_t stream) {
  return wc::drafter_forward_impl(dims, w, tokens_dev, feat, feat_ld, feat_row_dev, feat_row_add, rows, n_rows_dev,
                                  k_cache, v_cache, kv_dtype, capacity, offset_dev, offset_add, positions_dev,
                                  mask_dev, mask_ld, hidden_out, out_out, advance_dev, workspace, stream, nullptr);
}

int wc_drafter_forward_pending(const wc_drafter_dims* dims, const wc_drafter_weights* w, int32_t* token_out,
                               int32_t* row_out, const float* feat, int64_t feat_ld, const int32_t* feat_row_dev,
                               int feat_row_add, void* const* k_cache, void* const* v_cache, int kv_dtype,
                               int capacity, const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                               float* hidden_out, float* out_out, int32_t* advance_dev, void* workspace,
                               wc_stream_t stream) {
  const wc::PendTok pend{token_out, row_out};
  return wc::drafter_forward_impl(dims, w, nullptr, feat, feat_ld, feat_row_dev, feat_row_add, 1, nullptr, k_cache,
                                  v_cache, kv_dtype, capacity, offset_dev, offset_add, positions_dev, nullptr, 0,
                                  hidden_out, out_out, advance_dev, workspace, stream, &pend);
}

int wc_draft_head(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* out_rows, int64_t out_ld,
                  const int32_t* out_row_dev, int out_row_add, int rows, float* logits_out, int64_t logits_ld,
                  int32_t* token_out, int32_t* row_out, const wc_gumbel* gumbel, void* workspace,
                  wc_stream_t stream) {
  return wc::draft_head_impl(dims, w, out_rows, out_ld, out_row_dev, out_row_add, rows, nullptr, 0, logits_out,
                             logits_ld, token_out, row_out, gumbel, workspace, stream, false);
}

int wc_draft_head_norm(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* hidden_rows,
                       int64_t hidden_ld, const int32_t* row_dev, int row_add, float* out_norm, int64_t out_ld,
                       float* logits_out, int64_t logits_ld, int32_t* token_out, int32_t* row_out,
                       const wc_gumbel* gumbel, void* workspace, wc_stream_t stream) {
  WC_REQUIRE(dims && w && w->final_norm, "wc_draft_head_norm: final norm missing");
  WC_REQUIRE(out_norm == nullptr || (out_ld >= dims->hidden && out_ld % 4 == 0 && wc::aligned(out_norm, 16)),
             "wc_draft_head_norm: out rows must be 16-byte aligned with a stride >= hidden_size, multiple of 4");
  return wc::draft_head_impl(dims, w, hidden_rows, hidden_ld, row_dev, row_add, 1, out_norm, out_ld, logits_out,
                             logits_ld, token_out, row_out, gumbel, workspace, stream, true);
}

int wc_draft_head_norm_pending(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* hidden_rows,
                               int64_t hidden_ld, const int32_t* row_dev, int row_add, float* out_norm, int64_t out_ld,
                               float* logits_out, int64_t logits_ld, const wc_gumbel* gumbel, void* workspace,
                               wc_stream_t stream) {
  WC_REQUIRE(dims && w && w->final_norm, "wc_draft_head_norm_pending: final norm missing");
  WC_REQUIRE(out_norm == nullptr || (out_ld >= dims->hidden && out_ld % 4 == 0 && wc::aligned(out_norm, 16)),
             "wc_draft_head_norm_pending: out rows must be 16-byte aligned with a stride >= hidden_size, multiple of 4");
  return wc::draft_head_impl(dims, w, hidden_rows, hidden_ld, row_dev, row_add, 1, out_norm, out_ld, logits_out,
                             logits_ld, nullptr, nullptr, gumbel, workspace, stream, true, true);
}

}  // extern "C"
