// step.hip -- the drafter step for one token in ONE persistent launch.
//
// The step (python/woodcock/spec.py:346-350: the draft head's argmax over
// RMSNorm(h), then the drafter layer on the drafted token; drafter.py:85-127,
// 164-215) is a chain of six dependent phases:
//   H  head GEMV over RMSNorm(h) + argmax (keys into slots)   16384 x 2048
//   Q  QKV over the feedback row and the token's embedding   4096 x (2048 + 2048)
//   A  q/k norm, RoPE, KV append, split-KV attention + merge
//   O  o_proj + residual                                     2048 x 2048
//   G  gate / up + SiLU                                      2 x 6144 x 2048
//   D  down + residual -> h                                  2048 x 6144
// As separate launches each phase pays a launch, a ramp of first loads and a
// drain.  Here the grid is exactly as many blocks as the GPU holds at once
// (checked with the occupancy API), so every block is resident from the start
// and no block ever waits for another to be dispatched.  Every wave owns a
// fixed share of every phase: 4 head rows, 1 QKV row, then an attention item
// (blocks [0, a_blocks)) or an o_proj and a down row (the last waves), and one
// or two gate / up pairs (two on waves without o_proj / down rows).  A wave requests the weights of its next
// phase as soon as its current one is done, before it waits for the phase the
// next one depends on, so the layer's weights stream while the head's argmax,
// the attention and the hand-overs are in progress.  The input row of each
// GEMV phase is staged once per block in LDS (normalised there: one block-wide
// sum of squares), so a wave holds only its weights in registers.
// Hand-over between phases:
//   * every phase counter is kStepLeaves monotone 64-bit leaves (never reset);
//     the blocks add exactly kStepUnit per launch in total after their outputs
//     are published (agent-scope stores, waited for), so phase P of launch L is
//     complete once its leaves sum to (L + 1) kStepUnit;
//   * only the blocks that produce a phase's output arrive for it (every block
//     for the head, QKV and gate / up phases, the merging blocks for the
//     attention, the o_proj / down blocks for those two);
//   * L itself is the final phase's sum / kStepUnit read at block entry: every
//     block reads it before it arrives at the head phase, and no block arrives
//     at the final phase before the head phase is complete;
//   * data produced in the launch is read with agent-scope (sc1) loads;
//   * the head's argmax keys go to one of two slot sets by the parity of L;
//     the other set (the last launch's) is cleared by block 0.
// Every wait is bounded (wc_set_spin_limit): a block that gives up sets the
// sticky status word and goes on, so the launch always ends (its results are
// then invalid and the host reports it).
// The products of every phase are those of the per-op kernels (k_gemv1 /
// k_gemv1s / k_attn_decode) summed in the same order per lane; the RMSNorm
// sums of squares are block-wide here, so the values agree with the per-op
// launches within fp32 rounding.
#include <atomic>
#include <mutex>
#include <unordered_map>

#include "drafter_ws.h"

namespace wc {

constexpr int kStThreads = 256;
constexpr int kStWaves = kStThreads / kWave;
constexpr int kStD = 128;        // head_dim of the one-launch attention
constexpr int kStQV = 4;         // query vectors per kv head (GQA group) at most
constexpr int kStChunk = 32;     // keys per attention chunk
constexpr int kStHidden = 2048;  // the width this kernel is laid out for (8 elements per thread)
constexpr int kStS = kStHidden / 512;  // 512-wide steps of a hidden-wide row
constexpr int kStSI = 12;        // steps of the down projection's input (intermediate <= 6144)
constexpr int kStRH = 4;         // head rows per wave at most
constexpr int kStGX = 1;         // extra gate / up pairs per wave of the extra range
constexpr int kStLdsFloats = kStSI * 512;  // the block's staging area (the down projection's input)

struct StepArgs {
  int hidden, inter, H, Hk, head_rows, vocab, nqkv;
  float eps, scale;
  int splits;  // attention splits per kv head (a_blocks = splits * Hk)
  // layout of the work over the grid's waves
  int nb, nw;       // blocks, waves
  int a_blocks;     // blocks [0, a_blocks) run one attention item each
  int gx_w0, gx_n;  // waves [gx_w0, gx_w0 + gx_n) (none of them o_proj / down waves): kStGX extra gate / up pairs each
  int od_w0;        // waves [od_w0, nw): one o_proj row and one down row each (row = wave - od_w0)
  // the step's input row x[*row_dev + row_add]: the pre-norm hidden state (with
  // the head) or the layer's feature row (without)
  const float* x;
  int64_t ld_x;
  const int32_t* row_dev;
  int row_add;
  // head: out = RMSNorm(x row) * final_norm, written at the same row of `out`
  float* out;
  int64_t ld_out;
  const uint16_t* head_w;
  const uint16_t* final_norm;
  const int32_t* d2t;
  int32_t* token_out;
  int32_t* row_out;
  int fb_out;  // head: the layer's feature row is `out` (post_norm), else the x row
  // layer
  const int32_t* tokens_dev;  // without the head: the token of the aux stream
  const uint16_t* embed;
  const uint16_t *in_norm, *aux_norm, *post_norm, *q_norm, *k_norm;
  const uint16_t *wq, *wk, *wv, *aq, *ak, *av, *wo, *wg, *wu, *wd;
  const float *rope_cos, *rope_sin;
  int rope_max;
  void *kc, *vc;
  int cap;
  const int32_t* offset_dev;
  int offset_add;
  const int32_t* positions;
  int window;
  float *qkv, *attn, *h1, *act, *partial;
  float* hidden_out;
  unsigned long long* ctr;
  unsigned long long* slots;
  unsigned int* split_ctr;
  unsigned int* status;
  unsigned int spin_limit;
  unsigned long long* trace;  // diagnostics (NULL = off): per block and phase {waiting, resumed}
  int leaf_stride;            // uint64s between the leaves of a phase counter (1 .. kStepLeafStride)
  int poll_sleep;             // s_sleep between two polls: 0, 1, 4, 16 or 64 (x 64 clocks)
};

// ------------------------------------------------------------------ hand-over

// Diagnostic timestamp (the 100 MHz real-time counter, one clock for every CU)
// of this block's point k (2 per phase: waiting, resumed; 12 = entry, 13 = exit).
constexpr int kTraceSlots = 16;
__device__ __forceinline__ void tstamp(const StepArgs& a, int k) {
  if (a.trace != nullptr && threadIdx.x == 0)
    a.trace[blockIdx.x * kTraceSlots + k] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ unsigned long long* phase_ctr(const StepArgs& a, int ph) {
  return a.ctr + static_cast<size_t>(ph) * kStepLeaves * kStepLeafStride;
}

__device__ __forceinline__ void poll_pause(int mode) {
  switch (mode) {
    case 0: break;
    case 1: __builtin_amdgcn_s_sleep(1); break;
    case 4: __builtin_amdgcn_s_sleep(4); break;
    case 16: __builtin_amdgcn_s_sleep(16); break;
    default: __builtin_amdgcn_s_sleep(64); break;
  }
}

// Sum of a phase counter's leaves, by one whole wave (kStepLeaves / 64 leaves
// per lane, all loads issued together); the same value on every lane.
__device__ __forceinline__ unsigned long long ctr_sum(const unsigned long long* c, int stride) {
  static_assert(kStepLeaves % kWave == 0, "whole waves of leaves");
  const int lane = threadIdx.x % kWave;
  unsigned long long w[kStepLeaves / kWave];
#pragma unroll
  for (int j = 0; j < kStepLeaves / kWave; ++j) w[j] = atomic_load_u64(c + (lane + j * kWave) * stride);
  unsigned long long v = 0ull;
#pragma unroll
  for (int j = 0; j < kStepLeaves / kWave; ++j) v += w[j];
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// Block i of a phase of n blocks adds its share: kStepUnit per launch in total.
__device__ __forceinline__ void ctr_arrive(unsigned long long* c, int stride, int i, int n) {
  const unsigned long long v = i == 0 ? kStepUnit - static_cast<unsigned long long>(n - 1) : 1ull;
  __hip_atomic_fetch_add(c + (i % kStepLeaves) * stride, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every wave's published stores are done, then thread 0 arrives.
__device__ __forceinline__ void block_arrive(const StepArgs& a, int ph, int i, int n) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) ctr_arrive(phase_ctr(a, ph), a.leaf_stride, i, n);
}

// One wave polls phase `ph` until it reaches `target` (bounded; a give-up sets
// the sticky status).
__device__ __forceinline__ void wave_wait(const StepArgs& a, int ph, unsigned long long target) {
  for (unsigned int it = 0;; ++it) {
    if (ctr_sum(phase_ctr(a, ph), a.leaf_stride) >= target) break;
    if (it >= a.spin_limit) {
      if (threadIdx.x % kWave == 0) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    poll_pause(a.poll_sleep);
  }
  asm volatile("" ::: "memory");  // no load of the phase's outputs moves above the wait
}

// Block-wide wait for phase `ph` of launch L: wave 0 polls, the other waves
// wait at an LDS-only barrier (their loads in flight stay in flight); the
// compiler may move no memory access across it.
__device__ __forceinline__ void block_wait(const StepArgs& a, int ph, unsigned long long L) {
  tstamp(a, 2 * ph);
  if (threadIdx.x / kWave == 0) wave_wait(a, ph, (L + 1ull) * kStepUnit);
  lds_barrier();
  asm volatile("" ::: "memory");
  tstamp(a, 2 * ph + 1);
}

// 16-byte load of data published earlier in this launch, after the wait for
// its phase.  A plain load (it may be served by this XCD's L2): the L2s are
// invalidated at every kernel start, and no block reads these buffers before
// the phase that writes them is complete, so the first read on each XCD
// misses and fetches the published value; the other waves of that XCD hit.
// (Every wave reading the same few kilobytes with agent-scope loads
// serialises on those lines at the memory side.)
__device__ __forceinline__ uint4 ld_pub16(const float* p) { return *reinterpret_cast<const uint4*>(p); }

__device__ __forceinline__ float4 f4(const uint4 q) {
  return make_float4(__uint_as_float(q.x), __uint_as_float(q.y), __uint_as_float(q.z), __uint_as_float(q.w));
}

__device__ __forceinline__ int64_t step_row(const StepArgs& a) {
  return a.row_dev ? static_cast<int64_t>(*a.row_dev + a.row_add) : 0;
}

// Sum over the block (four waves); the same value in every thread.  s_red
// holds kStWaves floats; the trailing barrier lets the next call reuse it.
__device__ __forceinline__ float step_block_sum(float v, float* s_red) {
  v = wave_sum_dpp(v);
  if (threadIdx.x % kWave == 0) s_red[threadIdx.x / kWave] = v;
  lds_barrier();
  const float t = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  lds_barrier();
  return t;
}

// 8 consecutive fp32 / bf16 values -> float[8]
__device__ __forceinline__ void unpack_f32x8(const uint4 a, const uint4 b, float* x) {
  x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y); x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
  x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y); x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
}
__device__ __forceinline__ void unpack_bf16x8(const uint4 h, float* x) {
  x[0] = bf16_lo(h.x); x[1] = bf16_hi(h.x); x[2] = bf16_lo(h.y); x[3] = bf16_hi(h.y);
  x[4] = bf16_lo(h.z); x[5] = bf16_hi(h.z); x[6] = bf16_lo(h.w); x[7] = bf16_hi(h.w);
}

// Stage a hidden-wide row (thread t: elements 8t .. 8t + 7) as x * gain into
// xs (gain already widened in g) and return 1 / rms(x) from the block-wide sum
// of squares; as in the per-op kernels the scale is applied to the dot product.
__device__ __forceinline__ float stage_norm(const float* x, const float* g, float eps, float* xs, float* s_red) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  float4* dst = reinterpret_cast<float4*>(xs + threadIdx.x * 8);
  dst[0] = make_float4(x[0] * g[0], x[1] * g[1], x[2] * g[2], x[3] * g[3]);
  dst[1] = make_float4(x[4] * g[4], x[5] * g[5], x[6] * g[6], x[7] * g[7]);
  return 1.f / sqrtf(step_block_sum(ss, s_red) / static_cast<float>(kStHidden) + eps);
}

// part += dot(w row slice, staged row) over the kStS steps of a hidden-wide row
__device__ __forceinline__ float dot_staged(const uint4 (&w)[kStS], const float* xs, float part) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int u = 0; u < kStS; ++u) {
    const float* xp = xs + u * kWave * 8 + lane * 8;
    part += dot8(w[u], *reinterpret_cast<const float4*>(xp), *reinterpret_cast<const float4*>(xp + 4));
  }
  return part;
}

__device__ __forceinline__ void load_row(const uint16_t* row, uint4 (&w)[kStS]) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int u = 0; u < kStS; ++u) w[u] = *reinterpret_cast<const uint4*>(row + u * kWave * 8 + lane * 8);
}

// ------------------------------------------------------------------ A: attention

// The chunk of up to kStChunk keys at [c0, c0 + kStChunk) of one kv head:
// scores (group sums of the lanes' products), online softmax, probability-
// weighted V -- k_attn_decode's steps 2-4 for one chunk.
template <typename KT, int NL>
__device__ __forceinline__ void attn_chunk(const uint4 (&kreg)[NL], const uint4 (&vreg)[NL], int c0, int ke,
                                           int offset, int window, int QV, float scale, const float (*qs)[kStD],
                                           const float* nk, const float* nv, float (*vls)[kStD],
                                           float (*s_p)[kStChunk], float* s_m, float* s_l, float* s_alpha,
                                           float* o) {
  constexpr int D = kStD;
  constexpr int VE = 16 / static_cast<int>(sizeof(KT));
  constexpr int LK = D / VE;
  constexpr int KPB = kStThreads / LK;
  constexpr int OPT = kStQV * D / kStThreads;
  constexpr int VSTEP = kStThreads / D;
  const int t = threadIdx.x;
  const int kr = t / LK, e0 = (t % LK) * VE;
  const int n = min(kStChunk, ke - c0);
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int j = i * KPB + kr, tt = c0 + j;
    float kf[VE], vf[VE];
    if (tt >= offset) {
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        kf[e] = nk[e0 + e];
        vf[e] = nv[e0 + e];
      }
    } else {
      unpack16<KT>(kreg[i], kf);
      unpack16<KT>(vreg[i], vf);
    }
#pragma unroll
    for (int e = 0; e < VE; e += 4)
      *reinterpret_cast<float4*>(&vls[j][e0 + e]) = make_float4(vf[e], vf[e + 1], vf[e + 2], vf[e + 3]);
#pragma unroll
    for (int v = 0; v < kStQV; ++v) {
      if (v >= QV) break;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < VE; e += 4) {
        const float4 q = *reinterpret_cast<const float4*>(&qs[v][e0 + e]);
        d = fmaf(kf[e], q.x, d);
        d = fmaf(kf[e + 1], q.y, d);
        d = fmaf(kf[e + 2], q.z, d);
        d = fmaf(kf[e + 3], q.w, d);
      }
      d = group_sum<LK>(d);
      const bool vis = j < n && tt <= offset && (window <= 0 || tt > offset - window);
      if (t % LK == 0) s_p[v][j] = vis ? scale * d : -INFINITY;
    }
  }
  lds_barrier();
  if (t < kStQV * 16) {
    const int v = t / 16, g = t % 16;
    const bool live = v < QV;
    const float s0 = live && g < n ? s_p[v][g] : -INFINITY;
    const float s1 = live && g + 16 < n ? s_p[v][g + 16] : -INFINITY;
    const float mx = row16_max(fmaxf(s0, s1));
    const float m_old = s_m[v];
    const float m_new = fmaxf(m_old, mx);
    const float alpha = m_new == -INFINITY ? 1.f : (m_old == -INFINITY ? 0.f : expf(m_old - m_new));
    const float p0 = s0 == -INFINITY ? 0.f : expf(s0 - m_new);
    const float p1 = s1 == -INFINITY ? 0.f : expf(s1 - m_new);
    const float ls = row16_sum(p0 + p1);
    s_p[v][g] = p0;
    s_p[v][g + 16] = p1;
    if (g == 0) {
      s_m[v] = m_new;
      s_l[v] = s_l[v] * alpha + ls;
      s_alpha[v] = alpha;
    }
  }
  lds_barrier();
  const int od = t % D, ov0 = t / D;
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float acc0 = o[k] * s_alpha[v], acc1 = 0.f;
    int j = 0;
    for (; j + 1 < n; j += 2) {
      acc0 = fmaf(s_p[v][j], vls[j][od], acc0);
      acc1 = fmaf(s_p[v][j + 1], vls[j + 1][od], acc1);
    }
    if (j < n) acc0 = fmaf(s_p[v][j], vls[j][od], acc0);
    o[k] = acc0 + acc1;
  }
  lds_barrier();  // vls / s_p are rewritten by the next chunk
}

template <typename KT, int NL>
__device__ __forceinline__ void attn_load(const KT* kc, const KT* vc, int c0, int ke, uint4 (&kreg)[NL],
                                          uint4 (&vreg)[NL]) {
  constexpr int VE = 16 / static_cast<int>(sizeof(KT));
  constexpr int LK = kStD / VE;
  constexpr int KPB = kStThreads / LK;
  const int kr = threadIdx.x / LK, e0 = (threadIdx.x % LK) * VE;
  const int last = max(ke - 1, 0);
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t r = min(c0 + i * KPB + kr, last);
    kreg[i] = *reinterpret_cast<const uint4*>(kc + r * kStD + e0);
    vreg[i] = *reinterpret_cast<const uint4*>(vc + r * kStD + e0);
  }
}

struct AttnLds {
  float qs[kStQV][kStD];
  float nk[kStD], nv[kStD];
  float vls[kStChunk][kStD];
  float s_p[kStQV][kStChunk];
  float s_m[kStQV], s_l[kStQV], s_alpha[kStQV];
  float s_w[kStQV][kMaxSplits];
  float s_den[kStQV];
  int s_last;
};

// k_attn_decode<128, KT, 4> for one row: block (kv head kh, split).  Its first
// two chunks of cache rows, the RoPE row and the norm gains are requested
// before the wait for the QKV phase.  The last split of a kv head to finish
// merges all splits and arrives for the attention phase.
template <typename KT>
__device__ void ph_attn(const StepArgs& a, int i, unsigned long long L, AttnLds& m) {
  constexpr int D = kStD, half = D / 2;
  constexpr int VE = 16 / static_cast<int>(sizeof(KT));
  constexpr int LK = D / VE;
  constexpr int KPB = kStThreads / LK;
  constexpr int NL = kStChunk / KPB;
  constexpr int OPT = kStQV * D / kStThreads;
  constexpr int VSTEP = kStThreads / D;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int S = a.splits, kh = i / S, split = i % S;
  const int rep = a.H / a.Hk, QV = rep;
  const int offset = *a.offset_dev + a.offset_add;
  const int T = min(offset + 1, a.cap);
  const int per = (T + S - 1) / S;
  const int kb = min(T, split * per), ke = min(T, kb + per);
  KT* kc = static_cast<KT*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  KT* vc = static_cast<KT*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  // 1. cache rows of the first two chunks, RoPE row, gains
  uint4 ka[NL], va[NL], kb2[NL], vb2[NL];
  attn_load<KT, NL>(kc, vc, kb, ke, ka, va);
  attn_load<KT, NL>(kc, vc, kb + kStChunk, ke, kb2, vb2);
  const int pos = min(max(a.positions ? a.positions[0] : offset, 0), a.rope_max - 1);
  const float rc = a.rope_cos[static_cast<int64_t>(pos) * half + lane];
  const float rs = a.rope_sin[static_cast<int64_t>(pos) * half + lane];
  const float gql = bf16_to_float(a.q_norm[lane]), gqh = bf16_to_float(a.q_norm[lane + half]);
  const float gkl = bf16_to_float(a.k_norm[lane]), gkh = bf16_to_float(a.k_norm[lane + half]);
  if (t < kStQV) {
    m.s_m[t] = -INFINITY;
    m.s_l[t] = 0.f;
  }
  // 2. the QKV phase's q, k, v rows
  block_wait(a, kPhQkv, L);
  auto norm_rope = [&](float lo, float hi, float gl, float gh) {
    const float ss = wave_sum_dpp(fmaf(hi, hi, lo * lo));
    const float inv = 1.f / sqrtf(ss / static_cast<float>(D) + a.eps);
    const float x1 = lo * inv * gl, x2 = hi * inv * gh;
    return make_float2(x1 * rc - x2 * rs, x2 * rc + x1 * rs);
  };
  if (wave < QV) {
    const float* q = a.qkv + (kh * rep + wave) * D;
    const float2 r = norm_rope(q[lane], q[lane + half], gql, gqh);  // published: see ld_pub16
    m.qs[wave][lane] = r.x;
    m.qs[wave][lane + half] = r.y;
  }
  const int tt = offset;  // the appended row
  if (wave == kStWaves - 1 && tt >= kb && tt < ke) {
    const float* kn = a.qkv + (a.H + kh) * D;
    const float* vn = a.qkv + (a.H + a.Hk + kh) * D;
    const float kl = kn[lane], khv = kn[lane + half];
    const float vl = vn[lane], vh = vn[lane + half];
    const float2 r = norm_rope(kl, khv, gkl, gkh);
    m.nk[lane] = kv_store<KT>(kc, static_cast<int64_t>(tt) * D + lane, r.x);
    m.nk[lane + half] = kv_store<KT>(kc, static_cast<int64_t>(tt) * D + lane + half, r.y);
    m.nv[lane] = kv_store<KT>(vc, static_cast<int64_t>(tt) * D + lane, vl);
    m.nv[lane + half] = kv_store<KT>(vc, static_cast<int64_t>(tt) * D + lane + half, vh);
  }
  lds_barrier();
  // 3. chunks: two register sets, each refilled two chunks ahead
  float o[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) o[k] = 0.f;
  for (int c0 = kb; c0 < ke; c0 += 2 * kStChunk) {
    attn_chunk<KT, NL>(ka, va, c0, ke, offset, a.window, QV, a.scale, m.qs, m.nk, m.nv, m.vls, m.s_p, m.s_m, m.s_l,
                       m.s_alpha, o);
    if (c0 + 2 * kStChunk < ke) attn_load<KT, NL>(kc, vc, c0 + 2 * kStChunk, ke, ka, va);
    if (c0 + kStChunk < ke) {
      attn_chunk<KT, NL>(kb2, vb2, c0 + kStChunk, ke, offset, a.window, QV, a.scale, m.qs, m.nk, m.nv, m.vls, m.s_p,
                         m.s_m, m.s_l, m.s_alpha, o);
      if (c0 + 3 * kStChunk < ke) attn_load<KT, NL>(kc, vc, c0 + 3 * kStChunk, ke, kb2, vb2);
    }
  }
  // 4. this split's (m, l, o), published; an empty range leaves m = -inf, l = 0, o = 0
  const int od = t % D, ov0 = t / D;
  float* part = a.partial + (static_cast<int64_t>(kh) * S + split) * kStQV * (D + 2);
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float* pv = part + v * (D + 2);
    publish_f32(pv + 2 + od, o[k]);
    if (od == 0) {
      publish_f32(pv, m.s_m[v]);
      publish_f32(pv + 1, m.s_l[v]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    unsigned int* ctr = a.split_ctr + kh * kCounterStride;
    const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      static_cast<unsigned int>(S - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    m.s_last = last;
  }
  __syncthreads();
  if (!m.s_last) return;
  // 5. the last split of this kv head merges every split's (m, l, o)
  const float* base = a.partial + static_cast<int64_t>(kh) * S * kStQV * (D + 2);
  const int64_t sstride = static_cast<int64_t>(kStQV) * (D + 2);
  float ov[OPT][kMaxSplits];
#pragma unroll
  for (int k = 0; k < OPT; ++k)
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
      ov[k][sp] = fetch_f32(base + min(sp, S - 1) * sstride + min(ov0 + VSTEP * k, QV - 1) * (D + 2) + 2 + od);
  {
    const int v = min(wave, QV - 1);  // wave w: query vector w; lane = split
    const float ms = fetch_f32(base + min(lane, S - 1) * sstride + v * (D + 2));
    const float ls = fetch_f32(base + min(lane, S - 1) * sstride + v * (D + 2) + 1);
    if (wave < QV) {
      const float m_s = lane < S ? ms : -INFINITY;
      const float M = wave_max_dpp(m_s);
      const float wgt = m_s == -INFINITY ? 0.f : expf(m_s - M);
      const float den = wave_sum_dpp(lane < S ? ls * wgt : 0.f);
      if (lane < kMaxSplits) m.s_w[wave][lane] = lane < S ? wgt : 0.f;
      if (lane == 0) m.s_den[wave] = den;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float num = 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp) num = fmaf(m.s_w[v][sp], sp < S ? ov[k][sp] : 0.f, num);
    publish_f32(a.attn + (kh * rep + v) * D + od, num / m.s_den[v]);
  }
  block_arrive(a, kPhAttn, kh, a.Hk);
}

// ------------------------------------------------------------------ GEMV phases

// Weight row of logical QKV row n (q | k | v) in segment `aux`.
__device__ __forceinline__ const uint16_t* qkv_row(const StepArgs& a, int n, bool aux) {
  const int nq = a.H * kStD, nk = a.Hk * kStD;
  if (n < nq) return (aux ? a.aq : a.wq) + static_cast<int64_t>(n) * a.hidden;
  if (n < nq + nk) return (aux ? a.ak : a.wk) + static_cast<int64_t>(n - nq) * a.hidden;
  return (aux ? a.av : a.wv) + static_cast<int64_t>(n - nq - nk) * a.hidden;
}

// Gate / up weights of up to NP pairs (pair p: gate row p, up row p).
template <int NP>
struct Pairs {
  uint4 g[NP][kStS], u[NP][kStS];
  int row[NP];
  int n;
};

template <int NP>
__device__ __forceinline__ void pairs_load(const StepArgs& a, Pairs<NP>& p) {
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int r = min(max(p.row[j], 0), a.inter - 1);
    load_row(a.wg + static_cast<int64_t>(r) * a.hidden, p.g[j]);
    load_row(a.wu + static_cast<int64_t>(r) * a.hidden, p.u[j]);
  }
}

// G: wait for o_proj, stage RMSNorm(h1) * post_norm (coherent loads of h1), the
// wave's pairs -> act = silu(gate) * up, published; arrive.
template <int NP>
__device__ __forceinline__ void ph_gate_up(const StepArgs& a, const Pairs<NP>& p, unsigned long long L, float* xs,
                                           float* s_red) {
  const int t = threadIdx.x, lane = t % kWave;
  block_wait(a, kPhO, L);
  float x[8], g[8];
  unpack_f32x8(ld_pub16(a.h1 + 8 * t), ld_pub16(a.h1 + 8 * t + 4), x);
  unpack_bf16x8(*reinterpret_cast<const uint4*>(a.post_norm + t * 8), g);
  const float inv = stage_norm(x, g, a.eps, xs, s_red);
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    if (j >= p.n) break;  // wave-uniform
    const float gv = wave_sum_dpp(fmaf(dot_staged(p.g[j], xs, 0.f), inv, 0.f));
    const float uv = wave_sum_dpp(fmaf(dot_staged(p.u[j], xs, 0.f), inv, 0.f));
    if (lane == 0 && p.row[j] < a.inter) publish_f32(a.act + p.row[j], gv / (1.f + expf(-gv)) * uv);
  }
  block_arrive(a, kPhGateUp, blockIdx.x, a.nb);
}

// ------------------------------------------------------------------ the kernel

template <typename KT, bool HEAD, bool AUX>
__global__ __launch_bounds__(kStThreads) void k_step(StepArgs a) {
  constexpr size_t kAttnF = (sizeof(AttnLds) + 3) / 4;
  constexpr size_t kXsF = kStLdsFloats;
  __shared__ __attribute__((aligned(16))) float s_xs[kAttnF > kXsF ? kAttnF : kXsF];
  __shared__ float s_red[kStWaves];
  __shared__ unsigned long long s_key[kStWaves];
  __shared__ int s_tok;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int b = blockIdx.x, gw = b * kStWaves + wave;
  tstamp(a, 12);
  unsigned long long L = 0;
  if (wave == 0) L = ctr_sum(phase_ctr(a, kPhDown), a.leaf_stride) / kStepUnit;
  const int64_t xr = step_row(a);
  float xv[8];  // the thread's 8 elements of the step's input row
  {
    const float* xp = a.x + xr * a.ld_x + t * 8;
    unpack_f32x8(*reinterpret_cast<const uint4*>(xp), *reinterpret_cast<const uint4*>(xp + 4), xv);
  }

  // ---- H: head rows gw * kStRH .. + kStRH (rows past head_rows skipped)
  float fb[8];  // the layer's feature row (the thread's 8 elements)
  if constexpr (HEAD) {
    uint4 w[kStRH][kStS];
#pragma unroll
    for (int j = 0; j < kStRH; ++j)
      load_row(a.head_w + static_cast<int64_t>(min(gw * kStRH + j, a.head_rows - 1)) * a.hidden, w[j]);
    float gf[8];
    unpack_bf16x8(*reinterpret_cast<const uint4*>(a.final_norm + t * 8), gf);
    const float inv_f = stage_norm(xv, gf, a.eps, s_xs, s_red);
#pragma unroll
    for (int e = 0; e < 8; ++e) fb[e] = a.fb_out ? xv[e] * gf[e] * inv_f : xv[e];
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < kStRH; ++j) {
      const int r = gw * kStRH + j;
      if (r >= a.head_rows) break;  // wave-uniform
      const float z = wave_sum_dpp(fmaf(dot_staged(w[j], s_xs, 0.f), inv_f, 0.f));
      const unsigned long long key = argmax_key(z, r);
      best = key > best ? key : best;
    }
    if (lane == 0) s_key[wave] = best;
    lds_barrier();
    if (wave == 0) {
      // `out` (the drafter's output, the o_proj residual with post_norm), published
      if (b == 0 && a.out) {
        float* xo = a.out + xr * a.ld_out;
        for (int k = lane; k < kStHidden; k += kWave) publish_f32(xo + k, s_xs[k] * inv_f);
      }
      if (lane == 0) {
#pragma unroll
        for (int v = 1; v < kStWaves; ++v) best = s_key[v] > best ? s_key[v] : best;
        unsigned long long* set = a.slots + (L & 1ull) * kSlots * kSlotStride;
        if (best) atomic_max_u64(&set[(b % kSlots) * kSlotStride], best);
      }
      __builtin_amdgcn_s_waitcnt(0);
      if (lane == 0) ctr_arrive(phase_ctr(a, kPhHead), a.leaf_stride, b, a.nb);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) fb[e] = xv[e];
  }

  // ---- Q: row gw; the feature segment before the head's argmax is known
  {
    const int qrow = min(gw, a.nqkv - 1);
    uint4 w0[kStS], w1[kStS];
    load_row(qkv_row(a, qrow, false), w0);
    if (AUX) load_row(qkv_row(a, qrow, true), w1);
    float gi[8];
    unpack_bf16x8(*reinterpret_cast<const uint4*>(a.in_norm + t * 8), gi);
    float* xs0 = s_xs + kStHidden;
    const float inv0 = stage_norm(fb, gi, a.eps, xs0, s_red);
    float tq = fmaf(dot_staged(w0, xs0, 0.f), inv0, 0.f);
    if (AUX) {
      if (HEAD) {
        tstamp(a, 2 * kPhHead);
        if (wave == 0) {
          wave_wait(a, kPhHead, (L + 1ull) * kStepUnit);
          const unsigned long long* set = a.slots + (L & 1ull) * kSlots * kSlotStride;
          unsigned long long k = set[(lane % kSlots) * kSlotStride];  // complete: see ld_pub16
          k = wave_max_u64(k);
          const int hrow = min(max(argmax_key_index(k), 0), a.head_rows - 1);
          const int tok = min(max(a.d2t ? a.d2t[hrow] : hrow, 0), a.vocab - 1);
          if (lane == 0) {
            s_tok = tok;
            if (b == 0) {
              a.token_out[0] = tok;
              if (a.row_out) a.row_out[0] = hrow;
            }
          }
        }
      } else if (t == 0) {
        s_tok = min(max(a.tokens_dev[0], 0), a.vocab - 1);
      }
      lds_barrier();
      asm volatile("" ::: "memory");
      tstamp(a, 2 * kPhHead + 1);
      const uint16_t* er = a.embed + static_cast<int64_t>(s_tok) * a.hidden + t * 8;
      float e[8], ga[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(er), e);
      unpack_bf16x8(*reinterpret_cast<const uint4*>(a.aux_norm + t * 8), ga);
      float* xs1 = s_xs + 2 * kStHidden;
      const float inv1 = stage_norm(e, ga, a.eps, xs1, s_red);
      tq = fmaf(dot_staged(w1, xs1, 0.f), inv1, tq);
    }
    const float acc = wave_sum_dpp(tq);
    if (lane == 0 && gw < a.nqkv) publish_f32(a.qkv + gw, acc);
    if (b == 0 && t < kSlots) {
      // the last launch's slot set, for the next launch with the head
      unsigned long long* other = a.slots + ((L + 1ull) & 1ull) * kSlots * kSlotStride;
      atomic_store_u64(&other[t * kSlotStride], 0ull);
    }
    block_arrive(a, kPhQkv, b, a.nb);
    if (!HEAD && b == 0 && t == 0)  // no head phase: its counter advances all the same
      __hip_atomic_fetch_add(phase_ctr(a, kPhHead), kStepUnit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- the block's group: attention, extra gate / up pairs, or o_proj + down
  float* xs = s_xs;
  if (b < a.a_blocks) {
    ph_attn<KT>(a, b, L, *reinterpret_cast<AttnLds*>(s_xs));
    Pairs<1 + kStGX> p;
    const bool extra = gw >= a.gx_w0 && gw < a.gx_w0 + a.gx_n;
    p.row[0] = gw;
#pragma unroll
    for (int j = 0; j < kStGX; ++j) p.row[1 + j] = a.nw + (gw - a.gx_w0) * kStGX + j;
    p.n = gw >= a.inter ? 0 : !extra ? 1 : 1 + min(kStGX, max(0, a.inter - (a.nw + (gw - a.gx_w0) * kStGX)));
    pairs_load(a, p);
    ph_gate_up(a, p, L, xs, s_red);
  } else if (gw < a.od_w0) {
    Pairs<1 + kStGX> p;
    const bool extra = gw >= a.gx_w0 && gw < a.gx_w0 + a.gx_n;
    p.row[0] = gw;
#pragma unroll
    for (int j = 0; j < kStGX; ++j) p.row[1 + j] = a.nw + (gw - a.gx_w0) * kStGX + j;
    p.n = gw >= a.inter ? 0 : !extra ? 1 : 1 + min(kStGX, max(0, a.inter - (a.nw + (gw - a.gx_w0) * kStGX)));
    pairs_load(a, p);
    ph_gate_up(a, p, L, xs, s_red);
  } else {
    // o_proj row and down row r = gw - od_w0 (< hidden), one gate / up pair
    const int r = gw - a.od_w0;
    const int rc = min(r, a.hidden - 1);
    uint4 wo[kStS];
    load_row(a.wo + static_cast<int64_t>(rc) * a.hidden, wo);
    Pairs<1> p;
    p.row[0] = gw;
    p.n = gw < a.inter ? 1 : 0;
    pairs_load(a, p);
    // residual: the layer's feature row (`out` of this launch's head when it is the feature)
    float res = 0.f;
    if (!(HEAD && a.fb_out)) res = a.x[xr * a.ld_x + rc];
    block_wait(a, kPhAttn, L);
    if (HEAD && a.fb_out) res = a.out[xr * a.ld_out + rc];  // published: see ld_pub16
    float part = 0.f;
#pragma unroll
    for (int u = 0; u < kStS; ++u) {
      const int k = u * kWave * 8 + lane * 8;
      part = dot8_acc(wo[u], f4(ld_pub16(a.attn + k)), f4(ld_pub16(a.attn + k + 4)), part);
    }
    const float acc = wave_sum_dpp(fmaf(part, 1.f, 0.f));
    if (lane == 0 && r < a.hidden) publish_f32(a.h1 + r, res + acc);
    const int ob = b - a.od_w0 / kStWaves, on = a.nb - a.od_w0 / kStWaves;  // o_proj / down blocks
    block_arrive(a, kPhO, ob, on);
    uint4 wd[kStSI];
    const int steps = a.inter / (kWave * 8);
    {
      const uint16_t* wr = a.wd + static_cast<int64_t>(rc) * a.inter + lane * 8;
#pragma unroll
      for (int u = 0; u < kStSI; ++u) wd[u] = *reinterpret_cast<const uint4*>(wr + min(u, steps - 1) * kWave * 8);
    }
    ph_gate_up(a, p, L, xs, s_red);
    // D: down + residual
    block_wait(a, kPhGateUp, L);
    {
      constexpr int C = kStSI * 512 / (kStThreads * 8);
      uint4 sx[C][2];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k = min(c * kStThreads * 8 + t * 8, a.inter - 8);
        sx[c][0] = ld_pub16(a.act + k);
        sx[c][1] = ld_pub16(a.act + k + 4);
      }
      const float hres = a.h1[rc];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k = c * kStThreads * 8 + t * 8;
        if (k < a.inter) {
          *reinterpret_cast<uint4*>(xs + k) = sx[c][0];
          *reinterpret_cast<uint4*>(xs + k + 4) = sx[c][1];
        }
      }
      lds_barrier();
      float pd = 0.f;
#pragma unroll
      for (int u = 0; u < kStSI; ++u) {
        if (u >= steps) continue;
        const float* xp = xs + u * kWave * 8 + lane * 8;
        pd = dot8_acc(wd[u], *reinterpret_cast<const float4*>(xp), *reinterpret_cast<const float4*>(xp + 4), pd);
      }
      const float dsum = wave_sum_dpp(fmaf(pd, 1.f, 0.f));
      if (lane == 0 && r < a.hidden) a.hidden_out[r] = hres + dsum;
    }
    block_arrive(a, kPhDown, ob, on);
  }
  tstamp(a, 13);
}

// ------------------------------------------------------------------ host side

// Process-wide switch of the one-launch path (wc_set_one_launch_step).
static std::atomic<int> g_one_launch{1};
// Diagnostic per-block timestamps (wc_set_step_trace), NULL = off.
static std::atomic<unsigned long long*> g_trace{nullptr};
// Hand-over tuning (wc_set_step_tuning): leaf stride and poll pause.
static std::atomic<int> g_leaf_stride{kStepLeafStride};
static std::atomic<int> g_poll_sleep{1};

static const uint16_t* u16p(const void* p) { return static_cast<const uint16_t*>(p); }

// Shapes the one-launch step covers: the Qwen3-1.7B drafter width (hidden and q
// width 2048, head_dim 128, intermediate <= 6144, a GQA group of at most four).
static bool step_shape_ok(const wc_drafter_dims& d) {
  return d.head_dim == kStD && d.hidden == kStHidden && d.heads * kStD == kStHidden && d.heads % d.kv_heads == 0 &&
         d.heads / d.kv_heads <= kStQV && d.kv_heads <= kMaxKvHeads && d.inter % 512 == 0 &&
         d.inter <= kStSI * 512;
}

// Splits per kv head: one chunk of keys each up to kMaxSplits chunks (the
// per-op decode attention's split count).
static int step_splits(int capacity) {
  return std::max(1, std::min(kMaxSplits, (capacity + kStChunk - 1) / kStChunk));
}

template <typename KT, bool HEAD, bool AUX>
static const void* step_kernel() {
  return reinterpret_cast<const void*>(&k_step<KT, HEAD, AUX>);
}

static const void* step_kernel_for(int kv_dtype, bool head, bool aux) {
  if (kv_dtype == WC_BF16)
    return head ? step_kernel<uint16_t, true, true>() : aux ? step_kernel<uint16_t, false, true>()
                                                            : step_kernel<uint16_t, false, false>();
  return head ? step_kernel<float, true, true>() : aux ? step_kernel<float, false, true>()
                                                       : step_kernel<float, false, false>();
}

// Blocks of a step kernel the current device holds at once (per CU x CUs),
// queried once per (device, kernel).
static int step_capacity(const void* kern) {
  static std::mutex mu;
  static std::unordered_map<const void*, int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache[dev].find(kern);
  if (it != cache[dev].end()) return it->second;
  int cus = 0, per_cu = 0;
  if (device_cus(&cus) != WC_OK ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStThreads, 0) != hipSuccess)
    per_cu = 0;
  (void)hipGetLastError();
  const int n = cus * per_cu;
  cache[dev].emplace(kern, n);
  return n;
}

// The grid's layout (a.nb ...) for this shape on this device; false when the
// resident grid cannot hold the work (the per-op launches run instead).
static bool step_layout(StepArgs& a, bool head, const void* kern) {
  const int nb = step_capacity(kern);
  if (nb <= 0) return false;
  a.nb = nb;
  a.nw = nb * kStWaves;
  a.a_blocks = a.splits * a.Hk;
  a.gx_w0 = 0;
  const int extra = std::max(0, a.inter - a.nw);
  a.gx_n = (extra + kStGX - 1) / kStGX;
  a.od_w0 = a.nw - a.hidden;
  return (!head || a.head_rows <= a.nw * kStRH) && a.nqkv <= a.nw && a.a_blocks <= nb &&
         a.od_w0 % kStWaves == 0 && a.od_w0 >= a.gx_w0 + a.gx_n && a.inter <= a.nw + a.gx_n * kStGX;
}

// Common fields of the arguments.
static void step_layer_args(StepArgs& a, const wc_drafter_dims& d, const wc_drafter_weights& w, int layer,
                            const DrafterWs& ws, void* k_cache, void* v_cache, int capacity,
                            const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                            float* hidden_out) {
  const wc_layer_weights& L = w.layers[layer];
  a.hidden = d.hidden;
  a.inter = d.inter;
  a.H = d.heads;
  a.Hk = d.kv_heads;
  a.head_rows = d.head_rows;
  a.vocab = d.vocab;
  a.nqkv = (d.heads + 2 * d.kv_heads) * d.head_dim;
  a.eps = d.eps;
  a.scale = 1.f / sqrtf(static_cast<float>(d.head_dim));
  a.embed = u16p(w.embed);
  a.in_norm = u16p(L.in_norm);
  a.aux_norm = u16p(L.aux_norm);
  a.post_norm = u16p(L.post_norm);
  a.q_norm = u16p(L.q_norm);
  a.k_norm = u16p(L.k_norm);
  a.wq = u16p(L.q);
  a.wk = u16p(L.k);
  a.wv = u16p(L.v);
  a.aq = u16p(L.aux_q);
  a.ak = u16p(L.aux_k);
  a.av = u16p(L.aux_v);
  a.wo = u16p(L.o);
  a.wg = u16p(L.gate);
  a.wu = u16p(L.up);
  a.wd = u16p(L.down);
  a.rope_cos = w.rope_cos;
  a.rope_sin = w.rope_sin;
  a.rope_max = w.rope_max_pos;
  a.kc = k_cache;
  a.vc = v_cache;
  a.cap = capacity;
  a.offset_dev = offset_dev;
  a.offset_add = offset_add;
  a.positions = positions_dev;
  a.window = d.window;
  a.qkv = ws.qkv;
  a.attn = ws.attn;
  a.h1 = ws.h1;
  a.act = ws.act;
  a.partial = ws.partial;
  a.hidden_out = hidden_out;
  a.ctr = ws.step_ctr;
  a.slots = ws.step_slots;
  a.split_ctr = ws.step_split;
  a.status = ws.step_status;
  a.spin_limit = current_spin_limit();
  a.trace = g_trace.load(std::memory_order_relaxed);
  a.leaf_stride = g_leaf_stride.load(std::memory_order_relaxed);
  a.poll_sleep = g_poll_sleep.load(std::memory_order_relaxed);
  a.splits = step_splits(capacity);
}

static bool layer_ok(const wc_layer_weights& L) {
  auto al = [](const void* p) { return p != nullptr && aligned(p, 16); };
  return al(L.in_norm) && al(L.post_norm) && al(L.q) && al(L.k) && al(L.v) && al(L.o) && al(L.q_norm) &&
         al(L.k_norm) && al(L.gate) && al(L.up) && al(L.down) &&
         (L.aux_norm == nullptr || (al(L.aux_norm) && al(L.aux_q) && al(L.aux_k) && al(L.aux_v)));
}

static int step_launch(StepArgs& a, int kv_dtype, bool head, bool aux, hipStream_t s) {
  const dim3 grid(a.nb), block(kStThreads);
  if (kv_dtype == WC_BF16) {
    if (head)
      hipLaunchKernelGGL((k_step<uint16_t, true, true>), grid, block, 0, s, a);
    else if (aux)
      hipLaunchKernelGGL((k_step<uint16_t, false, true>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((k_step<uint16_t, false, false>), grid, block, 0, s, a);
  } else {
    if (head)
      hipLaunchKernelGGL((k_step<float, true, true>), grid, block, 0, s, a);
    else if (aux)
      hipLaunchKernelGGL((k_step<float, false, true>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((k_step<float, false, false>), grid, block, 0, s, a);
  }
  WC_LAUNCHED();
  return WC_OK;
}

bool step_layer_fits(const wc_drafter_dims& d, const wc_drafter_weights& w, int rows, const int32_t* n_rows_dev,
                     const uint8_t* mask_dev, int kv_dtype, const float* out_out, const int32_t* advance_dev) {
  if (!g_one_launch.load(std::memory_order_relaxed)) return false;
  if (rows != 1 || n_rows_dev || mask_dev || out_out || advance_dev) return false;
  if (kv_dtype != WC_BF16 && kv_dtype != WC_F32) return false;
  if (!step_shape_ok(d) || !w.embed || !aligned(w.embed, 16)) return false;
  for (int li = 0; li < d.num_layers; ++li)
    if (!layer_ok(w.layers[li])) return false;
  return true;
}

int step_layer_launch(const wc_drafter_dims& d, const wc_drafter_weights& w, int layer, const int32_t* tokens_dev,
                      const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add,
                      void* k_cache, void* v_cache, int kv_dtype, int capacity, const int32_t* offset_dev,
                      int offset_add, const int32_t* positions_dev, float* hidden_out, void* workspace,
                      hipStream_t s) {
  const DrafterWs ws = drafter_ws(d, workspace);
  StepArgs a{};
  step_layer_args(a, d, w, layer, ws, k_cache, v_cache, capacity, offset_dev, offset_add, positions_dev, hidden_out);
  a.x = feat;
  a.ld_x = feat_ld;
  a.row_dev = feat_row_dev;
  a.row_add = feat_row_add;
  a.tokens_dev = tokens_dev;
  const bool aux = w.layers[layer].aux_norm != nullptr;
  if (!step_layout(a, false, step_kernel_for(kv_dtype, false, aux)))
    return set_error(WC_E_UNSUPPORTED, "one-launch layer: the resident grid cannot hold this shape");
  return step_launch(a, kv_dtype, false, aux, s);
}

// Whether the one-launch layer runs for this call (the resident grid holds the work).
bool step_layer_grid_ok(const wc_drafter_dims& d, const wc_drafter_weights& w, int kv_dtype, int capacity) {
  StepArgs a{};
  a.hidden = d.hidden;
  a.inter = d.inter;
  a.Hk = d.kv_heads;
  a.head_rows = d.head_rows;
  a.nqkv = (d.heads + 2 * d.kv_heads) * d.head_dim;
  a.splits = step_splits(capacity);
  bool ok = true;
  for (int li = 0; li < d.num_layers && ok; ++li)
    ok = step_layout(a, false, step_kernel_for(kv_dtype, false, w.layers[li].aux_norm != nullptr));
  return ok;
}

}  // namespace wc

using namespace wc;

extern "C" {

int wc_draft_step(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* hidden_rows,
                  int64_t hidden_ld, const int32_t* row_dev, int row_add, float* out_norm, int64_t out_ld,
                  int32_t* token_out, int32_t* row_out, void* const* k_cache, void* const* v_cache, int kv_dtype,
                  int capacity, const int32_t* offset_dev, int offset_add, int feedback_out, float* hidden_out,
                  void* workspace, wc_stream_t stream) {
  WC_REQUIRE(dims && w && hidden_rows && token_out && k_cache && v_cache && offset_dev && hidden_out && workspace,
             "wc_draft_step: NULL argument");
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(w->head && w->final_norm && aligned(w->head, 16) && aligned(w->final_norm, 16),
             "wc_draft_step: head / final norm missing or not 16-byte aligned");
  WC_REQUIRE(hidden_ld >= d.hidden && hidden_ld % 4 == 0 && aligned(hidden_rows, 16),
             "wc_draft_step: hidden rows must be 16-byte aligned with a stride >= hidden_size, multiple of 4");
  WC_REQUIRE(out_norm == nullptr || (out_ld >= d.hidden && out_ld % 4 == 0 && aligned(out_norm, 16)),
             "wc_draft_step: out rows must be 16-byte aligned with a stride >= hidden_size, multiple of 4");
  WC_REQUIRE(out_norm != nullptr || !feedback_out, "wc_draft_step: a feedback of `out` needs out_norm");
  WC_REQUIRE(aligned(workspace, 16) && aligned(hidden_out, 16), "wc_draft_step: buffers must be 16-byte aligned");
  auto s = reinterpret_cast<hipStream_t>(stream);
  const float* feat = feedback_out ? out_norm : hidden_rows;
  const int64_t feat_ld = feedback_out ? out_ld : hidden_ld;
  bool one = d.num_layers == 1 && step_layer_fits(d, *w, 1, nullptr, nullptr, kv_dtype, nullptr, nullptr) &&
             w->layers[0].aux_norm != nullptr && k_cache[0] && v_cache[0] && aligned(k_cache[0], 16) &&
             aligned(v_cache[0], 16) && w->rope_cos && w->rope_sin && w->rope_max_pos >= capacity;
  StepArgs a{};
  if (one) {
    const DrafterWs ws = drafter_ws(d, workspace);
    step_layer_args(a, d, *w, 0, ws, k_cache[0], v_cache[0], capacity, offset_dev, offset_add, nullptr, hidden_out);
    one = step_layout(a, true, step_kernel_for(kv_dtype, true, true));
  }
  if (!one) {
    // the head launch, then the drafter forward on the drafted token
    if (int rc = wc_draft_head_norm(dims, w, hidden_rows, hidden_ld, row_dev, row_add, out_norm, out_ld, nullptr, 0,
                                    token_out, row_out, nullptr, workspace, stream))
      return rc;
    return wc_drafter_forward(dims, w, token_out, feat, feat_ld, row_dev, row_add, 1, nullptr, k_cache, v_cache,
                              kv_dtype, capacity, offset_dev, offset_add, nullptr, nullptr, 0, hidden_out, nullptr,
                              nullptr, workspace, stream);
  }
  a.x = hidden_rows;
  a.ld_x = hidden_ld;
  a.row_dev = row_dev;
  a.row_add = row_add;
  a.out = out_norm;
  a.ld_out = out_ld;
  a.head_w = u16p(w->head);
  a.final_norm = u16p(w->final_norm);
  a.d2t = w->d2t;
  a.token_out = token_out;
  a.row_out = row_out;
  a.fb_out = feedback_out ? 1 : 0;
  return step_launch(a, kv_dtype, true, true, s);
}

int wc_set_step_trace(void* buffer) {
  wc::g_trace.store(static_cast<unsigned long long*>(buffer), std::memory_order_relaxed);
  return WC_OK;
}

int wc_set_step_tuning(int leaf_stride, int poll_sleep) {
  WC_REQUIRE(leaf_stride >= 1 && leaf_stride <= kStepLeafStride, "wc_set_step_tuning: leaf stride in 1..%d",
             kStepLeafStride);
  WC_REQUIRE(poll_sleep == 0 || poll_sleep == 1 || poll_sleep == 4 || poll_sleep == 16 || poll_sleep == 64,
             "wc_set_step_tuning: poll pause 0, 1, 4, 16 or 64");
  wc::g_leaf_stride.store(leaf_stride, std::memory_order_relaxed);
  wc::g_poll_sleep.store(poll_sleep, std::memory_order_relaxed);
  return WC_OK;
}

int wc_set_one_launch_step(int enable) {
  wc::g_one_launch.store(enable ? 1 : 0, std::memory_order_relaxed);
  return WC_OK;
}

int wc_draft_step_grid(const wc_drafter_dims* dims, int kv_dtype) {
  if (!dims) return 0;
  return wc::step_capacity(wc::step_kernel_for(kv_dtype, true, true));
}

size_t wc_draft_step_status_offset(const wc_drafter_dims* dims) {
  if (!dims) return 0;
  return static_cast<size_t>(reinterpret_cast<char*>(drafter_ws(*dims, reinterpret_cast<void*>(256)).step_status) -
                             reinterpret_cast<char*>(256));
}

}  // extern "C"
