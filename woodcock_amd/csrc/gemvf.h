// gemvf.h -- few-row (2 <= M <= 16) streaming GEMV on the matrix cores of gfx950.
//
//   y[m][n] = sum_s inv_s[m] * sum_k W_s[n][k] * (x_s[m][k] * gain_s[k])
//
// The M input rows are the 16 columns of the B operand of
// v_mfma_f32_16x16x32_bf16 (columns past M are never read back), the weights
// are the A operand: lane l streams 16 bytes of weight row l % 16 at k group
// l / 16 of each 32-wide k step, TW 16-row tiles per wave.  A block is
// kGfWaves waves on the same rows, each streaming a contiguous share of the k
// steps of every input segment (kGfD steps in flight per wave); the partial
// tiles and the rows' partial sums of squares meet in LDS, so no product is
// reduced across lanes and no launch follows.  x * gain is split into three
// bf16 terms (hi + mid + lo equals the fp32 value to ~2^-25) and each weight
// tile is multiplied with all three, which keeps fp32 accuracy (the drafter's
// 1e-5 parity) at three MFMAs per tile and step.  Epilogues as the one-row
// kernel: store, residual, SiLU(gate) * up (PAIR: tile 0 gate rows, tile 1 the
// same up rows) and the head's argmax + d2t.
#pragma once
#include "gemv.h"

namespace wc {


typedef __bf16 gfbf16x8 __attribute__((ext_vector_type(8)));
typedef float gff32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t gf_pack2(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(b))) << 16);
}

// 8 fp32 -> three bf16 terms, each the rounding of what the previous ones left.
__device__ __forceinline__ void gf_split3(const float* x, gfbf16x8& hi, gfbf16x8& mid, gfbf16x8& lo) {
  float r1[8], r2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r1[e] = x[e] - static_cast<float>(static_cast<__bf16>(x[e]));
    r2[e] = r1[e] - static_cast<float>(static_cast<__bf16>(r1[e]));
  }
  hi = __builtin_bit_cast(gfbf16x8, make_uint4(gf_pack2(x[0], x[1]), gf_pack2(x[2], x[3]), gf_pack2(x[4], x[5]),
                                               gf_pack2(x[6], x[7])));
  mid = __builtin_bit_cast(gfbf16x8, make_uint4(gf_pack2(r1[0], r1[1]), gf_pack2(r1[2], r1[3]),
                                                gf_pack2(r1[4], r1[5]), gf_pack2(r1[6], r1[7])));
  lo = __builtin_bit_cast(gfbf16x8, make_uint4(gf_pack2(r2[0], r2[1]), gf_pack2(r2[2], r2[3]),
                                               gf_pack2(r2[4], r2[5]), gf_pack2(r2[6], r2[7])));
}

// K of input segment s (run time) by selects over the arguments' constant
// offsets: a run-time index into a register array would move the array to
// scratch memory, where every use waits on a load
template <int NIN>
__device__ __forceinline__ int gf_seg_k(const GemvArgs& a, int s) {
  int k = a.in[0].K;
  if constexpr (NIN > 1) k = s == 1 ? a.in[1].K : k;
  if constexpr (NIN > 2) k = s == 2 ? a.in[2].K : k;
  return k;
}
template <int NIN>
__device__ __forceinline__ int gf_seg_upr(const GemvArgs& a, int s, int unit) {
  return (gf_seg_k<NIN>(a, s) + unit - 1) / unit;
}
// start of segment s in the staged inputs [segment][M][K]
template <int NIN>
__device__ __forceinline__ int gf_seg_off(const GemvArgs& a, int s) {
  int o = 0;
  if constexpr (NIN > 1) o = s >= 1 ? a.M * a.in[0].K : o;
  if constexpr (NIN > 2) o = s >= 2 ? a.M * (a.in[0].K + a.in[1].K) : o;
  return o;
}

// Elements between consecutive k steps of a lane's weight stream: 32 along a
// row-major row, or one 1 KB fragment in the fragment-major layout
// (wc_weights_frag: chunk (T, s) of 16-row tile T at k step s holds lane l's
// W[16 T + l % 16][32 s + 8 (l / 16) .. + 8], so every load instruction of a
// wave is one contiguous kilobyte).
template <bool FRAG>
__device__ __forceinline__ constexpr int gf_step() { return FRAG ? 64 * 8 : 32; }

// Registers of one k step in flight: TW weight fragments, the lane's 8 inputs
// (fp32: two vectors; bf16: the first) and 8 gains.
template <int TW>
struct GfStep {
  uint4 w[TW];
  uint4 x0, x1, g;
};

// Issue the loads of step i (segment s, local step j of that segment).  STG:
// the lane's input row of segment S is staged in LDS as fp32 x * gain (xs).
template <int S, int TW, bool PAIR, int XB, int GB, bool STG, bool FRAG = false>
__device__ __forceinline__ void gf_load(const GemvArgs& a, const uint16_t* (*wrow)[TW], const int64_t* xoff,
                                        const float* const* xs, int j, GfStep<TW>& st) {
  const int kg = (threadIdx.x % kWave) / 16;
  const int k = j * 32 + kg * 8;
#pragma unroll
  for (int t = 0; t < TW; ++t) st.w[t] = *reinterpret_cast<const uint4*>(wrow[S][t] + j * gf_step<FRAG>());
  if constexpr (STG) {
    st.x0 = *reinterpret_cast<const uint4*>(xs[S] + k);
    st.x1 = *reinterpret_cast<const uint4*>(xs[S] + k + 4);
  } else if ((XB >> S) & 1) {
    st.x0 = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.in[S].x) + xoff[S] + k);
  } else {
    const float* xp = static_cast<const float*>(a.in[S].x) + xoff[S] + k;
    st.x0 = *reinterpret_cast<const uint4*>(xp);
    st.x1 = *reinterpret_cast<const uint4*>(xp + 4);
  }
  if ((GB >> S) & 1) st.g = *reinterpret_cast<const uint4*>(a.in[S].gain + k);
}

// Consume a landed step of segment S: sum of squares, x * gain, 3 x TW MFMAs
// (STG: x * gain comes staged, its sum of squares was taken while staging).
template <int S, int TW, int XB, int GB, bool STG>
__device__ __forceinline__ void gf_compute(const GfStep<TW>& st, gff32x4 (*acc)[TW], float* ss) {
  float x[8];
  if (STG || !((XB >> S) & 1)) {
    x[0] = __uint_as_float(st.x0.x); x[1] = __uint_as_float(st.x0.y);
    x[2] = __uint_as_float(st.x0.z); x[3] = __uint_as_float(st.x0.w);
    x[4] = __uint_as_float(st.x1.x); x[5] = __uint_as_float(st.x1.y);
    x[6] = __uint_as_float(st.x1.z); x[7] = __uint_as_float(st.x1.w);
  } else {
    x[0] = bf16_lo(st.x0.x); x[1] = bf16_hi(st.x0.x); x[2] = bf16_lo(st.x0.y); x[3] = bf16_hi(st.x0.y);
    x[4] = bf16_lo(st.x0.z); x[5] = bf16_hi(st.x0.z); x[6] = bf16_lo(st.x0.w); x[7] = bf16_hi(st.x0.w);
  }
  if constexpr (!STG) {
    float t = ss[S];
#pragma unroll
    for (int e = 0; e < 8; ++e) t = fmaf(x[e], x[e], t);
    ss[S] = t;
  }
  if (!STG && ((GB >> S) & 1)) {
    x[0] *= bf16_lo(st.g.x); x[1] *= bf16_hi(st.g.x); x[2] *= bf16_lo(st.g.y); x[3] *= bf16_hi(st.g.y);
    x[4] *= bf16_lo(st.g.z); x[5] *= bf16_hi(st.g.z); x[6] *= bf16_lo(st.g.w); x[7] *= bf16_hi(st.g.w);
  }
  gfbf16x8 hi, mid, lo;
  gf_split3(x, hi, mid, lo);
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) {
    const gfbf16x8 wv = __builtin_bit_cast(gfbf16x8, st.w[tt]);
    acc[S][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, hi, acc[S][tt], 0, 0, 0);
    acc[S][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, mid, acc[S][tt], 0, 0, 0);
    acc[S][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, lo, acc[S][tt], 0, 0, 0);
  }
}

// W waves per block and D k steps in flight per wave: 8 and 6 for
// single-tile waves, 4 and 4 for two-tile waves (their registers allow fewer
// waves per SIMD).
// STG: the M input rows of every segment are staged once per block in dynamic
// LDS as fp32 x * gain ([segment][row][K]; the host passes the size in
// a.lds_floats), with their sums of squares, so the k steps read x from LDS
// instead of every lane loading its 32 bytes of x and 16 of gain from memory.
constexpr int kGfUnit = 2048;  // staged elements per (wave, unit): 8 four-element chunks per lane
template <int TW, int W, int D, bool PAIR, int NIN, int XB, int GB, bool STG = false, bool FRAG = false>
__global__ __launch_bounds__(W * kWave) void k_gemvf(GemvArgs a) {
  static_assert(!FRAG || NIN == 1, "fragment-major weights: one input segment");
  constexpr int kGfWaves = W, kGfThreads = W * kWave, kGfD = D;
  static_assert(!PAIR || TW == 2, "the pair epilogue takes a gate tile and an up tile");
  constexpr int RB = PAIR ? 16 : 16 * TW;  // logical output rows per block
  // partial tiles of the waves; STG: in the dynamic region, over the staged x
  // once every wave is past its main loop
  __shared__ float s_c_static[STG ? 1 : kGfWaves][NIN][TW][4][kWave];
  __shared__ float s_ss[STG ? 1 : kGfWaves][NIN][kWave];
  __shared__ float s_inv[NIN][16];
  __shared__ unsigned long long s_key[kGemvWaves][kMaxM];
  extern __shared__ __attribute__((aligned(16))) float g_xs[];  // STG: [NIN][M][K_s] x * gain
  float(*s_c)[NIN][TW][4][kWave] =
      STG ? reinterpret_cast<float(*)[NIN][TW][4][kWave]>(g_xs) : s_c_static;
  constexpr int kMaxUnits = 3 * 16 * 3;                          // NIN * M * units per row, at most
  __shared__ float s_ssu[STG ? kMaxUnits : 1];                  // STG: sum of squares per unit
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int t = threadIdx.x;
  const int m_live = a.m_dev ? min(max(*a.m_dev, 0), a.M) : a.M;
  const int row0 = blockIdx.x * RB;
  const int lm = lane % 16, kg = lane / 16;

  // per-lane weight rows (clamped into the matrix) and input rows (clamped to the launch's rows)
  const uint16_t* wrow[NIN][TW];
  int64_t xoff[NIN];
  int nsteps[NIN];
  int total = 0;
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      const int n = PAIR ? min(row0 + lm, a.N - 1) : min(row0 + tt * 16 + lm, a.N - 1);
      if constexpr (FRAG) {
        // tile n / 16 of the fragment-major matrix (rows padded to 16), lane l's chunk
        const uint16_t* base = PAIR ? (tt ? a.w[1][s] : a.w[0][s]) : a.w[0][s];
        wrow[s][tt] = base + static_cast<int64_t>(n / 16) * (a.in[s].K / 32) * (64 * 8) + lane * 8;
      } else {
        wrow[s][tt] = row_ptr<PAIR>(a, n, PAIR ? tt : 0, s) + kg * 8;
      }
    }
    xoff[s] = static_cast<int64_t>(in_row(a.in[s], min(lm, a.M - 1))) * a.in[s].ld;
    nsteps[s] = a.in[s].K / 32;
    total += nsteps[s];
  }
  const int per = (total + kGfWaves - 1) / kGfWaves;
  const int i0 = min(total, wave * per), i1 = min(total, i0 + per);

  // STG, part 1: this wave's staging units (segment, row, 2048-element span),
  // loads issued before the weights so that waiting on them waits on nothing
  // else; a unit's 8 chunks of 4 elements per lane land in registers
  const float* xs[NIN];
  int soff[NIN + 1];
  soff[0] = 0;
#pragma unroll
  for (int s = 0; s < NIN; ++s) soff[s + 1] = soff[s] + a.M * a.in[s].K;
#pragma unroll
  for (int s = 0; s < NIN; ++s) xs[s] = g_xs + soff[s] + min(lm, a.M - 1) * a.in[s].K;
  int units = 0, upr[NIN];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    upr[s] = (a.in[s].K + kGfUnit - 1) / kGfUnit;
    units += a.M * upr[s];
  }
  constexpr int kCh = kGfUnit / (4 * kWave);
  uint4 sx[kCh];
  uint2 sg[kCh];
  auto unit_of = [&](int u, int& us, int& um, int& uk0) {
    us = 0;
#pragma unroll
    for (int s = 0; s + 1 < NIN; ++s)
      if (us == s && u >= a.M * upr[s]) {
        u -= a.M * upr[s];
        us = s + 1;
      }
    const int up = gf_seg_upr<NIN>(a, us, kGfUnit);
    um = u / up;
    uk0 = (u % up) * kGfUnit;
  };
  auto stage_issue = [&](int u) {
    int us, um, uk0;
    unit_of(u, us, um, uk0);
    const int K = a.in[us].K;
    const int64_t xr = static_cast<int64_t>(in_row(a.in[us], um)) * a.in[us].ld;
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int k = min(uk0 + (lane + c * kWave) * 4, K - 4);
      if ((XB >> us) & 1) {
        const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.in[us].x) + xr + k);
        sx[c] = make_uint4(h.x, h.y, 0u, 0u);
      } else {
        sx[c] = *reinterpret_cast<const uint4*>(static_cast<const float*>(a.in[us].x) + xr + k);
      }
      sg[c] = a.in[us].gain ? *reinterpret_cast<const uint2*>(a.in[us].gain + k) : make_uint2(0x3f803f80u, 0x3f803f80u);
    }
  };
  auto stage_store = [&](int u) {
    int us, um, uk0;
    unit_of(u, us, um, uk0);
    const int K = a.in[us].K;
    float t2 = 0.f;
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int k = uk0 + (lane + c * kWave) * 4;
      float x[4];
      if ((XB >> us) & 1) {
        x[0] = bf16_lo(sx[c].x); x[1] = bf16_hi(sx[c].x); x[2] = bf16_lo(sx[c].y); x[3] = bf16_hi(sx[c].y);
      } else {
        x[0] = __uint_as_float(sx[c].x); x[1] = __uint_as_float(sx[c].y);
        x[2] = __uint_as_float(sx[c].z); x[3] = __uint_as_float(sx[c].w);
      }
      if (k < K) {
#pragma unroll
        for (int e = 0; e < 4; ++e) t2 = fmaf(x[e], x[e], t2);
        const float4 v = make_float4(x[0] * bf16_lo(sg[c].x), x[1] * bf16_hi(sg[c].x), x[2] * bf16_lo(sg[c].y),
                                     x[3] * bf16_hi(sg[c].y));
        *reinterpret_cast<float4*>(g_xs + gf_seg_off<NIN>(a, us) + um * K + k) = v;
      }
    }
    t2 = wave_sum_dpp(t2);
    if (lane == 0) s_ssu[u] = t2;
  };
  const int u_first = wave;  // units wave, wave + W, ...
  if constexpr (STG) {
    if (u_first < units) stage_issue(u_first);
  }

  gff32x4 acc[NIN][TW];
  float ss[NIN];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    ss[s] = 0.f;
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) acc[s][tt] = gff32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (t < kGemvWaves * kMaxM) (&s_key[0][0])[t] = 0ull;

  // step i -> (segment, local step): segments are consecutive in the step list
#define GF_SEG(i, S_OUT, J_OUT)                                     \
  int S_OUT = 0, J_OUT = (i);                                       \
  if (NIN > 1 && J_OUT >= nsteps[0]) {                              \
    J_OUT -= nsteps[0];                                             \
    S_OUT = 1;                                                      \
    if (NIN > 2 && J_OUT >= nsteps[1 < NIN ? 1 : 0]) {              \
      J_OUT -= nsteps[1 < NIN ? 1 : 0];                             \
      S_OUT = 2;                                                    \
    }                                                               \
  }
#define GF_LOAD(i, ST)                                                                         \
  do {                                                                                         \
    GF_SEG(i, s_, j_);                                                                         \
    if (s_ == 0) gf_load<0, TW, PAIR, XB, GB, STG, FRAG>(a, wrow, xoff, xs, j_, ST);          \
    if constexpr (NIN > 1) if (s_ == 1) gf_load<1 < NIN ? 1 : 0, TW, PAIR, XB, GB, STG>(a, wrow, xoff, xs, j_, ST); \
    if constexpr (NIN > 2) if (s_ == 2) gf_load<2 < NIN ? 2 : 0, TW, PAIR, XB, GB, STG>(a, wrow, xoff, xs, j_, ST); \
  } while (0)
#define GF_COMPUTE(i, ST)                                                            \
  do {                                                                               \
    GF_SEG(i, s_, j_);                                                               \
    (void)j_;                                                                        \
    if (s_ == 0) gf_compute<0, TW, XB, GB, STG>(ST, acc, ss);                       \
    if constexpr (NIN > 1) if (s_ == 1) gf_compute<1 < NIN ? 1 : 0, TW, XB, GB, STG>(ST, acc, ss); \
    if constexpr (NIN > 2) if (s_ == 2) gf_compute<2 < NIN ? 2 : 0, TW, XB, GB, STG>(ST, acc, ss); \
  } while (0)

  GfStep<TW> ring[kGfD];
  if constexpr (STG) {
    // weights of the first steps in flight behind the staging loads; the x
    // reads of those steps follow the staging (LDS, after the barrier)
#pragma unroll
    for (int u = 0; u < kGfD; ++u)
      if (i0 + u < i1) {
        GF_SEG(i0 + u, s_, j_);
        // one load per segment branch: a select between the segments' row
        // pointers is folded into a runtime index of wrow, which then lives in
        // scratch memory and every weight load waits on a scratch load
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
          if (s_ == 0) ring[u].w[tt] = *reinterpret_cast<const uint4*>(wrow[0][tt] + j_ * gf_step<FRAG>());
          if constexpr (NIN > 1) if (s_ == 1) ring[u].w[tt] = *reinterpret_cast<const uint4*>(wrow[1 < NIN ? 1 : 0][tt] + j_ * 32);
          if constexpr (NIN > 2) if (s_ == 2) ring[u].w[tt] = *reinterpret_cast<const uint4*>(wrow[2 < NIN ? 2 : 0][tt] + j_ * 32);
        }
      }
    for (int u = u_first; u < units; u += kGfWaves) {
      if (u != u_first) stage_issue(u);
      stage_store(u);
    }
    lds_barrier();
    if (t < NIN * 16) {  // inverse RMS of (segment, row) from its units' sums, in unit order
      const int sgi = t / 16, m = t % 16;
      float tot = 0.f;
      if (m < a.M) {
        int base = 0;
        for (int s2 = 0; s2 < sgi; ++s2) base += a.M * upr[s2];
        const int up = gf_seg_upr<NIN>(a, sgi, kGfUnit);
        for (int q = 0; q < up; ++q) tot += s_ssu[base + m * up + q];
      }
      s_inv[sgi][m] = a.in[sgi].gain ? 1.f / sqrtf(tot / static_cast<float>(a.in[sgi].K) + a.eps) : 1.f;
    }
#pragma unroll
    for (int u = 0; u < kGfD; ++u)
      if (i0 + u < i1) {
        GF_SEG(i0 + u, s_, j_);
        const int kk = j_ * 32 + kg * 8;
        const float* xp = (s_ == 0 ? xs[0] : (s_ == 1 ? xs[NIN > 1 ? 1 : 0] : xs[NIN > 2 ? 2 : 0])) + kk;
        ring[u].x0 = *reinterpret_cast<const uint4*>(xp);
        ring[u].x1 = *reinterpret_cast<const uint4*>(xp + 4);
      }
  } else {
#pragma unroll
    for (int u = 0; u < kGfD; ++u)
      if (i0 + u < i1) GF_LOAD(i0 + u, ring[u]);
  }
  for (int b = i0; b < i1; b += kGfD) {
#pragma unroll
    for (int u = 0; u < kGfD; ++u) {
      const int i = b + u;
      if (i < i1) {
        GF_COMPUTE(i, ring[u]);
        if (i + kGfD < i1) GF_LOAD(i + kGfD, ring[u]);
      }
    }
  }
#undef GF_LOAD
#undef GF_COMPUTE
#undef GF_SEG

  // partial tiles and sums of squares -> LDS (STG: over the staged x, so every
  // wave's last reads of it come first)
  mfma_settle();
  if constexpr (STG) __syncthreads();
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) s_c[wave][s][tt][e][lane] = acc[s][tt][e];
    if constexpr (!STG) s_ss[wave][s][lane] = ss[s];
  }
  __syncthreads();
  if (!STG && t < NIN * 16) {
    const int s = t / 16, m = t % 16;
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kGfWaves; ++w)
#pragma unroll
      for (int g = 0; g < 4; ++g) tot += s_ss[w][s][g * 16 + m];
    s_inv[s][m] = a.in[s].gain ? 1.f / sqrtf(tot / static_cast<float>(a.in[s].K) + a.eps) : 1.f;
  }
  __syncthreads();

  // outputs (row r of the block, input row m), rows fastest
  for (int idx = t; idx < RB * a.M; idx += kGfThreads) {
    const int r = idx % RB, m = idx / RB;
    const int n = row0 + r;
    if (m >= m_live || n >= a.N) continue;
    const int tile = PAIR ? 0 : r / 16, i = r % 16;
    const int cl = (i / 4) * 16 + m, ce = i % 4;  // C fragment lane / element of (row i, column m)
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      float pg = 0.f, pu = 0.f;
#pragma unroll
      for (int w = 0; w < kGfWaves; ++w) {
        pg += s_c[w][s][tile][ce][cl];
        if (PAIR) pu += s_c[w][s][TW - 1][ce][cl];
      }
      g = fmaf(pg, s_inv[s][m], g);
      u = fmaf(pu, s_inv[s][m], u);
    }
    if (a.epi == kEpiArgmax) {
      const unsigned long long key = head_key(a, m, n, g);
      atomicMax(&s_key[0][m], key);
    } else {
      store_out<PAIR>(a, m, n, g, u, res_value(a, m, n));
    }
  }
  // the cache offset advance of the last projection (no block reads it here)
  if (a.adv_dst && blockIdx.x == 0 && t == 0) *a.adv_dst = *a.adv_src + a.adv_add + m_live;
  if (a.epi == kEpiArgmax) argmax_epilogue<kMaxM>(a, m_live, s_key);
}

// ------------------------------------------------------------------ staged, every step in flight
//
// k_gemvs: the staged few-row MFMA GEMV with every weight step of a wave
// requested at once (D >= the wave's share of the block's k steps; larger
// shares go in chunks of D).  Block (tile, piece): W waves on one 16-row tile
// (TW = 1), two tiles or a gate / up tile pair (TW = 2), over one part of one
// input segment: piece = segment * P + part, P = gridDim.y / NIN parts per
// segment.  The block stages its part of the M input rows once in dynamic LDS
// as fp32 x * gain ([m][part K + 4]) with their sums of squares and
// accumulates one MFMA tile per output tile, so a block never chooses between
// accumulators at run time (a branch-selected accumulator was shuffled through
// copies that read MFMA results early: wrong rows 2-3 of the tiles).  With
// one piece the block applies the RMS scale itself; otherwise every piece
// publishes its partial tile and sums of squares and the last block of the
// tile to finish adds them in piece order, applying each segment's scale
// (deterministic; the counter resets itself).  Nothing waits on a device
// value (row count, row index) before the weight loads are issued.
constexpr int kGsUnit = 1024;               // staged elements per (wave, unit): 4 four-element chunks per lane
constexpr int kGsMaxUnits = 16 * 10;        // rows x units per row (a part of K <= 10240)
constexpr int kGsPieceFloats = 1024;        // published per (tile, piece): tile(s) [row][m], then sums [m]
constexpr int kGsMaxPieces = 4096;          // tiles x pieces of one split launch

// Stage unit u (row um, span from ue0) of one segment: BF = bf16 input,
// GN = normed (gain); every load issued back to back, addresses clamped.
template <bool BF, bool GN>
__device__ __forceinline__ void gs_stage_issue(const void* x, int64_t xr, const uint16_t* gain, int ue0, int pk1,
                                               uint4* sx, uint2* sg) {
  const int lane = threadIdx.x % kWave;
  constexpr int kCh = kGsUnit / (4 * kWave);
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int k = min(ue0 + (lane + c * kWave) * 4, pk1 - 4);
    if constexpr (BF) {
      const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + xr + k);
      sx[c] = make_uint4(h.x, h.y, 0u, 0u);
    } else {
      sx[c] = *reinterpret_cast<const uint4*>(static_cast<const float*>(x) + xr + k);
    }
    if constexpr (GN) sg[c] = *reinterpret_cast<const uint2*>(gain + k);
  }
}
template <bool BF, bool GN>
__device__ __forceinline__ float gs_stage_store(const uint4* sx, const uint2* sg, float* dst, int ue0, int pk0, int pk1) {
  const int lane = threadIdx.x % kWave;
  constexpr int kCh = kGsUnit / (4 * kWave);
  float t2 = 0.f;
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int k = ue0 + (lane + c * kWave) * 4;
    float x[4];
    if constexpr (BF) {
      x[0] = bf16_lo(sx[c].x); x[1] = bf16_hi(sx[c].x); x[2] = bf16_lo(sx[c].y); x[3] = bf16_hi(sx[c].y);
    } else {
      x[0] = __uint_as_float(sx[c].x); x[1] = __uint_as_float(sx[c].y);
      x[2] = __uint_as_float(sx[c].z); x[3] = __uint_as_float(sx[c].w);
    }
    if (k < pk1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) t2 = fmaf(x[e], x[e], t2);
      float4 v = make_float4(x[0], x[1], x[2], x[3]);
      if constexpr (GN) {
        v.x *= bf16_lo(sg[c].x); v.y *= bf16_hi(sg[c].x); v.z *= bf16_lo(sg[c].y); v.w *= bf16_hi(sg[c].y);
      }
      *reinterpret_cast<float4*>(dst + (k - pk0)) = v;
    }
  }
  return wave_sum_dpp(t2);
}

template <int TW, int W, int D, bool PAIR, int NIN, int XB, int GB, bool GRP = false>
__global__ __launch_bounds__(W * kWave) void k_gemvs(GemvArgs a) {
  static_assert(!PAIR || TW == 2, "the pair epilogue takes a gate tile and an up tile");
  static_assert(!GRP || (NIN > 1 && W % NIN == 0), "wave groups: one group of W / NIN waves per segment");
  static_assert(NIN >= 1 && NIN <= 3, "one to three input segments");
  static_assert(GB == 0 || GB == (1 << NIN) - 1, "every segment normed or none");
  constexpr bool kGain = GB != 0;
  constexpr int kT = W * kWave;
  constexpr int RB = PAIR ? 16 : 16 * TW;  // logical output rows per block
  constexpr int kTiles = PAIR ? 2 : 1;     // published tiles per piece (gate, up)
  static_assert(RB * kMaxM <= kT, "one output per thread");
  static_assert(kTiles * RB * kMaxM + kMaxM <= kGsPieceFloats, "piece fits its slot");
  extern __shared__ __attribute__((aligned(16))) float g_x[];  // [M][xs]; after the main loop: partial tiles
  __shared__ float s_ssu[kGsMaxUnits];
  __shared__ float s_ss[NIN][16];
  __shared__ float s_inv[NIN][16];
  __shared__ unsigned long long s_key[kGemvWaves][kMaxM];
  __shared__ bool s_last;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int lm = lane % 16, kg = lane / 16;
  const int row0 = blockIdx.x * RB;
  const int M = a.M;
  // GRP: the block takes every segment whole, a group of W / NIN waves each;
  // else piece blockIdx.y = segment * P + part with all W waves on it
  constexpr int kWg = GRP ? W / NIN : W;  // waves on one segment
  const int KS = GRP ? 1 : gridDim.y, piece = GRP ? 0 : blockIdx.y, P = GRP ? 1 : KS / NIN;
  const int seg = GRP ? wave / kWg : piece / P, part = GRP ? 0 : piece - seg * P;
  const int wv = GRP ? wave - seg * kWg : wave;  // wave within its segment group
  constexpr int S1 = NIN > 1 ? 1 : 0, S2 = NIN > 2 ? 2 : 0;

  // this block's segment: every argument read at a constant offset, then
  // chosen by value (a segment struct picked by reference at run time turns
  // into chains of dependent argument loads)
  const void* sgx = a.in[0].x;
  int64_t sgld = a.in[0].ld;
  const int32_t* sgidx = a.in[0].row_idx;
  int sgadd = a.in[0].row_add, sgmax = a.in[0].max_row, K = a.in[0].K;
  const uint16_t* sgain = a.in[0].gain;
  int64_t ldw = a.ldw[0];
  if constexpr (NIN > 1) {
    const bool c = seg == 1;
    sgx = c ? a.in[S1].x : sgx;
    sgld = c ? a.in[S1].ld : sgld;
    sgidx = c ? a.in[S1].row_idx : sgidx;
    sgadd = c ? a.in[S1].row_add : sgadd;
    sgmax = c ? a.in[S1].max_row : sgmax;
    K = c ? a.in[S1].K : K;
    sgain = c ? a.in[S1].gain : sgain;
    ldw = c ? a.ldw[S1] : ldw;
  }
  if constexpr (NIN > 2) {
    const bool c = seg == 2;
    sgx = c ? a.in[S2].x : sgx;
    sgld = c ? a.in[S2].ld : sgld;
    sgidx = c ? a.in[S2].row_idx : sgidx;
    sgadd = c ? a.in[S2].row_add : sgadd;
    sgmax = c ? a.in[S2].max_row : sgmax;
    K = c ? a.in[S2].K : K;
    sgain = c ? a.in[S2].gain : sgain;
    ldw = c ? a.ldw[S2] : ldw;
  }
  const bool bf = (XB >> seg) & 1;
  const int ns = K / 32;
  const int pp = (ns + P - 1) / P;
  const int j0 = min(ns, part * pp), j1 = min(ns, j0 + pp);
  const int xs = (j1 - j0) * 32 + 4;
  const int per = (j1 - j0 + kWg - 1) / kWg;
  const int i0 = min(j1, j0 + wv * per), i1 = min(j1, i0 + per);
  // GRP: segment s's rows after segment s - 1's in LDS (equal row strides not assumed)
  const int K0a = a.in[0].K, K1a = NIN > 1 ? a.in[S1].K : 0;
  float* const gx_seg = g_x + (GRP ? (seg == 0 ? 0 : (seg == 1 ? M * (K0a + 4) : M * (K0a + 4 + K1a + 4))) : 0);
  float* const ssu = s_ssu + (GRP ? seg * (kGsMaxUnits / NIN) : 0);
  const int ilast = max(i1 - 1, 0);

  // per-lane weight rows of the segment (clamped into the matrix): the row
  // segments' bases of this input segment, then selects per lane (plain
  // values, no captured locals: a select between locals held in memory turns
  // into an indexed scratch load)
  const uint16_t* wr0;
  const uint16_t* wr1;
  {
    const uint16_t* B0 = a.w[0][0];
    const uint16_t* B1 = a.w[1][0];
    const uint16_t* B2 = a.w[2][0];
    if constexpr (NIN > 1) {
      B0 = seg == 1 ? a.w[0][S1] : B0;
      B1 = seg == 1 ? a.w[1][S1] : B1;
      B2 = seg == 1 ? a.w[2][S1] : B2;
    }
    if constexpr (NIN > 2) {
      B0 = seg == 2 ? a.w[0][S2] : B0;
      B1 = seg == 2 ? a.w[1][S2] : B1;
      B2 = seg == 2 ? a.w[2][S2] : B2;
    }
    const int nseg = a.n_seg, ss1 = a.seg_start[1], ss2 = a.seg_start[2];
    const int n0 = min(row0 + lm, a.N - 1);
    if constexpr (PAIR) {
      wr0 = B0 + static_cast<int64_t>(n0) * ldw + kg * 8;
      wr1 = B1 + static_cast<int64_t>(n0) * ldw + kg * 8;
    } else {
      const bool a1 = nseg > 1 && n0 >= ss1, a2 = nseg > 2 && n0 >= ss2;
      const uint16_t* ba = a2 ? B2 : (a1 ? B1 : B0);
      const int sa = a2 ? ss2 : (a1 ? ss1 : 0);
      wr0 = ba + static_cast<int64_t>(n0 - sa) * ldw + kg * 8;
      const int n1 = min(row0 + 16 + lm, a.N - 1);
      const bool b1 = nseg > 1 && n1 >= ss1, b2 = nseg > 2 && n1 >= ss2;
      const uint16_t* bb = b2 ? B2 : (b1 ? B1 : B0);
      const int sb = b2 ? ss2 : (b1 ? ss1 : 0);
      wr1 = TW > 1 ? bb + static_cast<int64_t>(n1 - sb) * ldw + kg * 8 : wr0;
    }
  }

  // staging units: (row, 1024-element span) of the part; the segment's wave wv
  // takes units wv, wv + its group's waves, ...
  const int pk0 = j0 * 32, pk1 = j1 * 32;
  const int upr = (pk1 - pk0 + kGsUnit - 1) / kGsUnit;
  const int units = M * upr;
  constexpr int kCh = kGsUnit / (4 * kWave);
  uint4 sx[kCh];
  uint2 sg[kCh];
  auto stage_issue = [&](int u) {
    const int um = u / upr, ue0 = pk0 + (u - um * upr) * kGsUnit;
    int xrow = (sgidx ? sgidx[um] : um) + sgadd;
    if (sgmax > 0) xrow = min(max(xrow, 0), sgmax - 1);
    const int64_t xr = static_cast<int64_t>(xrow) * sgld;
    if (bf)
      gs_stage_issue<true, kGain>(sgx, xr, sgain, ue0, pk1, sx, sg);
    else
      gs_stage_issue<false, kGain>(sgx, xr, sgain, ue0, pk1, sx, sg);
  };
  auto stage_store = [&](int u) {
    const int um = u / upr, ue0 = pk0 + (u - um * upr) * kGsUnit;
    const float t2 = bf ? gs_stage_store<true, kGain>(sx, sg, gx_seg + um * xs, ue0, pk0, pk1)
                        : gs_stage_store<false, kGain>(sx, sg, gx_seg + um * xs, ue0, pk0, pk1);
    if (lane == 0) ssu[u] = t2;
  };

  // 1. staging loads of the first unit (no row index: before the weights, so
  //    the staging waits on nothing the weights carry), every weight step of
  //    the first chunk, then the staging loads behind a row index
  const bool has_idx = sgidx != nullptr;
  const int u_first = wv;
  if (!has_idx && u_first < units) stage_issue(u_first);
  uint4 w[D][TW];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int j = min(i0 + u, ilast);
    w[u][0] = *reinterpret_cast<const uint4*>(wr0 + j * 32);
    if constexpr (TW > 1) w[u][1] = *reinterpret_cast<const uint4*>(wr1 + j * 32);
  }
  if (has_idx && u_first < units) stage_issue(u_first);
  if (t < kGemvWaves * kMaxM) (&s_key[0][0])[t] = 0ull;
  // the row count and this thread's residual (output t of the block, if any),
  // requested behind the weights and used only by the epilogue
  const int m_live = a.m_dev ? min(max(*a.m_dev, 0), M) : M;
  float resv = 0.f;
  if (a.epi == kEpiResidual) resv = res_value(a, min(t / RB, M - 1), min(row0 + t % RB, a.N - 1));

  // 2. x * gain -> LDS with the units' sums of squares; this part's sum of
  //    squares per row in unit order
  for (int u = u_first; u < units; u += kWg) {
    if (u != u_first) stage_issue(u);
    stage_store(u);
  }
  lds_barrier();
  {
    const int tg = t - (GRP ? seg * kWg * kWave : 0);  // thread within the segment's group
    if (tg < 16) {
      float tot = 0.f;
      if (tg < M)
        for (int q = 0; q < upr; ++q) tot += ssu[tg * upr + q];
      s_ss[GRP ? seg : 0][tg] = tot;
    }
  }

  // 3. the k steps: x from LDS (three-term bf16 split), 3 x TW MFMAs per step
  gff32x4 acc[TW];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) acc[tt] = gff32x4{0.f, 0.f, 0.f, 0.f};
  const float* xrow = gx_seg + min(lm, M - 1) * xs + kg * 8 - pk0;
  for (int c0 = i0; c0 < i1; c0 += D) {
    if (c0 != i0) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int j = min(c0 + u, ilast);
        w[u][0] = *reinterpret_cast<const uint4*>(wr0 + j * 32);
        if constexpr (TW > 1) w[u][1] = *reinterpret_cast<const uint4*>(wr1 + j * 32);
      }
    }
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int j = c0 + u;
      if (j < i1) {
        const float4 x0 = *reinterpret_cast<const float4*>(xrow + j * 32);
        const float4 x1 = *reinterpret_cast<const float4*>(xrow + j * 32 + 4);
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        gfbf16x8 hi, mid, lo;
        gf_split3(x, hi, mid, lo);
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
          const gfbf16x8 wv = __builtin_bit_cast(gfbf16x8, w[u][tt]);
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, hi, acc[tt], 0, 0, 0);
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, mid, acc[tt], 0, 0, 0);
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, lo, acc[tt], 0, 0, 0);
        }
      }
    }
  }

  // 4. partial tiles -> LDS over the staged x (every wave's last reads of it first)
  mfma_settle();
  __syncthreads();
  float(*s_c)[TW][4][kWave] = reinterpret_cast<float(*)[TW][4][kWave]>(g_x);
#pragma unroll
  for (int tt = 0; tt < TW; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_c[wave][tt][e][lane] = acc[tt][e];
  __syncthreads();

  // 5. this block's output (row r of the block, input row m), one per thread
  const int r = t % RB, m = t / RB;
  const int n = row0 + r;
  const int tile = PAIR ? 0 : r / 16, ri = r % 16;
  const int cl = (ri / 4) * 16 + min(m, 15), ce = ri % 4;  // C fragment lane / element of (row ri, column m)
  // per segment (GRP) or the block's one segment: the waves' partial tiles
  float pgs[GRP ? NIN : 1], pus[GRP ? NIN : 1];
#pragma unroll
  for (int sgi = 0; sgi < (GRP ? NIN : 1); ++sgi) {
    pgs[sgi] = 0.f;
    pus[sgi] = 0.f;
#pragma unroll
    for (int q = 0; q < kWg; ++q) {
      pgs[sgi] += s_c[sgi * kWg + q][tile][ce][cl];
      if (PAIR) pus[sgi] += s_c[sgi * kWg + q][TW - 1][ce][cl];
    }
  }
  const float pg = pgs[0], pu = pus[0];
  const bool mine = t < RB * M;
  // the cache offset advance of the last projection, by one block before any
  // block leaves early (none reads the offset here)
  if (a.adv_dst && blockIdx.x == 0 && piece == 0 && t == 0) *a.adv_dst = *a.adv_src + a.adv_add + m_live;
  float g = 0.f, u = 0.f;
  if (KS > 1) {
    // hand the piece over: gate [row][m] (pair: then up), then the sums [m]
    float* pub = a.gs_part + (static_cast<int64_t>(blockIdx.x) * KS + piece) * kGsPieceFloats;
    if (mine) {
      publish_f32(pub + r * M + m, pg);
      if (PAIR) publish_f32(pub + (RB + r) * M + m, pu);
    }
    if (t < M) publish_f32(pub + kTiles * RB * M + t, s_ss[0][t]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
      unsigned int* ctr = a.gs_ctr + blockIdx.x * kCounterStride;
      const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        static_cast<unsigned int>(KS - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // last block of the tile: every piece's partials and sums, in piece order
    const float* base = a.gs_part + static_cast<int64_t>(blockIdx.x) * KS * kGsPieceFloats;
    if (t < NIN * 16) {
      const int sgi = t / 16, mm = t % 16;
      float tot = 0.f;
      if (mm < M)
        for (int q = sgi * P; q < (sgi + 1) * P; ++q) tot += fetch_f32(base + q * kGsPieceFloats + kTiles * RB * M + mm);
      s_ss[sgi][mm] = tot;
    }
    float ps[NIN], us[NIN];
#pragma unroll
    for (int sgi = 0; sgi < NIN; ++sgi) {
      ps[sgi] = 0.f;
      us[sgi] = 0.f;
      for (int q = sgi * P; q < (sgi + 1) * P; ++q) {
        const float* pq = base + q * kGsPieceFloats;
        ps[sgi] += fetch_f32(pq + r * M + min(m, M - 1));
        if (PAIR) us[sgi] += fetch_f32(pq + (RB + r) * M + min(m, M - 1));
      }
    }
    __syncthreads();
    if (t < NIN * 16) {
      const int sgi = t / 16;
      const int Ks = sgi == 0 ? a.in[0].K : (sgi == 1 ? a.in[1 < NIN ? 1 : 0].K : a.in[2 < NIN ? 2 : 0].K);
      s_inv[sgi][t % 16] = ((GB >> sgi) & 1) ? 1.f / sqrtf(s_ss[sgi][t % 16] / static_cast<float>(Ks) + a.eps) : 1.f;
    }
    __syncthreads();
#pragma unroll
    for (int sgi = 0; sgi < NIN; ++sgi) {
      g = fmaf(ps[sgi], s_inv[sgi][min(m, 15)], g);
      u = fmaf(us[sgi], s_inv[sgi][min(m, 15)], u);
    }
  } else if constexpr (GRP) {
    if (t < NIN * 16) {
      const int sgi = t / 16;
      const int Ks = sgi == 0 ? a.in[0].K : (sgi == 1 ? a.in[S1].K : a.in[S2].K);
      s_inv[sgi][t % 16] = kGain ? 1.f / sqrtf(s_ss[sgi][t % 16] / static_cast<float>(Ks) + a.eps) : 1.f;
    }
    __syncthreads();
#pragma unroll
    for (int sgi = 0; sgi < NIN; ++sgi) {
      g = fmaf(pgs[sgi], s_inv[sgi][min(m, 15)], g);
      u = fmaf(pus[sgi], s_inv[sgi][min(m, 15)], u);
    }
  } else {
    if (t < 16) s_inv[0][t] = kGain ? 1.f / sqrtf(s_ss[0][t] / static_cast<float>(K) + a.eps) : 1.f;
    __syncthreads();
    g = pg * s_inv[0][min(m, 15)];
    u = pu * s_inv[0][min(m, 15)];
  }
  if (mine && m < m_live && n < a.N) {
    if (a.epi == kEpiArgmax) {
      const unsigned long long key = head_key(a, m, n, g);
      atomicMax(&s_key[0][m], key);
    } else {
      store_out<PAIR>(a, m, n, g, u, resv);
    }
  }
  if (a.epi == kEpiArgmax) argmax_epilogue<kMaxM>(a, m_live, s_key);  // one piece per tile (host)
}

}  // namespace wc
