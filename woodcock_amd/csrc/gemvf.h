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

// Registers of one k step in flight: TW weight fragments, the lane's 8 inputs
// (fp32: two vectors; bf16: the first) and 8 gains.
template <int TW>
struct GfStep {
  uint4 w[TW];
  uint4 x0, x1, g;
};

// Issue the loads of step i (segment s, local step j of that segment).  STG:
// the lane's input row of segment S is staged in LDS as fp32 x * gain (xs).
template <int S, int TW, bool PAIR, int XB, int GB, bool STG>
__device__ __forceinline__ void gf_load(const GemvArgs& a, const uint16_t* (*wrow)[TW], const int64_t* xoff,
                                        const float* const* xs, int j, GfStep<TW>& st) {
  const int kg = (threadIdx.x % kWave) / 16;
  const int k = j * 32 + kg * 8;
#pragma unroll
  for (int t = 0; t < TW; ++t) st.w[t] = *reinterpret_cast<const uint4*>(wrow[S][t] + j * 32);
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
template <int TW, int W, int D, bool PAIR, int NIN, int XB, int GB, bool STG = false>
__global__ __launch_bounds__(W * kWave) void k_gemvf(GemvArgs a) {
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
      wrow[s][tt] = row_ptr<PAIR>(a, n, PAIR ? tt : 0, s) + kg * 8;
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
    um = u / upr[us];
    uk0 = (u % upr[us]) * kGfUnit;
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
        *reinterpret_cast<float4*>(g_xs + soff[us] + um * K + k) = v;
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
    if (s_ == 0) gf_load<0, TW, PAIR, XB, GB, STG>(a, wrow, xoff, xs, j_, ST);                \
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
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
          const uint16_t* wp = s_ == 0 ? wrow[0][tt] : (s_ == 1 ? wrow[NIN > 1 ? 1 : 0][tt] : wrow[NIN > 2 ? 2 : 0][tt]);
          ring[u].w[tt] = *reinterpret_cast<const uint4*>(wp + j_ * 32);
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
        for (int q = 0; q < upr[sgi]; ++q) tot += s_ssu[base + m * upr[sgi] + q];
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

}  // namespace wc
