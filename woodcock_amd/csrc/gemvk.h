// gemvk.h -- few-row (2 <= M <= 8) streaming GEMV on the vector ALUs, the
// K dimension split over the waves of a block.
//
//   y[m][n] = sum_s inv_s[m] * sum_k W_s[n][k] * (x_s[m][k] * gain_s[k])
//
// The weights stream exactly as in the one-row kernel: lane j reads bf16
// k = 8j..8j+7 of a 512-wide step, so one load instruction of a wave is 1 KB
// of one weight row (the fastest pattern measured on gfx950; a 16-row MFMA
// fragment, 64 bytes from each of 16 rows per instruction, streams about a
// third slower).  Each wave owns S consecutive steps of ONE input segment for
// the block's R output rows (2R physical rows for the gate / up pair): it
// issues those weight loads first, then its own x slices of the live input
// rows and the gains, widens each weight to fp32 once and forms every
// (row, input row) product with fp32 FMAs.  A wave's x slices are its own (the
// waves of a block tile K), so nothing is staged in LDS and x is read once per
// block (the x rows are L2-resident after the first blocks), against once per
// block for all of K in an LDS-staged design.  Each wave's vector-ALU work
// between its loads' arrival and its partial sums (M fused multiply-adds per
// weight element, the lane reductions) sits on the block's critical path, so
// it is kept short: the weights are widened once (not once per input row),
// input rows past the device row count are skipped by wave-uniform branches,
// and the lanes are reduced within 16-lane rows only (four DPP steps per
// value).  (Counters show 8-26% VALU busy over the launch: the limit is the
// latency of each block's load -> compute -> reduce chain, not ALU throughput.)
// Per (output row, input row) each 16-lane row of the wave is summed with DPP
// moves and leaves its total of the partial product and of the partial sum of
// squares in LDS;
// after one barrier the block applies each segment's 1/rms (sums of squares
// added in wave order) and adds the waves' partials in wave order, so the
// result does not depend on timing.  No device counter, no second launch.
#pragma once
#include "gemv.h"

namespace wc {

constexpr int kGkWavesMax = 16;  // waves of a block, at most

// sum over each 16-lane row by DPP moves; every lane of a row holds its row's total
__device__ __forceinline__ float row16_total(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x124>(v);  // row_ror:4
  v += dpp_move<0x128>(v);  // row_ror:8
  return v;
}

// Last block of the launch (device counter, reset by the finisher): the final
// RMSNorm of the m produced rows, read back coherently (they were published),
// into fin_out, and the offset advance.  Every row's values and the gains are
// requested at once (one round trip for all rows, from clamped addresses) when
// a row is at most kFinPer values per thread; sums in wave order.
constexpr int kFinPer = 8;
template <int MM>
__device__ __forceinline__ void gk_fin_epilogue(const GemvArgs& a, int m, float (*s_red)[kGkWavesMax], int blk,
                                                int nblk) {
  if (!last_block_done(a.fin_counter, nblk, blk)) return;
  const int nt = blockDim.x, nw = nt / kWave, lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int t = threadIdx.x;
  const int adv = (t == 0 && a.adv_dst) ? *a.adv_src : 0;
  if (a.N <= kFinPer * nt) {
    float v[MM][kFinPer];
    uint32_t gw[kFinPer];
#pragma unroll
    for (int mi = 0; mi < MM; ++mi)
#pragma unroll
      for (int j = 0; j < kFinPer; ++j)
        v[mi][j] = fetch_f32(a.y + min(mi, max(m - 1, 0)) * a.ldy + min(t + j * nt, a.N - 1));
#pragma unroll
    for (int j = 0; j < kFinPer; ++j) gw[j] = a.fin_gain[min(t + j * nt, a.N - 1)];
#pragma unroll
    for (int j = 0; j < kFinPer; ++j) pin(gw[j]);
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kFinPer; ++j) {
        const float x = t + j * nt < a.N ? v[mi][j] : 0.f;
        ss = fmaf(x, x, ss);
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) s_red[mi][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      if (mi >= m) continue;
      float tot = 0.f;
      for (int w = 0; w < nw; ++w) tot += s_red[mi][w];
      const float inv = 1.f / sqrtf(tot / static_cast<float>(a.N) + a.eps);
#pragma unroll
      for (int j = 0; j < kFinPer; ++j) {
        const int k = t + j * nt;
        if (k < a.N) a.fin_out[mi * a.ld_fin + k] = v[mi][j] * inv * bf16_to_float(static_cast<uint16_t>(gw[j]));
      }
    }
  } else {
    for (int mi = 0; mi < m; ++mi) {
      const float* yr = a.y + mi * a.ldy;
      float ss = 0.f;
      for (int k = t; k < a.N; k += nt) {
        const float x = fetch_f32(yr + k);
        ss = fmaf(x, x, ss);
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) s_red[0][wave] = ss;
      __syncthreads();
      float tot = 0.f;
      for (int w = 0; w < nw; ++w) tot += s_red[0][w];
      const float inv = 1.f / sqrtf(tot / static_cast<float>(a.N) + a.eps);
      for (int k = t; k < a.N; k += nt)
        a.fin_out[mi * a.ld_fin + k] = fetch_f32(yr + k) * inv * bf16_to_float(a.fin_gain[k]);
      __syncthreads();
    }
  }
  if (t == 0 && a.adv_dst) *a.adv_dst = adv + a.adv_add + m;
}

// R: logical output rows per block (gate rows for PAIR); S: 512-wide k steps
// per wave; MM: compile-time bound on the input rows (run time: a.M, and the
// live rows *a.m_dev <= a.M); WB: waves per block the launch bounds allow (the
// launch uses blockDim.x / 64 waves).  Waves are segment-aligned: the host
// checks that every segment's step count is a multiple of S, except with one
// segment, where the last wave's steps past the end are zeroed.
// One block of the GEMV: block blk of nblk (a kernel of its own, or the GEMV
// part of a launch that runs other work in its other blocks).
template <int R, bool PAIR, int NIN, int S, int MM, int XB, int GB, int WB>
__device__ __forceinline__ void gemvk_block(const GemvArgs& a, const int blk, const int nblk) {
  static_assert(NIN >= 1 && NIN <= 3, "one to three input segments");
  static_assert(GB == 0 || GB == (1 << NIN) - 1, "every segment normed or none");
  constexpr int P = PAIR ? 2 : 1;
  constexpr bool kGain = GB != 0;
  __shared__ float s_ss[WB][MM][4];
  __shared__ float s_dot[WB][R * P][MM][4];
  __shared__ float s_inv[NIN][MM];
  __shared__ float s_fin[MM][kGkWavesMax];
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int nw = blockDim.x / kWave;
  const int row0 = blk * R;
  constexpr int S1 = NIN > 1 ? 1 : 0, S2 = NIN > 2 ? 2 : 0;

  // this wave's segment and first local step (scalar selects over arguments
  // read at constant offsets; a run-time index into the argument arrays would
  // copy them to scratch memory)
  int seg = 0, j0 = wave * S;
  int nst = a.in[0].K / 512;
  if constexpr (NIN > 1) {
    if (j0 >= nst) {
      j0 -= nst;
      seg = 1;
      nst = a.in[S1].K / 512;
      if constexpr (NIN > 2) {
        if (j0 >= nst) {
          j0 -= nst;
          seg = 2;
          nst = a.in[S2].K / 512;
        }
      }
    }
  }
  const void* sgx = a.in[0].x;
  int64_t sgld = a.in[0].ld;
  const int32_t* sgidx = a.in[0].row_idx;
  int sgadd = a.in[0].row_add, sgmax = a.in[0].max_row;
  const uint16_t* sgain = a.in[0].gain;
  if constexpr (NIN > 1) {
    const bool c = seg == 1;
    sgx = c ? a.in[S1].x : sgx;
    sgld = c ? a.in[S1].ld : sgld;
    sgidx = c ? a.in[S1].row_idx : sgidx;
    sgadd = c ? a.in[S1].row_add : sgadd;
    sgmax = c ? a.in[S1].max_row : sgmax;
    sgain = c ? a.in[S1].gain : sgain;
  }
  if constexpr (NIN > 2) {
    const bool c = seg == 2;
    sgx = c ? a.in[S2].x : sgx;
    sgld = c ? a.in[S2].ld : sgld;
    sgidx = c ? a.in[S2].row_idx : sgidx;
    sgadd = c ? a.in[S2].row_add : sgadd;
    sgmax = c ? a.in[S2].max_row : sgmax;
    sgain = c ? a.in[S2].gain : sgain;
  }
  const bool bf = (XB >> seg) & 1;

  // 1. weights of the block's rows over this wave's steps (addresses clamped
  //    into the matrix: every load unconditional, issued back to back)
  uint4 w[R][P][S];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(row0 + r, a.N - 1);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint16_t* wr = row_ptr<PAIR>(a, n, p, 0);
      if constexpr (NIN > 1) wr = seg == 1 ? row_ptr<PAIR>(a, n, p, S1) : wr;
      if constexpr (NIN > 2) wr = seg == 2 ? row_ptr<PAIR>(a, n, p, S2) : wr;
      wr += lane * 8;
#pragma unroll
      for (int u = 0; u < S; ++u) w[r][p][u] = *reinterpret_cast<const uint4*>(wr + min(j0 + u, nst - 1) * 512);
    }
  }
  const int m_live = a.m_dev ? min(max(*a.m_dev, 0), a.M) : a.M;

  // 2. the x slices of the live input rows, then the gains
  uint4 xq[S][MM][2];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m < m_live) {
      int r = (sgidx ? sgidx[m] : m) + sgadd;
      if (sgmax > 0) r = min(max(r, 0), sgmax - 1);
      const int64_t xr = static_cast<int64_t>(r) * sgld;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int k = min(j0 + u, nst - 1) * 512 + lane * 8;
        if (bf) {
          xq[u][m][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(sgx) + xr + k);
        } else {
          const float* xp = static_cast<const float*>(sgx) + xr + k;
          xq[u][m][0] = *reinterpret_cast<const uint4*>(xp);
          xq[u][m][1] = *reinterpret_cast<const uint4*>(xp + 4);
        }
      }
    }
  }
  uint4 gq[S];
  if constexpr (kGain) {
#pragma unroll
    for (int u = 0; u < S; ++u)
      gq[u] = *reinterpret_cast<const uint4*>(sgain + min(j0 + u, nst - 1) * 512 + lane * 8);
  }

  // 3. products: the weights widened to fp32 once, then per live input row its
  //    sum of squares and R x P dot products
  float wf[R][P][S][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const uint4 q = w[r][p][u];
        wf[r][p][u][0] = bf16_lo(q.x); wf[r][p][u][1] = bf16_hi(q.x);
        wf[r][p][u][2] = bf16_lo(q.y); wf[r][p][u][3] = bf16_hi(q.y);
        wf[r][p][u][4] = bf16_lo(q.z); wf[r][p][u][5] = bf16_hi(q.z);
        wf[r][p][u][6] = bf16_lo(q.w); wf[r][p][u][7] = bf16_hi(q.w);
      }
  float ss[MM];
  float acc[R][P][MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    ss[m] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) acc[r][p][m] = 0.f;
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m < m_live) {
#pragma unroll
      for (int u = 0; u < S; ++u) {
        float4 x0, x1;
        if (bf) {
          const uint4 h = xq[u][m][0];
          x0 = make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
          x1 = make_float4(bf16_lo(h.z), bf16_hi(h.z), bf16_lo(h.w), bf16_hi(h.w));
        } else {
          x0 = make_float4(__uint_as_float(xq[u][m][0].x), __uint_as_float(xq[u][m][0].y),
                           __uint_as_float(xq[u][m][0].z), __uint_as_float(xq[u][m][0].w));
          x1 = make_float4(__uint_as_float(xq[u][m][1].x), __uint_as_float(xq[u][m][1].y),
                           __uint_as_float(xq[u][m][1].z), __uint_as_float(xq[u][m][1].w));
        }
        if (j0 + u >= nst) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);  // ragged last wave (one segment)
        if constexpr (kGain) {
          float q = ss[m];
          q = fmaf(x0.x, x0.x, q); q = fmaf(x0.y, x0.y, q); q = fmaf(x0.z, x0.z, q); q = fmaf(x0.w, x0.w, q);
          q = fmaf(x1.x, x1.x, q); q = fmaf(x1.y, x1.y, q); q = fmaf(x1.z, x1.z, q); q = fmaf(x1.w, x1.w, q);
          ss[m] = q;
          const uint4 g = gq[u];
          x0 = make_float4(x0.x * bf16_lo(g.x), x0.y * bf16_hi(g.x), x0.z * bf16_lo(g.y), x0.w * bf16_hi(g.y));
          x1 = make_float4(x1.x * bf16_lo(g.z), x1.y * bf16_hi(g.z), x1.z * bf16_lo(g.w), x1.w * bf16_hi(g.w));
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const float* f = wf[r][p][u];
            float d = acc[r][p][m];
            d = fmaf(f[0], x0.x, d); d = fmaf(f[1], x0.y, d); d = fmaf(f[2], x0.z, d); d = fmaf(f[3], x0.w, d);
            d = fmaf(f[4], x1.x, d); d = fmaf(f[5], x1.y, d); d = fmaf(f[6], x1.z, d); d = fmaf(f[7], x1.w, d);
            acc[r][p][m] = d;
          }
      }
    }
  }

  // 4. lane sums: each 16-lane row summed by DPP moves, the rows' four totals
  //    (lanes 15, 31, 47, 63) left in LDS
  const int q4 = lane / 16;
  const bool row_end = lane % 16 == 15;
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m < m_live) {
      if constexpr (kGain) {
        const float q = row16_total(ss[m]);
        if (row_end) s_ss[wave][m][q4] = q;
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const float d = row16_total(acc[r][p][m]);
          if (row_end) s_dot[wave][r * P + p][m][q4] = d;
        }
    }
  }
  __syncthreads();

  // 5. 1/rms of (segment, input row): its waves' sums in wave order
  const int w1 = (a.in[0].K / 512 + S - 1) / S;              // first wave of segment 1
  const int w2 = NIN > 2 ? w1 + a.in[S1].K / 512 / S : nw;   // first wave of segment 2
  if (t < NIN * MM) {
    const int sg = t / MM, m = t % MM;
    const int lo = sg == 0 ? 0 : (sg == 1 ? w1 : w2), hi = sg == 0 ? (NIN > 1 ? w1 : nw) : (sg == 1 ? (NIN > 2 ? w2 : nw) : nw);
    float tot = 0.f;
    if (kGain && m < m_live)
      for (int v = lo; v < hi; ++v) tot += (s_ss[v][m][0] + s_ss[v][m][1]) + (s_ss[v][m][2] + s_ss[v][m][3]);
    const int K = sg == 0 ? a.in[0].K : (sg == 1 ? a.in[S1].K : a.in[S2].K);
    s_inv[sg][m] = kGain ? 1.f / sqrtf(tot / static_cast<float>(K) + a.eps) : 1.f;
  }
  __syncthreads();

  // 6. outputs (row r of the block, input row m), rows fastest
  for (int idx = t; idx < R * MM; idx += blockDim.x) {
    const int r = idx % R, m = idx / R;
    const int n = row0 + r;
    if (m >= m_live || n >= a.N) continue;
    float g = 0.f, u = 0.f;
    for (int v = 0; v < nw; ++v) {
      const int sg = v < w1 ? 0 : (NIN > 2 && v >= w2 ? 2 : (NIN > 1 ? 1 : 0));
      const float inv = s_inv[sg][m];
      const float* dg = s_dot[v][r * P][m];
      g = fmaf((dg[0] + dg[1]) + (dg[2] + dg[3]), inv, g);
      if (PAIR) {
        const float* du = s_dot[v][r * P + P - 1][m];
        u = fmaf((du[0] + du[1]) + (du[2] + du[3]), inv, u);
      }
    }
    store_out<PAIR>(a, m, n, g, u, res_value(a, m, n));
  }
  // the final RMSNorm of the produced rows (the drafter's `out`) by the last
  // block, which then also advances the offset
  if (a.fin_gain) {
    gk_fin_epilogue<MM>(a, m_live, s_fin, blk, nblk);
    return;
  }
  // otherwise the cache offset advance of the last projection (no block reads it here)
  if (a.adv_dst && blk == 0 && t == 0) *a.adv_dst = *a.adv_src + a.adv_add + m_live;
}

template <int R, bool PAIR, int NIN, int S, int MM, int XB, int GB, int WB>
__global__ __launch_bounds__(WB * kWave) void k_gemvk(GemvArgs a) {
  gemvk_block<R, PAIR, NIN, S, MM, XB, GB, WB>(a, blockIdx.x, gridDim.x);
}

}  // namespace wc
