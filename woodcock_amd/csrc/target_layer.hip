// target_layer.hip -- one Qwen3 decoder layer over a verify block of M <= 64
// rows (the tree / chain verify forward of the target model,
// python/woodcock/target.py:82-116,142-156; src/core/qwen3.cpp:75-114):
//   h  = x + W_o . attn(q_norm(W_q xn), k_norm(W_k xn), W_v xn),  xn = RMS_in(x)
//   x' = h + W_down . (silu(W_gate hn) * W_up hn),                  hn = RMS_post(h)
// with RoPE at explicit positions and an explicit boolean mask over the cache
// slots (the tree mask, python/woodcock/sampling.py:118-128), appending the
// block's K/V at the cache offset.
//
// The projections are skinny GEMMs (M <= 64 rows against weight matrices of
// 2048..12288 rows), HBM-bound on the weight stream: bf16 MFMA
// (v_mfma_f32_16x16x32_bf16) with the fp32 activations split into bf16 hi + lo
// parts (x = hi + lo to ~2^-17 relative) so the products keep fp32-level
// accuracy.  The activations are written once, already split and in MFMA
// fragment order (xa_index), by whoever produces them -- a prep kernel for the
// layer input, the attention merge, the o_proj and gate/up epilogues -- with
// the next RMSNorm's gain folded in and per-row sums of squares on the side
// (the norm's 1/rms scales the products afterwards).  k_mm_stream streams the
// weights straight into B fragments eight k steps ahead while a three-slot LDS
// ring hands each k step of activations to the block's four waves; blocks
// split K when the projection is too narrow to fill the GPU, each split
// storing its fp32 tile with plain stores, and k_mm_fix (the next launch, over
// column ranges x 16-row groups) sums the splits in a fixed order and runs the
// epilogue (store, residual, SiLU(gate) * up, next activations, or the QKV
// head epilogue) -- no device-scope hand-over inside the GEMM, except for
// blocks of at most 16 rows, whose small tiles the last split of each column
// range sums in the same order inside the GEMM launch (k_mm_wave's FTW).
#include <array>

#include "attention.h"

namespace wc {

// ------------------------------------------------------------------ activation prep
// x [M][ldx] fp32 (times gain when given) -> fragment-major hi / lo, plus the
// rows' sums of squares of x per 256-wide k block: ss [K / 256][64].  Block
// (b, r) covers k [256 b, 256 b + 256) of rows 16 r .. 16 r + 15 (rows >= M are
// zero); thread t row 16 r + t / 16, k [256 b + 16 (t % 16), + 16).
struct XaPrepArgs {
  const float* x;
  int64_t ldx;
  int M, K;
  const uint16_t* gain;
  uint16_t* xa;
  float* ss;
};

__global__ __launch_bounds__(256) void k_xa_prep(XaPrepArgs a) {
  const int t = threadIdx.x, m = blockIdx.y * 16 + t / 16, k0 = blockIdx.x * 256 + (t % 16) * 16;
  const bool live = m < a.M;
  const float* xr = a.x + static_cast<int64_t>(min(m, a.M - 1)) * a.ldx + k0;
  float4 xv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const float4*>(xr + 4 * i);
  uint4 gv[2];
  if (a.gain) {
#pragma unroll
    for (int i = 0; i < 2; ++i) gv[i] = *reinterpret_cast<const uint4*>(a.gain + k0 + 8 * i);
  }
  float ss = 0.f;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    float v[8] = {xv[2 * g].x, xv[2 * g].y, xv[2 * g].z, xv[2 * g].w,
                  xv[2 * g + 1].x, xv[2 * g + 1].y, xv[2 * g + 1].z, xv[2 * g + 1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (!live) v[e] = 0.f;
      ss = fmaf(v[e], v[e], ss);
    }
    if (a.gain) {
      const uint4 q = gv[g];
      v[0] *= bf16_lo(q.x); v[1] *= bf16_hi(q.x); v[2] *= bf16_lo(q.y); v[3] *= bf16_hi(q.y);
      v[4] *= bf16_lo(q.z); v[5] *= bf16_hi(q.z); v[6] *= bf16_lo(q.w); v[7] *= bf16_hi(q.w);
    }
    uint4 hi, lo;
    split8(v, hi, lo);
    *reinterpret_cast<uint4*>(a.xa + xa_index(m, k0 + 8 * g, 0)) = hi;
    *reinterpret_cast<uint4*>(a.xa + xa_index(m, k0 + 8 * g, 1)) = lo;
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o);
  if (t % 16 == 0) a.ss[blockIdx.x * 64 + m] = ss;
}

// ------------------------------------------------------------------ streaming skinny GEMM

enum SkEpi { kSkRaw = 0, kSkStore = 1, kSkResidual = 2, kSkSiluPair = 3, kSkQkvHead = 4 };
constexpr int kSkMaxSeg = 3;
constexpr int kSkP = 8;            // k steps of weights / activations in flight

struct SkArgs {
  const uint16_t* xa;  // fragment-major activations, K / 32 steps
  const float* ss;     // row scale: inv = 1 / sqrt(sum_p ss[p][m] / ss_k + eps); NULL = 1
  int n_ss, ss_k;
  float eps;
  const uint16_t* w[kSkMaxSeg];  // weight segments [rows][K] bf16
  int seg_start[kSkMaxSeg + 1];
  int n_seg;
  int M, N, K, ks;  // N weight rows (SiLU pair: gate rows then up rows); ks = K splits
  int epi;
  float* out;  // [M][ldo] (N columns, N / 2 for the pair); may be NULL for the pair
  int64_t ldo;
  const float* res;  // residual [M][ldr]
  int64_t ldr;
  uint16_t* xa_next;         // optional: the output as the next projection's activations
  const uint16_t* gain_next; // its RMSNorm gain (NULL = none)
  float* ss_next;            // with xa_next: per-row sums of squares of the output, [gridDim.x][64]
  float* part;               // ks > 1: [ks][64][cols] partials (summed by k_mm_fix)
  unsigned int* fix_ctr;     // <= 16 rows: one zeroed counter per column range (the fix-up in the GEMM)
  // kSkQkvHead (column ranges of one 128-wide head): q / k heads get their
  // RMSNorm (q_gain / k_gain) and rotate-half RoPE at the row's position; q
  // rows land in out [M][ldo], k / v rows in the cache at slot offset + row
  int nq, nk;
  const uint16_t *q_gain, *k_gain;
  const float *rope_cos, *rope_sin;
  int rope_max;
  const int32_t* positions;  // [M] or NULL: offset + row
  const int32_t* offset_dev;
  void *kc, *vc;  // [Hk][cap][128]
  int kv_bf16, cap;
};

// Operands of the epilogue that do not depend on the tile: the row scale's
// partial sums of squares (thread t sums parts t % 4 + 4 q of row t / 4), the
// residuals and the next gains of the thread's columns.  Loaded on their own so
// that a caller can issue them before the loads the tile waits on.
constexpr int kSsMax = 16;  // row-scale parts <= 64
template <int TW, bool QKV = false>
struct EpiOps {
  float ssv[kSsMax], resv[16 * TW];
  uint16_t gnv[16 * TW];
  // the QKV head epilogue: the row's cache offset / position, and the cos, sin
  // and head-norm gains of the thread's columns
  int offset, pos;
  float cs[QKV ? 16 * TW : 1], sn[QKV ? 16 * TW : 1];
  uint16_t hg[QKV ? 16 * TW : 1];
};

template <int TW, bool QKV = false>
__device__ __forceinline__ void sk_epi_load(const SkArgs& a, int cb, EpiOps<TW, QKV>& o) {
  constexpr int FB = 64 * TW, CQ = FB / 4;
  const int t = threadIdx.x;
  const bool pair = a.epi == kSkSiluPair;
  const int m = t / 4, g = t % 4;
  const int n0 = pair ? cb * 64 + g * 16 : cb * FB + g * CQ;
  const int mr = min(m, a.M - 1);
  if constexpr (QKV) {  // one 128-wide head per column range: 16-byte loads of the thread's 32 columns
    static_assert(FB == 128, "one head per column range");
    const int col0 = cb * FB, d0 = g * CQ;
    const bool is_q = col0 < a.nq, is_k = !is_q && col0 < a.nq + a.nk;
    o.offset = *a.offset_dev;
    o.pos = a.positions ? a.positions[mr] : -1;  // resolved (and the table read) by sk_epi_rope
    if (is_q || is_k) {
      const uint4* gp = reinterpret_cast<const uint4*>((is_q ? a.q_gain : a.k_gain) + d0);
      uint4 gv[CQ / 8];
#pragma unroll
      for (int i = 0; i < CQ / 8; ++i) gv[i] = gp[i];
#pragma unroll
      for (int i = 0; i < CQ / 8; ++i) {
        const uint32_t w4[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) o.hg[8 * i + e] = static_cast<uint16_t>(w4[e / 2] >> (16 * (e % 2)));
      }
    }
  }

#pragma unroll
  for (int q = 0; q < kSsMax; ++q) {
    const int pp = g + 4 * q;
    o.ssv[q] = (a.ss && pp < a.n_ss) ? a.ss[pp * 64 + m] : 0.f;
  }
  if constexpr (QKV) return;  // the head epilogue reads no residual and no next gain
  // residuals and gains as 16-byte loads where the thread's columns are whole
  // and aligned (scalar loads of 16 rows x 4 column runs per instruction cost
  // as much as the partial sums they wait beside)
  const bool res = !pair && a.epi == kSkResidual;
  const float* rp = res ? a.res + static_cast<int64_t>(mr) * a.ldr + n0 : nullptr;
  if (res && n0 + CQ <= a.N && (reinterpret_cast<uintptr_t>(rp) & 15) == 0) {
    float4 rv[CQ / 4];
#pragma unroll
    for (int i = 0; i < CQ / 4; ++i) rv[i] = reinterpret_cast<const float4*>(rp)[i];
#pragma unroll
    for (int i = 0; i < CQ / 4; ++i) {
      o.resv[4 * i] = rv[i].x;
      o.resv[4 * i + 1] = rv[i].y;
      o.resv[4 * i + 2] = rv[i].z;
      o.resv[4 * i + 3] = rv[i].w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < CQ; ++c)
      o.resv[c] = res ? a.res[static_cast<int64_t>(mr) * a.ldr + min(n0 + c, a.N - 1)] : 0.f;
  }
  constexpr int NG = 16 * TW;  // gains read: CQ (one per output column), the pair's first 16
  const int ng = pair ? 16 : CQ;
  const uint16_t* gp = a.gain_next ? a.gain_next + n0 : nullptr;
  if (a.xa_next && gp && (reinterpret_cast<uintptr_t>(gp) & 15) == 0 && (pair || n0 + CQ <= a.N)) {
    uint4 gq[NG / 8];
#pragma unroll
    for (int i = 0; i < NG / 8; ++i) gq[i] = reinterpret_cast<const uint4*>(gp)[min(i, ng / 8 - 1)];
#pragma unroll
    for (int i = 0; i < NG / 8; ++i) {
      const uint32_t w4[4] = {gq[i].x, gq[i].y, gq[i].z, gq[i].w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o.gnv[8 * i + e] = 8 * i < ng ? static_cast<uint16_t>(w4[e / 2] >> (16 * (e % 2))) : 0;
    }
  } else if (a.xa_next && gp) {  // every gain load issued before the first is used
    uint32_t gw[CQ];
#pragma unroll
    for (int c = 0; c < CQ; ++c) gw[c] = a.gain_next[n0 + min(c, pair ? 15 : CQ - 1)];
#pragma unroll
    for (int c = 0; c < CQ; ++c) pin(gw[c]);
#pragma unroll
    for (int c = 0; c < CQ; ++c) o.gnv[c] = (!pair || c < 16) ? static_cast<uint16_t>(gw[c]) : 0;
  } else {
#pragma unroll
    for (int c = 0; c < CQ; ++c) o.gnv[c] = 0;
  }
}

// The QKV head epilogue's cos / sin at the row's position: a load that waits
// for the position, so callers issue it after the loads that do not.
template <int TW, bool QKV>
__device__ __forceinline__ void sk_epi_rope(const SkArgs& a, int cb, EpiOps<TW, QKV>& o) {
  if constexpr (QKV) {
    constexpr int FB = 64 * TW, CQ = FB / 4;
    const int t = threadIdx.x, m = t / 4, g = t % 4, d0 = g * CQ, col0 = cb * FB;
    const bool is_q = col0 < a.nq, is_k = !is_q && col0 < a.nq + a.nk;
    o.pos = min(max(o.pos >= 0 ? o.pos : o.offset + min(m, a.M - 1), 0), a.rope_max - 1);
    if (is_q || is_k) {
      const float4* cp = reinterpret_cast<const float4*>(a.rope_cos + static_cast<int64_t>(o.pos) * (FB / 2) + d0 % (FB / 2));
      const float4* sp = reinterpret_cast<const float4*>(a.rope_sin + static_cast<int64_t>(o.pos) * (FB / 2) + d0 % (FB / 2));
      float4 cv[CQ / 4], sv[CQ / 4];
#pragma unroll
      for (int i = 0; i < CQ / 4; ++i) {
        cv[i] = cp[i];
        sv[i] = sp[i];
      }
#pragma unroll
      for (int i = 0; i < CQ / 4; ++i) {
        o.cs[4 * i] = cv[i].x; o.cs[4 * i + 1] = cv[i].y; o.cs[4 * i + 2] = cv[i].z; o.cs[4 * i + 3] = cv[i].w;
        o.sn[4 * i] = sv[i].x; o.sn[4 * i + 1] = sv[i].y; o.sn[4 * i + 2] = sv[i].z; o.sn[4 * i + 3] = sv[i].w;
      }
    }
  }
}

// Epilogue of a column range for rows [r0, r1) of the tile in s_c (row r,
// column c at s_c[r * (FB + 4) + c]): the row scale, then store / residual /
// SiLU(gate) * up / the next activations, or the QKV head epilogue.  Every
// thread of the block calls it; rows outside [r0, r1) or >= M write nothing.
template <int TW, bool QKV = false>
__device__ __forceinline__ void sk_epi_run(const SkArgs& a, float* s_c, float* s_inv, int cb, int r0, int r1,
                                           const EpiOps<TW, QKV>& ops) {
  constexpr int FB = 64 * TW;
  constexpr int LDC = FB + 4;
  const int t = threadIdx.x;
  const bool pair = a.epi == kSkSiluPair;
  const int m = t / 4, g = t % 4;  // row m, column quarter g
  const bool live = m < a.M && m >= r0 && m < r1;
  constexpr int CQ = FB / 4;
  const int n0 = pair ? cb * 64 + g * 16 : cb * FB + g * CQ;  // first output column of this thread
  const float* ssv = ops.ssv;
  const float* resv = ops.resv;
  const uint16_t* gnv = ops.gnv;
  {
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kSsMax; ++q) tot += ssv[q];
    tot += __shfl_xor(tot, 1);
    tot += __shfl_xor(tot, 2);
    if (g == 0) s_inv[m] = a.ss ? 1.f / sqrtf(tot / static_cast<float>(a.ss_k) + a.eps) : 1.f;
  }
  __syncthreads();
  if (QKV || a.epi == kSkQkvHead) {
    // one head per column range: RMS_in scale, then for q / k heads the per-head
    // RMSNorm (q_norm / k_norm gains) and rotate-half RoPE at the row's position
    // (src/backends/cpu_ops.cpp:61-77), in the order x1 = x inv g,
    // lo' = x1 c - x2 s, hi' = x2 c + x1 s.  q lands in out; K and V rows go
    // straight to the cache at slot offset + row, so the attention that follows
    // reads every key, old or new, from the cache.
    const int col0 = cb * FB, d0 = g * CQ;
    const bool is_q = col0 < a.nq, is_k = !is_q && col0 < a.nq + a.nk;
    const float inv = s_inv[m];
    float y[CQ];
    float hs = 0.f;
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      y[c] = s_c[m * LDC + d0 + c] * inv;
      hs = fmaf(y[c], y[c], hs);
    }
    hs += __shfl_xor(hs, 1);
    hs += __shfl_xor(hs, 2);
    int offset, pos;
    if constexpr (QKV) {
      offset = ops.offset;
      pos = ops.pos;
    } else {
      offset = *a.offset_dev;
      pos = min(max(a.positions ? a.positions[min(m, a.M - 1)] : offset + m, 0), a.rope_max - 1);
    }
    if (is_q || is_k) {
      const float invh = 1.f / sqrtf(hs / static_cast<float>(FB) + a.eps);
      const uint16_t* gain = is_q ? a.q_gain : a.k_gain;
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        float gc;
        if constexpr (QKV) gc = bf16_to_float(ops.hg[c]);
        else gc = bf16_to_float(gain[d0 + c]);
        y[c] = y[c] * invh * gc;
        s_c[m * LDC + d0 + c] = y[c];
      }
    }
    __syncthreads();
    if (!live) return;
    if (is_q || is_k) {
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        const int dd = d0 + c, pi = dd % (FB / 2);
        const float xp = s_c[m * LDC + (dd ^ (FB / 2))];
        float cs, sn;
        if constexpr (QKV) {
          cs = ops.cs[c];
          sn = ops.sn[c];
        } else {
          cs = a.rope_cos[static_cast<int64_t>(pos) * (FB / 2) + pi];
          sn = a.rope_sin[static_cast<int64_t>(pos) * (FB / 2) + pi];
        }
        y[c] = dd < FB / 2 ? y[c] * cs - xp * sn : y[c] * cs + xp * sn;
      }
    }
    if (is_q) {
      float* op = a.out + static_cast<int64_t>(m) * a.ldo + col0 + d0;
      if ((reinterpret_cast<uintptr_t>(op) & 15) == 0) {
#pragma unroll
        for (int c = 0; c < CQ; c += 4) *reinterpret_cast<float4*>(op + c) = float4{y[c], y[c + 1], y[c + 2], y[c + 3]};
      } else {
#pragma unroll
        for (int c = 0; c < CQ; ++c) op[c] = y[c];
      }
      return;
    }
    const int slot = offset + m;
    if (slot < 0 || slot >= a.cap) return;
    const int head = is_k ? (col0 - a.nq) / FB : (col0 - a.nq - a.nk) / FB;
    const int64_t at = (static_cast<int64_t>(head) * a.cap + slot) * FB + d0;
    void* base = is_k ? a.kc : a.vc;
    if (a.kv_bf16) {
      uint16_t* dst = static_cast<uint16_t*>(base) + at;
#pragma unroll
      for (int c = 0; c < CQ; c += 8)  // d0 is a multiple of 32: 16-byte aligned rows of 128 bf16
        *reinterpret_cast<uint4*>(dst + c) = make_uint4(
            static_cast<uint32_t>(float_to_bf16(y[c])) | (static_cast<uint32_t>(float_to_bf16(y[c + 1])) << 16),
            static_cast<uint32_t>(float_to_bf16(y[c + 2])) | (static_cast<uint32_t>(float_to_bf16(y[c + 3])) << 16),
            static_cast<uint32_t>(float_to_bf16(y[c + 4])) | (static_cast<uint32_t>(float_to_bf16(y[c + 5])) << 16),
            static_cast<uint32_t>(float_to_bf16(y[c + 6])) | (static_cast<uint32_t>(float_to_bf16(y[c + 7])) << 16));
    } else {
      float* dst = static_cast<float*>(base) + at;
#pragma unroll
      for (int c = 0; c < CQ; c += 4) *reinterpret_cast<float4*>(dst + c) = float4{y[c], y[c + 1], y[c + 2], y[c + 3]};
    }
    return;
  }
  if (!live) return;
  const float inv = s_inv[m];
  // this thread's outputs: 8-wide groups of consecutive output columns
  constexpr int NC = CQ < 16 ? CQ : 16;  // the pair's outputs per thread
  float ss = 0.f;
#pragma unroll
  for (int c0 = 0; c0 < CQ; c0 += 8) {
    if (pair && c0 >= NC) continue;
    float z[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = c0 + e;
      float y;
      if (pair) {
        const int af = g * 16 + c;  // act feature within the block
        const int gc = (af / 16) * 32 + af % 16;
        const float gv = s_c[m * LDC + gc] * inv, uv = s_c[m * LDC + gc + 16] * inv;
        y = gv / (1.f + expf(-gv)) * uv;
      } else {
        const float sv = s_c[m * LDC + g * CQ + c];
        y = (a.epi == kSkRaw ? sv : sv * inv) + resv[c];
      }
      z[e] = y;
    }
    if (a.out) {
      float* op = a.out + static_cast<int64_t>(m) * a.ldo + n0 + c0;
      if (pair || n0 + c0 + 8 <= a.N) {
#pragma unroll
        for (int e = 0; e < 8; ++e) op[e] = z[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n0 + c0 + e < a.N) op[e] = z[e];
      }
    }
    if (a.xa_next) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ss = fmaf(z[e], z[e], ss);
        if (a.gain_next) z[e] *= bf16_to_float(gnv[c0 + e]);
      }
      uint4 hi, lo;
      split8(z, hi, lo);
      *reinterpret_cast<uint4*>(a.xa_next + xa_index(m, n0 + c0, 0)) = hi;
      *reinterpret_cast<uint4*>(a.xa_next + xa_index(m, n0 + c0, 1)) = lo;
    }
  }
  if (a.xa_next && a.ss_next) {
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    if (g == 0) a.ss_next[cb * 64 + m] = ss;
  }
}

template <int TW>
__device__ __forceinline__ void sk_epilogue(const SkArgs& a, float* s_c, float* s_inv, int cb, int r0, int r1) {
  EpiOps<TW> ops;
  sk_epi_load<TW>(a, cb, ops);
  sk_epi_run<TW>(a, s_c, s_inv, cb, r0, r1, ops);
}

// Block (column range cb, K split kz), 4 waves.  TW = tiles of 16 weight rows
// per wave (block columns FB = 64 TW); wave w owns tiles w TW .. w TW + TW - 1
// (the SiLU pair: wave w's gate tile and up tile of act features 64 cb + 16 w ..).
template <int MT, int TW>
__global__ __launch_bounds__(256) void k_mm_stream(SkArgs a) {
  constexpr int FB = 64 * TW;
  constexpr int AQ = MT * 128;                // uint4 of activations per k step
  constexpr int AR = (AQ + 255) / 256;        // per thread
  constexpr int LDC = FB + 4;
  __shared__ __attribute__((aligned(16))) uint4 s_a[3][AQ];
  __shared__ __attribute__((aligned(16))) float s_c[64 * LDC];
  __shared__ float s_inv[64];
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int cb = blockIdx.x, kz = blockIdx.y;
  const bool pair = a.epi == kSkSiluPair;

  // weights are fragment-major (wc_weights_frag): the A fragment of 16-row
  // tile T at k step s is 64 lanes x 8 bf16 at ((T S + s) 64 + lane) 8, so
  // every weight load is one contiguous kilobyte
  const int S = a.K / 32, per = (S + a.ks - 1) / a.ks;
  const uint16_t* wp[TW];
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    int tb = pair ? (j == 0 ? 0 : a.N / 2) + cb * 64 + wave * 16 : cb * FB + (wave * TW + j) * 16;
    tb = min(tb, ((a.N + 15) / 16 - 1) * 16);  // a tile past the last one re-reads it (its columns are not stored)
    int seg = 0;
#pragma unroll
    for (int q = 1; q < kSkMaxSeg; ++q)
      if (q < a.n_seg && tb >= a.seg_start[q]) seg = q;
    const uint16_t* base = seg == 0 ? a.w[0] : seg == 1 ? a.w[1] : a.w[2];
    const int s0r = seg == 0 ? a.seg_start[0] : seg == 1 ? a.seg_start[1] : a.seg_start[2];
    wp[j] = base + (static_cast<int64_t>((tb - s0r) >> 4) * S * 64 + lane) * 8;
  }
  const int s0 = min(S, kz * per), ns = min(S, s0 + per) - s0;

  af32x4 acc[TW][MT];
#pragma unroll
  for (int j = 0; j < TW; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = af32x4{0.f, 0.f, 0.f, 0.f};
  // P steps of weights and activations in flight; the activations of step i
  // are staged in LDS slot i % 3 just before step i's barrier (the barrier of
  // step i - 1 guarantees every wave is done with the slot, last read by step
  // i - 3).  Native vectors (not the uint4 struct) keep the buffers in registers.
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  uint4 wb[kSkP][TW];
  u32x4v ab[kSkP][AR];
#pragma unroll
  for (int u = 0; u < kSkP; ++u) {
    if (u < ns) {
#pragma unroll
      for (int j_ = 0; j_ < TW; ++j_) wb[u][j_] = *reinterpret_cast<const uint4*>(wp[j_] + static_cast<int64_t>(s0 + u) * 512);
      const uint4* ap_ = reinterpret_cast<const uint4*>(a.xa + static_cast<int64_t>(s0 + u) * kXaStepElems);
#pragma unroll
      for (int r_ = 0; r_ < AR; ++r_) ab[u][r_] = reinterpret_cast<const u32x4v*>(ap_)[(t + r_ * 256) % AQ];
    }
  }
  for (int b = 0; b < ns; b += kSkP) {
#pragma unroll
    for (int u = 0; u < kSkP; ++u) {
      const int i = b + u;
      if (i < ns) {
        const int slot = i % 3;
#pragma unroll
        for (int r_ = 0; r_ < AR; ++r_) reinterpret_cast<u32x4v*>(s_a[slot])[(t + r_ * 256) % AQ] = ab[u][r_];
        lds_barrier();
        abf16x8 ah[MT], al[MT];
#pragma unroll
        for (int q = 0; q < MT; ++q) {
          ah[q] = __builtin_bit_cast(abf16x8, s_a[slot][(2 * q) * 64 + lane]);
          al[q] = __builtin_bit_cast(abf16x8, s_a[slot][(2 * q + 1) * 64 + lane]);
        }
#pragma unroll
        for (int q = 0; q < MT; ++q)
#pragma unroll
          for (int j = 0; j < TW; ++j)
            acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[q], __builtin_bit_cast(abf16x8, wb[u][j]),
                                                                acc[j][q], 0, 0, 0);
#pragma unroll
        for (int q = 0; q < MT; ++q)
#pragma unroll
          for (int j = 0; j < TW; ++j)
            acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[q], __builtin_bit_cast(abf16x8, wb[u][j]),
                                                                acc[j][q], 0, 0, 0);
        if (i + kSkP < ns) {
#pragma unroll
          for (int j_ = 0; j_ < TW; ++j_) wb[u][j_] = *reinterpret_cast<const uint4*>(wp[j_] + static_cast<int64_t>(s0 + i + kSkP) * 512);
          const uint4* ap_ = reinterpret_cast<const uint4*>(a.xa + static_cast<int64_t>(s0 + i + kSkP) * kXaStepElems);
#pragma unroll
          for (int r_ = 0; r_ < AR; ++r_) ab[u][r_] = reinterpret_cast<const u32x4v*>(ap_)[(t + r_ * 256) % AQ];
        }
      }
    }
  }

  // the block's tile -> LDS: row i 16 + 4 (lane / 16) + e, column (w TW + j) 16 + lane % 16
  mfma_settle();
#pragma unroll
  for (int j = 0; j < TW; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s_c[(i * 16 + (lane / 16) * 4 + e) * LDC + (wave * TW + j) * 16 + lane % 16] = acc[j][i][e];
  __syncthreads();

  if (a.ks > 1) {
    // this split's tile, rows < M, as plain coalesced stores (a wave per row,
    // lanes along the columns); k_mm_fix sums the splits after the launch
    const int cols = gridDim.x * FB;
    float* base = a.part + static_cast<int64_t>(cb) * FB;
    for (int r = wave; r < a.M; r += 4)
#pragma unroll
      for (int c = lane * 4; c < FB; c += kWave * 4)
        *reinterpret_cast<float4*>(base + (static_cast<int64_t>(kz) * 64 + r) * cols + c) =
            *reinterpret_cast<const float4*>(&s_c[r * LDC + c]);
    return;
  }
  sk_epilogue<TW>(a, s_c, s_inv, cb, 0, 64);
}

// Barrier-free skinny GEMM for the layer's projections.  Block (column group
// cg, K split kz), 4 waves; the group is G 16-column tiles, tile tau covering
// output columns 16 tau .. 16 tau + 15 (the SiLU pair interleaves gate and up
// tiles: tau = 8 cb + 2 w + j is gate (j = 0) or up (j = 1) rows
// 64 cb + 16 w ..).  Wave w takes the split's k steps w, w + 4, ..., so the
// four waves read each tile's consecutive fragment-major kilobytes together.
// Per k step a wave loads its G weight fragments and the 2 MT activation
// fragments straight into registers (each load one contiguous kilobyte) and
// runs 2 MT G MFMAs: every activation fragment feeds G tiles, with no LDS and
// no barrier in the loop.  The four waves' tiles are summed in LDS in wave
// order and stored as this split's partial (k_mm_fix sums the splits and runs
// the epilogue).
constexpr int kMwG = 4;  // column tiles per block
constexpr int kMwP = 3;  // k steps in flight per wave

// The split-K fix-up inside the GEMM launch, for at most 16 rows: every block
// publishes its partial tile with device-coherent stores and counts itself on
// its column range's counter; the last of the range's ks x FTW blocks sums the
// partials in split order -- the order k_mm_fix uses, so the results are the
// same bits -- and runs the range's epilogue.  At 16 rows a split's tile is
// 4 KB, so the coherent hand-over costs less than the fix-up launch (its
// launch gap and first loads); with 64 rows the tiles are four times larger
// and the separate launch stays.
constexpr int kFixRanges = 256;    // column ranges with a counter of their own
constexpr int kFixFusedRows = 16;  // rows up to which the fix-up runs in the GEMM

// The last of `total` blocks counting on one counter: each thread first waits
// for its own device-coherent stores, the block barriers, one relaxed
// device-scope RMW orders the blocks; the last resets the counter.
__device__ __forceinline__ bool last_of(unsigned int* ctr, unsigned int total) {
  __shared__ bool s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  return s_last;
}

// k_mm_fix's work for column range cb and rows 0..15, run by the last block of
// the range: the partials read with device-coherent 16-byte loads (all splits
// in flight at once), summed in split order into s_c, then the epilogue.  For
// the QKV head epilogue the caller has loaded the cache offset and the row's
// position already, so the RoPE table loads go out with the others.
template <int TW, bool QKV>
__device__ __forceinline__ void sk_fix_last(const SkArgs& a, int cb, float* s_c, int offset, int pos) {
  constexpr int FB = 64 * TW, LDC = FB + 4;
  constexpr int V4 = 16 * FB / 4 / 256;  // float4 per thread: 16 rows x FB columns
  __shared__ float s_inv[64];
  const int t = threadIdx.x, cols = a.N;
  EpiOps<TW, QKV> ops;
  sk_epi_load<TW, QKV>(a, cb, ops);
  if constexpr (QKV) {
    ops.offset = offset;
    ops.pos = pos;
    sk_epi_rope<TW, QKV>(a, cb, ops);
  }
  const int64_t first = static_cast<int64_t>(cb) * FB;
  const __amdgpu_buffer_rsrc_t rs =
      buffer_rsrc(a.part + first, static_cast<int>((static_cast<int64_t>(a.ks) * 64 * cols - first) * 4));
  float4 u[8][V4];
#pragma unroll
  for (int h = 0; h < 8; ++h)
#pragma unroll
    for (int i = 0; i < V4; ++i) {
      const int e = (t + 256 * i) * 4, r = min(e / FB, a.M - 1), c = e % FB;
      const int zz = min(h, a.ks - 1);
      u[h][i] = fetch_f32x4(rs, ((zz * 64 + r) * cols + c) * 4);
    }
  float4 acc[V4];
#pragma unroll
  for (int i = 0; i < V4; ++i) acc[i] = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 8; ++h)
    if (h < a.ks)
#pragma unroll
      for (int i = 0; i < V4; ++i) {
        acc[i].x += u[h][i].x;
        acc[i].y += u[h][i].y;
        acc[i].z += u[h][i].z;
        acc[i].w += u[h][i].w;
      }
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int e = (t + 256 * i) * 4;
    *reinterpret_cast<float4*>(&s_c[(e / FB) * LDC + e % FB]) = acc[i];
  }
  __syncthreads();
  sk_epi_run<TW, QKV>(a, s_c, s_inv, cb, 0, 16, ops);
}

// PE: the SiLU pair with K unsplit (ks = 1): the block owns its 32 act
// features outright, so instead of a partial it runs the pair's epilogue
// itself (row scale from the ss parts, SiLU(gate) * up, the next projection's
// activations), and no fix-up launch follows.
// FTW > 0 (MT = 1): the fix-up of column ranges of 64 FTW runs in this launch
// (sk_fix_last), with the QKV head epilogue when FQKV.
template <int MT, bool PE = false, int FTW = 0, bool FQKV = false>
__global__ __launch_bounds__(256) void k_mm_wave(SkArgs a) {
  static_assert(FTW == 0 || (MT == 1 && !PE), "the fix-up in the GEMM takes one row tile");
  constexpr int G = kMwG, FB = 16 * G, LDR = FB + 4;
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) float s_red[4][64 * LDR];
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int cg = blockIdx.x, kz = blockIdx.y;
  const bool pair = a.epi == kSkSiluPair;
  const int S = a.K / 32, per = (S + a.ks - 1) / a.ks;
  const int sb = min(S, kz * per), se = min(S, sb + per);
  const int nw = sb + wave < se ? (se - sb - wave + 3) / 4 : 0;  // this wave's steps
  const uint16_t* wp[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int tau = cg * G + g;
    int tb = pair ? ((tau & 1) ? a.N / 2 : 0) + 64 * (tau >> 3) + 16 * ((tau >> 1) & 3) : 16 * tau;
    tb = min(tb, ((a.N + 15) / 16 - 1) * 16);
    int seg = 0;
#pragma unroll
    for (int q = 1; q < kSkMaxSeg; ++q)
      if (q < a.n_seg && tb >= a.seg_start[q]) seg = q;
    const uint16_t* base = seg == 0 ? a.w[0] : seg == 1 ? a.w[1] : a.w[2];
    const int s0r = seg == 0 ? a.seg_start[0] : seg == 1 ? a.seg_start[1] : a.seg_start[2];
    wp[g] = base + (static_cast<int64_t>((tb - s0r) >> 4) * S * 64 + lane) * 8;
  }
  const u32x4v* xa4 = reinterpret_cast<const u32x4v*>(a.xa);
  af32x4 acc[G][MT];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int q = 0; q < MT; ++q) acc[g][q] = af32x4{0.f, 0.f, 0.f, 0.f};
  u32x4v wb[kMwP][G], ab[kMwP][2 * MT];
  auto issue = [&](int slot, int i) {
    const int st = min(sb + wave + 4 * i, S - 1);
#pragma unroll
    for (int g = 0; g < G; ++g)
      wb[slot][g] = *reinterpret_cast<const u32x4v*>(wp[g] + static_cast<int64_t>(st) * 512);
#pragma unroll
    for (int h = 0; h < 2 * MT; ++h)
      ab[slot][h] = xa4[static_cast<int64_t>(st) * (kXaStepElems / 8) + h * 64 + lane];
  };
#pragma unroll
  for (int u = 0; u < kMwP; ++u)
    if (u < nw) issue(u, u);
  for (int b = 0; b < nw; b += kMwP) {
#pragma unroll
    for (int u = 0; u < kMwP; ++u) {
      const int i = b + u;
      if (i < nw) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int q = 0; q < MT; ++q)
#pragma unroll
            for (int g = 0; g < G; ++g)
              acc[g][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(abf16x8, ab[u][2 * q + h]),
                                                                 __builtin_bit_cast(abf16x8, wb[u][g]), acc[g][q], 0,
                                                                 0, 0);
        if (i + kMwP < nw) issue(u, i + kMwP);
      }
    }
  }
  // the QKV head epilogue's cache offset and row position (thread t: row t / 4),
  // in flight during the LDS reduction and the hand-over
  int fx_offset = 0, fx_pos = -1;
  if constexpr (FQKV) {
    fx_offset = *a.offset_dev;
    fx_pos = a.positions ? a.positions[min(t / 4, a.M - 1)] : -1;
  }
  // the pair's row-scale parts (thread t: row t / 4, parts t % 4 + 4 q), in
  // flight during the LDS reduction
  float ssv[PE ? kSsMax : 1];
  if constexpr (PE) {
#pragma unroll
    for (int q = 0; q < kSsMax; ++q) {
      const int pp = t % 4 + 4 * q;
      ssv[q] = (a.ss && pp < a.n_ss) ? a.ss[pp * 64 + t / 4] : 0.f;
    }
  }
  // the wave's tile -> LDS (row 16 q + 4 (lane / 16) + e, column 16 g + lane % 16)
  mfma_settle();
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int q = 0; q < MT; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) s_red[wave][(q * 16 + (lane / 16) * 4 + e) * LDR + g * 16 + lane % 16] = acc[g][q][e];
  __syncthreads();
  if constexpr (PE) {
    // four waves summed in order into wave 0's tile, then the pair epilogue
    // of thread (row m, 8 act features from g * 8): gate at column
    // 32 (f / 16) + f % 16 of the tile, up 16 columns further
    for (int e = t * 4; e < a.M * FB; e += 256 * 4) {
      const int r = e / FB, c = e % FB;
      float4 v = *reinterpret_cast<const float4*>(&s_red[0][r * LDR + c]);
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float4 o = *reinterpret_cast<const float4*>(&s_red[w][r * LDR + c]);
        v.x += o.x;
        v.y += o.y;
        v.z += o.z;
        v.w += o.w;
      }
      *reinterpret_cast<float4*>(&s_red[0][r * LDR + c]) = v;
    }
    __shared__ float s_inv[64];
    const int m = t / 4, g = t % 4;
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kSsMax; ++q) tot += ssv[q];
    tot += __shfl_xor(tot, 1);
    tot += __shfl_xor(tot, 2);
    if (g == 0) s_inv[m] = a.ss ? 1.f / sqrtf(tot / static_cast<float>(a.ss_k) + a.eps) : 1.f;
    __syncthreads();
    if (m >= a.M) return;
    const float inv = s_inv[m];
    float z[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int f = g * 8 + e, gc = (f / 16) * 32 + f % 16;
      const float gv = s_red[0][m * LDR + gc] * inv, uv = s_red[0][m * LDR + gc + 16] * inv;
      z[e] = gv / (1.f + expf(-gv)) * uv;
    }
    const int n0 = (cg >> 1) * 64 + (cg & 1) * 32 + g * 8;
    uint4 hi, lo;
    split8(z, hi, lo);
    *reinterpret_cast<uint4*>(a.xa_next + xa_index(m, n0, 0)) = hi;
    *reinterpret_cast<uint4*>(a.xa_next + xa_index(m, n0, 1)) = lo;
    return;
  }
  // four waves summed in order; rows < M as this split's partial
  const int cols = gridDim.x * FB;
  float* base = a.part + static_cast<int64_t>(cg) * FB;
  for (int e = t * 4; e < a.M * FB; e += 256 * 4) {
    const int r = e / FB, c = e % FB;
    float4 v = *reinterpret_cast<const float4*>(&s_red[0][r * LDR + c]);
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float4 o = *reinterpret_cast<const float4*>(&s_red[w][r * LDR + c]);
      v.x += o.x;
      v.y += o.y;
      v.z += o.z;
      v.w += o.w;
    }
    float* dst = base + (static_cast<int64_t>(kz) * 64 + r) * cols + c;
    if constexpr (FTW > 0) {
      publish_f32(dst, v.x);
      publish_f32(dst + 1, v.y);
      publish_f32(dst + 2, v.z);
      publish_f32(dst + 3, v.w);
    } else {
      *reinterpret_cast<float4*>(dst) = v;
    }
  }
  if constexpr (FTW > 0) {
    const int fr = cg / FTW;
    if (last_of(a.fix_ctr + static_cast<int64_t>(fr) * kCounterStride, a.ks * FTW))
      sk_fix_last<FTW, FQKV>(a, fr, &s_red[0][0], fx_offset, fx_pos);
  }
}

// The split-K fix-up of a column range and a quarter of the rows: the ks
// partial tiles summed in split order (deterministic), then the epilogue.
// Launched after k_mm_stream, so plain loads see every split's stores.
template <int TW, bool QKV = false>
__global__ __launch_bounds__(256) void k_mm_fix(SkArgs a) {
  constexpr int FB = 64 * TW;
  constexpr int LDC = FB + 4;
  constexpr int V4 = 16 * FB / 4 / 256;  // float4 per thread: 16 rows x FB columns
  __shared__ __attribute__((aligned(16))) float s_c[64 * LDC];
  __shared__ float s_inv[64];
  const int t = threadIdx.x, cb = blockIdx.x, r0 = blockIdx.y * 16;
  const int cols = gridDim.x * FB;
  const float* base = a.part + static_cast<int64_t>(cb) * FB;
  EpiOps<TW, QKV> ops;  // issued first: one round trip covers them and the partials
  sk_epi_load<TW, QKV>(a, cb, ops);
  float4 acc[V4];
#pragma unroll
  for (int i = 0; i < V4; ++i) acc[i] = float4{0.f, 0.f, 0.f, 0.f};
  // every split's loads in flight at once (ks <= 8), then the loads that wait on the position
  float4 u[8][V4];
#pragma unroll
  for (int h = 0; h < 8; ++h)
#pragma unroll
    for (int i = 0; i < V4; ++i) {
      const int e = (t + 256 * i) * 4, r = min(r0 + e / FB, a.M - 1), c = e % FB;
      const int zz = min(h, a.ks - 1);
      u[h][i] = *reinterpret_cast<const float4*>(base + (static_cast<int64_t>(zz) * 64 + r) * cols + c);
    }
  sk_epi_rope<TW, QKV>(a, cb, ops);
#pragma unroll
  for (int h = 0; h < 8; ++h)
    if (h < a.ks)
#pragma unroll
      for (int i = 0; i < V4; ++i) {
        acc[i].x += u[h][i].x;
        acc[i].y += u[h][i].y;
        acc[i].z += u[h][i].z;
        acc[i].w += u[h][i].w;
      }
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int e = (t + 256 * i) * 4, r = r0 + e / FB, c = e % FB;
    *reinterpret_cast<float4*>(&s_c[r * LDC + c]) = acc[i];
  }
  __syncthreads();
  sk_epi_run<TW, QKV>(a, s_c, s_inv, cb, r0, r0 + 16, ops);
}

struct GemmPlan {
  int tw, cols, ks;
};

// Column ranges of 64 TW weight rows (TW = 2 for the SiLU pair and wide
// projections), K split into at most 8 parts of >= 8 k steps so that about
// 256 blocks stream at once (each split stores an M x 64 TW fp32 tile that
// k_mm_fix sums: 8 ks M bytes per weight row against 2 K bytes of weights).
static GemmPlan plan_gemm(int n_rows, int K, bool pair, int tw = 0) {
  GemmPlan p{};
  p.tw = tw ? tw : (pair || n_rows >= 8192) ? 2 : 1;
  p.cols = pair ? n_rows / 2 / 64 : (n_rows + 64 * p.tw - 1) / (64 * p.tw);
  const int steps = K / 32;
  p.ks = std::max(1, std::min(std::min(8, steps / 8), (256 + p.cols - 1) / p.cols));
  return p;
}

template <int TW>
static int launch_stream_t(const SkArgs& g, const GemmPlan& p, hipStream_t s) {
  const dim3 grid(p.cols, p.ks);
  switch ((g.M + 15) / 16) {
    case 1: hipLaunchKernelGGL((k_mm_stream<1, TW>), grid, dim3(256), 0, s, g); break;
    case 2: hipLaunchKernelGGL((k_mm_stream<2, TW>), grid, dim3(256), 0, s, g); break;
    case 3: hipLaunchKernelGGL((k_mm_stream<3, TW>), grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL((k_mm_stream<4, TW>), grid, dim3(256), 0, s, g); break;
  }
  WC_LAUNCHED();
  if (p.ks > 1) {
    hipLaunchKernelGGL((k_mm_fix<TW>), dim3(p.cols, (g.M + 15) / 16), dim3(256), 0, s, g);
    WC_LAUNCHED();
  }
  return WC_OK;
}

static int launch_stream(SkArgs g, const GemmPlan& p, hipStream_t s) {
  WC_REQUIRE(g.M >= 1 && g.M <= 64, "target layer: rows must be in 1..64");
  WC_REQUIRE(g.K % 256 == 0, "target layer: K %d must be a multiple of 256", g.K);
  WC_REQUIRE(g.N >= 1, "target layer: no weight rows");
  WC_REQUIRE(g.n_ss <= 64, "target layer: at most 64 row-scale parts");
  g.ks = p.ks;
  return p.tw == 2 ? launch_stream_t<2>(g, p, s) : launch_stream_t<1>(g, p, s);
}

// k_mm_wave over column groups of 64 and K splits (at most 256 blocks, one per
// CU, with >= 4 k steps each), then k_mm_fix with column ranges of 64 fix_tw
// (the epilogue's own width: one 128-wide head for QKV, 64 act features for the
// pair).  The split count rounds down: rounding up put a second block on some
// CUs (280 blocks for the Qwen3-4B o / down projections, 288 for its QKV), and
// those CUs set the launch's end -- the 36-layer 8-row verify forward took
// 3.45 ms that way against 3.19 ms with 240 and 192 blocks.
static int wave_ks(int N, int K) {
  const int cg = N / (16 * kMwG), steps = K / 32;
  return std::max(1, std::min(std::min(8, steps / 4), 256 / cg));
}

static int launch_wave(SkArgs g, int fix_tw, hipStream_t s) {
  WC_REQUIRE(g.M >= 1 && g.M <= 64, "target layer: rows must be in 1..64");
  WC_REQUIRE(g.K % 256 == 0, "target layer: K %d must be a multiple of 256", g.K);
  WC_REQUIRE(g.N % (64 * fix_tw) == 0, "target layer: %d weight rows must be a multiple of %d", g.N, 64 * fix_tw);
  WC_REQUIRE(g.n_ss <= 64, "target layer: at most 64 row-scale parts");
  g.ks = wave_ks(g.N, g.K);  // <= 8: k_mm_fix issues every split's loads at once
  // the SiLU pair over >= 128 column groups: K unsplit, the epilogue in the GEMM
  if (g.epi == kSkSiluPair && fix_tw == 2 && g.xa_next && !g.out && g.N / (16 * kMwG) >= 128 &&
      g.n_ss <= 4 * kSsMax) {
    g.ks = 1;
    const dim3 grid1(g.N / (16 * kMwG), 1);
    switch ((g.M + 15) / 16) {
      case 1: hipLaunchKernelGGL((k_mm_wave<1, true>), grid1, dim3(256), 0, s, g); break;
      case 2: hipLaunchKernelGGL((k_mm_wave<2, true>), grid1, dim3(256), 0, s, g); break;
      case 3: hipLaunchKernelGGL((k_mm_wave<3, true>), grid1, dim3(256), 0, s, g); break;
      default: hipLaunchKernelGGL((k_mm_wave<4, true>), grid1, dim3(256), 0, s, g); break;
    }
    WC_LAUNCHED();
    return WC_OK;
  }
  const dim3 grid(g.N / (16 * kMwG), g.ks);
  if (g.M <= kFixFusedRows && g.fix_ctr && g.N / (64 * fix_tw) <= kFixRanges) {
    if (g.epi == kSkQkvHead) {
      WC_REQUIRE(fix_tw == 2, "target layer: the QKV head epilogue takes 128-column ranges");
      hipLaunchKernelGGL((k_mm_wave<1, false, 2, true>), grid, dim3(256), 0, s, g);
    } else if (fix_tw == 2)
      hipLaunchKernelGGL((k_mm_wave<1, false, 2>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((k_mm_wave<1, false, 1>), grid, dim3(256), 0, s, g);
    WC_LAUNCHED();
    return WC_OK;
  }
  switch ((g.M + 15) / 16) {
    case 1: hipLaunchKernelGGL((k_mm_wave<1>), grid, dim3(256), 0, s, g); break;
    case 2: hipLaunchKernelGGL((k_mm_wave<2>), grid, dim3(256), 0, s, g); break;
    case 3: hipLaunchKernelGGL((k_mm_wave<3>), grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL((k_mm_wave<4>), grid, dim3(256), 0, s, g); break;
  }
  WC_LAUNCHED();
  const dim3 fgrid(g.N / (64 * fix_tw), (g.M + 15) / 16);
  if (g.epi == kSkQkvHead) {
    WC_REQUIRE(fix_tw == 2, "target layer: the QKV head epilogue takes 128-column ranges");
    hipLaunchKernelGGL((k_mm_fix<2, true>), fgrid, dim3(256), 0, s, g);
  } else if (fix_tw == 2)
    hipLaunchKernelGGL((k_mm_fix<2>), fgrid, dim3(256), 0, s, g);
  else
    hipLaunchKernelGGL((k_mm_fix<1>), fgrid, dim3(256), 0, s, g);
  WC_LAUNCHED();
  return WC_OK;
}

static int launch_xa_prep(const float* x, int64_t ldx, int M, int K, const uint16_t* gain, uint16_t* xa, float* ss,
                          hipStream_t s) {
  XaPrepArgs a{x, ldx, M, K, gain, xa, ss};
  hipLaunchKernelGGL(k_xa_prep, dim3(K / 256, 4), dim3(256), 0, s, a);
  WC_LAUNCHED();
  return WC_OK;
}

constexpr int kVaD = 128;  // head_dim of the verify-width path

// ------------------------------------------------------------------ verify attention
// Split-KV GQA attention for a verify block (head_dim 128, bf16 cache) whose q
// rows are already normalised / rotated and whose K / V rows are already in
// the cache.  Block (split, kv head, group): group z covers query vectors
// 64 z .. 64 z + 63, wave w of them 16 w .. 16 w + 15, loaded straight into
// MFMA A fragments (fp32 split into bf16 hi + lo).  Per chunk of 64 keys:
// S^T = K Q^T by v_mfma_f32_16x16x32_bf16 (four independent key tiles), an
// online softmax in base 2 in registers (one query row per lane), O^T += V^T
// P^T with P^T straight from the registers and the V^T fragments read from
// the chunk's V rows by transposing LDS reads.  The next chunk's K / V and
// mask bytes load while the current one is consumed.  Partial (m, l, o) per
// split (m in natural units) go to k_attn_merge.
constexpr int kVaCH = 64;            // keys per chunk
constexpr int kVaLdK = kVaD + 8;     // row stride (bf16) of the K chunk: B-fragment reads spread over the banks
constexpr int kVaLdV = kVaD + 16;    // row stride (bf16) of the V chunk: a transposing read's four rows on distinct banks
constexpr int kVaGroup = 64;         // query vectors per block
constexpr int kVaMaxRows = 64;       // rows per launch (mask rows staged per chunk)
constexpr int kVaMaxSplits = kMaxSplits;
constexpr float kLog2e = 1.4426950408889634f;

// One chunk of the split in registers: K and V as [key][d] (thread t: key
// t / 16 + 16 i, d chunk t % 16: coalesced); the mask bytes of row t / 4, keys
// 16 (t % 4) .. + 16.  Buffer loads: rows past the capacity read as zeros.
struct VaChunk {
  uint4 k[4], v[4];
  uint4 mw;  // the 16 mask bytes (one 16-byte load) or their nonzero bits (byte loads)
};

// bit e: byte e of w nonzero (bytes spread to bits 0 / 8 / 16 / 24, then
// gathered by one multiply: byte e's bit lands at 21 + e, no two terms collide)
__device__ __forceinline__ uint32_t va_nz4(uint32_t w) {
  const uint32_t h = ((((w & 0x7f7f7f7fu) + 0x7f7f7f7fu) | w) & 0x80808080u) >> 7;
  return (h * 0x00204081u) >> 21 & 0xfu;
}

struct VaSrc {
  __amdgpu_buffer_rsrc_t kr, vr, mr;
  int kvo;          // per-thread byte offset of the K / V loads
  int mo;           // byte offset of the thread's mask bytes at key 0
  bool mask_vec;    // mask rows 16-byte aligned: one 16-byte load per chunk
};

// (the chunk offset rides in the vector offset, which the buffer range check covers)
template <bool MASK>
__device__ __forceinline__ void va_chunk_load(const VaSrc& src, int c0, VaChunk& ch) {
  const int ko = src.kvo + c0 * (kVaD * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ch.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.kr, ko + i * 16 * (kVaD * 2), 0, 0));
    ch.v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.vr, ko + i * 16 * (kVaD * 2), 0, 0));
  }
  if constexpr (MASK) {
    const int mo = src.mo + c0;
    if (src.mask_vec) {
      ch.mw = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.mr, mo, 0, 0));
    } else {
      uint32_t b = 0;
#pragma unroll
      for (int e = 0; e < 16; ++e) b |= (__builtin_amdgcn_raw_buffer_load_b8(src.mr, mo + e, 0, 0) != 0 ? 1u : 0u) << e;
      ch.mw = make_uint4(b, 0, 0, 0);
    }
  }
}

template <bool MASK>
__device__ __forceinline__ uint32_t va_mask_bits(const VaSrc& src, const VaChunk& ch) {
  if (!src.mask_vec) return ch.mw.x;
  return va_nz4(ch.mw.x) | va_nz4(ch.mw.y) << 4 | va_nz4(ch.mw.z) << 8 | va_nz4(ch.mw.w) << 12;
}


// MASK: visibility from the explicit mask rows; otherwise causal (and the
// sliding window).  Split ranges are fixed by the capacity (whole chunks), so a
// block requests its first chunk before the cache offset arrives; splits past
// the live keys leave m = -inf, l = 0.
template <bool MASK>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_verify_attention(AttnArgs a) {
  constexpr int D = kVaD, CH = kVaCH;
  __shared__ __attribute__((aligned(16))) uint16_t ksb[CH * kVaLdK];   // [key][d]
  __shared__ __attribute__((aligned(16))) uint16_t vsb[CH * kVaLdV];   // [key][d]
  __shared__ __attribute__((aligned(16))) uint16_t s_mb[kVaMaxRows * 4];  // mask bits [row][key / 16]

  const int kh = blockIdx.y, split = blockIdx.x, S = gridDim.x, z = blockIdx.z;
  const int rep = a.H / a.Hk;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int dg = (lane / 16) * 8;
  const int per = ((a.cap + S - 1) / S + CH - 1) / CH * CH;  // whole chunks per split
  const int kb = min(a.cap, split * per);
  const int QVb = a.rows * rep;

  VaSrc src;
  src.kr = buffer_rsrc(static_cast<const uint16_t*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D, a.cap * D * 2);
  src.vr = buffer_rsrc(static_cast<const uint16_t*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D, a.cap * D * 2);
  src.kvo = (t / 16) * (D * 2) + (t % 16) * 16;
  src.mask_vec = false;
  src.mo = 0;
  if constexpr (MASK) {
    src.mr = buffer_rsrc(a.mask, static_cast<int>(a.rows * a.mask_ld));
    src.mask_vec = (a.mask_ld & 15) == 0 && (reinterpret_cast<uintptr_t>(a.mask) & 15) == 0;
    src.mo = static_cast<int>(min(t / 4, a.rows - 1) * a.mask_ld) + (t % 4) * 16;
  }

  // q tile (this lane: vector vq, dims 32 st + dg .. + 8), then the first chunk
  const int vq = z * kVaGroup + wave * 16 + lane % 16;
  const int vqc = min(vq, QVb - 1);
  const float* qsrc = a.qkv + static_cast<int64_t>(vqc / rep) * a.ld_qkv + (kh * rep + vqc % rep) * D + dg;
  float4 qf[8];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    qf[2 * st] = *reinterpret_cast<const float4*>(qsrc + st * 32);
    qf[2 * st + 1] = *reinterpret_cast<const float4*>(qsrc + st * 32 + 4);
  }
  VaChunk ch;
  va_chunk_load<MASK>(src, kb, ch);
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  const int offset = *a.offset_dev + a.offset_add;
  const int T = min(offset + nr, a.cap);
  const int QV = nr * rep;
  const int ke = min(T, kb + per);
  // q scaled by scale * log2(e) before the split: the scores come out in base 2
  const float sc = a.scale * kLog2e;
  abf16x8 qh[4], ql[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const float g = vq < QV ? sc : 0.f;
    const float4 u = qf[2 * st], w = qf[2 * st + 1];
    const float x[8] = {u.x * g, u.y * g, u.z * g, u.w * g, w.x * g, w.y * g, w.z * g, w.w * g};
    split8(x, qh[st], ql[st]);
  }

  // S^T = K Q^T per 16-key tile: lane l holds query vector q = l % 16 of the
  // wave's 16 (its softmax row: live or not, mask row, causal / window limits)
  // and keys 16 kt + 4 g + e of the chunk (g = l / 16); the four lane groups
  // share a row, so its max and sum are the lane's 16 values then two
  // cross-group shuffles.  P^T then feeds O^T = V^T P^T straight from the
  // lane's registers: the MFMA's k slots 8 g .. 8 g + 7 of key block kk take
  // keys 32 kk + 4 g + {0..3} and 32 kk + 16 + 4 g + {0..3}, and the V^T
  // fragments are read from the transposed chunk in that same key order.
  const int kl = lane % 16, gq = lane / 16;
  const int vrow = z * kVaGroup + wave * 16 + kl;
  const bool rlive = vrow < QV;
  const int mrow = min(vrow, QVb - 1) / rep;
  const int lim = offset + mrow;
  const int wlo = a.window > 0 ? offset + mrow - a.window : -0x7fffffff;
  float m_r = -INFINITY, l_r = 0.f;
  af32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = af32x4{0.f, 0.f, 0.f, 0.f};
  const bool tile_live = z * kVaGroup + wave * 16 < QV;
  uint16_t* kdst = ksb + (t / 16) * kVaLdK + (t % 16) * 8;
  uint16_t* vdst = vsb + (t / 16) * kVaLdV + (t % 16) * 8;
  // the lane's transposing V reads: source lane 4 e + a of its 16-lane group
  // points at key (kk block) + 4 g + e, dims 16 dt + 4 a .. + 3, so that lane
  // i of the group receives V[key + e][16 dt + i] for e = 0..3 (the lane holds
  // M[i / 4 + 4 e][i % 4] of its group's 16 x 4 block of reads)
  const int vr0 = 4 * (lane / 16) + (lane % 16) / 4, vc0 = 4 * ((lane % 16) % 4);

  for (int c0 = kb; c0 < ke; c0 += CH) {
    const int n = min(CH, ke - c0);
    lds_barrier();  // the previous chunk is consumed
    if (n < CH) {
      // the split's last, partial chunk: V rows past the range zeroed (the
      // cache there may hold anything; P is 0 for them)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (t / 16 + 16 * i >= n) ch.v[i] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint4*>(kdst + 16 * i * kVaLdK) = ch.k[i];
      *reinterpret_cast<uint4*>(vdst + 16 * i * kVaLdV) = ch.v[i];
    }
    if constexpr (MASK) s_mb[t] = static_cast<uint16_t>(va_mask_bits<MASK>(src, ch));
    lds_barrier();
    if (c0 + CH < ke) va_chunk_load<MASK>(src, c0 + CH, ch);  // next chunk

    if (tile_live) {
      // S^T, four independent key tiles (K fragments as A, q as B)
      af32x4 sacc[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) sacc[kt] = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        abf16x8 b[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          b[kt] = __builtin_bit_cast(
              abf16x8, *reinterpret_cast<const uint4*>(ksb + (kt * 16 + kl) * kVaLdK + st * 32 + dg));
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[kt], qh[st], sacc[kt], 0, 0, 0);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[kt], ql[st], sacc[kt], 0, 0, 0);
      }
      // the row's visible keys of this chunk (key j = bit j), then the lane's
      // four 4-key runs 16 kt + 4 g ..
      uint64_t bits;
      if constexpr (MASK) {
        const uint2 mw = *reinterpret_cast<const uint2*>(s_mb + mrow * 4);
        bits = static_cast<uint64_t>(mw.y) << 32 | mw.x;
      } else {
        bits = low_bits64(lim - c0 + 1) & ~low_bits64(wlo - c0 + 1);
      }
      bits = rlive ? bits & low_bits64(n) : 0ull;
      const uint32_t blo = static_cast<uint32_t>(bits), bhi = static_cast<uint32_t>(bits >> 32);
      mfma_settle();
      float sv[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint32_t nib = __builtin_amdgcn_ubfe(kt < 2 ? blo : bhi, (kt & 1) * 16 + 4 * gq, 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[kt][e] = (nib >> e) & 1u ? sacc[kt][e] : -INFINITY;
          mx = fmaxf(mx, sv[kt][e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_r, mx);
      const float mb = m_new == -INFINITY ? 0.f : m_new;  // all hidden so far: exp2(-inf) = 0 below
      const float alpha = __builtin_amdgcn_exp2f(m_r - mb);
      float p[4][4], rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[kt][e] = __builtin_amdgcn_exp2f(sv[kt][e] - mb);
          rs += p[kt][e];
        }
      rs += __shfl_xor(rs, 16);
      rs += __shfl_xor(rs, 32);
      l_r = l_r * alpha + rs;
      m_r = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[dt][e] *= alpha;
      // O^T += V^T P^T over the two 32-key blocks
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const float px[8] = {p[2 * kk][0], p[2 * kk][1], p[2 * kk][2], p[2 * kk][3],
                             p[2 * kk + 1][0], p[2 * kk + 1][1], p[2 * kk + 1][2], p[2 * kk + 1][3]};
        abf16x8 ph, pl;
        split8(px, ph, pl);
        abf16x8 va[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          uint16_t* vp = vsb + (kk * 32 + vr0) * kVaLdV + dt * 16 + vc0;
          const vs16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_vs16x4*)(vp));
          const vs16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_vs16x4*)(vp + 16 * kVaLdV));
          va[dt] = __builtin_bit_cast(abf16x8, vs16x8{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]});
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], ph, o[dt], 0, 0, 0);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pl, o[dt], 0, 0, 0);
      }
    }
  }

  // this split's (m, l, o) per query vector (lane: dims 16 dt + 4 g .. + 4 of
  // vector vrow); m back to natural units
  mfma_settle();
  if (!rlive) return;
  float* part = a.partial + ((static_cast<int64_t>(kh) * S + split) * a.qv_ld + vrow) * (D + 2);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    float2* pp = reinterpret_cast<float2*>(part + 2 + dt * 16 + 4 * gq);
    pp[0] = make_float2(o[dt][0], o[dt][1]);
    pp[1] = make_float2(o[dt][2], o[dt][3]);
  }
  if (gq == 0) *reinterpret_cast<float2*>(part) = make_float2(m_r == -INFINITY ? -INFINITY : m_r / kLog2e, l_r);
}

static int launch_verify_attention(const AttnArgs& a, int splits, hipStream_t s) {
  WC_REQUIRE(a.rows >= 1 && a.rows <= kVaMaxRows, "verify attention: rows must be in 1..%d", kVaMaxRows);
  WC_REQUIRE(splits >= 1 && splits <= kVaMaxSplits, "verify attention: 1..%d splits", kVaMaxSplits);
  const int qvb = a.rows * (a.H / a.Hk);
  WC_REQUIRE(a.qv_ld >= qvb, "verify attention: partial stride too small");
  WC_REQUIRE(static_cast<int64_t>(a.cap) * kVaD * 2 < (int64_t{1} << 31) &&
                 (!a.mask || static_cast<int64_t>(a.rows) * a.mask_ld < (int64_t{1} << 31)),
             "verify attention: cache or mask too large for 32-bit offsets");
  const unsigned groups = static_cast<unsigned>((qvb + kVaGroup - 1) / kVaGroup);
  if (a.mask)
    hipLaunchKernelGGL(k_verify_attention<true>, dim3(splits, a.Hk, groups), dim3(kAttnThreads), 0, s, a);
  else
    hipLaunchKernelGGL(k_verify_attention<false>, dim3(splits, a.Hk, groups), dim3(kAttnThreads), 0, s, a);
  WC_LAUNCHED();
  launch_merge<kVaD>(a, qvb, splits, s);
  WC_LAUNCHED();
  return WC_OK;
}

// ------------------------------------------------------------------ weight layout
// W [rows][cols] bf16 row-major -> fragment-major: chunk c = (T S + s) 64 + l
// (S = cols / 32) holds W[16 T + l % 16][32 s + 8 (l / 16) .. + 8], the A
// fragment lane l of v_mfma_f32_16x16x32_bf16 needs for 16-row tile T at k step s.
__global__ __launch_bounds__(256) void k_frag_layout(const uint16_t* __restrict__ w, int rows, int cols,
                                                     uint16_t* __restrict__ out) {
  const int64_t chunks = static_cast<int64_t>(rows) * cols / 8;
  const int S = cols / 32;
  for (int64_t c = blockIdx.x * 256ll + threadIdx.x; c < chunks; c += static_cast<int64_t>(gridDim.x) * 256) {
    const int l = static_cast<int>(c % 64);
    const int64_t ts = c / 64;
    const int s = static_cast<int>(ts % S);
    const int64_t T = ts / S;
    const int64_t row = 16 * T + l % 16;
    const int col = 32 * s + 8 * (l / 16);
    *reinterpret_cast<uint4*>(out + c * 8) = *reinterpret_cast<const uint4*>(w + row * cols + col);
  }
}

// ------------------------------------------------------------------ embedding
// out[m] = table[tokens[m]] (bf16 -> fp32), token ids clamped into the table
// (python/woodcock/target.py:70-71).
__global__ __launch_bounds__(256) void k_embed_rows(const uint16_t* __restrict__ table, int vocab, int hidden,
                                                    const int32_t* __restrict__ tokens, float* __restrict__ out,
                                                    int64_t ld) {
  const int m = blockIdx.x;
  const int tok = min(max(tokens[m], 0), vocab - 1);
  const uint16_t* src = table + static_cast<int64_t>(tok) * hidden;
  for (int k = threadIdx.x; k < hidden; k += 256) out[static_cast<int64_t>(m) * ld + k] = bf16_to_float(src[k]);
}

struct TargetWs {
  uint16_t *xa_x, *xa_attn, *xa_h1, *xa_act;
  float *ss_x, *ss_h1, *qkv, *q, *attn, *h1, *part, *apart;
  unsigned int* fix_ctr;
  size_t bytes;
};

struct LayerPlans {
  GemmPlan qkv, o, gu, down;
};

static LayerPlans layer_plans(const wc_drafter_dims& d) {
  const int nq = d.heads * d.head_dim, nqkv = nq + 2 * d.kv_heads * d.head_dim;
  return {plan_gemm(nqkv, d.hidden, false, 2), plan_gemm(d.hidden, nq, false), plan_gemm(2 * d.inter, d.hidden, true),
          plan_gemm(d.hidden, d.inter, false)};
}

static TargetWs target_ws(const wc_drafter_dims& d, int max_rows, void* base) {
  TargetWs w{};
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = (off + bytes + 255) / 256 * 256;
    return q;
  };
  const size_t M = static_cast<size_t>(max_rows);
  const size_t nq = static_cast<size_t>(d.heads) * d.head_dim;
  const size_t nqkv = nq + 2 * static_cast<size_t>(d.kv_heads) * d.head_dim;
  const LayerPlans pl = layer_plans(d);
  // activations in fragment order: K / 32 steps of 8 KB = 256 bytes per k
  w.xa_x = reinterpret_cast<uint16_t*>(take(256 * static_cast<size_t>(d.hidden)));
  w.xa_attn = reinterpret_cast<uint16_t*>(take(256 * nq));
  w.xa_h1 = reinterpret_cast<uint16_t*>(take(256 * static_cast<size_t>(d.hidden)));
  w.xa_act = reinterpret_cast<uint16_t*>(take(256 * static_cast<size_t>(d.inter)));
  // parts of the layer input's row sums of squares: the prep's (one per 256 k) or a down epilogue's (one per 64 columns)
  w.ss_x = reinterpret_cast<float*>(take(4 * 64 * static_cast<size_t>(std::max(d.hidden / 64, 4))));
  // o_proj epilogue parts (one per column range) or the fallback attention prep's (one per 256 k)
  const size_t ss_parts = std::max(static_cast<size_t>(d.hidden / 64), nq / 256);
  w.ss_h1 = reinterpret_cast<float*>(take(4 * 64 * ss_parts));
  w.qkv = reinterpret_cast<float*>(take(4 * M * nqkv));
  w.q = reinterpret_cast<float*>(take(4 * M * nq));
  w.attn = reinterpret_cast<float*>(take(4 * M * nq));
  w.h1 = reinterpret_cast<float*>(take(4 * M * d.hidden));
  size_t part = 0;
  for (const GemmPlan* g : {&pl.qkv, &pl.o, &pl.gu, &pl.down}) {
    part = std::max(part, static_cast<size_t>(g->ks) * 64 * g->cols * 64 * g->tw);
  }
  for (const int* nk : {std::array<int, 2>{static_cast<int>(nqkv), d.hidden}.data(),
                        std::array<int, 2>{d.hidden, static_cast<int>(nq)}.data(),
                        std::array<int, 2>{2 * d.inter, d.hidden}.data(),
                        std::array<int, 2>{d.hidden, d.inter}.data()})
    part = std::max(part, static_cast<size_t>(wave_ks(nk[0], nk[1])) * 64 * nk[0]);
  w.part = reinterpret_cast<float*>(take(4 * part));
  const size_t qv = M * static_cast<size_t>(d.heads / std::max(d.kv_heads, 1));
  w.apart = reinterpret_cast<float*>(
      take(4 * static_cast<size_t>(d.kv_heads) * std::max(kMaxSplits, kVaMaxSplits) * qv * (d.head_dim + 2)));
  w.fix_ctr = reinterpret_cast<unsigned int*>(take(4 * static_cast<size_t>(kCounterStride) * kFixRanges));
  w.bytes = off;
  return w;
}

}  // namespace wc

extern "C" {

size_t wc_target_workspace_bytes(const wc_drafter_dims* dims, int max_rows) {
  if (!dims || max_rows < 1) return 0;
  return wc::target_ws(*dims, max_rows, nullptr).bytes;
}

int wc_target_layer(const wc_drafter_dims* dims, const wc_layer_weights* L, const float* rope_cos,
                    const float* rope_sin, int rope_max_pos, float* x, int rows, const int32_t* positions_dev,
                    const uint8_t* mask_dev, int64_t mask_ld, void* k_cache, void* v_cache, int kv_dtype,
                    int capacity, const int32_t* offset_dev, const void* next_norm, int input_prepared,
                    void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(dims && L && x && k_cache && v_cache && offset_dev && workspace, "wc_target_layer: NULL argument");
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(rows >= 1 && rows <= 64, "wc_target_layer: rows must be in 1..64 (got %d)", rows);
  WC_REQUIRE(d.heads >= 1 && d.kv_heads >= 1 && d.heads % d.kv_heads == 0, "wc_target_layer: bad head counts");
  WC_REQUIRE(d.hidden % 256 == 0 && (d.heads * d.head_dim) % 256 == 0 && d.inter % 256 == 0,
             "wc_target_layer: hidden, heads*head_dim and inter must be multiples of 256");
  WC_REQUIRE(d.head_dim % 32 == 0, "wc_target_layer: head_dim must be a multiple of 32");
  WC_REQUIRE(d.hidden <= 4096, "wc_target_layer: hidden_size above 4096 is not supported");
  WC_REQUIRE(kv_dtype == WC_F32 || kv_dtype == WC_BF16, "wc_target_layer: kv_dtype must be WC_F32 or WC_BF16");
  WC_REQUIRE(L->in_norm && L->post_norm && L->q && L->k && L->v && L->o && L->q_norm && L->k_norm && L->gate &&
                 L->up && L->down,
             "wc_target_layer: NULL layer weight");
  WC_REQUIRE(rope_cos && rope_sin && rope_max_pos >= 1, "wc_target_layer: rope table missing");
  WC_REQUIRE(mask_dev == nullptr || mask_ld >= rows, "wc_target_layer: mask row stride too small");
  WC_REQUIRE(aligned(x, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(workspace, 16),
             "wc_target_layer: buffers must be 16-byte aligned");
  const int H = d.heads, Hk = d.kv_heads, D = d.head_dim, rep = H / Hk;
  WC_REQUIRE(Hk <= kMaxKvHeads && rep <= kMaxQV, "wc_target_layer: head grouping not supported");
  const int nq = H * D, nk = Hk * D, nqkv = nq + 2 * nk;
  const TargetWs ws = target_ws(d, rows, workspace);
  const LayerPlans pl = layer_plans(d);
  auto s = reinterpret_cast<hipStream_t>(stream);
  auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
  const bool verify_path = D == kVaD && kv_dtype == WC_BF16;

  // 1. the layer input as activations: x * in_norm, row sums of squares (or
  //    already there: the previous layer's down epilogue wrote them)
  if (!input_prepared)
    if (int rc = launch_xa_prep(x, d.hidden, rows, d.hidden, u16(L->in_norm), ws.xa_x, ws.ss_x, s)) return rc;
  const int n_ss_x = input_prepared ? pl.down.cols : d.hidden / 256;

  // 2. QKV = W . RMS_in(x): unscaled sums for the verify epilogue, scaled otherwise
  SkArgs g{};
  g.xa = ws.xa_x;
  g.eps = d.eps;
  g.w[0] = u16(L->q);
  g.w[1] = u16(L->k);
  g.w[2] = u16(L->v);
  g.seg_start[0] = 0;
  g.seg_start[1] = nq;
  g.seg_start[2] = nq + nk;
  g.seg_start[3] = nqkv;
  g.n_seg = 3;
  g.M = rows;
  g.N = nqkv;
  g.K = d.hidden;
  g.epi = verify_path ? kSkQkvHead : kSkStore;
  g.ss = ws.ss_x;
  g.n_ss = n_ss_x;
  g.ss_k = d.hidden;
  g.out = verify_path ? ws.q : ws.qkv;
  g.ldo = verify_path ? nq : nqkv;
  g.part = ws.part;
  g.fix_ctr = ws.fix_ctr;
  if (verify_path) {
    // head_dim 128 with a bf16 cache: the QKV epilogue normalises / rotates q
    // and k and appends K / V, so the attention reads every key from the cache
    g.nq = nq;
    g.nk = nk;
    g.q_gain = u16(L->q_norm);
    g.k_gain = u16(L->k_norm);
    g.rope_cos = rope_cos;
    g.rope_sin = rope_sin;
    g.rope_max = rope_max_pos;
    g.positions = positions_dev;
    g.offset_dev = offset_dev;
    g.kc = k_cache;
    g.vc = v_cache;
    g.kv_bf16 = 1;
    g.cap = capacity;
  }
  if (int rc = launch_wave(g, 2, s)) return rc;

  const int splits = std::max(1, std::min(kMaxSplits, (capacity + kAttnChunkMax - 1) / kAttnChunkMax));
  if (verify_path) {
    // one MFMA attention launch covers every row
    AttnArgs at{};
    at.qkv = ws.q;
    at.ld_qkv = nq;
    at.H = H;
    at.Hk = Hk;
    at.rows = rows;
    at.scale = 1.f / sqrtf(static_cast<float>(D));
    at.kc = k_cache;
    at.vc = v_cache;
    at.cap = capacity;
    at.offset_dev = offset_dev;
    at.mask = mask_dev;
    at.mask_ld = mask_ld;
    at.window = d.window;
    at.partial = ws.apart;
    at.qv_ld = rows * rep;
    at.out = ws.attn;
    at.ld_out = nq;
    at.xa_out = ws.xa_attn;
    // the fewest chunks per split (at least two) that keep the grid within one
    // block per CU: one chunk per split measured slower (the split's fixed costs
    // dominate and the merge reads twice the partials), and CUs given a second
    // block set the launch's tail
    int cus = 0;
    if (int rc = device_cus(&cus)) return rc;
    const int groups = (rows * rep + kVaGroup - 1) / kVaGroup;
    const int chunks = (capacity + kVaCH - 1) / kVaCH;
    const int slots = std::max(1, cus / (Hk * groups));
    const int cps = std::max(2, (chunks + slots - 1) / slots);
    const int vsplits = std::max(1, std::min(kVaMaxSplits, (chunks + cps - 1) / cps));
    if (int rc = launch_verify_attention(at, vsplits, s)) return rc;
  } else {
    // other head sizes / an fp32 cache: the decode attention over tiles of rows
    // whose query vectors fit one block (it normalises, rotates and appends on
    // the fly), then the output as activations
    const int tile = std::max(1, std::min(kMaxQV / rep, WC_MAX_NODES));
    for (int t0 = 0; t0 < rows; t0 += tile) {
      AttnArgs at{};
      at.qkv = ws.qkv + static_cast<int64_t>(t0) * nqkv;
      at.ld_qkv = nqkv;
      at.H = H;
      at.Hk = Hk;
      at.rows = std::min(tile, rows - t0);
      at.q_gain = u16(L->q_norm);
      at.k_gain = u16(L->k_norm);
      at.eps = d.eps;
      at.scale = 1.f / sqrtf(static_cast<float>(D));
      at.rope_cos = rope_cos;
      at.rope_sin = rope_sin;
      at.rope_max = rope_max_pos;
      at.positions = positions_dev ? positions_dev + t0 : nullptr;
      at.kc = k_cache;
      at.vc = v_cache;
      at.cap = capacity;
      at.offset_dev = offset_dev;
      at.offset_add = t0;
      at.mask = mask_dev ? mask_dev + static_cast<int64_t>(t0) * mask_ld : nullptr;
      at.mask_ld = mask_ld;
      at.window = d.window;
      at.partial = ws.apart;
      at.qv_ld = std::min(tile, rows) * rep;
      at.out = ws.attn + static_cast<int64_t>(t0) * nq;
      at.ld_out = nq;
      if (int rc = launch_attention(at, D, kv_dtype, splits, s)) return rc;
    }
    if (int rc = launch_xa_prep(ws.attn, nq, rows, nq, nullptr, ws.xa_attn, ws.ss_h1, s)) return rc;
  }

  // 3. h1 = x + W_o . attn; the epilogue also writes h1 * post_norm as activations
  g = SkArgs{};
  g.xa = ws.xa_attn;
  g.w[0] = u16(L->o);
  g.seg_start[1] = d.hidden;
  g.n_seg = 1;
  g.M = rows;
  g.N = d.hidden;
  g.K = nq;
  g.epi = kSkResidual;
  g.out = ws.h1;
  g.ldo = d.hidden;
  g.res = x;
  g.ldr = d.hidden;
  g.xa_next = ws.xa_h1;
  g.gain_next = u16(L->post_norm);
  g.ss_next = ws.ss_h1;
  g.part = ws.part;
  g.fix_ctr = ws.fix_ctr;
  if (int rc = launch_wave(g, 1, s)) return rc;

  // 4. act = silu(W_gate . RMS_post(h1)) * (W_up . RMS_post(h1)), as activations only
  g = SkArgs{};
  g.xa = ws.xa_h1;
  g.ss = ws.ss_h1;
  g.n_ss = pl.o.cols;
  g.ss_k = d.hidden;
  g.eps = d.eps;
  g.w[0] = u16(L->gate);
  g.w[1] = u16(L->up);
  g.seg_start[1] = d.inter;
  g.seg_start[2] = 2 * d.inter;
  g.n_seg = 2;
  g.M = rows;
  g.N = 2 * d.inter;
  g.K = d.hidden;
  g.epi = kSkSiluPair;
  g.xa_next = ws.xa_act;
  g.part = ws.part;
  g.fix_ctr = ws.fix_ctr;
  if (int rc = launch_wave(g, 2, s)) return rc;

  // 5. x = h1 + W_down . act
  g = SkArgs{};
  g.xa = ws.xa_act;
  g.w[0] = u16(L->down);
  g.seg_start[1] = d.hidden;
  g.n_seg = 1;
  g.M = rows;
  g.N = d.hidden;
  g.K = d.inter;
  g.epi = kSkResidual;
  g.out = x;
  g.ldo = d.hidden;
  g.res = ws.h1;
  g.ldr = d.hidden;
  if (next_norm) {  // the next layer's (or the final) norm: its activations written here
    g.xa_next = ws.xa_x;
    g.gain_next = u16(next_norm);
    g.ss_next = ws.ss_x;
  }
  g.part = ws.part;
  g.fix_ctr = ws.fix_ctr;
  return launch_wave(g, 1, s);
}

int wc_weights_frag(const void* w, int rows, int cols, void* out, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(w && out && w != out, "wc_weights_frag: NULL or aliased buffer");
  WC_REQUIRE(rows >= 16 && rows % 16 == 0 && cols >= 32 && cols % 32 == 0,
             "wc_weights_frag: rows must be a multiple of 16 and cols a multiple of 32 (got %d x %d)", rows, cols);
  WC_REQUIRE(aligned(w, 16) && aligned(out, 16), "wc_weights_frag: buffers must be 16-byte aligned");
  const int64_t chunks = static_cast<int64_t>(rows) * cols / 8;
  const int grid = static_cast<int>(std::min<int64_t>((chunks + 255) / 256, 8192));
  hipLaunchKernelGGL(k_frag_layout, dim3(grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(w), rows, cols, static_cast<uint16_t*>(out));
  WC_LAUNCHED();
  return WC_OK;
}

int wc_target_embed(const void* table, int vocab, int hidden, const int32_t* tokens_dev, int rows, float* out,
                    int64_t ld, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(table && tokens_dev && out, "wc_target_embed: NULL buffer");
  WC_REQUIRE(rows >= 1 && vocab >= 1 && hidden >= 1 && ld >= hidden, "wc_target_embed: bad sizes");
  hipLaunchKernelGGL(k_embed_rows, dim3(rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(table), vocab, hidden, tokens_dev, out, ld);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_target_head(const wc_drafter_dims* dims, const void* head_w, const void* final_norm, const float* x, int rows,
                   int vocab, float* logits_out, int64_t ld, int input_prepared, void* workspace,
                   wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(dims && head_w && final_norm && x && logits_out && workspace, "wc_target_head: NULL argument");
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(rows >= 1 && rows <= 64, "wc_target_head: rows must be in 1..64 (got %d)", rows);
  WC_REQUIRE(d.hidden % 256 == 0 && d.hidden <= 4096, "wc_target_head: hidden_size must be a multiple of 256, <= 4096");
  WC_REQUIRE(vocab >= 1 && ld >= vocab, "wc_target_head: logits row stride smaller than the vocabulary");
  WC_REQUIRE(aligned(head_w, 16) && aligned(x, 16) && aligned(workspace, 16), "wc_target_head: misaligned buffer");
  const TargetWs ws = target_ws(d, rows, workspace);
  auto s = reinterpret_cast<hipStream_t>(stream);
  // final RMSNorm folded in: x * gain as activations (or already there: the last
  // layer's down epilogue wrote them), 1/rms scales the logits
  if (!input_prepared)
    if (int rc = launch_xa_prep(x, d.hidden, rows, d.hidden, static_cast<const uint16_t*>(final_norm), ws.xa_x,
                                ws.ss_x, s))
      return rc;
  GemmPlan p = plan_gemm(vocab, d.hidden, false);
  p.ks = 1;  // one column range per block: the vocabulary fills the GPU
  SkArgs g{};
  g.xa = ws.xa_x;
  g.ss = ws.ss_x;
  g.n_ss = input_prepared ? layer_plans(d).down.cols : d.hidden / 256;
  g.ss_k = d.hidden;
  g.eps = d.eps;
  g.w[0] = static_cast<const uint16_t*>(head_w);
  g.seg_start[1] = vocab;
  g.n_seg = 1;
  g.M = rows;
  g.N = vocab;
  g.K = d.hidden;
  g.epi = kSkStore;
  g.out = logits_out;
  g.ldo = ld;
  return launch_stream(g, p, s);
}

}  // extern "C"
