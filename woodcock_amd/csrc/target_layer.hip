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
// 2048..12288 rows): bf16 MFMA (v_mfma_f32_16x16x32_bf16) with the fp32
// activations split into bf16 hi + lo parts (x = hi + lo to ~2^-17 relative),
// so the products keep fp32-level accuracy.  Each block owns 128 output
// features and one 256-wide K chunk (split-K, so every CU gets work and the
// activations are read ~N/128 times, not once per row); a second launch sums
// the K chunks in a fixed order (deterministic), applies the RMSNorm scale and
// the epilogue (store, residual, SiLU(gate) * up).
#include "attention.h"

namespace wc {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMmThreads = 256;           // 4 waves
constexpr int kMmNT = 128;                // output features per block: 4 waves x 2 tiles of 16
constexpr int kMmKC = 256;                // K per block: 8 MFMA steps of 32
constexpr int kMmMaxRows = 64;            // 4 row tiles of 16
constexpr int kMmLdsRow = kMmKC * 2 + 16; // bytes per LDS row of bf16 (16 B pad against bank conflicts)
constexpr int kMmMaxSeg = 3;

struct MmArgs {
  const float* x;  // [M][ldx] fp32 rows
  int64_t ldx;
  const uint16_t* gain;  // [K] bf16 RMSNorm gain, or NULL (no norm)
  const uint16_t* w[kMmMaxSeg];  // per output segment: [rows][K] bf16
  int seg_start[kMmMaxSeg + 1];  // output feature boundaries (multiples of kMmNT)
  int n_seg;
  int M, N, K, kchunks;
  float* part;  // [kchunks][M][N]
  float* ss;    // [kchunks][M] sums of squares of x over each chunk (with a gain)
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const __bf16 x = static_cast<__bf16>(a), y = static_cast<__bf16>(b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, x)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y)) << 16);
}

// Block (n tile, K chunk): partial products of its 128 features over its chunk.
template <int MT>
__global__ __launch_bounds__(kMmThreads) void k_mm_partial(MmArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char s_hi[kMmMaxRows * kMmLdsRow];
  __shared__ __attribute__((aligned(16))) unsigned char s_lo[kMmMaxRows * kMmLdsRow];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nb = blockIdx.x * kMmNT, kc = blockIdx.y, k0 = kc * kMmKC;

  // 1. this wave's weights: 2 tiles of 16 features x 8 steps, one 16-byte
  //    fragment per lane each (feature lane%16, k group lane/16)
  int seg = 0;
#pragma unroll
  for (int j = 1; j < kMmMaxSeg; ++j)
    if (j < a.n_seg && nb >= a.seg_start[j]) seg = j;
  const uint16_t* wbase = seg == 0 ? a.w[0] : seg == 1 ? a.w[1] : a.w[2];
  const int sbeg = seg == 0 ? a.seg_start[0] : seg == 1 ? a.seg_start[1] : a.seg_start[2];
  uint4 wf[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = min(nb + wave * 32 + j * 16 + lane % 16, a.N - 1) - sbeg;
    const uint16_t* wr = wbase + static_cast<int64_t>(n) * a.K + k0 + (lane / 16) * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s) wf[j][s] = *reinterpret_cast<const uint4*>(wr + s * 32);
  }

  // 2. activation chunk -> LDS as bf16 hi / lo of x * gain; thread t owns row
  //    t/4, columns (t%4)*64 .. +64 of the chunk
  {
    const int r = threadIdx.x / 4, q = threadIdx.x % 4;
    const bool live = r < a.M;
    const float* xr = a.x + static_cast<int64_t>(min(r, a.M - 1)) * a.ldx + k0 + q * 64;
    float4 xv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = *reinterpret_cast<const float4*>(xr + 4 * i);
    uint4 gv[8];
    if (a.gain) {
#pragma unroll
      for (int i = 0; i < 8; ++i) gv[i] = *reinterpret_cast<const uint4*>(a.gain + k0 + q * 64 + 8 * i);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v[8] = {xv[2 * i].x, xv[2 * i].y, xv[2 * i].z, xv[2 * i].w,
                    xv[2 * i + 1].x, xv[2 * i + 1].y, xv[2 * i + 1].z, xv[2 * i + 1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (!live) v[e] = 0.f;
        ss = fmaf(v[e], v[e], ss);
      }
      if (a.gain) {
        const uint4 g = gv[i];
        v[0] *= bf16_lo(g.x); v[1] *= bf16_hi(g.x); v[2] *= bf16_lo(g.y); v[3] *= bf16_hi(g.y);
        v[4] *= bf16_lo(g.z); v[5] *= bf16_hi(g.z); v[6] *= bf16_lo(g.w); v[7] *= bf16_hi(g.w);
      }
      float lo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) lo[e] = v[e] - static_cast<float>(static_cast<__bf16>(v[e]));
      const uint4 hq = make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                                  pack_bf16(v[6], v[7]));
      const uint4 lq = make_uint4(pack_bf16(lo[0], lo[1]), pack_bf16(lo[2], lo[3]), pack_bf16(lo[4], lo[5]),
                                  pack_bf16(lo[6], lo[7]));
      const int off = r * kMmLdsRow + (q * 64 + 8 * i) * 2;
      *reinterpret_cast<uint4*>(s_hi + off) = hq;
      *reinterpret_cast<uint4*>(s_lo + off) = lq;
    }
    // the row's four threads are adjacent lanes: combine, one of them records
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    if (a.gain && q == 0 && live && blockIdx.x == 0) a.ss[static_cast<int64_t>(kc) * a.M + r] = ss;
  }
  lds_barrier();

  // 3. MFMA: rows tile i (MT of them) x features tile j (2), 8 steps, hi and lo
  f32x4 acc[2][MT];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 8; ++s) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int off = (i * 16 + lane % 16) * kMmLdsRow + (s * 32 + (lane / 16) * 8) * 2;
      const bf16x8 ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(s_hi + off));
      const bf16x8 al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(s_lo + off));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16x8 b = __builtin_bit_cast(bf16x8, wf[j][s]);
        acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b, acc[j][i], 0, 0, 0);
        acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b, acc[j][i], 0, 0, 0);
      }
    }
  }

  // 4. partials: lane holds feature lane%16, rows (lane/16)*4 + e of each tile
  float* pp = a.part + static_cast<int64_t>(kc) * a.M * a.N;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = nb + wave * 32 + j * 16 + lane % 16;
    if (n >= a.N) continue;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = i * 16 + (lane / 16) * 4 + e;
        if (m < a.M) pp[static_cast<int64_t>(m) * a.N + n] = acc[j][i][e];
      }
  }
}

enum MmEpi { kMmStore = 0, kMmResidual = 1, kMmSiluPair = 2 };

struct MmReduceArgs {
  const float* part;
  const float* ss;  // NULL: no norm
  int M, N, K, kchunks;
  float eps;
  int epi;
  float* out;  // [M][ldo]
  int64_t ldo;
  const float* res;  // residual [M][ldr]
  int64_t ldr;
};

// Sum the K chunks in order, scale by the row's 1/rms, epilogue.  Block
// (feature range, row); for the SiLU pair the features are [gate | up] halves.
__global__ __launch_bounds__(256) void k_mm_reduce(MmReduceArgs a) {
  __shared__ float s_inv;
  const int m = blockIdx.y;
  if (threadIdx.x == 0) {
    float inv = 1.f;
    if (a.ss) {
      float t = 0.f;
      for (int c = 0; c < a.kchunks; ++c) t += a.ss[static_cast<int64_t>(c) * a.M + m];
      inv = 1.f / sqrtf(t / static_cast<float>(a.K) + a.eps);
    }
    s_inv = inv;
  }
  __syncthreads();
  const float inv = s_inv;
  const int nout = a.epi == kMmSiluPair ? a.N / 2 : a.N;
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= nout) return;
  const int64_t stride = static_cast<int64_t>(a.M) * a.N;
  const float* p = a.part + static_cast<int64_t>(m) * a.N + n;
  float y = 0.f, u = 0.f;
  for (int c = 0; c < a.kchunks; ++c) {
    y += p[c * stride];
    if (a.epi == kMmSiluPair) u += p[c * stride + nout];
  }
  y *= inv;
  float v;
  if (a.epi == kMmSiluPair) {
    u *= inv;
    v = y / (1.f + expf(-y)) * u;
  } else if (a.epi == kMmResidual) {
    v = a.res[static_cast<int64_t>(m) * a.ldr + n] + y;
  } else {
    v = y;
  }
  a.out[static_cast<int64_t>(m) * a.ldo + n] = v;
}

static int launch_mm_partial(const MmArgs& g, hipStream_t s) {
  WC_REQUIRE(g.M >= 1 && g.M <= kMmMaxRows, "target layer: rows must be in 1..%d", kMmMaxRows);
  WC_REQUIRE(g.K % kMmKC == 0, "target layer: K %d must be a multiple of %d", g.K, kMmKC);
  for (int j = 0; j < g.n_seg; ++j)
    WC_REQUIRE(g.seg_start[j] % kMmNT == 0, "target layer: projection widths must be multiples of %d", kMmNT);
  const dim3 grid((g.N + kMmNT - 1) / kMmNT, g.kchunks);
  switch ((g.M + 15) / 16) {
    case 1: hipLaunchKernelGGL(k_mm_partial<1>, grid, dim3(kMmThreads), 0, s, g); break;
    case 2: hipLaunchKernelGGL(k_mm_partial<2>, grid, dim3(kMmThreads), 0, s, g); break;
    case 3: hipLaunchKernelGGL(k_mm_partial<3>, grid, dim3(kMmThreads), 0, s, g); break;
    default: hipLaunchKernelGGL(k_mm_partial<4>, grid, dim3(kMmThreads), 0, s, g); break;
  }
  WC_LAUNCHED();
  return WC_OK;
}

static int launch_mm(const MmArgs& g, const MmReduceArgs& r, hipStream_t s) {
  if (int rc = launch_mm_partial(g, s)) return rc;
  const int nout = r.epi == kMmSiluPair ? r.N / 2 : r.N;
  hipLaunchKernelGGL(k_mm_reduce, dim3((nout + 255) / 256, r.M), dim3(256), 0, s, r);
  WC_LAUNCHED();
  return WC_OK;
}

// ------------------------------------------------------------------ QKV epilogue
// The QKV projection's reduce kernel, for head_dim 128: per (row, 256 output
// features = two heads) it sums the K chunks, applies RMS_in, then for q and k
// heads the per-head RMSNorm (q_norm / k_norm gains) and rotate-half RoPE at
// the row's position (src/backends/cpu_ops.cpp:61-77), in the order
// x1 = x inv g, lo' = x1 c - x2 s, hi' = x2 c + x1 s.  q lands in q_out; the
// block's K and V rows go straight to the cache at slot offset + row, so the
// attention that follows reads every key, old or new, from the cache.
constexpr int kVaD = 128;  // head_dim of the verify-width path

struct QkvEpiArgs {
  const float* part;  // [kchunks][M][N]
  const float* ss;    // [kchunks][M]
  int M, N, K, kchunks;
  float eps;
  float* q_out;  // [M][nq]
  int64_t ldq;
  int nq, nk;
  const uint16_t *q_gain, *k_gain;
  const float *rope_cos, *rope_sin;
  int rope_max;
  const int32_t* positions;  // [M] or NULL: offset + row
  const int32_t* offset_dev;
  void *kc, *vc;  // [Hk][cap][128]
  int kv_bf16, cap;
};

__global__ __launch_bounds__(256) void k_mm_reduce_qkv(QkvEpiArgs a) {
  __shared__ float s_red[256 / kWave];
  __shared__ float s_x[256];
  const int m = blockIdx.y, t = threadIdx.x, wave = t / kWave;
  const int n = min(blockIdx.x * 256 + t, a.N - 1);
  const bool live = blockIdx.x * 256 + t < a.N;
  // every load first: the row's chunk sums of squares, this feature's partials,
  // the position and the cache offset
  float ssum = 0.f;
  for (int c = 0; c < a.kchunks; ++c) ssum += a.ss[static_cast<int64_t>(c) * a.M + m];
  const int64_t stride = static_cast<int64_t>(a.M) * a.N;
  const float* p = a.part + static_cast<int64_t>(m) * a.N + n;
  float y = 0.f;
  for (int c = 0; c < a.kchunks; ++c) y += p[c * stride];
  const int offset = *a.offset_dev;
  const int pos = min(max(a.positions ? a.positions[m] : offset + m, 0), a.rope_max - 1);
  y *= 1.f / sqrtf(ssum / static_cast<float>(a.K) + a.eps);

  const int d = n % kVaD;
  const bool is_q = n < a.nq, is_k = !is_q && n < a.nq + a.nk;  // uniform per head (128 threads)
  float x = y;
  {
    // per-head RMSNorm: a head is two waves
    float hs = wave_sum_dpp(y * y);
    if (t % kWave == 0) s_red[wave] = hs;
    lds_barrier();
    hs = s_red[wave & ~1] + s_red[wave | 1];
    const float inv = 1.f / sqrtf(hs / static_cast<float>(kVaD) + a.eps);
    const float g = bf16_to_float(is_q ? a.q_gain[d] : a.k_gain[min(d, kVaD - 1)]);
    x = y * inv * g;
    s_x[t] = x;
    lds_barrier();
    const float xp = s_x[t ^ (kVaD / 2)];  // the rotate-half partner, same head
    const int pi = d % (kVaD / 2);
    const float c = a.rope_cos[static_cast<int64_t>(pos) * (kVaD / 2) + pi];
    const float s = a.rope_sin[static_cast<int64_t>(pos) * (kVaD / 2) + pi];
    if (is_q || is_k) x = d < kVaD / 2 ? x * c - xp * s : x * c + xp * s;
  }
  if (!live) return;
  if (is_q) {
    a.q_out[static_cast<int64_t>(m) * a.ldq + n] = x;
    return;
  }
  const int slot = offset + m;
  if (slot < 0 || slot >= a.cap) return;
  const int j = is_k ? n - a.nq : n - a.nq - a.nk;
  const int64_t at = (static_cast<int64_t>(j / kVaD) * a.cap + slot) * kVaD + d;
  void* base = is_k ? a.kc : a.vc;
  const float v = is_k ? x : y;
  if (a.kv_bf16)
    static_cast<uint16_t*>(base)[at] = float_to_bf16(v);
  else
    static_cast<float*>(base)[at] = v;
}

// ------------------------------------------------------------------ verify attention
// Split-KV GQA attention for a verify block (head_dim 128, bf16 cache) whose q
// rows are already normalised / rotated and whose K / V rows are already in
// the cache.  Block (split, kv head, group): group z covers query vectors
// 64 z .. 64 z + 63, wave w of them 16 w .. 16 w + 15, loaded straight into
// MFMA A fragments (fp32 split into bf16 hi + lo).  Per chunk of 64 keys:
// S = Q K^T by v_mfma_f32_16x16x32_bf16 (four independent key tiles), an
// online softmax in base 2 in registers (a query row is one 16-lane DPP row),
// P through the wave's LDS tile into the A layout (hi + lo), O += P V against
// the chunk's transposed V.  The next chunk's K / V and mask bytes load while
// the current one is consumed.  Partial (m, l, o) per split (m in natural
// units) go to k_attn_merge.
typedef __bf16 abf16x8 __attribute__((ext_vector_type(8)));
typedef float af32x4 __attribute__((ext_vector_type(4)));

constexpr int kVaCH = 64;            // keys per chunk
constexpr int kVaLdK = kVaD + 8;     // row stride (bf16) of the K chunk: B-fragment reads spread over the banks
constexpr int kVaLdT = kVaCH + 8;    // row stride (bf16) of the transposed V chunk
constexpr int kVaLdP = kVaCH + 4;    // row stride (fp32) of a wave's P tile
constexpr int kVaGroup = 64;         // query vectors per block
constexpr int kVaMaxRows = 64;       // rows per launch (mask rows staged per chunk)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(b))) << 16);
}

// 8 fp32 -> bf16 hi (round to nearest) and lo (the rounding remainder, rounded):
// hi + lo equals x to ~2^-17 relative, so bf16 MFMA products keep fp32 accuracy.
__device__ __forceinline__ void split8(const float* x, abf16x8& hi, abf16x8& lo) {
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = x[e] - static_cast<float>(static_cast<__bf16>(x[e]));
  const uint4 h = make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]), pack2_bf16(x[4], x[5]),
                             pack2_bf16(x[6], x[7]));
  const uint4 l = make_uint4(pack2_bf16(r[0], r[1]), pack2_bf16(r[2], r[3]), pack2_bf16(r[4], r[5]),
                             pack2_bf16(r[6], r[7]));
  hi = __builtin_bit_cast(abf16x8, h);
  lo = __builtin_bit_cast(abf16x8, l);
}

struct VaChunk {
  uint4 k[4], v[4];
  uint8_t mb[16];  // mask bytes: this thread's row, keys 16 (t % 4) .. + 16 (packed when staged)
};

// K as [key][d] (thread t: key t / 16 + 16 i, d chunk t % 16: coalesced); V
// with lanes along keys (lane l: key l % 32 + 32 (i & 1), d chunk l / 32 + 2 w
// + 8 (i >> 1)) so that the transposed LDS writes of a wave cover two
// contiguous 64-byte runs; mask bytes of row t / 4, keys 16 (t % 4) .. + 16.
// Rows clamp into [0, last].
__device__ __forceinline__ void va_chunk_load(const uint16_t* kc, const uint16_t* vc, int c0, int last,
                                              const uint8_t* mask, int64_t mask_ld, int nr, int ke, VaChunk& ch) {
  const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kj = min(c0 + t / 16 + 16 * i, last);
    ch.k[i] = *reinterpret_cast<const uint4*>(kc + static_cast<int64_t>(kj) * kVaD + (t % 16) * 8);
    const int vj = min(c0 + lane % 32 + 32 * (i & 1), last);
    const int dc = lane / 32 + 2 * w + 8 * (i >> 1);
    ch.v[i] = *reinterpret_cast<const uint4*>(vc + static_cast<int64_t>(vj) * kVaD + dc * 8);
  }
  if (mask) {
    const int r = min(t / 4, max(nr - 1, 0));
    const uint8_t* mr = mask + static_cast<int64_t>(r) * mask_ld;
#pragma unroll
    for (int e = 0; e < 16; ++e) ch.mb[e] = mr[min(c0 + (t % 4) * 16 + e, max(ke - 1, 0))];
  }
}

template <int UNUSED = 0>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_verify_attention(AttnArgs a) {
  constexpr int D = kVaD, CH = kVaCH;
  constexpr int nw = kAttnThreads / kWave;
  __shared__ __attribute__((aligned(16))) float pb[nw * 16 * kVaLdP];  // per-wave P tiles
  __shared__ __attribute__((aligned(16))) uint16_t ksb[CH * kVaLdK];   // [key][d]
  __shared__ __attribute__((aligned(16))) uint16_t vst[D * kVaLdT];    // [d][key]
  __shared__ __attribute__((aligned(16))) uint16_t s_mb[kVaMaxRows * 4];  // mask bits [row][key / 16]

  const int kh = blockIdx.y, split = blockIdx.x, S = gridDim.x, z = blockIdx.z;
  const int rep = a.H / a.Hk;
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  const int offset = *a.offset_dev + a.offset_add;
  const int T = min(offset + nr, a.cap);
  const int QV = nr * rep, QVb = a.rows * rep;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int dg = (lane / 16) * 8;
  const uint16_t* kc = static_cast<const uint16_t*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  const uint16_t* vc = static_cast<const uint16_t*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  const int per = ((T + S - 1) / S + CH - 1) / CH * CH;  // whole chunks per split
  const int kb = min(T, split * per), ke = min(T, kb + per);
  const int last = max(a.cap - 1, 0);

  // q tile (this lane: vector vq, dims 32 st + dg .. + 8) and the first chunk
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
  va_chunk_load(kc, vc, kb, last, a.mask, a.mask_ld, nr, ke, ch);
  abf16x8 qh[4], ql[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const bool lv = vq < QV;
    const float4 u = qf[2 * st], w = qf[2 * st + 1];
    const float x[8] = {lv ? u.x : 0.f, lv ? u.y : 0.f, lv ? u.z : 0.f, lv ? u.w : 0.f,
                        lv ? w.x : 0.f, lv ? w.y : 0.f, lv ? w.z : 0.f, lv ? w.w : 0.f};
    split8(x, qh[st], ql[st]);
  }

  // the lane's softmax rows 16 w + 4 (lane / 16) + e: visibility limits in
  // cache slots (causal and window), or the mask row
  int lim[4], wlo[4], mrow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = z * kVaGroup + wave * 16 + (lane / 16) * 4 + e;
    const int l = min(v, QVb - 1) / rep;
    mrow[e] = l;
    lim[e] = v < QV ? (a.mask ? 0x7fffffff : offset + l) : -1;
    wlo[e] = (!a.mask && a.window > 0) ? offset + l - a.window : -0x7fffffff;
  }
  const float sc = a.scale * kLog2e;
  float m_r[4], l_r[4];
  af32x4 o[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m_r[e] = -INFINITY;
    l_r[e] = 0.f;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = af32x4{0.f, 0.f, 0.f, 0.f};
  const bool tile_live = z * kVaGroup + wave * 16 < QV;
  float* pw = pb + wave * 16 * kVaLdP;

  for (int c0 = kb; c0 < ke; c0 += CH) {
    const int n = min(CH, ke - c0);
    lds_barrier();  // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kj = t / 16 + 16 * i;
      *reinterpret_cast<uint4*>(ksb + kj * kVaLdK + (t % 16) * 8) = kj < n ? ch.k[i] : make_uint4(0, 0, 0, 0);
      const int vj = lane % 32 + 32 * (i & 1), d0 = (lane / 32 + 2 * wave + 8 * (i >> 1)) * 8;
      const uint4 vv = vj < n ? ch.v[i] : make_uint4(0, 0, 0, 0);
      const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vst[(d0 + 2 * e) * kVaLdT + vj] = static_cast<uint16_t>(vw[e] & 0xffffu);
        vst[(d0 + 2 * e + 1) * kVaLdT + vj] = static_cast<uint16_t>(vw[e] >> 16);
      }
    }
    if (a.mask) {
      uint32_t mbits = 0;
#pragma unroll
      for (int e = 0; e < 16; ++e) mbits |= (ch.mb[e] != 0 ? 1u : 0u) << e;
      s_mb[t] = static_cast<uint16_t>(mbits);
    }
    lds_barrier();
    if (c0 + CH < ke) va_chunk_load(kc, vc, c0 + CH, last, a.mask, a.mask_ld, nr, ke, ch);  // next chunk

    if (tile_live) {
      // S = Q K^T, four independent key tiles
      af32x4 sacc[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) sacc[kt] = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        abf16x8 b[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          b[kt] = __builtin_bit_cast(
              abf16x8, *reinterpret_cast<const uint4*>(ksb + (kt * 16 + lane % 16) * kVaLdK + st * 32 + dg));
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh[st], b[kt], sacc[kt], 0, 0, 0);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql[st], b[kt], sacc[kt], 0, 0, 0);
      }
      // lane holds key kt * 16 + lane % 16 of rows 4 (lane / 16) + e
      float p[4][4], alpha[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t bits = 0xffffffffu, bits2 = 0xffffffffu;
        if (a.mask) {
          const uint2 mw = *reinterpret_cast<const uint2*>(s_mb + mrow[e] * 4);
          bits = mw.x;
          bits2 = mw.y;
        }
        float sv[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const int j = kt * 16 + lane % 16, tk = c0 + j;
          const uint32_t bw = kt < 2 ? bits : bits2;
          const bool vis = j < n && tk <= lim[e] && tk > wlo[e] && ((bw >> (j & 31)) & 1u);
          sv[kt] = vis ? sc * sacc[kt][e] : -INFINITY;
        }
        const float mx = row16_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
        const float m_new = fmaxf(m_r[e], mx);
        const float mb = m_new == -INFINITY ? 0.f : m_new;  // all hidden so far: exp2(-inf) = 0 below
        alpha[e] = __builtin_amdgcn_exp2f(m_r[e] - mb);
        float rs = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          p[kt][e] = __builtin_amdgcn_exp2f(sv[kt] - mb);
          rs += p[kt][e];
        }
        l_r[e] = l_r[e] * alpha[e] + row16_sum(rs);
        m_r[e] = m_new;
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[dt][e] *= alpha[e];
      // P through the wave's LDS tile into the A layout (row lane % 16, keys 32 kk + dg ..)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) pw[((lane / 16) * 4 + e) * kVaLdP + kt * 16 + lane % 16] = p[kt][e];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const float4 u = *reinterpret_cast<const float4*>(pw + (lane % 16) * kVaLdP + kk * 32 + dg);
        const float4 w = *reinterpret_cast<const float4*>(pw + (lane % 16) * kVaLdP + kk * 32 + dg + 4);
        const float px[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
        abf16x8 ph, pl;
        split8(px, ph, pl);
        abf16x8 b[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
          b[dt] = __builtin_bit_cast(
              abf16x8, *reinterpret_cast<const uint4*>(vst + (dt * 16 + lane % 16) * kVaLdT + kk * 32 + dg));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, b[dt], o[dt], 0, 0, 0);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, b[dt], o[dt], 0, 0, 0);
      }
    }
  }

  // this split's (m, l, o) per query vector; m back to natural units
  float* part = a.partial + (static_cast<int64_t>(kh) * S + split) * a.qv_ld * (D + 2);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = z * kVaGroup + wave * 16 + (lane / 16) * 4 + e;
    if (v >= QV) continue;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) part[v * (D + 2) + 2 + dt * 16 + lane % 16] = o[dt][e];
    if (lane % 16 == 0) {
      part[v * (D + 2)] = m_r[e] == -INFINITY ? -INFINITY : m_r[e] / kLog2e;
      part[v * (D + 2) + 1] = l_r[e];
    }
  }
}

static int launch_verify_attention(const AttnArgs& a, int splits, hipStream_t s) {
  WC_REQUIRE(a.rows >= 1 && a.rows <= kVaMaxRows, "verify attention: rows must be in 1..%d", kVaMaxRows);
  const int qvb = a.rows * (a.H / a.Hk);
  WC_REQUIRE(a.qv_ld >= qvb, "verify attention: partial stride too small");
  const unsigned groups = static_cast<unsigned>((qvb + kVaGroup - 1) / kVaGroup);
  hipLaunchKernelGGL(k_verify_attention<0>, dim3(splits, a.Hk, groups), dim3(kAttnThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL((k_attn_merge<kVaD>), dim3(static_cast<unsigned>(qvb), a.Hk), dim3(kAttnThreads), 0, s, a,
                     splits);
  WC_LAUNCHED();
  return WC_OK;
}

struct TargetWs {
  float *qkv, *attn, *h1, *act, *part, *ss, *apart;
  size_t bytes;
};

static TargetWs target_ws(const wc_drafter_dims& d, int max_rows, void* base) {
  TargetWs w{};
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off = (off + bytes + 255) / 256 * 256;
    return reinterpret_cast<float*>(q);
  };
  const size_t M = static_cast<size_t>(max_rows);
  const size_t nqkv = static_cast<size_t>(d.heads + 2 * d.kv_heads) * d.head_dim;
  const size_t hd = static_cast<size_t>(d.heads) * d.head_dim;
  const size_t kmax = std::max<size_t>(std::max<size_t>(d.hidden, hd), d.inter);
  const size_t nmax = std::max<size_t>(std::max<size_t>(nqkv, 2 * static_cast<size_t>(d.inter)), d.hidden);
  w.qkv = take(4 * M * nqkv);
  w.attn = take(4 * M * hd);
  w.h1 = take(4 * M * d.hidden);
  w.act = take(4 * M * d.inter);
  w.part = take(4 * (kmax / kMmKC) * M * nmax);
  w.ss = take(4 * (kmax / kMmKC) * M);
  const size_t qv = M * static_cast<size_t>(d.heads / std::max(d.kv_heads, 1));
  w.apart = take(4 * static_cast<size_t>(d.kv_heads) * kMaxSplits * qv * (d.head_dim + 2));
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
                    int capacity, const int32_t* offset_dev, void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(dims && L && x && k_cache && v_cache && offset_dev && workspace, "wc_target_layer: NULL argument");
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(rows >= 1 && rows <= kMmMaxRows, "wc_target_layer: rows must be in 1..%d (got %d)", kMmMaxRows, rows);
  WC_REQUIRE(d.heads >= 1 && d.kv_heads >= 1 && d.heads % d.kv_heads == 0, "wc_target_layer: bad head counts");
  WC_REQUIRE(d.hidden % kMmKC == 0 && (d.heads * d.head_dim) % kMmKC == 0 && d.inter % kMmKC == 0,
             "wc_target_layer: hidden, heads*head_dim and inter must be multiples of %d", kMmKC);
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
  auto s = reinterpret_cast<hipStream_t>(stream);
  auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };

  // 1. QKV = W . RMS_in(x)
  MmArgs g{};
  g.x = x;
  g.ldx = d.hidden;
  g.gain = u16(L->in_norm);
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
  g.kchunks = d.hidden / kMmKC;
  g.part = ws.part;
  g.ss = ws.ss;
  MmReduceArgs r{};
  r.part = ws.part;
  r.ss = ws.ss;
  r.M = rows;
  r.N = nqkv;
  r.K = d.hidden;
  r.kchunks = g.kchunks;
  r.eps = d.eps;
  r.epi = kMmStore;
  r.out = ws.qkv;
  r.ldo = nqkv;
  const int splits = std::max(1, std::min(kMaxSplits, (capacity + kAttnChunkMax - 1) / kAttnChunkMax));
  // head_dim 128 with a bf16 cache: the QKV epilogue normalises / rotates q and
  // k and appends K / V, then one MFMA attention launch covers every row
  const bool verify_path = D == kVaD && kv_dtype == WC_BF16 && rows <= kVaMaxRows;
  if (verify_path) {
    if (int rc = launch_mm_partial(g, s)) return rc;
    QkvEpiArgs e{};
    e.part = ws.part;
    e.ss = ws.ss;
    e.M = rows;
    e.N = nqkv;
    e.K = d.hidden;
    e.kchunks = g.kchunks;
    e.eps = d.eps;
    e.q_out = ws.qkv;
    e.ldq = nq;
    e.nq = nq;
    e.nk = nk;
    e.q_gain = u16(L->q_norm);
    e.k_gain = u16(L->k_norm);
    e.rope_cos = rope_cos;
    e.rope_sin = rope_sin;
    e.rope_max = rope_max_pos;
    e.positions = positions_dev;
    e.offset_dev = offset_dev;
    e.kc = k_cache;
    e.vc = v_cache;
    e.kv_bf16 = 1;
    e.cap = capacity;
    hipLaunchKernelGGL(k_mm_reduce_qkv, dim3((nqkv + 255) / 256, rows), dim3(256), 0, s, e);
    WC_LAUNCHED();
    AttnArgs at{};
    at.qkv = ws.qkv;
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
    // about two chunks of keys per split
    const int vsplits = std::max(1, std::min(kMaxSplits, (capacity + 2 * kVaCH - 1) / (2 * kVaCH)));
    if (int rc = launch_verify_attention(at, vsplits, s)) return rc;
  } else if (int rc = launch_mm(g, r, s)) {
    return rc;
  }

  // 2. (other head sizes / fp32 cache) attention with the decode kernel over
  //    tiles of rows whose query vectors fit one block; it normalises, rotates
  //    and appends on the fly
  const int tile = verify_path ? rows : std::max(1, std::min(kMaxQV / rep, WC_MAX_NODES));
  for (int t0 = 0; t0 < rows && !verify_path; t0 += tile) {
    AttnArgs at{};
    at.qkv = ws.qkv + static_cast<int64_t>(t0) * nqkv;
    at.ld_qkv = nqkv;
    at.H = H;
    at.Hk = Hk;
    at.rows = std::min(tile, rows - t0);
    at.n_rows_dev = nullptr;
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

  // 3. h1 = x + W_o . attn
  g = MmArgs{};
  g.x = ws.attn;
  g.ldx = nq;
  g.w[0] = u16(L->o);
  g.seg_start[1] = d.hidden;
  g.n_seg = 1;
  g.M = rows;
  g.N = d.hidden;
  g.K = nq;
  g.kchunks = nq / kMmKC;
  g.part = ws.part;
  g.ss = ws.ss;
  r = MmReduceArgs{};
  r.part = ws.part;
  r.M = rows;
  r.N = d.hidden;
  r.K = nq;
  r.kchunks = g.kchunks;
  r.epi = kMmResidual;
  r.out = ws.h1;
  r.ldo = d.hidden;
  r.res = x;
  r.ldr = d.hidden;
  if (int rc = launch_mm(g, r, s)) return rc;

  // 4. act = silu(W_gate . RMS_post(h1)) * (W_up . RMS_post(h1))
  g = MmArgs{};
  g.x = ws.h1;
  g.ldx = d.hidden;
  g.gain = u16(L->post_norm);
  g.w[0] = u16(L->gate);
  g.w[1] = u16(L->up);
  g.seg_start[1] = d.inter;
  g.seg_start[2] = 2 * d.inter;
  g.n_seg = 2;
  g.M = rows;
  g.N = 2 * d.inter;
  g.K = d.hidden;
  g.kchunks = d.hidden / kMmKC;
  g.part = ws.part;
  g.ss = ws.ss;
  r = MmReduceArgs{};
  r.part = ws.part;
  r.ss = ws.ss;
  r.M = rows;
  r.N = 2 * d.inter;
  r.K = d.hidden;
  r.kchunks = g.kchunks;
  r.eps = d.eps;
  r.epi = kMmSiluPair;
  r.out = ws.act;
  r.ldo = d.inter;
  if (int rc = launch_mm(g, r, s)) return rc;

  // 5. x = h1 + W_down . act
  g = MmArgs{};
  g.x = ws.act;
  g.ldx = d.inter;
  g.w[0] = u16(L->down);
  g.seg_start[1] = d.hidden;
  g.n_seg = 1;
  g.M = rows;
  g.N = d.hidden;
  g.K = d.inter;
  g.kchunks = d.inter / kMmKC;
  g.part = ws.part;
  g.ss = ws.ss;
  r = MmReduceArgs{};
  r.part = ws.part;
  r.M = rows;
  r.N = d.hidden;
  r.K = d.inter;
  r.kchunks = g.kchunks;
  r.epi = kMmResidual;
  r.out = x;
  r.ldo = d.hidden;
  r.res = ws.h1;
  r.ldr = d.hidden;
  return launch_mm(g, r, s);
}

}  // extern "C"
