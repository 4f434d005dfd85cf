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

static int launch_mm(const MmArgs& g, const MmReduceArgs& r, hipStream_t s) {
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
  const int nout = r.epi == kMmSiluPair ? r.N / 2 : r.N;
  hipLaunchKernelGGL(k_mm_reduce, dim3((nout + 255) / 256, r.M), dim3(256), 0, s, r);
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
  w.apart = take(4 * static_cast<size_t>(d.kv_heads) * kMaxSplits * kMaxQV * (d.head_dim + 2));
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
  if (int rc = launch_mm(g, r, s)) return rc;

  // 2. attention over the cache + this block (explicit positions / mask), in
  //    tiles of rows whose query vectors fit one block
  const int tile = std::max(1, std::min(kMaxQV / rep, WC_MAX_NODES));
  const int splits = std::max(1, std::min(kMaxSplits, (capacity + kAttnChunkMax - 1) / kAttnChunkMax));
  for (int t0 = 0; t0 < rows; t0 += tile) {
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
