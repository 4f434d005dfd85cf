// ops.hip -- the backend-interface operations of the reference runtime
// (include/woodcock/ops.h:9-24, src/backends/cpu_ops.cpp:45-115) on device
// buffers, plus the KV cache's append / trim (include/woodcock/cache.h:17-21).
//
// These are the building blocks a HIP backend under the reference's own C++
// runtime (Drafter::forward, src/core/drafter.cpp:106-133; Qwen3::forward,
// src/core/qwen3.cpp:86-111) calls one at a time; the fused entry points of
// drafter.hip / target_layer.hip are what the hot path uses.  Arithmetic
// follows cpu_ops.cpp where it fixes results: fp64 sums of squares (rmsnorm)
// and of exponentials (softmax) as in cpu_ops.cpp:50-59,86-96, the reference's
// powf RoPE frequencies (cpu_ops.cpp:61-77), products kept unfused (contraction
// off) where the reference rounds them separately.  Layouts are the reference's: activations
// [rows][cols], the attention's K / V as its KVCache rows [T][Hk][D].
#include <cmath>
#include <vector>

#include "wc_common.h"

namespace wc {

constexpr int kOpThreads = 256;

__device__ __forceinline__ float ld_w(const void* w, int dtype, int64_t i) {
  return dtype == WC_BF16 ? __uint_as_float(static_cast<unsigned int>(static_cast<const uint16_t*>(w)[i]) << 16)
                          : static_cast<const float*>(w)[i];
}

// fp64 block sum over kOpThreads threads; the same value in every thread
__device__ __forceinline__ double op_block_sum(double v, double* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kOpThreads / kWave; ++w) t += red[w];
  return t;
}

__device__ __forceinline__ float op_block_max(float v, float* red) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kOpThreads / kWave; ++w) t = fmaxf(t, red[w]);
  return t;
}

// ------------------------------------------------------------------ rmsnorm

// one block per row: y = x * (1 / sqrt(mean(x^2) + eps)) * w, the mean from an fp64 sum
__global__ __launch_bounds__(kOpThreads) void k_op_rmsnorm(const float* x, float* y, int d, const void* w,
                                                           int w_dtype, float eps) {
  __shared__ double red[kOpThreads / kWave];
  const float* xr = x + static_cast<int64_t>(blockIdx.x) * d;
  float* yr = y + static_cast<int64_t>(blockIdx.x) * d;
  double ss = 0.0;
  for (int i = threadIdx.x; i < d; i += kOpThreads) ss += static_cast<double>(xr[i]) * xr[i];
  ss = op_block_sum(ss, red);
  const float inv = 1.f / sqrtf(static_cast<float>(ss / d) + eps);
  __syncthreads();  // x and y may alias: every read of the row is done
  for (int i = threadIdx.x; i < d; i += kOpThreads) yr[i] = __fmul_rn(__fmul_rn(xr[i], inv), ld_w(w, w_dtype, i));
}

// ------------------------------------------------------------------ rope

struct RopeInv {
  float inv[128];  // powf(base, -2i/D), i < D/2 <= 128, formed on the host as the reference forms it
};

// block (row l, head h), thread i < D/2: rotate-half at positions[l]
__global__ void k_op_rope(float* x, int heads, int D, const int32_t* positions, RopeInv r, const float* cos_t,
                          const float* sin_t, int max_pos) {
  const int l = blockIdx.x, h = blockIdx.y, i = threadIdx.x, half = D / 2;
  if (i >= half) return;
  const int pos = positions[l];
  float c, s;
  if (cos_t != nullptr && pos >= 0 && pos < max_pos) {
    c = cos_t[static_cast<int64_t>(pos) * half + i];
    s = sin_t[static_cast<int64_t>(pos) * half + i];
  } else {
    const float a = __fmul_rn(static_cast<float>(pos), r.inv[i]);
    c = cosf(a);
    s = sinf(a);
  }
  float* v = x + (static_cast<int64_t>(l) * heads + h) * D;
  const float x1 = v[i], x2 = v[i + half];
  {
    // each product rounded on its own, as the reference computes them (no fma)
#pragma clang fp contract(off)
    v[i] = x1 * c - x2 * s;
    v[i + half] = x2 * c + x1 * s;
  }
}

// ------------------------------------------------------------------ silu_mul

__global__ void k_op_silu_mul(float* gate, const float* up, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
    const float g = gate[i];
    gate[i] = __fmul_rn(g / (1.f + expf(-g)), up[i]);
  }
}

// ------------------------------------------------------------------ softmax

// one block per row, in place: e = exp(x - max) (0 where x = -inf), s = fp64 sum,
// x = e * (float)(1 / s)
__global__ __launch_bounds__(kOpThreads) void k_op_softmax(float* x, int n) {
  __shared__ float redf[kOpThreads / kWave];
  __shared__ double redd[kOpThreads / kWave];
  float* xr = x + static_cast<int64_t>(blockIdx.x) * n;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n; i += kOpThreads) m = fmaxf(m, xr[i]);
  m = op_block_max(m, redf);
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += kOpThreads) {
    const float v = xr[i];
    const float e = (isinf(v) && v < 0.f) ? 0.f : expf(v - m);
    xr[i] = e;
    s += e;
  }
  s = op_block_sum(s, redd);
  const float inv = static_cast<float>(1.0 / s);
  for (int i = threadIdx.x; i < n; i += kOpThreads) xr[i] = __fmul_rn(xr[i], inv);
}

// ------------------------------------------------------------------ attention

// block (query row l, head h): softmax(scale * q K^T + mask) V over T keys of kv
// head h / (H / Hk), 256 keys per chunk with a running max; thread d < D owns
// output element d.
__global__ __launch_bounds__(kOpThreads) void k_op_attention(const float* q, int H, int Hk, int D, const float* K,
                                                             const float* V, int T, const uint8_t* mask, float* out,
                                                             float scale) {
  __shared__ float s_q[256];
  __shared__ float s_p[kOpThreads];
  __shared__ float redf[kOpThreads / kWave];
  __shared__ double redd[kOpThreads / kWave];
  const int l = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
  const int kh = h / (H / Hk);
  const int64_t kv_ld = static_cast<int64_t>(Hk) * D;
  if (t < D) s_q[t] = q[(static_cast<int64_t>(l) * H + h) * D + t];
  __syncthreads();
  float m = -INFINITY;
  double lsum = 0.0;
  float acc = 0.f;
  for (int t0 = 0; t0 < T; t0 += kOpThreads) {
    const int j = t0 + t;
    float sc = -INFINITY;
    if (j < T && (mask == nullptr || mask[static_cast<int64_t>(l) * T + j])) {
      const float* kr = K + j * kv_ld + static_cast<int64_t>(kh) * D;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(s_q[d], kr[d], dot);
      sc = __fmul_rn(scale, dot);
    }
    const float cm = op_block_max(sc, redf);
    const float mn = fmaxf(m, cm);
    // rescale what was accumulated under the old max
    const float alpha = mn == -INFINITY ? 1.f : expf(m - mn);
    const float p = sc == -INFINITY ? 0.f : expf(sc - mn);
    __syncthreads();
    s_p[t] = p;
    const double ps = op_block_sum(static_cast<double>(p), redd);
    lsum = lsum * alpha + ps;
    m = mn;
    if (t < D) {
      float a = acc * alpha;
      const int n = min(kOpThreads, T - t0);
      const float* vr = V + t0 * kv_ld + static_cast<int64_t>(kh) * D + t;
      for (int k = 0; k < n; ++k) a = fmaf(s_p[k], vr[k * kv_ld], a);
      acc = a;
    }
    __syncthreads();
  }
  if (t < D) out[(static_cast<int64_t>(l) * H + h) * D + t] = __fmul_rn(acc, static_cast<float>(1.0 / lsum));
}

// ------------------------------------------------------------------ linear

// y[l][n] (+)= sum_k x[l][k] * W[n][k]: wave = one output row n, up to kLinRows
// input rows per block; lanes stride over k; DPP wave sums.
constexpr int kLinRows = 8;
__global__ __launch_bounds__(kOpThreads) void k_op_linear(const float* x, int L, int in, const void* W, int w_dtype,
                                                          int out, float* y, int accumulate) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int n = blockIdx.x * (kOpThreads / kWave) + wave;
  const int l0 = blockIdx.y * kLinRows;
  if (n >= out) return;
  const int nl = min(kLinRows, L - l0);
  float s[kLinRows];
#pragma unroll
  for (int r = 0; r < kLinRows; ++r) s[r] = 0.f;
  const int64_t wrow = static_cast<int64_t>(n) * in;
  for (int k = lane; k < in; k += kWave) {
    const float wv = ld_w(W, w_dtype, wrow + k);
#pragma unroll
    for (int r = 0; r < kLinRows; ++r)
      if (r < nl) s[r] = fmaf(x[static_cast<int64_t>(l0 + r) * in + k], wv, s[r]);
  }
#pragma unroll
  for (int r = 0; r < kLinRows; ++r) {
    const float v = wave_sum_dpp(s[r]);
    if (r < nl && lane == 0) {
      float* yp = y + static_cast<int64_t>(l0 + r) * out + n;
      *yp = accumulate ? *yp + v : v;
    }
  }
}

// ------------------------------------------------------------------ KV cache rows

// rows [L][row] of K and V into the caches at rows *offset_dev + l, [cap][row]
// (rows outside [0, cap) are dropped; the host checks what it can)
__global__ void k_op_kv_append(float* kc, float* vc, int row, int cap, const float* k, const float* v, int L,
                               const int32_t* offset_dev) {
  const int off = *offset_dev;
  const int64_t n = static_cast<int64_t>(L) * row;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t l = i / row;
    if (off + l >= 0 && off + l < cap) {
      kc[(off + l) * row + i % row] = k[i];
      vc[(off + l) * row + i % row] = v[i];
    }
  }
}

// *dst = *src + add clamped into [0, cap] (one thread; src may be dst): an
// offset never points past the rows an append could write
__global__ void k_op_advance_i32(int32_t* dst, const int32_t* src, int add, int cap) {
  *dst = min(max(*src + add, 0), cap);
}

__global__ void k_op_set_i32(int32_t* p, int v) { *p = v; }

}  // namespace wc

using namespace wc;

extern "C" {

int wc_rmsnorm(const float* x, float* y, int rows, int d, const void* w, int w_dtype, float eps, wc_stream_t stream) {
  WC_REQUIRE(x && y && w, "wc_rmsnorm: NULL buffer");
  WC_REQUIRE(rows >= 0 && d >= 1, "wc_rmsnorm: bad shape rows=%d d=%d", rows, d);
  WC_REQUIRE(w_dtype == WC_F32 || w_dtype == WC_BF16, "wc_rmsnorm: weight dtype must be f32 or bf16");
  if (rows == 0) return WC_OK;
  hipLaunchKernelGGL(k_op_rmsnorm, dim3(rows), dim3(kOpThreads), 0, reinterpret_cast<hipStream_t>(stream), x, y, d,
                     w, w_dtype, eps);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_rope(float* x, int L, int heads, int head_dim, const int32_t* positions_dev, float base, const float* cos_table,
            const float* sin_table, int max_pos, wc_stream_t stream) {
  WC_REQUIRE(x && positions_dev, "wc_rope: NULL buffer");
  WC_REQUIRE(L >= 0 && heads >= 1, "wc_rope: bad shape");
  WC_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 256, "wc_rope: head_dim must be even and <= 256");
  WC_REQUIRE((cos_table == nullptr) == (sin_table == nullptr), "wc_rope: give both tables or neither");
  if (L == 0) return WC_OK;
  RopeInv r{};
  for (int i = 0; i < head_dim / 2; ++i) r.inv[i] = std::pow(base, -2.f * static_cast<float>(i) / head_dim);
  hipLaunchKernelGGL(k_op_rope, dim3(L, heads), dim3(std::max(head_dim / 2, 64)), 0,
                     reinterpret_cast<hipStream_t>(stream), x, heads, head_dim, positions_dev, r, cos_table, sin_table,
                     cos_table ? max_pos : 0);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_silu_mul(float* gate, const float* up, int64_t n, wc_stream_t stream) {
  WC_REQUIRE(gate && up, "wc_silu_mul: NULL buffer");
  WC_REQUIRE(n >= 0, "wc_silu_mul: negative length");
  if (n == 0) return WC_OK;
  const int64_t blocks = std::min<int64_t>((n + kOpThreads - 1) / kOpThreads, 8192);
  hipLaunchKernelGGL(k_op_silu_mul, dim3(static_cast<unsigned>(blocks)), dim3(kOpThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), gate, up, n);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_softmax(float* x, int rows, int n, wc_stream_t stream) {
  WC_REQUIRE(x, "wc_softmax: NULL buffer");
  WC_REQUIRE(rows >= 0 && n >= 1, "wc_softmax: bad shape rows=%d n=%d", rows, n);
  if (rows == 0) return WC_OK;
  hipLaunchKernelGGL(k_op_softmax, dim3(rows), dim3(kOpThreads), 0, reinterpret_cast<hipStream_t>(stream), x, n);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_attention(const float* q, int L, int H, int Hk, int D, const float* K, const float* V, int T,
                 const uint8_t* mask, float* out, float scale, wc_stream_t stream) {
  WC_REQUIRE(q && K && V && out, "wc_attention: NULL buffer");
  WC_REQUIRE(L >= 0 && T >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0, "wc_attention: bad shape L=%d T=%d H=%d Hk=%d", L,
             T, H, Hk);
  WC_REQUIRE(D >= 1 && D <= 256, "wc_attention: head_dim %d outside 1..256", D);
  if (L == 0) return WC_OK;
  hipLaunchKernelGGL(k_op_attention, dim3(L, H), dim3(kOpThreads), 0, reinterpret_cast<hipStream_t>(stream), q, H, Hk,
                     D, K, V, T, mask, out, scale);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_linear(const float* x, int L, int in, const void* W, int w_dtype, int out, float* y, int accumulate,
              wc_stream_t stream) {
  WC_REQUIRE(x && W && y, "wc_linear: NULL buffer");
  WC_REQUIRE(L >= 0 && in >= 1 && out >= 1, "wc_linear: bad shape L=%d in=%d out=%d", L, in, out);
  WC_REQUIRE(w_dtype == WC_F32 || w_dtype == WC_BF16, "wc_linear: weight dtype must be f32 or bf16");
  if (L == 0) return WC_OK;
  const dim3 grid((out + kOpThreads / kWave - 1) / (kOpThreads / kWave), (L + kLinRows - 1) / kLinRows);
  hipLaunchKernelGGL(k_op_linear, grid, dim3(kOpThreads), 0, reinterpret_cast<hipStream_t>(stream), x, L, in, W,
                     w_dtype, out, y, accumulate);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_kv_append(float* k_cache, float* v_cache, int capacity, int row, const float* k, const float* v, int L,
                 const int32_t* offset_dev, int32_t* advance_dev, wc_stream_t stream) {
  WC_REQUIRE(k_cache && v_cache && k && v && offset_dev, "wc_kv_append: NULL buffer");
  WC_REQUIRE(L >= 0 && row >= 1 && capacity >= 1, "wc_kv_append: bad shape");
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (L > 0) {
    const int64_t n = static_cast<int64_t>(L) * row;
    const int64_t blocks = std::min<int64_t>((n + kOpThreads - 1) / kOpThreads, 4096);
    hipLaunchKernelGGL(k_op_kv_append, dim3(static_cast<unsigned>(blocks)), dim3(kOpThreads), 0, s, k_cache, v_cache,
                       row, capacity, k, v, L, offset_dev);
    WC_LAUNCHED();
  }
  if (advance_dev != nullptr) {  // after every block has read the offset (stream order): commit(L)
    hipLaunchKernelGGL(k_op_advance_i32, dim3(1), dim3(1), 0, s, advance_dev, offset_dev, L, capacity);
    WC_LAUNCHED();
  }
  return WC_OK;
}

int wc_kv_set_offset(int32_t* offset_dev, int n, wc_stream_t stream) {
  WC_REQUIRE(offset_dev, "wc_kv_set_offset: NULL offset");
  WC_REQUIRE(n >= 0, "wc_kv_set_offset: negative offset %d", n);
  hipLaunchKernelGGL(k_op_set_i32, dim3(1), dim3(1), 0, reinterpret_cast<hipStream_t>(stream), offset_dev, n);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
