// attention.h -- decode / verify-width attention for gfx950: q/k RMSNorm,
// rotate-half RoPE, KV append and split-KV GQA attention with an optional
// explicit mask (python/woodcock/drafter.py:85-97,186-188;
// python/woodcock/target.py:142-156; src/backends/cpu_ops.cpp:61-77,98-115).
// Shared by the drafter step and the verify-width target layer.
#pragma once
#include "wc_common.h"

namespace wc {

constexpr int kAttnThreads = 256;
constexpr int kAttnChunkMax = 32;  // keys staged per iteration (fewer for head_dim 256)
template <int D>
constexpr int attn_chunk() { return D >= 256 ? 16 : kAttnChunkMax; }
constexpr int kMaxQV = 64;      // query vectors (rows x GQA group) per attention block
constexpr int kMaxSplits = 32;
constexpr int kMaxKvHeads = 64;

// ------------------------------------------------------------------ fragment-major activations
// Element (m, k) of a block of 64 fp32 rows, split into bf16 hi (round to
// nearest) and lo (the rounding remainder), stored where one lane's 16-byte A
// fragment of v_mfma_f32_16x16x32_bf16 reads it: 32-wide k step s = k / 32,
// row tile m / 16, part h (0 hi, 1 lo), lane (m % 16) + 16 ((k % 32) / 8),
// element k % 8.  One k step of all four row tiles is a contiguous 8 KB run.
constexpr int kXaRowTiles = 4;
constexpr int kXaStepElems = kXaRowTiles * 2 * 512;  // bf16 per k step
__device__ __forceinline__ int64_t xa_index(int m, int k, int h) {
  return (static_cast<int64_t>(k >> 5) * kXaRowTiles + (m >> 4)) * 1024 + h * 512 +
         ((m & 15) + 16 * ((k & 31) >> 3)) * 8 + (k & 7);
}

// ------------------------------------------------------------------ attention

struct AttnArgs {
  const float* qkv;  // [rows][ld_qkv] raw q | k | v
  int64_t ld_qkv;
  int H, Hk, rows;
  const int32_t* n_rows_dev;
  const uint16_t *q_gain, *k_gain;
  float eps, scale;
  const float *rope_cos, *rope_sin;
  int rope_max;
  const int32_t* positions;  // [rows] or NULL
  void *kc, *vc;             // [Hk][cap][D]
  int cap;
  const int32_t* offset_dev;
  int offset_add;
  const uint8_t* mask;  // [rows][mask_ld] or NULL
  int64_t mask_ld;
  int window;
  float* partial;  // [Hk][S][qv_ld][D+2]
  int qv_ld;       // query vectors per (kv head, split) in `partial` (>= rows x group)
  float* out;  // [rows][H*D]
  uint16_t* xa_out;  // optional: the output also as fragment-major bf16 hi / lo (see xa_index), or NULL
  int64_t ld_out;
  unsigned int* ctr;  // [Hk][kCounterStride] zeroed split counters, or NULL (decode kernel: merge launch)
  // optional: the kSlots keys of a pending draft-head argmax (stride kSlotStride)
  // that the launch before this one consumed; the first block clears them
  unsigned long long* clear_slots;
};

template <typename KT>
__device__ __forceinline__ float kv_load(const KT* p, int64_t i);
template <>
__device__ __forceinline__ float kv_load<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float kv_load<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_float(p[i]);
}
// store to the cache, return the stored value as read back (bf16 rounding)
template <typename KT>
__device__ __forceinline__ float kv_store(KT* p, int64_t i, float v);
template <>
__device__ __forceinline__ float kv_store<float>(float* p, int64_t i, float v) {
  p[i] = v;
  return v;
}
template <>
__device__ __forceinline__ float kv_store<uint16_t>(uint16_t* p, int64_t i, float v) {
  const uint16_t b = float_to_bf16(v);
  p[i] = b;
  return bf16_to_float(b);
}

// The value a cache entry takes (bf16 rounding), and the store of such a value.
template <typename KT>
__device__ __forceinline__ float kv_round(float v) {
  if constexpr (sizeof(KT) == 2) return bf16_to_float(float_to_bf16(v));
  return v;
}
template <typename KT>
__device__ __forceinline__ void kv_put(KT* p, int64_t i, float rounded) {
  if constexpr (sizeof(KT) == 2)
    p[i] = float_to_bf16(rounded);
  else
    p[i] = rounded;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < static_cast<int>(blockDim.x) / kWave; ++w) t += red[w];
  return t;
}

// One head vector held by one wave for q/k RMSNorm + rotate-half RoPE
// (src/backends/cpu_ops.cpp:61-77): lane j owns the pairs (p, p + D/2) for
// p = j, j + 64, ..., so every value a lane produces was computed by that lane
// alone.  Loads go to clamped addresses (always in bounds) and lanes with
// p >= D/2 are masked when the values are used, so a load never sits behind a
// branch.
template <int D>
struct HeadVec {
  static constexpr int kHalf = D / 2;
  static constexpr int kPPL = (kHalf + kWave - 1) / kWave;
  float lo[kPPL], hi[kPPL];
  uint16_t glo[kPPL], ghi[kPPL];  // raw bf16 gains, widened where used
  float c[kPPL], sn[kPPL];        // RoPE row of the vector's position
};

template <int D>
__device__ __forceinline__ void head_vec_load(const float* src, const uint16_t* gain, HeadVec<D>& r) {
  const int lane = threadIdx.x % kWave;
  constexpr int half = HeadVec<D>::kHalf;
#pragma unroll
  for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
    const int p = min(lane + e * kWave, half - 1);
    r.lo[e] = src[p];
    r.hi[e] = src[p + half];
    r.glo[e] = gain[p];
    r.ghi[e] = gain[p + half];
  }
}

template <int D>
__device__ __forceinline__ void head_vec_rope_load(const float* ct, const float* st, int pos, HeadVec<D>& r) {
  const int lane = threadIdx.x % kWave;
  constexpr int half = HeadVec<D>::kHalf;
#pragma unroll
  for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
    const int p = min(lane + e * kWave, half - 1);
    r.c[e] = ct[static_cast<int64_t>(pos) * half + p];
    r.sn[e] = st[static_cast<int64_t>(pos) * half + p];
  }
}

// Normalise and rotate in place (after head_vec_load and head_vec_rope_load).
template <int D>
__device__ __forceinline__ void head_vec_norm_rope(HeadVec<D>& r, float eps) {
  const int lane = threadIdx.x % kWave;
  constexpr int half = HeadVec<D>::kHalf, PPL = HeadVec<D>::kPPL;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < PPL; ++e) {
    if (lane + e * kWave >= half) r.lo[e] = r.hi[e] = 0.f;
    ss = fmaf(r.lo[e], r.lo[e], ss);
    ss = fmaf(r.hi[e], r.hi[e], ss);
  }
  ss = wave_sum_dpp(ss);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
  for (int e = 0; e < PPL; ++e) {
    const float x1 = r.lo[e] * inv * bf16_to_float(r.glo[e]);
    const float x2 = r.hi[e] * inv * bf16_to_float(r.ghi[e]);
    r.lo[e] = x1 * r.c[e] - x2 * r.sn[e];
    r.hi[e] = x2 * r.c[e] + x1 * r.sn[e];
  }
}

// Key/value chunk staging: CH rows x D elements of one kv head, read as
// 16-byte vectors (VE cache elements each), kNL vectors per thread per tensor.
template <int D, typename KT>
struct KvChunk {
  static constexpr int kCH = attn_chunk<D>();
  static constexpr int kVE = 16 / static_cast<int>(sizeof(KT));
  static constexpr int kNL = (kCH * D / kVE + kAttnThreads - 1) / kAttnThreads;
  uint4 k[kNL], v[kNL];
};

// Issue the loads of rows [c0, c0 + CH) (clamped into the cache; rows past the
// chunk's end are loaded and ignored).
template <int D, typename KT>
__device__ __forceinline__ void kv_chunk_load(const KT* kc, const KT* vc, int cap, int c0, KvChunk<D, KT>& r) {
  using C = KvChunk<D, KT>;
  const uint4* k4 = reinterpret_cast<const uint4*>(kc);
  const uint4* v4 = reinterpret_cast<const uint4*>(vc);
  const int64_t last = static_cast<int64_t>(cap) * D / C::kVE - 1;
#pragma unroll
  for (int i = 0; i < C::kNL; ++i) {
    const int64_t e = min(static_cast<int64_t>(c0) * D / C::kVE + threadIdx.x + i * kAttnThreads, last);
    r.k[i] = k4[e];
    r.v[i] = v4[e];
  }
}

template <typename KT>
__device__ __forceinline__ void unpack16(const uint4 q, float* out);
template <>
__device__ __forceinline__ void unpack16<uint16_t>(const uint4 q, float* out) {
  out[0] = bf16_lo(q.x); out[1] = bf16_hi(q.x); out[2] = bf16_lo(q.y); out[3] = bf16_hi(q.y);
  out[4] = bf16_lo(q.z); out[5] = bf16_hi(q.z); out[6] = bf16_lo(q.w); out[7] = bf16_hi(q.w);
}
template <>
__device__ __forceinline__ void unpack16<float>(const uint4 q, float* out) {
  out[0] = __uint_as_float(q.x); out[1] = __uint_as_float(q.y);
  out[2] = __uint_as_float(q.z); out[3] = __uint_as_float(q.w);
}

// Write the n staged rows of chunk c0 into LDS; rows at or past `offset` are
// this launch's appended rows and come from nk / nv instead of the loads.
template <int D, typename KT>
__device__ __forceinline__ void kv_chunk_fill(const KvChunk<D, KT>& r, int c0, int n, int offset, const float* nk,
                                              const float* nv, float* ks, float* vs) {
  using C = KvChunk<D, KT>;
#pragma unroll
  for (int i = 0; i < C::kNL; ++i) {
    const int e = threadIdx.x + i * kAttnThreads;
    const int el = e * C::kVE;  // element index within the chunk
    if (el >= n * D) continue;
    const int t = c0 + el / D;
    if (t < offset) {
      unpack16<KT>(r.k[i], ks + el);
      unpack16<KT>(r.v[i], vs + el);
    } else {
      const int src = (t - offset) * D + el % D;
#pragma unroll
      for (int j = 0; j < C::kVE; ++j) {
        ks[el + j] = nk[src + j];
        vs[el + j] = nv[src + j];
      }
    }
  }
}

// One block per (split, kv head).  The block's key range [kb, ke) of the
// visible rows [0, T) is staged in chunks; the q vectors of the head group are
// normalised and rotated into LDS; rows appended by this launch (t >= offset)
// whose slot lies in [kb, ke) are normalised/rotated and written to the cache
// by this block, which also takes them from LDS rather than reading them back.
// Every load that does not depend on another is issued before the first wait:
// q / new-row sources and gains, then the first chunk, then the RoPE rows.
template <int D, typename KT>
__global__ __launch_bounds__(kAttnThreads) void k_attention(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];  // 16-byte aligned for b128 accesses
  constexpr int CH = attn_chunk<D>();
  constexpr int ACC = (kMaxQV * D + kAttnThreads - 1) / kAttnThreads;
  if (a.clear_slots && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < kSlots)
    a.clear_slots[threadIdx.x * kSlotStride] = 0ull;
  const int kh = blockIdx.y, split = blockIdx.x, S = gridDim.x;
  const int rep = a.H / a.Hk;
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  const int offset = *a.offset_dev + a.offset_add;
  const int T = min(offset + nr, a.cap);  // never past the cache capacity
  const int QV = nr * rep, QVb = a.rows * rep;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  constexpr int nw = kAttnThreads / kWave;

  float* qs = lds;                 // [QVb][D]
  float* ks = qs + QVb * D;        // [CH][D]
  float* vs = ks + CH * D;         // [CH][D]
  float* sc = vs + CH * D;         // [QVb][CH]
  float* nk = sc + QVb * CH;       // [rows][D] appended keys (cache-rounded)
  float* nv = nk + a.rows * D;     // [rows][D] appended values (cache-rounded)
  __shared__ float s_m[kMaxQV], s_l[kMaxQV], s_alpha[kMaxQV];
  __shared__ uint8_t s_mask[kMaxQV * kAttnChunkMax];  // mask bytes of the current chunk, [row][key]

  KT* kc = static_cast<KT*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  KT* vc = static_cast<KT*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  const int per = (T + S - 1) / S;
  const int kb = min(T, split * per), ke = min(T, kb + per);

  // first q vector and first appended row of this wave: sources and gains
  const int v0 = wave, l0 = nw - 1 - wave;  // appended rows from the last wave down
  // (loaded unconditionally from clamped rows so that no load sits in a branch)
  HeadVec<D> qv0, kv0;
  {
    const int v = min(v0, QVb - 1), l = v / rep, h = kh * rep + v % rep;
    head_vec_load<D>(a.qkv + l * a.ld_qkv + h * D, a.q_gain, qv0);
  }
  const bool app0 = l0 < nr && offset + l0 >= kb && offset + l0 < ke;
  constexpr int VPL = (D + kWave - 1) / kWave;
  float vv0[VPL];
  {
    const int l = min(l0, a.rows - 1);
    head_vec_load<D>(a.qkv + l * a.ld_qkv + (a.H + kh) * D, a.k_gain, kv0);
    const float* vsrc = a.qkv + l * a.ld_qkv + (a.H + a.Hk + kh) * D;
#pragma unroll
    for (int e = 0; e < VPL; ++e) vv0[e] = vsrc[min(lane + e * kWave, D - 1)];
  }
  // first chunk
  KvChunk<D, KT> ch;
  kv_chunk_load<D, KT>(kc, vc, a.cap, kb, ch);

  auto row_pos = [&](int l) {
    const int pos = a.positions ? a.positions[l] : offset + l;
    return min(max(pos, 0), a.rope_max - 1);
  };
  auto put_q = [&](int v, HeadVec<D>& r) {
    head_vec_norm_rope<D>(r, a.eps);
#pragma unroll
    for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
      const int p = lane + e * kWave;
      if (p < D / 2) {
        qs[v * D + p] = r.lo[e];
        qs[v * D + p + D / 2] = r.hi[e];
      }
    }
  };
  auto put_kv = [&](int l, HeadVec<D>& r, const float* vv) {
    const int t = offset + l;
    head_vec_norm_rope<D>(r, a.eps);
#pragma unroll
    for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
      const int p = lane + e * kWave;
      if (p < D / 2) {
        nk[l * D + p] = kv_store<KT>(kc, static_cast<int64_t>(t) * D + p, r.lo[e]);
        nk[l * D + p + D / 2] = kv_store<KT>(kc, static_cast<int64_t>(t) * D + p + D / 2, r.hi[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      const int i = lane + e * kWave;
      if (i < D) nv[l * D + i] = kv_store<KT>(vc, static_cast<int64_t>(t) * D + i, vv[e]);
    }
  };

  head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(min(v0, QVb - 1) / rep), qv0);
  head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(min(l0, a.rows - 1)), kv0);
  if (v0 < QV) put_q(v0, qv0);
  if (app0) put_kv(l0, kv0, vv0);
  for (int v = v0 + nw; v < QV; v += nw) {
    HeadVec<D> r;
    const int l = v / rep, h = kh * rep + v % rep;
    head_vec_load<D>(a.qkv + l * a.ld_qkv + h * D, a.q_gain, r);
    head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(l), r);
    put_q(v, r);
  }
  for (int l = l0 + nw; l < nr; l += nw) {
    if (offset + l < kb || offset + l >= ke) continue;
    HeadVec<D> r;
    float vv[VPL];
    head_vec_load<D>(a.qkv + l * a.ld_qkv + (a.H + kh) * D, a.k_gain, r);
    const float* vsrc = a.qkv + l * a.ld_qkv + (a.H + a.Hk + kh) * D;
#pragma unroll
    for (int e = 0; e < VPL; ++e) vv[e] = vsrc[min(lane + e * kWave, D - 1)];
    head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(l), r);
    put_kv(l, r, vv);
  }
  if (threadIdx.x < kMaxQV) {
    s_m[threadIdx.x] = -INFINITY;
    s_l[threadIdx.x] = 0.f;
  }
  __syncthreads();

  float acc[ACC];
#pragma unroll
  for (int e = 0; e < ACC; ++e) acc[e] = 0.f;
  int qv_group = 32;  // lanes per query vector in the softmax update
  while (qv_group > 1 && qv_group * QV > kAttnThreads) qv_group >>= 1;

  for (int c0 = kb; c0 < ke; c0 += CH) {
    const int n = min(CH, ke - c0);
    kv_chunk_fill<D, KT>(ch, c0, n, offset, nk, nv, ks, vs);
    if (a.mask) {  // the chunk's mask bytes, every load issued at once
      for (int e = threadIdx.x; e < nr * n; e += kAttnThreads) {
        const int l = e / n, j = e - l * n;
        s_mask[l * CH + j] = a.mask[static_cast<int64_t>(l) * a.mask_ld + c0 + j];
      }
    }
    __syncthreads();
    if (c0 + CH < ke) kv_chunk_load<D, KT>(kc, vc, a.cap, c0 + CH, ch);  // next chunk in flight
    for (int e = threadIdx.x; e < QV * n; e += kAttnThreads) {
      const int v = e / n, j = e - v * n;
      const int l = v / rep, t = c0 + j;
      bool vis;
      if (a.mask)
        vis = s_mask[l * CH + j] != 0;
      else
        vis = t <= offset + l && (a.window <= 0 || t > offset + l - a.window);
      float s = -INFINITY;
      if (vis) {
        // four independent partial sums (shorter dependency chain)
        float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
        const float4* q = reinterpret_cast<const float4*>(qs + v * D);
        const float4* k = reinterpret_cast<const float4*>(ks + j * D);
#pragma unroll 4
        for (int i = 0; i < D / 4; ++i) {
          const float4 x = q[i], y = k[i];
          d0 = fmaf(x.x, y.x, d0);
          d1 = fmaf(x.y, y.y, d1);
          d2 = fmaf(x.z, y.z, d2);
          d3 = fmaf(x.w, y.w, d3);
        }
        s = a.scale * ((d0 + d1) + (d2 + d3));
      }
      sc[v * CH + j] = s;
    }
    __syncthreads();
    // online softmax update: G adjacent lanes per query vector (G = 256 / QV
    // rounded down to a power of two, at most 32), each lane a stride-G subset
    // of the chunk's keys; max and sum reduce within the group
    {
      const int G = qv_group;
      const int v = threadIdx.x / G, g = threadIdx.x % G;
      const bool active = v < QV;
      float sv[kAttnChunkMax / 1];
      float mx = -INFINITY;
      int cnt = 0;
      for (int j = g; j < n; j += G) {
        sv[cnt] = active ? sc[v * CH + j] : -INFINITY;
        mx = fmaxf(mx, sv[cnt]);
        ++cnt;
      }
      for (int o = 1; o < G; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_old = active ? s_m[v] : -INFINITY;
      const float m_new = fmaxf(m_old, mx);
      float alpha = 1.f, lsum = 0.f;
      if (m_new != -INFINITY) alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
      cnt = 0;
      for (int j = g; j < n; j += G) {
        const float p = (m_new == -INFINITY || sv[cnt] == -INFINITY) ? 0.f : expf(sv[cnt] - m_new);
        if (active) sc[v * CH + j] = p;
        lsum += p;
        ++cnt;
      }
      for (int o = 1; o < G; o <<= 1) lsum += __shfl_xor(lsum, o);
      if (active && g == 0) {
        s_m[v] = m_new;
        s_l[v] = s_l[v] * alpha + lsum;
        s_alpha[v] = alpha;
      }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < ACC; ++e) {
      const int idx = threadIdx.x + e * kAttnThreads;
      if (idx < QV * D) {
        const int v = idx / D, i = idx - v * D;
        float o = acc[e] * s_alpha[v];
        for (int j = 0; j < n; ++j) o = fmaf(sc[v * CH + j], vs[j * D + i], o);
        acc[e] = o;
      }
    }
    __syncthreads();
  }

  // this split's (m, l, o); an empty range leaves m = -inf, l = 0
  float* part = a.partial + (static_cast<int64_t>(kh) * S + split) * a.qv_ld * (D + 2);
#pragma unroll
  for (int e = 0; e < ACC; ++e) {
    const int idx = threadIdx.x + e * kAttnThreads;
    if (idx < QV * D) {
      const int v = idx / D, i = idx - v * D;
      part[v * (D + 2) + 2 + i] = acc[e];
    }
  }
  if (threadIdx.x < QV) {
    part[threadIdx.x * (D + 2)] = s_m[threadIdx.x];
    part[threadIdx.x * (D + 2) + 1] = s_l[threadIdx.x];
  }
}

// Merge the splits: one block per (vector, kv head), of kAttnThreads threads
// or of D >= 64 threads (thread t < D writes dim t).  Every load -- the splits'
// (m, l) and this vector's partial outputs -- is issued up front from
// addresses that do not depend on the row count; the block then exits if its
// vector is past the live rows.  Runs after k_attention (stream order), so
// plain loads see the partials.
template <int D, int FS = kMaxSplits>
__global__ __launch_bounds__(kAttnThreads) void k_attn_merge(AttnArgs a, int S) {
  constexpr int kPer = (D + kAttnThreads - 1) / kAttnThreads;  // elements per thread (D <= 256: 1)
  static_assert(kPer == 1, "head_dim up to the block size");
  static_assert(FS <= kWave, "one lane per split");
  __shared__ float s_w[FS];
  __shared__ float s_den;
  const int v = blockIdx.x, kh = blockIdx.y;
  const int rep = a.H / a.Hk;
  const int t = threadIdx.x;
  const float* base = a.partial + static_cast<int64_t>(kh) * S * a.qv_ld * (D + 2) + v * (D + 2);
  const int64_t kSplitStride = static_cast<int64_t>(a.qv_ld) * (D + 2);
  const int i = min(t, D - 1);
  float o[FS];
#pragma unroll
  for (int sp = 0; sp < FS; ++sp) o[sp] = base[min(sp, S - 1) * kSplitStride + 2 + i];
  float ms = -INFINITY, ls = 0.f;
  if (t < S) {
    ms = base[t * kSplitStride];
    ls = base[t * kSplitStride + 1];
  }
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  if (v >= nr * rep) return;  // uniform per block
  if (t < kWave) {  // wave 0, lane = split: weights exp(m_s - M) and the denominator
    const float M = wave_max(ms);
    const float wgt = ms == -INFINITY ? 0.f : expf(ms - M);
    const float den = wave_sum(ls * wgt);
    if (t < S) s_w[t] = wgt;
    if (t == 0) s_den = den;
  }
  __syncthreads();
  float num = 0.f;
#pragma unroll
  for (int sp = 0; sp < FS; ++sp)
    if (sp < S) num = fmaf(s_w[sp], o[sp], num);
  if (t < D) {
    const int l = v / rep, h = kh * rep + v % rep;
    const float y = num / s_den;
    a.out[l * a.ld_out + h * D + t] = y;
    if (a.xa_out) {
      const __bf16 hi = static_cast<__bf16>(y);
      a.xa_out[xa_index(l, h * D + t, 0)] = __builtin_bit_cast(uint16_t, hi);
      a.xa_out[xa_index(l, h * D + t, 1)] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(y - static_cast<float>(hi)));
    }
  }
}

// The merge launch: one thread per output dim where D fills whole waves, one
// load per split slot (16 slots when they cover the splits).
template <int D>
static void launch_merge(const AttnArgs& a, int qvb, int splits, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(qvb), a.Hk), block(D >= kWave && D % kWave == 0 ? D : kAttnThreads);
  if (splits <= 16)
    hipLaunchKernelGGL((k_attn_merge<D, 16>), grid, block, 0, stream, a, splits);
  else
    hipLaunchKernelGGL((k_attn_merge<D>), grid, block, 0, stream, a, splits);
}

// ------------------------------------------------------------------ decode-width attention

// Sum over groups of LK adjacent lanes (8, 16 or 32); every lane of a group
// receives its group's sum.
template <int LK>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_move<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);  // quad_perm [2,3,0,1]
  if constexpr (LK == 8) {
    v += dpp_move<0x141>(v);  // row_half_mirror: the other quad of the 8
  } else {
    v += dpp_move<0x124>(v);  // row_ror:4
    v += dpp_move<0x128>(v);  // row_ror:8
    if constexpr (LK == 32) v += __shfl_xor(v, 16);
  }
  return v;
}

// Few query vectors (rows x GQA group <= QVM), causal / sliding-window
// visibility, no explicit mask.  One block per (split, kv head); the split's
// keys go through in chunks of 32: the K and V rows of a chunk are loaded
// straight into registers (LK lanes per row, 16 bytes per lane, the next chunk
// requested as soon as the current one is consumed), scores are group sums of
// the lanes' partial dot products, V goes to LDS once for the
// probability-weighted sums.  q vectors and appended rows are normalised and
// rotated by the block while its first chunk is in flight.  With `ctr` (and
// QVM <= 4) the last split to finish for a kv head merges all splits of that
// head (device-coherent hand-over of the partials), so no merge launch
// follows; otherwise the partials go to k_attn_merge.
template <int D, typename KT, int QVM>
__global__ __launch_bounds__(kAttnThreads) void k_attn_decode(AttnArgs a) {
  constexpr int VE = 16 / static_cast<int>(sizeof(KT));  // cache elements per 16-byte load
  constexpr int LK = D / VE;                             // lanes per key row
  constexpr int KPB = kAttnThreads / LK;                 // key rows per block-wide load
  constexpr int CHK = 32;
  constexpr int NL = CHK / KPB;  // loads per thread and tensor per chunk
  constexpr int OPT = QVM * D / kAttnThreads > 0 ? QVM * D / kAttnThreads : 1;  // outputs per thread
  constexpr int VSTEP = kAttnThreads / D;                                         // v stride of a thread's outputs
  static_assert(LK == 8 || LK == 16 || LK == 32, "8, 16 or 32 lanes per key row");
  static_assert(NL >= 1 && NL * KPB == CHK, "whole key rows per chunk");
  static_assert(QVM * D >= kAttnThreads && D <= kAttnThreads, "at least one output per thread");
  __shared__ __attribute__((aligned(16))) float qs[QVM][D];
  __shared__ __attribute__((aligned(16))) float nks[QVM][D];  // appended rows of this block (cache-rounded)
  __shared__ __attribute__((aligned(16))) float nvs[QVM][D];
  __shared__ __attribute__((aligned(16))) float vls[CHK][D];
  __shared__ float s_p[QVM][CHK];
  __shared__ float s_m[QVM], s_l[QVM], s_alpha[QVM];
  // the merge's operands fit the registers for <= 4 query vectors (a fused
  // merge of 8 over half the splits measured slower than split + merge launch)
  constexpr bool kFuse = QVM <= 4;
  constexpr int kFS = kMaxSplits;
  __shared__ float s_w[kFuse ? QVM : 1][kFS];
  __shared__ float s_den[QVM];
  __shared__ bool s_last;

  if (a.clear_slots && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < kSlots)
    a.clear_slots[threadIdx.x * kSlotStride] = 0ull;
  const int kh = blockIdx.y, split = blockIdx.x, S = gridDim.x;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int rep = a.H / a.Hk;
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  const int offset = *a.offset_dev + a.offset_add;
  const int T = min(offset + nr, a.cap);
  const int QV = nr * rep;
  KT* kc = static_cast<KT*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  KT* vc = static_cast<KT*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  const int per = (T + S - 1) / S;
  const int kb = min(T, split * per), ke = min(T, kb + per);
  const int kr = t / LK, e0 = (t % LK) * VE;  // key row within a load, first element

  // 1. the first chunk in flight, then q vectors and appended rows
  uint4 kreg[NL], vreg[NL];
  const int64_t last_row = static_cast<int64_t>(a.cap) - 1;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t r = min(static_cast<int64_t>(kb + i * KPB + kr), last_row);
    kreg[i] = *reinterpret_cast<const uint4*>(kc + r * D + e0);
    vreg[i] = *reinterpret_cast<const uint4*>(vc + r * D + e0);
  }
  auto row_pos = [&](int l) {
    const int pos = a.positions ? a.positions[l] : offset + l;
    return min(max(pos, 0), a.rope_max - 1);
  };
  for (int v = wave; v < QV; v += kAttnThreads / kWave) {
    HeadVec<D> r;
    const int l = v / rep, h = kh * rep + v % rep;
    head_vec_load<D>(a.qkv + l * a.ld_qkv + h * D, a.q_gain, r);
    head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(l), r);
    head_vec_norm_rope<D>(r, a.eps);
#pragma unroll
    for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
      const int p = lane + e * kWave;
      if (p < D / 2) {
        qs[v][p] = r.lo[e];
        qs[v][p + D / 2] = r.hi[e];
      }
    }
  }
  for (int l = kAttnThreads / kWave - 1 - wave; l < nr; l += kAttnThreads / kWave) {
    const int tt = offset + l;
    if (tt < kb || tt >= ke) continue;
    HeadVec<D> r;
    head_vec_load<D>(a.qkv + l * a.ld_qkv + (a.H + kh) * D, a.k_gain, r);
    head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(l), r);
    const float* vsrc = a.qkv + l * a.ld_qkv + (a.H + a.Hk + kh) * D;
    head_vec_norm_rope<D>(r, a.eps);
#pragma unroll
    for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
      const int p = lane + e * kWave;
      if (p < D / 2) {
        nks[l][p] = kv_store<KT>(kc, static_cast<int64_t>(tt) * D + p, r.lo[e]);
        nks[l][p + D / 2] = kv_store<KT>(kc, static_cast<int64_t>(tt) * D + p + D / 2, r.hi[e]);
      }
    }
    for (int i = lane; i < D; i += kWave) nvs[l][i] = kv_store<KT>(vc, static_cast<int64_t>(tt) * D + i, vsrc[i]);
  }
  if (t < QVM) {
    s_m[t] = -INFINITY;
    s_l[t] = 0.f;
  }
  __syncthreads();

  float o[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) o[k] = 0.f;
  const int od = t % D, ov0 = t / D;  // outputs (ov0 + VSTEP k, od)

  for (int c0 = kb; c0 < ke; c0 += CHK) {
    const int n = min(CHK, ke - c0);
    // 2. scores of the chunk (group sums), V rows -> LDS as fp32
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int j = i * KPB + kr, tt = c0 + j;
      float kf[VE], vf[VE];
      if (tt >= offset) {
        const int l = min(tt - offset, QVM - 1);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          kf[e] = nks[l][e0 + e];
          vf[e] = nvs[l][e0 + e];
        }
      } else {
        unpack16<KT>(kreg[i], kf);
        unpack16<KT>(vreg[i], vf);
      }
#pragma unroll
      for (int e = 0; e < VE; e += 4)
        *reinterpret_cast<float4*>(&vls[j][e0 + e]) = make_float4(vf[e], vf[e + 1], vf[e + 2], vf[e + 3]);
#pragma unroll
      for (int v = 0; v < QVM; ++v) {
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
        const int l = v / rep;
        const bool vis = j < n && tt <= offset + l && (a.window <= 0 || tt > offset + l - a.window);
        if (t % LK == 0) s_p[v][j] = vis ? a.scale * d : -INFINITY;
      }
    }
    if (c0 + CHK < ke) {  // next chunk in flight during the softmax and the weighted sums
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int64_t r = min(static_cast<int64_t>(c0 + CHK + i * KPB + kr), last_row);
        kreg[i] = *reinterpret_cast<const uint4*>(kc + r * D + e0);
        vreg[i] = *reinterpret_cast<const uint4*>(vc + r * D + e0);
      }
    }
    lds_barrier();
    // 3. online softmax: 16 lanes per query vector, keys g and g + 16
    if (t < QVM * 16) {
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
    // 4. probability-weighted V rows
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
    if (c0 + CHK < ke) lds_barrier();  // vls / s_p are rewritten by the next chunk
  }

  // 5. this split's (m, l, o); an empty range leaves m = -inf, l = 0, o = 0
  float* part = a.partial + (static_cast<int64_t>(kh) * S + split) * a.qv_ld * (D + 2);
  const bool fused = kFuse && a.ctr != nullptr;
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float* pv = part + v * (D + 2);
    if (fused) {
      publish_f32(pv + 2 + od, o[k]);
      if (od == 0) {
        publish_f32(pv, s_m[v]);
        publish_f32(pv + 1, s_l[v]);
      }
    } else {
      pv[2 + od] = o[k];
      if (od == 0) {
        pv[0] = s_m[v];
        pv[1] = s_l[v];
      }
    }
  }
  if constexpr (kFuse) {
  if (!fused) return;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    unsigned int* ctr = a.ctr + kh * kCounterStride;
    const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      static_cast<unsigned int>(S - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;

  // 6. last split of this kv head: merge every split's (m, l, o)
  const float* base = a.partial + static_cast<int64_t>(kh) * S * a.qv_ld * (D + 2);
  const int64_t sstride = static_cast<int64_t>(a.qv_ld) * (D + 2);
  // every partial loaded from clamped addresses before any is used
  float ov[OPT][kFS];
#pragma unroll
  for (int k = 0; k < OPT; ++k)
#pragma unroll
    for (int sp = 0; sp < kFS; ++sp)
      ov[k][sp] = fetch_f32(base + min(sp, S - 1) * sstride + min(ov0 + VSTEP * k, max(QV - 1, 0)) * (D + 2) + 2 + od);
  constexpr int kNw = kAttnThreads / kWave;
  float ms[(QVM + kNw - 1) / kNw], ls[(QVM + kNw - 1) / kNw];
#pragma unroll
  for (int q = 0; q < (QVM + kNw - 1) / kNw; ++q) {  // wave w: query vectors w, w + 4, ...; lane = split
    const int v = min(wave + q * kNw, max(QV - 1, 0));
    ms[q] = fetch_f32(base + min(lane, S - 1) * sstride + v * (D + 2));
    ls[q] = fetch_f32(base + min(lane, S - 1) * sstride + v * (D + 2) + 1);
  }
#pragma unroll
  for (int q = 0; q < (QVM + kNw - 1) / kNw; ++q) {
    const int v = wave + q * kNw;
    if (v >= QV || v >= QVM) continue;  // wave-uniform
    const float m_s = lane < S ? ms[q] : -INFINITY;
    const float M = wave_max_dpp(m_s);
    const float wgt = m_s == -INFINITY ? 0.f : expf(m_s - M);
    const float den = wave_sum_dpp(lane < S ? ls[q] * wgt : 0.f);
    if (lane < kFS) s_w[v][lane] = lane < S ? wgt : 0.f;
    if (lane == 0) s_den[v] = den;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float num = 0.f;
#pragma unroll
    for (int sp = 0; sp < kFS; ++sp) num = fmaf(s_w[v][sp], sp < S ? ov[k][sp] : 0.f, num);
    const float y = num / s_den[v];
    const int l = v / rep, h = kh * rep + v % rep;
    a.out[l * a.ld_out + h * D + od] = y;
    if (a.xa_out) {
      const __bf16 hi = static_cast<__bf16>(y);
      a.xa_out[xa_index(l, h * D + od, 0)] = __builtin_bit_cast(uint16_t, hi);
      a.xa_out[xa_index(l, h * D + od, 1)] =
          __builtin_bit_cast(uint16_t, static_cast<__bf16>(y - static_cast<float>(hi)));
    }
  }
  }  // kFuse
}

// Decode attention over fixed key ranges, for up to 4 query vectors with the
// merge fused: split s of kv head kh owns keys [s * per, s * per + per), per =
// a multiple of 32 chosen from the capacity, so every block requests its first
// CPS chunks of K and V, its raw q row and appended k / v rows at entry, before
// the offset (and with it the live length) has been read; later chunks follow
// in a ring of CPS register slots, each refilled as soon as its chunk is
// consumed.  Splits whose range starts past the live length skip the work.
// The appended rows are rounded into LDS at once and stored to the cache after
// the chunks, so no wait in the chunk loop covers those stores.  The chunk
// math is latency-bound (a wave or two per SIMD), so blocks of one-chunk
// splits have 512 threads (two waves per SIMD), others 256, and the math is
// written as independent chains: the four query vectors' dot products side by side
// (vectors past the live count are computed and masked), and the weighted V
// sums over all 32 keys with every LDS read issued first (rows past the chunk
// end are zero, their probabilities too).  The last split of a kv head to
// finish merges the live splits in one round of 16-byte coherent loads (wave v
// takes query vector v; a lane holds 4 dims of every other split).
constexpr int kFxMaxSplits = 64;
constexpr int kFxMaxRows = 8;  // rows of one launch (appended rows held in LDS)
constexpr int kFxThreads = 512;  // block size of the one-chunk splits
constexpr int kFxRec = 132;  // floats per (split, vector) record: o[128], m, l, 2 pad (16-byte multiple)

// 16-byte device-coherent load from a buffer resource; reads past num_records
// return zeros without a memory access.
__device__ __forceinline__ float4 fetch_f32x4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16 /* sc1 */));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}


typedef __bf16 abf16x8 __attribute__((ext_vector_type(8)));
typedef float af32x4 __attribute__((ext_vector_type(4)));
// operands of ds_read_b64_tr_b16: within each 16-lane group, lane i receives
// element i % 4 of the 8-byte reads of lanes i / 4 + 4 e (e = 0..3)
typedef short vs16x4 __attribute__((ext_vector_type(4)));
typedef short vs16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) vs16x4 lds_vs16x4;

// keys [0, k) of a 64-key chunk as bits
__device__ __forceinline__ uint64_t low_bits64(int k) {
  return k >= 64 ? ~0ull : k <= 0 ? 0ull : (1ull << k) - 1;
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(b))) << 16);
}

// 8 fp32 -> bf16 hi (round to nearest) and lo (the rounding remainder, rounded):
// hi + lo equals x to ~2^-17 relative, so bf16 MFMA products keep fp32 accuracy.
__device__ __forceinline__ void split8(const float* x, uint4& hi, uint4& lo) {
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = x[e] - static_cast<float>(static_cast<__bf16>(x[e]));
  hi = make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]), pack2_bf16(x[4], x[5]), pack2_bf16(x[6], x[7]));
  lo = make_uint4(pack2_bf16(r[0], r[1]), pack2_bf16(r[2], r[3]), pack2_bf16(r[4], r[5]), pack2_bf16(r[6], r[7]));
}
__device__ __forceinline__ void split8(const float* x, abf16x8& hi, abf16x8& lo) {
  uint4 h, l;
  split8(x, h, l);
  hi = __builtin_bit_cast(abf16x8, h);
  lo = __builtin_bit_cast(abf16x8, l);
}

// This split's (m, l, o) records of the fixed-range decode kernels, handed
// over coherently (outputs (ov0 + VSTEP k, od) of thread t, ov0 = t / 128).
template <int OPT, int VSTEP>
__device__ __forceinline__ void fx_publish(const AttnArgs& a, const float* o, const float* s_m, const float* s_l,
                                           int QV, int64_t rec) {
  constexpr int D = 128, QVM = 4;
  const int t = threadIdx.x, od = t % D, ov0 = t / D;
  float* part = a.partial + rec * QVM * kFxRec;
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int v = ov0 + VSTEP * k;
    if (v >= QV) break;
    float* pv = part + v * kFxRec;
    publish_f32(pv + od, o[k]);
    if (od == 0) {
      publish_f32(pv + D, s_m[v]);
      publish_f32(pv + D + 1, s_l[v]);
    }
  }
}

// Split counter of this (kv head, row group) -- group g = kh * Z + z; the
// last split to arrive merges the SL live splits in one round of coherent
// 16-byte loads (records of splits >= SL lie past the resource's range and
// read as zeros): wave v takes query vector v (row lz0 + v / rep), lane j split
// j's (m, l), and each lane 4 dims of every other split.
__device__ __forceinline__ void fx_merge(const AttnArgs& a, float (*s_w)[kFxMaxSplits], bool& s_last, int T, int per,
                                         int QV, int rep, int lz0) {
  constexpr int D = 128, QVM = 4;
  const int kh = blockIdx.y, S = gridDim.x, g = blockIdx.y * gridDim.z + blockIdx.z;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    unsigned int* ctr = a.ctr + g * kCounterStride;
    const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      static_cast<unsigned int>(S - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  const int SL = min(S, (T + per - 1) / per);
  if (wave >= QV || SL <= 0) return;  // wave-uniform
  const int rec_bytes = QVM * kFxRec * 4;  // one split's records
  const __amdgpu_buffer_rsrc_t rs =
      buffer_rsrc(a.partial + static_cast<int64_t>(g) * S * QVM * kFxRec, SL * rec_bytes);
  const int half = lane / 32, d4 = lane % 32;
  float4 ov[kFxMaxSplits / 2];
#pragma unroll
  for (int jj = 0; jj < kFxMaxSplits / 2; ++jj)
    ov[jj] = fetch_f32x4(rs, (2 * jj + half) * rec_bytes + wave * kFxRec * 4 + 16 * d4);
  const float4 ml = fetch_f32x4(rs, lane * rec_bytes + wave * kFxRec * 4 + 4 * D);  // (m, l, pad, pad)
  const float m_s = lane < SL ? ml.x : -INFINITY;
  const float M = wave_max_dpp(m_s);
  const float wgt = m_s == -INFINITY ? 0.f : expf(m_s - M);
  const float den = wave_sum_dpp(lane < SL ? ml.y * wgt : 0.f);
  s_w[wave][lane] = wgt;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int jj = 0; jj < kFxMaxSplits / 2; ++jj) {
    const float w = s_w[wave][2 * jj + half];
    num.x = fmaf(w, ov[jj].x, num.x);
    num.y = fmaf(w, ov[jj].y, num.y);
    num.z = fmaf(w, ov[jj].z, num.z);
    num.w = fmaf(w, ov[jj].w, num.w);
  }
  num.x += __shfl_xor(num.x, 32);
  num.y += __shfl_xor(num.y, 32);
  num.z += __shfl_xor(num.z, 32);
  num.w += __shfl_xor(num.w, 32);
  if (half) return;
  const int l = lz0 + wave / rep, h = kh * rep + wave % rep;
  const float y[4] = {num.x / den, num.y / den, num.z / den, num.w / den};
  *reinterpret_cast<float4*>(a.out + l * a.ld_out + h * D + 4 * d4) = make_float4(y[0], y[1], y[2], y[3]);
  if (a.xa_out) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = h * D + 4 * d4 + q;
      const __bf16 hi = static_cast<__bf16>(y[q]);
      a.xa_out[xa_index(l, col, 0)] = __builtin_bit_cast(uint16_t, hi);
      a.xa_out[xa_index(l, col, 1)] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(y[q] - static_cast<float>(hi)));
    }
  }
}

template <int D, typename KT, int CPS, int NT>
__global__ __launch_bounds__(NT) void k_attn_decode_fx(AttnArgs a, int per) {
  constexpr int QVM = 4;
  constexpr int VE = 16 / static_cast<int>(sizeof(KT));
  constexpr int LK = D / VE;
  constexpr int KPB = NT / LK;
  constexpr int CHK = 32;
  constexpr int NL = CHK / KPB;
  constexpr int OPT = QVM * D / NT;
  constexpr int VSTEP = NT / D;
  static_assert(D == 128 && kFxRec >= D + 2 && kFxRec % 4 == 0, "record layout");
  static_assert(LK == 16 || LK == 32, "16 or 32 lanes per key row");
  static_assert(NL >= 1 && NL * KPB == CHK, "whole key rows per chunk");
  static_assert(NT / kWave >= QVM && OPT >= 1, "a wave per query vector, an output per thread");
  __shared__ __attribute__((aligned(16))) float qs[QVM][D];
  __shared__ __attribute__((aligned(16))) float nks[kFxMaxRows][D];  // appended rows (cache-rounded)
  __shared__ __attribute__((aligned(16))) float nvs[kFxMaxRows][D];
  __shared__ __attribute__((aligned(16))) float vls[CHK][D];
  __shared__ __attribute__((aligned(16))) float s_p[QVM][CHK];
  __shared__ float s_m[QVM], s_l[QVM], s_alpha[QVM];
  __shared__ float s_w[QVM][kFxMaxSplits];
  __shared__ uint8_t s_mk[CPS][QVM][CHK];  // explicit mask bytes of the group's rows, chunk by chunk
  __shared__ bool s_last;

  const int kh = blockIdx.y, split = blockIdx.x;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  KT* kc = static_cast<KT*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  KT* vc = static_cast<KT*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  const int kb = split * per;
  const int kr = t / LK, e0 = (t % LK) * VE;
  const int64_t last_row = static_cast<int64_t>(a.cap) - 1;
  const int rep = a.H / a.Hk;
  // row group z of the block: rows lz0 .. lz0 + rpz - 1 (rep query vectors each)
  const int z = blockIdx.z, rpz = QVM / rep, lz0 = z * rpz;
  constexpr int NW = NT / kWave;
  constexpr int RPW = (kFxMaxRows + NW - 1) / NW;  // appended rows per wave (rows w, w + NW, ...)

  // 0. the offset and the live row count, requested before anything else
  const int off_raw = *a.offset_dev;
  const int nr_raw = *(a.n_rows_dev ? a.n_rows_dev : a.offset_dev);
  if (a.clear_slots && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && t < kSlots)
    a.clear_slots[t * kSlotStride] = 0ull;

  // 1. in flight at entry: the split's first CPS chunks, the raw q vector of
  // this wave (v = wave) and the raw k / v rows of rows wave + NW i
  uint4 kreg[CPS][NL], vreg[CPS][NL];
#pragma unroll
  for (int c = 0; c < CPS; ++c)
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int64_t r = min(static_cast<int64_t>(kb + c * CHK + i * KPB + kr), last_row);
      kreg[c][i] = *reinterpret_cast<const uint4*>(kc + r * D + e0);
      vreg[c][i] = *reinterpret_cast<const uint4*>(vc + r * D + e0);
    }
  // with an explicit mask (every chunk of the split in flight: no ring), its
  // bytes for the group's rows: thread t row t / 32, key t % 32 of each chunk;
  // one register per byte (packing them would wait for the loads here), and
  // loaded without a branch (without a mask from the offset word, unused): a
  // conditional load becomes a select whose other arm waits for the chunk loads
  uint32_t mb[CPS];
  {
    const int mr = min(lz0 + (t / CHK) % QVM, a.rows - 1);
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      const uint8_t* mp = a.mask ? a.mask + static_cast<int64_t>(mr) * a.mask_ld +
                                       min(static_cast<int64_t>(kb + c * CHK + t % CHK), a.mask_ld - 1)
                                 : reinterpret_cast<const uint8_t*>(a.offset_dev);
      mb[c] = *mp;
    }
  }
  const int vq = wave, lq = min(lz0 + vq / rep, a.rows - 1), hq = kh * rep + vq % rep;
  HeadVec<D> rq;
  head_vec_load<D>(a.qkv + lq * a.ld_qkv + hq * D, a.q_gain, rq);
  HeadVec<D> rk[RPW];
  float vraw[RPW][D / kWave];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int lk = min(wave + NW * r, a.rows - 1);
    head_vec_load<D>(a.qkv + lk * a.ld_qkv + (a.H + kh) * D, a.k_gain, rk[r]);
    const float* vsrc = a.qkv + lk * a.ld_qkv + (a.H + a.Hk + kh) * D;
#pragma unroll
    for (int i = 0; i < D / kWave; ++i) vraw[r][i] = vsrc[lane + i * kWave];
  }

  const int nr = a.n_rows_dev ? min(max(nr_raw, 0), a.rows) : a.rows;
  const int offset = off_raw + a.offset_add;
  const int T = min(offset + nr, a.cap);
  const int nlast = min(nr, lz0 + rpz);           // rows 0 .. nlast - 1 are visible to this group
  const int nvis = a.mask ? nr : nlast;           // appended rows the group may see (a mask may show any)
  const int QV = max(0, nlast - lz0) * rep;       // live query vectors of this group
  const int ke = min(T, kb + per);
  const bool live = kb < ke && QV > 0;

  if (live) {
    auto row_pos = [&](int l) {
      const int pos = a.positions ? a.positions[l] : offset + l;
      return min(max(pos, 0), a.rope_max - 1);
    };
    if (vq < QV) {
      head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(lq), rq);
      head_vec_norm_rope<D>(rq, a.eps);
#pragma unroll
      for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
        const int p = lane + e * kWave;
        if (p < D / 2) {
          qs[vq][p] = rq.lo[e];
          qs[vq][p + D / 2] = rq.hi[e];
        }
      }
    }
    // appended rows of this split's key range that the group's rows see
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int l = wave + NW * r, tk = offset + l;
      if (!(l < nvis && tk >= kb && tk < ke)) continue;  // wave-uniform
      head_vec_rope_load<D>(a.rope_cos, a.rope_sin, row_pos(l), rk[r]);
      head_vec_norm_rope<D>(rk[r], a.eps);
#pragma unroll
      for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
        const int p = lane + e * kWave;
        if (p < D / 2) {
          nks[l][p] = kv_round<KT>(rk[r].lo[e]);
          nks[l][p + D / 2] = kv_round<KT>(rk[r].hi[e]);
        }
      }
#pragma unroll
      for (int i = 0; i < D / kWave; ++i) nvs[l][lane + i * kWave] = kv_round<KT>(vraw[r][i]);
    }
    if (t < QVM) {
      s_m[t] = -INFINITY;
      s_l[t] = 0.f;
    }
    if (a.mask && t < QVM * CHK) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) s_mk[c][t / CHK][t % CHK] = static_cast<uint8_t>(mb[c]);
    }
    __syncthreads();

    float o[OPT];
#pragma unroll
    for (int k = 0; k < OPT; ++k) o[k] = 0.f;
    const int od = t % D, ov0 = t / D;

    for (int g0 = kb; g0 < ke; g0 += CPS * CHK) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) {
        const int c0 = g0 + c * CHK;
        if (c0 >= ke) break;  // block-uniform
        const int n = min(CHK, ke - c0);
        // 2. scores of the chunk (group sums of the four vectors side by side), V rows -> LDS
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          const int j = i * KPB + kr, tt = c0 + j;
          float kf[VE], vf[VE];
          unpack16<KT>(kreg[c][i], kf);
          unpack16<KT>(vreg[c][i], vf);
          if (tt >= offset) {  // appended rows: this launch's values (zero past the group's last row)
            const int l = min(tt - offset, kFxMaxRows - 1);
            const bool mine = tt - offset < nvis;
#pragma unroll
            for (int e = 0; e < VE; ++e) {
              kf[e] = mine ? nks[l][e0 + e] : 0.f;
              vf[e] = mine ? nvs[l][e0 + e] : 0.f;
            }
          }
          if (j >= n) {
#pragma unroll
            for (int e = 0; e < VE; ++e) vf[e] = 0.f;
          }
#pragma unroll
          for (int e = 0; e < VE; e += 4)
            *reinterpret_cast<float4*>(&vls[j][e0 + e]) = make_float4(vf[e], vf[e + 1], vf[e + 2], vf[e + 3]);
          float d0[QVM], d1[QVM];
#pragma unroll
          for (int v = 0; v < QVM; ++v) {
            d0[v] = 0.f;
            d1[v] = 0.f;
          }
#pragma unroll
          for (int e = 0; e < VE; e += 4) {
#pragma unroll
            for (int v = 0; v < QVM; ++v) {
              const float4 q = *reinterpret_cast<const float4*>(&qs[v][e0 + e]);
              d0[v] = fmaf(kf[e], q.x, d0[v]);
              d1[v] = fmaf(kf[e + 1], q.y, d1[v]);
              d0[v] = fmaf(kf[e + 2], q.z, d0[v]);
              d1[v] = fmaf(kf[e + 3], q.w, d1[v]);
            }
          }
          float dv[QVM];
#pragma unroll
          for (int v = 0; v < QVM; ++v) dv[v] = group_sum<LK>(d0[v] + d1[v]);
          if (t % LK == 0) {
#pragma unroll
            for (int v = 0; v < QVM; ++v) {
              const int l = lz0 + v / rep;
              const bool seen = a.mask ? s_mk[c][v / rep][j] != 0
                                       : tt <= offset + l && (a.window <= 0 || tt > offset + l - a.window);
              const bool vis = v < QV && j < n && seen;
              s_p[v][j] = vis ? a.scale * dv[v] : -INFINITY;
            }
          }
        }
        // the slot's next chunk in flight during the softmax and the weighted sums
        if (c0 + CPS * CHK < ke) {
#pragma unroll
          for (int i = 0; i < NL; ++i) {
            const int64_t r = min(static_cast<int64_t>(c0 + CPS * CHK + i * KPB + kr), last_row);
            kreg[c][i] = *reinterpret_cast<const uint4*>(kc + r * D + e0);
            vreg[c][i] = *reinterpret_cast<const uint4*>(vc + r * D + e0);
          }
        }
        lds_barrier();
        // 3. online softmax: 16 lanes per query vector, keys g and g + 16
        if (t < QVM * 16) {
          const int v = t / 16, g = t % 16;
          const float s0 = s_p[v][g];
          const float s1 = s_p[v][g + 16];
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
        // 4. probability-weighted V rows: every read first, four accumulators
#pragma unroll
        for (int k = 0; k < OPT; ++k) {
          const int v = ov0 + VSTEP * k;
          float vv[CHK];
#pragma unroll
          for (int j = 0; j < CHK; ++j) vv[j] = vls[j][od];
          float4 pp[CHK / 4];
#pragma unroll
          for (int j = 0; j < CHK / 4; ++j) pp[j] = *reinterpret_cast<const float4*>(&s_p[v][4 * j]);
          float acc[4] = {o[k] * s_alpha[v], 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < CHK / 4; ++j) {
            acc[0] = fmaf(pp[j].x, vv[4 * j], acc[0]);
            acc[1] = fmaf(pp[j].y, vv[4 * j + 1], acc[1]);
            acc[2] = fmaf(pp[j].z, vv[4 * j + 2], acc[2]);
            acc[3] = fmaf(pp[j].w, vv[4 * j + 3], acc[3]);
          }
          o[k] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        }
        lds_barrier();  // vls / s_p are rewritten by the next chunk
      }
    }

    // the appended rows into the cache (after the chunks, so no wait in the
    // chunk loop covers these stores), each by the group holding its row; the
    // lanes that wrote nks / nvs read them
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int l = wave + NW * r, tk = offset + l;
      if (!(l < nlast && l >= lz0 && tk >= kb && tk < ke)) continue;  // wave-uniform
#pragma unroll
      for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
        const int p = lane + e * kWave;
        if (p < D / 2) {
          kv_put<KT>(kc, static_cast<int64_t>(tk) * D + p, nks[l][p]);
          kv_put<KT>(kc, static_cast<int64_t>(tk) * D + p + D / 2, nks[l][p + D / 2]);
        }
      }
#pragma unroll
      for (int i = 0; i < D / kWave; ++i)
        kv_put<KT>(vc, static_cast<int64_t>(tk) * D + lane + i * kWave, nvs[l][lane + i * kWave]);
    }
    fx_publish<OPT, VSTEP>(a, o, s_m, s_l, QV,
                           (static_cast<int64_t>(kh) * gridDim.z + z) * gridDim.x + split);
  }
  fx_merge(a, s_w, s_last, T, per, QV, rep, lz0);
}

// ------------------------------------------------------------------ decode attention on the matrix cores
// One query row (a draft step) with up to four query vectors per kv head,
// head_dim 128, bf16 cache, causal with no mask or window -- the long-context
// case, where the fixed-range kernel above runs several dependent 32-key
// chunks per split on the vector ALUs.  Block (split, kv head) of four waves;
// split s owns keys [s per, s per + per) (per = 4 KPW, fixed by the capacity),
// and wave w the KPW-key chunk s per + KPW w, all four independent until their
// (m, l, o) meet in LDS.  The launch uses KPW = 64 (32 keys per wave, twice
// the splits, measured slower: the merge reads twice the records), from a
// capacity of 1024 (Qwen3-1.7B step: 52.7 against 53.4 us at context 1024 and
// against 54.1 at 2048; 52.3 against 49.8 at 512, where the fixed-range kernel
// stays).  A wave's chunk is requested at entry: its K straight
// into v_mfma_f32_16x16x32_bf16 A fragments (lane l: key 16 kt + l % 16, dims
// 32 st + 8 (l / 16) .. + 8) and its V rows, which go to the wave's own LDS
// region as [key][d].  The block normalises and rotates q (the B operand,
// split into bf16 hi + lo, scaled into base 2) and the appended row, which
// replaces the cache row in the wave holding it (the cache gets it at the
// end).  S^T = K Q^T leaves each lane one query vector (l % 16; lanes past the
// group's vectors see nothing) and keys 16 kt + 4 (l / 16) + e; the softmax
// runs on those 16 values and two cross-group shuffles, and O^T = V^T P^T
// takes P^T from the registers with the V^T fragments read by transposing LDS
// reads in the same key order.  The block's record goes to the last split of
// the kv head (fx_publish / fx_merge), so no merge launch follows.
constexpr int kMfNW = 4;              // waves per block
constexpr int kMfLdV = 128 + 16;      // row stride (bf16) of a wave's V chunk
// Capacities below kMfMinCap keep the fixed-range kernel.  Both kernels size
// their grids from the capacity (the live length is on the device), and this
// one takes 256 keys per block: at capacity 1024 that is 4 splits per kv head,
// so a 513-key context runs on 16 blocks of the 32 (10.5 us against 6.7 on
// the fixed-range kernel's 32-key splits); at 4112 it is 17 splits (4097 keys:
// 11.7 against 16.5 us)
constexpr int kMfMinCap = 2048;

__device__ __forceinline__ uint4 mf_pack8(const float* x) {
  return make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]), pack2_bf16(x[4], x[5]), pack2_bf16(x[6], x[7]));
}

template <int D, int KPW>
__global__ __launch_bounds__(256) void k_attn_decode_mf(AttnArgs a) {
  static_assert(D == 128, "head_dim 128: two 64-dim halves per lane pair, 16-dim MFMA tiles");
  static_assert(KPW == 32 || KPW == 64, "32 or 64 keys per wave: whole 32-key blocks of the V^T product");
  constexpr int QVM = 4, NW = kMfNW, CH = KPW, KTL = KPW / 16, NVR = KPW / 4, PER = NW * KPW;
  constexpr int OPT = QVM * D / 256, VSTEP = 256 / D;  // the record layout of fx_publish
  __shared__ __attribute__((aligned(16))) uint16_t vsb[NW][CH * kMfLdV];  // each wave's V rows [key][d]
  __shared__ __attribute__((aligned(16))) float qs[QVM][D];              // q, normalised, rotated, base-2 scaled
  __shared__ __attribute__((aligned(16))) float nkv[2][D];               // the appended row's k and v (cache-rounded)
  __shared__ __attribute__((aligned(16))) float s_wo[NW][QVM][D];        // each wave's o
  __shared__ float s_wm[NW][QVM], s_wl[NW][QVM];
  __shared__ float s_m[QVM], s_l[QVM];
  __shared__ float s_w[QVM][kFxMaxSplits];
  __shared__ bool s_last;

  const int kh = blockIdx.y, split = blockIdx.x;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int kl = lane % 16, gq = lane / 16;
  const int rep = a.H / a.Hk;
  const int kb = split * PER, c0 = kb + CH * wave;

  // 0. the offset, requested before anything else
  const int off_raw = *a.offset_dev;
  if (a.clear_slots && blockIdx.x == 0 && blockIdx.y == 0 && t < kSlots) a.clear_slots[t * kSlotStride] = 0ull;

  // 1. in flight at entry: the wave's K fragments and V rows (rows past the
  // capacity read as zeros), this wave's raw q vector (v = wave) and the raw
  // k / v of the appended row (every wave loads them: no load behind a branch)
  const __amdgpu_buffer_rsrc_t kr =
      buffer_rsrc(static_cast<const uint16_t*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D, a.cap * D * 2);
  const __amdgpu_buffer_rsrc_t vr =
      buffer_rsrc(static_cast<const uint16_t*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D, a.cap * D * 2);
  uint4 kf[KTL][4], vrow[NVR];
#pragma unroll
  for (int kt = 0; kt < KTL; ++kt)
#pragma unroll
    for (int st = 0; st < 4; ++st)
      kf[kt][st] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, ((c0 + 16 * kt + kl) * D + 32 * st + 8 * gq) * 2, 0, 0));
#pragma unroll
  for (int i = 0; i < NVR; ++i)  // key c0 + l / 16 + 4 i, dims 8 (l % 16) .. + 8
    vrow[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, ((c0 + gq + 4 * i) * D + 8 * kl) * 2, 0, 0));
  const int vq = wave, hq = kh * rep + min(vq, rep - 1);
  HeadVec<D> rq, rk;
  head_vec_load<D>(a.qkv + hq * D, a.q_gain, rq);
  head_vec_load<D>(a.qkv + (a.H + kh) * D, a.k_gain, rk);
  float vraw[D / kWave];
#pragma unroll
  for (int i = 0; i < D / kWave; ++i) vraw[i] = a.qkv[(a.H + a.Hk + kh) * D + lane + i * kWave];

  const int offset = off_raw + a.offset_add;
  const int T = min(offset + 1, a.cap);
  const int ke = min(T, kb + PER);
  uint16_t* kc = static_cast<uint16_t*>(a.kc) + static_cast<int64_t>(kh) * a.cap * D;
  uint16_t* vc = static_cast<uint16_t*>(a.vc) + static_cast<int64_t>(kh) * a.cap * D;
  const bool holds = kb <= offset && offset < ke;  // this split holds the appended row
  if (kb < ke) {
    const int pos = min(max(a.positions ? a.positions[0] : offset, 0), a.rope_max - 1);
    if (vq < rep) {
      head_vec_rope_load<D>(a.rope_cos, a.rope_sin, pos, rq);
      head_vec_norm_rope<D>(rq, a.eps);
      const float sc = a.scale * 1.4426950408889634f;
#pragma unroll
      for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
        const int p = lane + e * kWave;
        if (p < D / 2) {
          qs[vq][p] = rq.lo[e] * sc;
          qs[vq][p + D / 2] = rq.hi[e] * sc;
        }
      }
    }
    if (holds && wave == 0) {
      head_vec_rope_load<D>(a.rope_cos, a.rope_sin, pos, rk);
      head_vec_norm_rope<D>(rk, a.eps);
#pragma unroll
      for (int e = 0; e < HeadVec<D>::kPPL; ++e) {
        const int p = lane + e * kWave;
        if (p < D / 2) {
          nkv[0][p] = kv_round<uint16_t>(rk.lo[e]);
          nkv[0][p + D / 2] = kv_round<uint16_t>(rk.hi[e]);
        }
      }
#pragma unroll
      for (int i = 0; i < D / kWave; ++i) nkv[1][lane + i * kWave] = kv_round<uint16_t>(vraw[i]);
    }
    lds_barrier();  // q and the appended row in LDS; the chunk loads stay in flight

    // q as the B operand: lane (kl, gq) supplies vector kl (zero past the
    // group's vectors), dims 32 st + 8 gq .. + 8
    abf16x8 qh[4], ql[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = kl < rep ? qs[min(kl, QVM - 1)][32 * st + 8 * gq + e] : 0.f;
      split8(x, qh[st], ql[st]);
    }
    float m_r = -INFINITY, l_r = 0.f;
    af32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = af32x4{0.f, 0.f, 0.f, 0.f};
    const int n = min(CH, ke - c0);  // the wave's live keys (none when its chunk starts past them)
    if (n > 0) {
      const int jr = offset - c0;  // the appended row's key within the chunk
      if (jr >= 0 && jr < CH) {
#pragma unroll
        for (int kt = 0; kt < KTL; ++kt)
          if (16 * kt + kl == jr) {
#pragma unroll
            for (int st = 0; st < 4; ++st) kf[kt][st] = mf_pack8(&nkv[0][32 * st + 8 * gq]);
          }
#pragma unroll
        for (int i = 0; i < NVR; ++i)
          if (gq + 4 * i == jr) vrow[i] = mf_pack8(&nkv[1][8 * kl]);
      }
      if (n < CH) {  // V rows past the live keys zeroed (the cache there may hold anything; P is 0 for them)
#pragma unroll
        for (int i = 0; i < NVR; ++i)
          if (gq + 4 * i >= n) vrow[i] = make_uint4(0, 0, 0, 0);
      }
      uint16_t* vw = vsb[wave];
#pragma unroll
      for (int i = 0; i < NVR; ++i) *reinterpret_cast<uint4*>(vw + (gq + 4 * i) * kMfLdV + 8 * kl) = vrow[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      // S^T, four independent key tiles
      af32x4 sacc[KTL];
#pragma unroll
      for (int kt = 0; kt < KTL; ++kt) sacc[kt] = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
#pragma unroll
        for (int kt = 0; kt < KTL; ++kt)
          sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(abf16x8, kf[kt][st]), qh[st], sacc[kt], 0, 0, 0);
#pragma unroll
        for (int kt = 0; kt < KTL; ++kt)
          sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(abf16x8, kf[kt][st]), ql[st], sacc[kt], 0, 0, 0);
      }
      // every key of the chunk is at or before the query's position
      const uint64_t bits = kl < rep ? low_bits64(n) : 0ull;
      const uint32_t blo = static_cast<uint32_t>(bits), bhi = static_cast<uint32_t>(bits >> 32);
      mfma_settle();
      float sv[KTL][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < KTL; ++kt) {
        const uint32_t nib = __builtin_amdgcn_ubfe(kt < 2 ? blo : bhi, (kt & 1) * 16 + 4 * gq, 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[kt][e] = (nib >> e) & 1u ? sacc[kt][e] : -INFINITY;
          mx = fmaxf(mx, sv[kt][e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      m_r = mx;
      const float mb = mx == -INFINITY ? 0.f : mx;
      float p[KTL][4], rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < KTL; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[kt][e] = __builtin_amdgcn_exp2f(sv[kt][e] - mb);
          rs += p[kt][e];
        }
      rs += __shfl_xor(rs, 16);
      rs += __shfl_xor(rs, 32);
      l_r = rs;
      // O^T = V^T P^T over the two 32-key blocks; the lane's transposing reads:
      // source lane 4 e + a of its group points at key 32 kk + 4 g + e, dims
      // 16 dt + 4 a .. + 3 (and the same 16 keys further)
      const int vr0 = 4 * gq + kl / 4, vc0 = 4 * (kl % 4);
#pragma unroll
      for (int kk = 0; kk < KTL / 2; ++kk) {
        const float px[8] = {p[2 * kk][0], p[2 * kk][1], p[2 * kk][2], p[2 * kk][3],
                             p[2 * kk + 1][0], p[2 * kk + 1][1], p[2 * kk + 1][2], p[2 * kk + 1][3]};
        abf16x8 ph, pl;
        split8(px, ph, pl);
        abf16x8 va[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          uint16_t* vp = vw + (kk * 32 + vr0) * kMfLdV + dt * 16 + vc0;
          const vs16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_vs16x4*)(vp));
          const vs16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_vs16x4*)(vp + 16 * kMfLdV));
          va[dt] = __builtin_bit_cast(abf16x8, vs16x8{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]});
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], ph, o[dt], 0, 0, 0);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pl, o[dt], 0, 0, 0);
      }
      mfma_settle();
    }
    // the wave's (m, l, o): lane (kl, gq) holds O^T[16 dt + 4 gq + e][vector kl]
    if (kl < QVM) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<float4*>(&s_wo[wave][kl][16 * dt + 4 * gq]) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
      if (gq == 0) {
        s_wm[wave][kl] = m_r;
        s_wl[wave][kl] = l_r;
      }
    }
    __syncthreads();
    // the block's record (thread: vectors ov0 + VSTEP k, dim od), m in natural units
    float ob[OPT];
    const int od = t % D, ov0 = t / D;
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int v = ov0 + VSTEP * k;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w][v]);
      float acc = 0.f, ls = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = s_wm[w][v];
        const float wt = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        acc = fmaf(wt, s_wo[w][v][od], acc);
        ls = fmaf(wt, s_wl[w][v], ls);
      }
      ob[k] = acc;
      if (od == 0) {
        s_m[v] = M == -INFINITY ? -INFINITY : M / 1.4426950408889634f;
        s_l[v] = ls;
      }
    }
    fx_publish<OPT, VSTEP>(a, ob, s_m, s_l, rep, static_cast<int64_t>(kh) * gridDim.x + split);
    // the appended row into the cache, after the chunk loads
    if (holds && wave == 0) {
#pragma unroll
      for (int i = 0; i < D / kWave; ++i) {
        kv_put<uint16_t>(kc, static_cast<int64_t>(offset) * D + lane + i * kWave, nkv[0][lane + i * kWave]);
        kv_put<uint16_t>(vc, static_cast<int64_t>(offset) * D + lane + i * kWave, nkv[1][lane + i * kWave]);
      }
    }
  }
  fx_merge(a, s_w, s_last, T, PER, rep, rep, 0);
}

// Fixed-range decode split plan for a capacity: chunks of 32 keys, at most
// kFxMaxSplits splits, per = keys per split (whole chunks), cps = chunks per split.
struct FxPlan {
  int splits, per, cps;
};
inline FxPlan fx_plan(int cap, int chunk) {
  const int chunks = (cap + chunk - 1) / chunk;
  const int cps = std::max(1, (chunks + kFxMaxSplits - 1) / kFxMaxSplits);
  const int splits = std::max(1, (chunks + cps - 1) / cps);
  return FxPlan{splits, cps * chunk, cps};
}

template <int D, typename KT>
static int launch_attention_t(const AttnArgs& a, int splits, hipStream_t stream) {
  constexpr int CH = attn_chunk<D>();
  const size_t qvb = static_cast<size_t>(a.rows) * (a.H / a.Hk);
  if constexpr (D == 64 || D == 128) {
    if constexpr (D == 128) {
    const int rep = a.H / std::max(a.Hk, 1);
    const int groups = rep >= 1 && rep <= 4 ? (a.rows * rep + 3) / 4 : 0;  // row groups of <= 4 query vectors
    // one query row at long contexts: the matrix-core kernel, one 64-key chunk per wave
    if constexpr (sizeof(KT) == 2) {
      const int mf_splits = (a.cap + kMfNW * 64 - 1) / (kMfNW * 64);
      if (a.rows == 1 && !a.mask && !a.n_rows_dev && a.window <= 0 && a.ctr && rep >= 1 && rep <= 4 &&
          a.cap >= kMfMinCap && mf_splits <= kFxMaxSplits && a.Hk <= kMaxKvHeads && a.ld_out % 4 == 0 &&
          aligned(a.out, 16) &&
          static_cast<size_t>(a.qv_ld) * kMaxSplits * (D + 2) >= static_cast<size_t>(kFxMaxSplits) * 4 * kFxRec) {
        hipLaunchKernelGGL((k_attn_decode_mf<D, 64>), dim3(mf_splits, a.Hk), dim3(256), 0, stream, a);
        WC_LAUNCHED();
        return WC_OK;
      }
    }
    // an explicit mask needs every chunk of a split in flight at entry (its bytes are fetched then)
    const int fx_cps = fx_plan(a.cap, 32).cps;
    if ((!a.mask || fx_cps <= 4) && a.ctr && groups >= 1 && a.rows <= kFxMaxRows && a.Hk * groups <= kMaxKvHeads &&
        a.ld_out % 4 == 0 && aligned(a.out, 16) &&
        static_cast<size_t>(a.qv_ld) * kMaxSplits * (D + 2) >=
            static_cast<size_t>(groups) * kFxMaxSplits * 4 * kFxRec) {
      // fixed key ranges from the capacity, merge fused per (kv head, row
      // group); the partials as (group, split, vector) records of kFxRec
      // floats, 4 vectors per split, in the same workspace
      constexpr int NT = kAttnThreads;
      const FxPlan pl = fx_plan(a.cap, 32);
      const dim3 grid(pl.splits, a.Hk, groups);
      if (pl.cps == 1 && groups == 1)  // one chunk per split: two waves per SIMD share its latency-bound math
        hipLaunchKernelGGL((k_attn_decode_fx<D, KT, 1, kFxThreads>), grid, dim3(kFxThreads), 0, stream, a, pl.per);
      else if (pl.cps == 1)  // several row groups: 256-thread blocks keep the grid resident at once
        hipLaunchKernelGGL((k_attn_decode_fx<D, KT, 1, NT>), grid, dim3(NT), 0, stream, a, pl.per);
      else if (pl.cps == 2)
        hipLaunchKernelGGL((k_attn_decode_fx<D, KT, 2, NT>), grid, dim3(NT), 0, stream, a, pl.per);
      else if (pl.cps == 3)
        hipLaunchKernelGGL((k_attn_decode_fx<D, KT, 3, NT>), grid, dim3(NT), 0, stream, a, pl.per);
      else  // four chunks in flight, the rest through the ring
        hipLaunchKernelGGL((k_attn_decode_fx<D, KT, 4, NT>), grid, dim3(NT), 0, stream, a, pl.per);
      WC_LAUNCHED();
      return WC_OK;
    }
    }
    if (!a.mask && qvb <= 16) {  // decode width: chunked registers, merge fused for <= 4 query vectors
      if (qvb <= 4) {
        hipLaunchKernelGGL((k_attn_decode<D, KT, 4>), dim3(splits, a.Hk), dim3(kAttnThreads), 0, stream, a);
      } else {
        hipLaunchKernelGGL((k_attn_decode<D, KT, 16>), dim3(splits, a.Hk), dim3(kAttnThreads), 0, stream, a);
      }
      WC_LAUNCHED();
      if (qvb <= 4 && a.ctr) return WC_OK;
      launch_merge<D>(a, qvb, splits, stream);
      WC_LAUNCHED();
      return WC_OK;
    }
  }
  const size_t lds = sizeof(float) * (qvb * D + 2 * CH * D + qvb * CH + 2 * static_cast<size_t>(a.rows) * D);
  static size_t attr_bytes = 64 * 1024;  // default dynamic-LDS limit
  if (lds > attr_bytes) {
    WC_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attention<D, KT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr_bytes = lds;
  }
  hipLaunchKernelGGL((k_attention<D, KT>), dim3(splits, a.Hk), dim3(kAttnThreads), lds, stream, a);
  WC_LAUNCHED();
  launch_merge<D>(a, qvb, splits, stream);
  WC_LAUNCHED();
  return WC_OK;
}

static int launch_attention(const AttnArgs& a, int D, int kv_dtype, int splits, hipStream_t s) {
#define WC_ATT(DD)                                                                                  \
  case DD:                                                                                          \
    return kv_dtype == WC_BF16 ? launch_attention_t<DD, uint16_t>(a, splits, s)                   \
                               : launch_attention_t<DD, float>(a, splits, s);
  switch (D) {
    WC_ATT(8)
    WC_ATT(16)
    WC_ATT(32)
    WC_ATT(64)
    WC_ATT(128)
    WC_ATT(256)
    default:
      return set_error(WC_E_UNSUPPORTED, "head_dim %d not supported (8, 16, 32, 64, 128, 256)", D);
  }
#undef WC_ATT
}

}  // namespace wc
