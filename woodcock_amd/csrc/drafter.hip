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
#include "gemv.h"

namespace wc {

// ------------------------------------------------------------------ workspace

constexpr int kAttnThreads = 256;
constexpr int kAttnChunkMax = 32;  // keys staged per iteration (fewer for head_dim 256)
template <int D>
constexpr int attn_chunk() { return D >= 256 ? 16 : kAttnChunkMax; }
constexpr int kMaxQV = 64;      // query vectors (rows x GQA group) per attention block
constexpr int kMaxSplits = 32;
constexpr int kMaxKvHeads = 64;

struct DrafterWs {
  unsigned int* head_ctr;  // tree counters (kTreeCounterBytes each)
  unsigned int* fin_ctr;
  unsigned long long* slots;
  float* qkv;
  float* attn;
  float* h1;
  float* act;
  float* partial;
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
  w.slots = reinterpret_cast<unsigned long long*>(take(8 * R * kSlots * kSlotStride));
  w.qkv = reinterpret_cast<float*>(take(4 * R * nqkv));
  w.attn = reinterpret_cast<float*>(take(4 * R * d.heads * d.head_dim));
  w.h1 = reinterpret_cast<float*>(take(4 * R * d.hidden));
  w.act = reinterpret_cast<float*>(take(4 * R * d.inter));
  w.partial = reinterpret_cast<float*>(take(4 * static_cast<size_t>(d.kv_heads) * kMaxSplits * kMaxQV *
                                            (d.head_dim + 2)));
  w.bytes = off;
  return w;
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
  float* partial;  // [Hk][S][kMaxQV][D+2]
  float* out;  // [rows][H*D]
  int64_t ld_out;
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

  for (int c0 = kb; c0 < ke; c0 += CH) {
    const int n = min(CH, ke - c0);
    kv_chunk_fill<D, KT>(ch, c0, n, offset, nk, nv, ks, vs);
    __syncthreads();
    if (c0 + CH < ke) kv_chunk_load<D, KT>(kc, vc, a.cap, c0 + CH, ch);  // next chunk in flight
    for (int e = threadIdx.x; e < QV * n; e += kAttnThreads) {
      const int v = e / n, j = e - v * n;
      const int l = v / rep, t = c0 + j;
      bool vis;
      if (a.mask)
        vis = a.mask[l * a.mask_ld + t] != 0;
      else
        vis = t <= offset + l && (a.window <= 0 || t > offset + l - a.window);
      float s = -INFINITY;
      if (vis) {
        float d = 0.f;
        const float4* q = reinterpret_cast<const float4*>(qs + v * D);
        const float4* k = reinterpret_cast<const float4*>(ks + j * D);
#pragma unroll 4
        for (int i = 0; i < D / 4; ++i) {
          const float4 x = q[i], y = k[i];
          d = fmaf(x.x, y.x, d);
          d = fmaf(x.y, y.y, d);
          d = fmaf(x.z, y.z, d);
          d = fmaf(x.w, y.w, d);
        }
        s = a.scale * d;
      }
      sc[v * CH + j] = s;
    }
    __syncthreads();
    if (threadIdx.x < QV) {
      const int v = threadIdx.x;
      const float m_old = s_m[v];
      float m_new = m_old;
      for (int j = 0; j < n; ++j) m_new = fmaxf(m_new, sc[v * CH + j]);
      float alpha = 1.f, lsum = 0.f;
      if (m_new != -INFINITY) {
        alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
        for (int j = 0; j < n; ++j) {
          const float sv = sc[v * CH + j];
          const float p = sv == -INFINITY ? 0.f : expf(sv - m_new);
          sc[v * CH + j] = p;
          lsum += p;
        }
      } else {
        for (int j = 0; j < n; ++j) sc[v * CH + j] = 0.f;
      }
      s_m[v] = m_new;
      s_l[v] = s_l[v] * alpha + lsum;
      s_alpha[v] = alpha;
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
  float* part = a.partial + (static_cast<int64_t>(kh) * S + split) * kMaxQV * (D + 2);
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

// Merge the splits: one block per (vector, kv head).  Every load -- the
// splits' (m, l) and this vector's partial outputs -- is issued up front from
// addresses that do not depend on the row count; the block then exits if its
// vector is past the live rows.  Runs after k_attention (stream order), so
// plain loads see the partials.
template <int D>
__global__ __launch_bounds__(kAttnThreads) void k_attn_merge(AttnArgs a, int S) {
  constexpr int kPer = (D + kAttnThreads - 1) / kAttnThreads;  // elements per thread (D <= 256: 1)
  static_assert(kPer == 1, "head_dim up to the block size");
  __shared__ float s_w[kMaxSplits], s_lsum[kMaxSplits];
  const int v = blockIdx.x, kh = blockIdx.y;
  const int rep = a.H / a.Hk;
  const int t = threadIdx.x;
  const float* base = a.partial + static_cast<int64_t>(kh) * S * kMaxQV * (D + 2) + v * (D + 2);
  constexpr int64_t kSplitStride = static_cast<int64_t>(kMaxQV) * (D + 2);
  const int i = min(t, D - 1);
  float o[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) o[sp] = base[min(sp, S - 1) * kSplitStride + 2 + i];
  if (t < S) {
    s_w[t] = base[t * kSplitStride];
    s_lsum[t] = base[t * kSplitStride + 1];
  }
  const int nr = a.n_rows_dev ? min(max(*a.n_rows_dev, 0), a.rows) : a.rows;
  if (v >= nr * rep) return;  // uniform per block
  __syncthreads();
  float M = -INFINITY;
  for (int sp = 0; sp < S; ++sp) M = fmaxf(M, s_w[sp]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    if (sp < S) {
      const float ms = s_w[sp];
      const float wgt = ms == -INFINITY ? 0.f : expf(ms - M);
      den = fmaf(s_lsum[sp], wgt, den);
      num = fmaf(wgt, o[sp], num);
    }
  }
  if (t < D) {
    const int l = v / rep, h = kh * rep + v % rep;
    a.out[l * a.ld_out + h * D + t] = num / den;
  }
}

template <int D, typename KT>
static int launch_attention_t(const AttnArgs& a, int splits, hipStream_t stream) {
  constexpr int CH = attn_chunk<D>();
  const size_t qvb = static_cast<size_t>(a.rows) * (a.H / a.Hk);
  const size_t lds = sizeof(float) * (qvb * D + 2 * CH * D + qvb * CH + 2 * static_cast<size_t>(a.rows) * D);
  static size_t attr_bytes = 64 * 1024;  // default dynamic-LDS limit
  if (lds > attr_bytes) {
    WC_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attention<D, KT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr_bytes = lds;
  }
  hipLaunchKernelGGL((k_attention<D, KT>), dim3(splits, a.Hk), dim3(kAttnThreads), lds, stream, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL((k_attn_merge<D>), dim3(static_cast<unsigned>(qvb), a.Hk), dim3(kAttnThreads), 0, stream, a,
                     splits);
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
    const dim3 grid((a.N + kGemvWaves * R - 1) / (kGemvWaves * R)), block(kGemvThreads);
    hipLaunchKernelGGL((k_gemv1<R, PAIR, NIN, S, XB>), grid, block, 0, s, a);
    return true;
  }
}

template <int R, bool PAIR, int NIN, int XB>
static bool launch_gemv1(const GemvArgs& a, int steps, hipStream_t s) {
  if (steps <= 4) return launch_gemv1_s<R, PAIR, NIN, 4, XB>(a, s);
  if (steps <= 8) return launch_gemv1_s<R, PAIR, NIN, 8, XB>(a, s);
  if (steps <= 12) return launch_gemv1_s<R, PAIR, NIN, 12, XB>(a, s);
  return false;
}

// Largest rows-per-wave that keeps at least 512 blocks and fits the budget.
template <bool PAIR, int NIN, int XB>
static bool launch_gemv1_r(const GemvArgs& a, int steps, hipStream_t s) {
  if (a.N >= 4 * kGemvWaves * 512 && launch_gemv1<4, PAIR, NIN, XB>(a, steps, s)) return true;
  if (a.N >= 2 * kGemvWaves * 512 && launch_gemv1<2, PAIR, NIN, XB>(a, steps, s)) return true;
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

// Every K a multiple of 512 (up to 6144): one row goes to the register-resident
// kernel, 2..8 rows to the LDS-staged few-row kernel; anything else to the
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
  if (a.M > 1 && k512) {
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

int wc_drafter_fuse(const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps, int tap_dtype,
                    int64_t tap_ld, const int32_t* tap_rows_dev, int rows, const int32_t* n_rows_dev, float* g_out,
                    int64_t g_ld, void* workspace, wc_stream_t stream) {
  if (int rc = check_dims(dims)) return rc;
  WC_REQUIRE(w && taps && g_out, "wc_drafter_fuse: NULL argument");
  WC_REQUIRE(w->fc && al16(w->fc), "wc_drafter_fuse: fc weight missing or not 16-byte aligned");
  WC_REQUIRE(tap_dtype == WC_F32 || tap_dtype == WC_BF16, "wc_drafter_fuse: tap dtype must be f32 or bf16");
  WC_REQUIRE(tap_ld >= dims->target_hidden && g_ld >= dims->hidden, "wc_drafter_fuse: bad row stride");
  WC_REQUIRE(tap_ld % 8 == 0 && g_ld % 4 == 0, "wc_drafter_fuse: row strides must be multiples of 8 (taps) / 4");
  WC_REQUIRE(rows >= 1, "wc_drafter_fuse: rows must be positive");
  WC_REQUIRE(n_rows_dev == nullptr || rows <= WC_MAX_STEP_ROWS,
             "wc_drafter_fuse: a device row count needs rows <= %d", WC_MAX_STEP_ROWS);
  auto s = reinterpret_cast<hipStream_t>(stream);
  const int nf = dims->num_features, Dt = dims->target_hidden;
  for (int t0 = 0; t0 < rows; t0 += WC_MAX_STEP_ROWS) {
    const int tr = std::min(WC_MAX_STEP_ROWS, rows - t0);
    GemvArgs g = gemv_defaults();
    g.n_in = nf;
    for (int f = 0; f < nf; ++f) {
      WC_REQUIRE(taps[f] != nullptr && al16(taps[f]), "wc_drafter_fuse: tap %d is NULL or not 16-byte aligned", f);
      g.in[f].x = static_cast<const char*>(taps[f]) + (tap_rows_dev ? 0 : t0 * tap_ld * (tap_dtype ? 2 : 4));
      g.in[f].ld = tap_ld;
      g.in[f].dtype = tap_dtype;
      g.in[f].row_idx = tap_rows_dev ? tap_rows_dev + t0 : nullptr;
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

int wc_drafter_forward(const wc_drafter_dims* dims, const wc_drafter_weights* w, const int32_t* tokens_dev,
                       const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add, int rows,
                       const int32_t* n_rows_dev, void* const* k_cache, void* const* v_cache, int kv_dtype,
                       int capacity, const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                       const uint8_t* mask_dev, int64_t mask_ld, float* hidden_out, float* out_out,
                       int32_t* advance_dev, void* workspace, wc_stream_t stream) {
  if (int rc = check_dims(dims)) return rc;
  const wc_drafter_dims& d = *dims;
  WC_REQUIRE(w && tokens_dev && feat && hidden_out && out_out && workspace && offset_dev && k_cache && v_cache,
             "wc_drafter_forward: NULL argument");
  WC_REQUIRE(al16(workspace), "wc_drafter_forward: workspace must be 16-byte aligned");
  WC_REQUIRE(rows >= 1, "wc_drafter_forward: rows must be positive");
  WC_REQUIRE(kv_dtype == WC_F32 || kv_dtype == WC_BF16, "wc_drafter_forward: kv dtype must be f32 or bf16");
  WC_REQUIRE(feat_ld >= d.hidden && feat_ld % 4 == 0,
             "wc_drafter_forward: feature row stride must be >= hidden_size and a multiple of 4");
  WC_REQUIRE(al16(feat) && al16(hidden_out) && al16(out_out), "wc_drafter_forward: buffers must be 16-byte aligned");
  WC_REQUIRE(feat_row_dev == nullptr || rows == 1, "wc_drafter_forward: a gathered feature row needs rows == 1");
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
        xin.row_idx = feat_row_dev;
        xin.row_add = feat_row_dev ? feat_row_add : 0;
      } else {
        xin.x = hidden_out + t0 * d.hidden;
        xin.ld = d.hidden;
      }

      // 1. QKV (dual stream on layers with the token embedding)
      GemvArgs q = gemv_defaults();
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
        e.row_idx = tokens_dev + t0;
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
      at.out = ws.attn;
      at.ld_out = H * D;
      if (int rc = launch_attention(at, D, kv_dtype, splits, s)) return rc;

      // 3. o_proj with the residual: h1 = h + W_o . o
      GemvArgs o = gemv_defaults();
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
      gu.in[0].x = ws.h1;
      gu.in[0].ld = d.hidden;
      gu.in[0].dtype = WC_F32;
      gu.in[0].gain = u16(L.post_norm);
      gu.in[0].K = d.hidden;
      gu.n_in = 1;
      gu.ldw[0] = d.hidden;
      gu.w[0][0] = u16(L.gate);
      gu.w[1][0] = u16(L.up);
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
      if (last_layer) {
        dn.fin_counter = ws.fin_ctr;
        dn.fin_gain = u16(w->final_norm);
        dn.fin_out = out_out + t0 * d.hidden;
        dn.ld_fin = d.hidden;
        if (advance_dev && last_tile) {
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

int wc_draft_head(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* out_rows, int64_t out_ld,
                  const int32_t* out_row_dev, int out_row_add, int rows, float* logits_out, int64_t logits_ld,
                  int32_t* token_out, int32_t* row_out, const wc_gumbel* gumbel, void* workspace,
                  wc_stream_t stream) {
  if (int rc = check_dims(dims)) return rc;
  WC_REQUIRE(w && w->head && out_rows && token_out && workspace, "wc_draft_head: NULL argument");
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
  for (int t0 = 0; t0 < rows; t0 += WC_MAX_STEP_ROWS) {
    const int tr = std::min(WC_MAX_STEP_ROWS, rows - t0);
    GemvArgs h = gemv_defaults();
    h.in[0].x = out_rows + (out_row_dev ? 0 : t0 * out_ld);
    h.in[0].ld = out_ld;
    h.in[0].dtype = WC_F32;
    h.in[0].row_idx = out_row_dev;
    h.in[0].row_add = out_row_dev ? out_row_add : 0;
    h.in[0].K = dims->hidden;
    h.n_in = 1;
    h.ldw[0] = dims->hidden;
    h.w[0][0] = u16(w->head);
    h.N = dims->head_rows;
    h.seg_start[1] = h.N;
    h.M = tr;
    h.eps = dims->eps;
    h.epi = kEpiArgmax;
    h.y = logits_out ? logits_out + t0 * logits_ld : nullptr;
    h.ldy = logits_ld;
    h.slots = ws.slots;
    h.counter = ws.head_ctr;
    h.d2t = w->d2t;
    h.tok_out = token_out + t0;
    h.row_out = row_out ? row_out + t0 : nullptr;
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

}  // extern "C"
