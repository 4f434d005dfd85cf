/*
 * wc_oracle.c -- CPU restatement of Woodcock's per-round speculative-decoding
 * arithmetic (drafter step, KV compaction, Philox uniforms).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product (woodcock_amd/) never links or calls it.
 *
 * What it restates (reference paths relative to the reference repository):
 *   rmsnorm          src/backends/cpu_ops.cpp:50-59   (fp64 sum of squares, x*inv*w)
 *   rope             src/backends/cpu_ops.cpp:61-77   (rotate-half, powf/cosf/sinf recipe)
 *   silu_mul         src/backends/cpu_ops.cpp:79-84
 *   softmax          src/backends/cpu_ops.cpp:86-96   (fp64 sum, -inf -> 0)
 *   attention        src/backends/cpu_ops.cpp:98-115  (GQA kh = h / rep, uint8 mask)
 *   Drafter::fuse    src/core/drafter.cpp:75-89       (python/woodcock/drafter.py:149-153)
 *   Drafter::forward src/core/drafter.cpp:91-136      (python/woodcock/drafter.py:164-191)
 *   causal_mask      src/core/qwen3.cpp:44-53         (python/woodcock/drafter.py:196-202)
 *   logits/head      python/woodcock/drafter.py:204-229 (restricted head = W[ids])
 *   argmax           src/sampling/sampling.cpp:47     (lowest index wins a tie)
 *   KV compaction    python/woodcock/target.py:159-175, src/cache/kv_cache.cpp:21-31
 *
 * Deliberate, documented differences from the reference C++ runtime:
 *   - weights are bf16 and widened exactly to fp32 on use (the reference
 *     widens them once at load, src/core/weights.cpp:100-122: same values);
 *   - dot products accumulate in fp32 over 8 interleaved partial sums
 *     instead of one running sum (same precision class, different order);
 *   - the KV cache is laid out [kv_head][capacity][head_dim] per layer (the
 *     mlx-lm layout, python/woodcock/drafter.py:92-94) instead of the C++
 *     [position][kv_head][head_dim]; optionally stored as bf16.
 *
 * Philox4x64-10 follows Salmon et al., "Parallel random numbers: as easy as
 * 1, 2, 3" (SC'11), and is checked bit-for-bit against numpy.random.Philox.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

static inline float bf16f(uint16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round to nearest even; NaN stays NaN */
static inline uint16_t f2bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void or_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f2bf16(x[i]);
}

void or_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int or_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ Philox4x64-10 */

static inline uint64_t mulhi64(uint64_t a, uint64_t b) { return (uint64_t)(((unsigned __int128)a * b) >> 64); }

void or_philox4x64_10(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]) {
  uint64_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint64_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B97F4A7C15ull;
      k1 += 0xBB67AE8584CAA73Bull;
    }
    const uint64_t lo0 = 0xD2E7470EE14C6C93ull * c0, hi0 = mulhi64(0xD2E7470EE14C6C93ull, c0);
    const uint64_t lo1 = 0xCA5A826395121157ull * c2, hi1 = mulhi64(0xCA5A826395121157ull, c2);
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

/* uniform i of stream (round, purpose) under `seed`: counter (i/4, round, purpose, 0),
 * key (seed, 0), word i%4, 53-bit double as numpy's Generator.random does */
void or_uniforms(uint64_t seed, uint64_t round, uint64_t purpose, uint64_t start, int64_t n, double* out) {
  uint64_t blk[4];
  uint64_t have = ~0ull;
  for (int64_t j = 0; j < n; ++j) {
    const uint64_t i = start + (uint64_t)j;
    if ((i >> 2) != have) {
      const uint64_t ctr[4] = {i >> 2, round, purpose, 0};
      const uint64_t key[2] = {seed, 0};
      or_philox4x64_10(ctr, key, blk);
      have = i >> 2;
    }
    out[j] = (double)(blk[i & 3] >> 11) * (1.0 / 9007199254740992.0);
  }
}

/* ------------------------------------------------------------------ basic ops */

/* y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w ; fp64 sum of squares (cpu_ops.cpp:50-59) */
void or_rmsnorm(const float* x, float* y, int rows, int d, const uint16_t* w, float eps) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (int64_t)r * d;
    float* yr = y + (int64_t)r * d;
    double ss = 0.0;
    for (int i = 0; i < d; ++i) ss += (double)xr[i] * xr[i];
    const float inv = 1.f / sqrtf((float)(ss / d) + eps);
    for (int i = 0; i < d; ++i) yr[i] = xr[i] * inv * (w ? bf16f(w[i]) : 1.f);
  }
}

/* cos/sin table [max_pos][D/2] with the reference recipe: inv_i = powf(base, -2i/D),
 * angle = (float)pos * inv_i (cpu_ops.cpp:63-68) */
void or_rope_table(float* cos_t, float* sin_t, int max_pos, int D, float base) {
  const int half = D / 2;
  float* inv = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; ++i) inv[i] = powf(base, -2.f * (float)i / (float)D);
  for (int p = 0; p < max_pos; ++p)
    for (int i = 0; i < half; ++i) {
      const float a = (float)p * inv[i];
      cos_t[(int64_t)p * half + i] = cosf(a);
      sin_t[(int64_t)p * half + i] = sinf(a);
    }
  free(inv);
}

/* rotate-half RoPE on x[L][heads][D] at positions (cpu_ops.cpp:61-77) */
static void rope(float* x, int L, int heads, int D, const int* pos, const float* ct, const float* st) {
  const int half = D / 2;
  for (int l = 0; l < L; ++l)
    for (int i = 0; i < half; ++i) {
      const float c = ct[(int64_t)pos[l] * half + i], s = st[(int64_t)pos[l] * half + i];
      for (int h = 0; h < heads; ++h) {
        float* v = x + ((int64_t)l * heads + h) * D;
        const float x1 = v[i], x2 = v[i + half];
        v[i] = x1 * c - x2 * s;
        v[i + half] = x2 * c + x1 * s;
      }
    }
}

typedef float v8f __attribute__((vector_size(32)));
typedef uint32_t v8u __attribute__((vector_size(32)));
typedef uint16_t v8h __attribute__((vector_size(16)));

/* dot(x fp32, w bf16) over n, 8 interleaved fp32 partial sums */
static inline float dot_bf16(const float* x, const uint16_t* w, int n) {
  v8f acc = {0, 0, 0, 0, 0, 0, 0, 0};
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    v8h wh;
    memcpy(&wh, w + k, 16);
    v8u wu = __builtin_convertvector(wh, v8u) << 16;
    v8f wf;
    memcpy(&wf, &wu, 32);
    v8f xv;
    memcpy(&xv, x + k, 32);
    acc += xv * wf;
  }
  float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  for (; k < n; ++k) s += x[k] * bf16f(w[k]);
  return s;
}

/* y[L][out] (+)= x[L][in] . W[out][in]^T with W bf16 (cpu_ops.cpp:45-48) */
void or_linear(const float* x, int L, int in, const uint16_t* W, int out, float* y, int accumulate) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < out; ++n)
    for (int l = 0; l < L; ++l) {
      const float s = dot_bf16(x + (int64_t)l * in, W + (int64_t)n * in, in);
      float* dst = y + (int64_t)l * out + n;
      *dst = accumulate ? *dst + s : s;
    }
}

/* softmax in place with an fp64 sum; -inf entries become 0 (cpu_ops.cpp:86-96) */
static void softmax_row(float* x, int n) {
  float m = -INFINITY;
  for (int i = 0; i < n; ++i) m = x[i] > m ? x[i] : m;
  double s = 0.0;
  for (int i = 0; i < n; ++i) {
    x[i] = (isinf(x[i]) && x[i] < 0) ? 0.f : expf(x[i] - m);
    s += x[i];
  }
  const float inv = (float)(1.0 / s);
  for (int i = 0; i < n; ++i) x[i] *= inv;
}

static inline float kv_get(const void* base, int kv_bf16, int64_t idx) {
  return kv_bf16 ? bf16f(((const uint16_t*)base)[idx]) : ((const float*)base)[idx];
}

static inline void kv_put(void* base, int kv_bf16, int64_t idx, float v) {
  if (kv_bf16)
    ((uint16_t*)base)[idx] = f2bf16(v);
  else
    ((float*)base)[idx] = v;
}

/* q[L][H][D]; cache K,V [Hk][cap][D]; mask[L][T] (1 = visible); out[L][H][D]
 * (cpu_ops.cpp:98-115: scores = scale * q.k, masked -> -inf, softmax, P.V) */
void or_attention(const float* q, int L, int H, int Hk, int D, const void* kc, const void* vc, int kv_bf16, int cap,
                  int T, const uint8_t* mask, float* out, float scale) {
  const int rep = H / Hk;
#pragma omp parallel for schedule(static)
  for (int h = 0; h < H; ++h) {
    const int kh = h / rep;
    float* S = (float*)malloc(sizeof(float) * (size_t)T);
    for (int l = 0; l < L; ++l) {
      const float* qr = q + ((int64_t)l * H + h) * D;
      for (int t = 0; t < T; ++t) {
        float s = 0.f;
        for (int i = 0; i < D; ++i) s += qr[i] * kv_get(kc, kv_bf16, ((int64_t)kh * cap + t) * D + i);
        S[t] = scale * s;
        if (mask && !mask[(int64_t)l * T + t]) S[t] = -INFINITY;
      }
      softmax_row(S, T);
      float* o = out + ((int64_t)l * H + h) * D;
      for (int i = 0; i < D; ++i) {
        float acc = 0.f;
        for (int t = 0; t < T; ++t) acc += S[t] * kv_get(vc, kv_bf16, ((int64_t)kh * cap + t) * D + i);
        o[i] = acc;
      }
    }
    free(S);
  }
}

/* ------------------------------------------------------------------ drafter */

typedef struct {
  int hidden, num_layers, heads, kv_heads, head_dim, inter, target_hidden, num_features, head_rows, vocab;
  float eps, rope_theta;
  int post_norm, feature_norm, window;
} or_dims;

typedef struct {
  const uint16_t *in_norm, *aux_norm, *post_norm; /* aux_norm NULL for layers without the aux stream */
  const uint16_t *q, *k, *v, *o, *aux_q, *aux_k, *aux_v, *q_norm, *k_norm, *gate, *up, *down;
} or_layer_w;

typedef struct {
  const uint16_t* embed;     /* [vocab][hidden] */
  const uint16_t* fc;        /* [hidden][num_features * target_hidden] */
  const uint16_t* fnorm[8];  /* [target_hidden] each (feature_norm) */
  const uint16_t* final_norm;
  const uint16_t* head;      /* [head_rows][hidden] (restricted rows already gathered) */
  const or_layer_w* layers;  /* [num_layers] */
} or_weights;

/* g[L][hidden] = fc(concat_f RMS_f(tap_f)) (drafter.cpp:75-89) */
void or_drafter_fuse(const or_dims* c, const or_weights* w, const float* const* taps, int L, float* g) {
  const int Dt = c->target_hidden, F = c->num_features;
  float* cat = (float*)malloc(sizeof(float) * (size_t)L * F * Dt);
  for (int f = 0; f < F; ++f)
    for (int l = 0; l < L; ++l) {
      const float* src = taps[f] + (int64_t)l * Dt;
      float* dst = cat + ((int64_t)l * F + f) * Dt;
      if (c->feature_norm)
        or_rmsnorm(src, dst, 1, Dt, w->fnorm[f], c->eps);
      else
        memcpy(dst, src, sizeof(float) * (size_t)Dt);
    }
  or_linear(cat, L, F * Dt, w->fc, c->hidden, g, 0);
  free(cat);
}

/* One drafter forward over L tokens appended at cache offset `offset`
 * (drafter.cpp:91-136).  kc/vc: per layer [kv_heads][cap][head_dim].
 * positions: NULL = offset + l; mask: NULL = causal with window (qwen3.cpp:44-53),
 * else [L][offset + L].  Returns 0, or -1 when offset + L > cap. */
int or_drafter_forward(const or_dims* c, const or_weights* w, const int* tokens, int L, const float* feat, void** kc,
                       void** vc, int kv_bf16, int cap, int offset, const int* positions, const uint8_t* mask,
                       const float* rope_cos, const float* rope_sin, float* hidden, float* out) {
  const int d = c->hidden, H = c->heads, Hk = c->kv_heads, D = c->head_dim, FF = c->inter;
  const int T = offset + L;
  if (T > cap) return -1;
  int* pos = (int*)malloc(sizeof(int) * (size_t)L);
  for (int l = 0; l < L; ++l) pos[l] = positions ? positions[l] : offset + l;
  uint8_t* m = (uint8_t*)malloc((size_t)L * T);
  if (mask) {
    memcpy(m, mask, (size_t)L * T);
  } else {
    for (int l = 0; l < L; ++l) {
      const int qp = offset + l;
      const int lo = c->window > 0 ? (qp - c->window + 1 > 0 ? qp - c->window + 1 : 0) : 0;
      for (int t = 0; t < T; ++t) m[(int64_t)l * T + t] = (t >= lo && t <= qp);
    }
  }
  float* e = (float*)malloc(sizeof(float) * (size_t)L * d);
  for (int l = 0; l < L; ++l)
    for (int i = 0; i < d; ++i) e[(int64_t)l * d + i] = bf16f(w->embed[(int64_t)tokens[l] * d + i]);
  float* h = hidden;
  memcpy(h, feat, sizeof(float) * (size_t)L * d);
  float* x = (float*)malloc(sizeof(float) * (size_t)L * d);
  float* a = (float*)malloc(sizeof(float) * (size_t)L * d);
  float* q = (float*)malloc(sizeof(float) * (size_t)L * H * D);
  float* k = (float*)malloc(sizeof(float) * (size_t)L * Hk * D);
  float* v = (float*)malloc(sizeof(float) * (size_t)L * Hk * D);
  float* att = (float*)malloc(sizeof(float) * (size_t)L * H * D);
  float* gt = (float*)malloc(sizeof(float) * (size_t)L * FF);
  float* up = (float*)malloc(sizeof(float) * (size_t)L * FF);
  for (int li = 0; li < c->num_layers; ++li) {
    const or_layer_w* Ly = &w->layers[li];
    or_rmsnorm(h, x, L, d, Ly->in_norm, c->eps);
    or_linear(x, L, d, Ly->q, H * D, q, 0);
    or_linear(x, L, d, Ly->k, Hk * D, k, 0);
    or_linear(x, L, d, Ly->v, Hk * D, v, 0);
    if (Ly->aux_norm) {
      or_rmsnorm(e, a, L, d, Ly->aux_norm, c->eps);
      or_linear(a, L, d, Ly->aux_q, H * D, q, 1);
      or_linear(a, L, d, Ly->aux_k, Hk * D, k, 1);
      or_linear(a, L, d, Ly->aux_v, Hk * D, v, 1);
    }
    or_rmsnorm(q, q, L * H, D, Ly->q_norm, c->eps);
    or_rmsnorm(k, k, L * Hk, D, Ly->k_norm, c->eps);
    rope(q, L, H, D, pos, rope_cos, rope_sin);
    rope(k, L, Hk, D, pos, rope_cos, rope_sin);
    for (int l = 0; l < L; ++l)
      for (int kh = 0; kh < Hk; ++kh)
        for (int i = 0; i < D; ++i) {
          const int64_t dst = ((int64_t)kh * cap + offset + l) * D + i;
          kv_put(kc[li], kv_bf16, dst, k[((int64_t)l * Hk + kh) * D + i]);
          kv_put(vc[li], kv_bf16, dst, v[((int64_t)l * Hk + kh) * D + i]);
        }
    or_attention(q, L, H, Hk, D, kc[li], vc[li], kv_bf16, cap, T, m, att, 1.f / sqrtf((float)D));
    or_linear(att, L, H * D, Ly->o, d, h, 1);
    or_rmsnorm(h, x, L, d, Ly->post_norm, c->eps);
    or_linear(x, L, d, Ly->gate, FF, gt, 0);
    or_linear(x, L, d, Ly->up, FF, up, 0);
    for (int64_t i = 0; i < (int64_t)L * FF; ++i) {
      const float g = gt[i];
      gt[i] = g / (1.f + expf(-g)) * up[i];
    }
    or_linear(gt, L, FF, Ly->down, d, h, 1);
  }
  or_rmsnorm(h, out, L, d, w->final_norm, c->eps);
  free(pos);
  free(m);
  free(e);
  free(x);
  free(a);
  free(q);
  free(k);
  free(v);
  free(att);
  free(gt);
  free(up);
  return 0;
}

/* z[L][head_rows] = out . W_head^T (drafter.py:204-207) */
void or_head_logits(const or_dims* c, const or_weights* w, const float* out, int L, float* z) {
  or_linear(out, L, c->hidden, w->head, c->head_rows, z, 0);
}

/* first index of the maximum (sampling.cpp:47, numpy argmax); NaN never wins */
int or_argmax(const float* z, int n) {
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (z[i] > z[best]) best = i;
  return best;
}

void or_argmax_rows(const float* z, int rows, int n, int* out) {
  for (int r = 0; r < rows; ++r) out[r] = or_argmax(z + (int64_t)r * n, n);
}

/* ------------------------------------------------------------------ KV compaction */

/* For every layer: rows start + keep[i] -> start + i in every kv head, gathered
 * first then written (target.py:170-177); nothing moves when keep is the identity.
 * Layout per layer [kv_heads][cap][row_bytes]. */
void or_kv_compact(void** k_layers, void** v_layers, int n_layers, int kv_heads, int cap, int row_bytes, int start,
                   const int* keep, int n_keep) {
  int ident = 1;
  for (int i = 0; i < n_keep; ++i) ident &= keep[i] == i;
  if (ident) return;
  unsigned char* tmp = (unsigned char*)malloc((size_t)n_keep * row_bytes);
  for (int l = 0; l < n_layers; ++l)
    for (int kv = 0; kv < 2; ++kv) {
      unsigned char* base = (unsigned char*)(kv ? v_layers[l] : k_layers[l]);
      for (int hh = 0; hh < kv_heads; ++hh) {
        unsigned char* hb = base + (int64_t)hh * cap * row_bytes;
        for (int i = 0; i < n_keep; ++i) memcpy(tmp + (int64_t)i * row_bytes, hb + (int64_t)(start + keep[i]) * row_bytes, (size_t)row_bytes);
        for (int i = 0; i < n_keep; ++i) memcpy(hb + (int64_t)(start + i) * row_bytes, tmp + (int64_t)i * row_bytes, (size_t)row_bytes);
      }
    }
  free(tmp);
}
