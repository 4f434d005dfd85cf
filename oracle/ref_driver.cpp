// ref_driver.cpp -- extern "C" shim over the reference's own C++ runtime.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's sources where they lie (src/backends/cpu_ops.cpp,
// src/core/{drafter,weights,json,qwen3}.cpp, src/cache/kv_cache.cpp,
// src/sampling/sampling.cpp) into oracle/_ref/libwcref.so.  Nothing of the
// reference is copied here: this file only calls its public interface
// (include/woodcock/{drafter,cache,sampling,ops,model}.h) so that Python
// tests can produce golden vectors and cross-check the restatement in
// oracle/wc_oracle.c.  Exceptions never cross the ABI: every entry point
// returns 0 on success and -1 on error (message via wcref_last_error).
#include <array>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "woodcock/cache.h"
#include "woodcock/drafter.h"
#include "woodcock/model.h"
#include "woodcock/ops.h"
#include "woodcock/sampling.h"

using namespace woodcock;

static thread_local std::string g_err;

#define GUARD(...)                   \
  try {                              \
    __VA_ARGS__;                     \
    return 0;                        \
  } catch (const std::exception& e) { \
    g_err = e.what();                \
    return -1;                       \
  }

extern "C" {

const char* wcref_last_error() { return g_err.c_str(); }

// ------------------------------------------------------------------ drafter (drafter.h:48-58)

int wcref_drafter_open(const char* dir, void** out) { GUARD(*out = new Drafter(dir)) }
void wcref_drafter_close(void* d) { delete static_cast<Drafter*>(d); }

int wcref_drafter_cache_new(void* d, void** out) {
  GUARD(*out = new KVCache(static_cast<Drafter*>(d)->make_cache()))
}

// fuse: taps[f] is [L][target_hidden] fp32 (drafter.h:54)
int wcref_drafter_fuse(void* d, const float* const* taps, int n_taps, int L, float* g) {
  GUARD({
    const auto& c = static_cast<Drafter*>(d)->config();
    std::vector<std::vector<float>> t(static_cast<size_t>(n_taps));
    for (int f = 0; f < n_taps; ++f) t[size_t(f)].assign(taps[f], taps[f] + int64_t(L) * c.target_hidden);
    auto r = static_cast<Drafter*>(d)->fuse(t, L);
    std::memcpy(g, r.data(), sizeof(float) * r.size());
  })
}

// forward (drafter.h:56-58): positions [L] and mask [L][cache+L] are optional
int wcref_drafter_forward(void* d, const int* tokens, int L, const float* feat, void* cache, const int* positions,
                          const uint8_t* mask, float* hidden, float* out) {
  GUARD({
    auto* dr = static_cast<Drafter*>(d);
    auto* kv = static_cast<KVCache*>(cache);
    const int dd = dr->config().hidden;
    std::vector<int> tok(tokens, tokens + L);
    std::vector<float> f(feat, feat + int64_t(L) * dd);
    std::vector<int> pos;
    std::vector<uint8_t> m;
    if (positions) pos.assign(positions, positions + L);
    if (mask) m.assign(mask, mask + int64_t(L) * (kv->size() + L));
    DraftOut o = dr->forward(tok, f, *kv, positions ? &pos : nullptr, mask ? &m : nullptr);
    std::memcpy(hidden, o.hidden.data(), sizeof(float) * o.hidden.size());
    std::memcpy(out, o.out.data(), sizeof(float) * o.out.size());
  })
}

// full logits of one row: z has config().vocab entries (drafter.h:62-63)
int wcref_drafter_logits(void* d, const float* out_row, float* z) {
  GUARD({
    std::vector<float> r;
    static_cast<Drafter*>(d)->logits(out_row, r);
    std::memcpy(z, r.data(), sizeof(float) * r.size());
  })
}

// ------------------------------------------------------------------ KV cache (cache.h:9-28)

int wcref_cache_new(int layers, int kv_heads, int head_dim, void** out) { GUARD(*out = new KVCache(layers, kv_heads, head_dim)) }
void wcref_cache_free(void* c) { delete static_cast<KVCache*>(c); }
int wcref_cache_size(void* c) { return static_cast<KVCache*>(c)->size(); }
int wcref_cache_append(void* c, int layer, const float* k, const float* v, int L) {
  GUARD(static_cast<KVCache*>(c)->append(layer, k, v, L))
}
void wcref_cache_commit(void* c, int L) { static_cast<KVCache*>(c)->commit(L); }
void wcref_cache_trim_to(void* c, int n) { static_cast<KVCache*>(c)->trim_to(n); }
int wcref_cache_compact(void* c, int start, const int* keep, int n_keep) {
  GUARD(static_cast<KVCache*>(c)->compact(start, std::vector<int>(keep, keep + n_keep)))
}
// copy rows [0, n) of layer's K (which=0) or V (which=1): [n][kv_heads*head_dim]
int wcref_cache_rows(void* c, int layer, int which, int n, float* dst) {
  GUARD({
    auto* kv = static_cast<KVCache*>(c);
    const float* src = which ? kv->values(layer) : kv->keys(layer);
    std::memcpy(dst, src, sizeof(float) * size_t(n) * size_t(kv->row()));
  })
}

// ------------------------------------------------------------------ target model (model.h:19-48)

int wcref_qwen3_open(const char* dir, int t0, int t1, int t2, void** out) {
  GUARD(*out = new Qwen3(dir, std::array<int, 3>{t0, t1, t2}))
}
void wcref_qwen3_close(void* m) { delete static_cast<Qwen3*>(m); }
int wcref_qwen3_cache_new(void* m, void** out) { GUARD(*out = new KVCache(static_cast<Qwen3*>(m)->make_cache())) }

// forward (model.h:36-37): positions [L] and mask [L][cache + L] optional;
// logits [L][vocab]; taps [3][L][hidden] in the order the forward pushes them
int wcref_qwen3_forward(void* m, const int* tokens, int L, void* cache, const int* positions, const uint8_t* mask,
                        float* logits, float* taps) {
  GUARD({
    auto* q = static_cast<Qwen3*>(m);
    auto* kv = static_cast<KVCache*>(cache);
    std::vector<int> tok(tokens, tokens + L), pos;
    std::vector<uint8_t> msk;
    ForwardArgs a;
    if (positions) {
      pos.assign(positions, positions + L);
      a.positions = &pos;
    }
    if (mask) {
      msk.assign(mask, mask + int64_t(L) * (kv->size() + L));
      a.mask = &msk;
    }
    ForwardOut o = q->forward(tok, *kv, a);
    std::memcpy(logits, o.logits.data(), sizeof(float) * o.logits.size());
    for (size_t i = 0; i < o.taps.size(); ++i)
      std::memcpy(taps + i * o.taps[i].size(), o.taps[i].data(), sizeof(float) * o.taps[i].size());
  })
}

// ------------------------------------------------------------------ sampling (sampling.h:21-45)

int wcref_argmax(const float* z, int n) { return argmax(z, n); }

int wcref_probs_from_logits(const float* z, int n, float temperature, int top_k, float top_p, float* p) {
  GUARD({
    SamplingParams sp;
    sp.temperature = temperature;
    sp.top_k = top_k;
    sp.top_p = top_p;
    auto r = probs_from_logits(z, n, sp);
    std::memcpy(p, r.data(), sizeof(float) * r.size());
  })
}

static DraftTree make_tree(const int* tokens, const int* parents, const int* depth, int N) {
  DraftTree t;
  t.tokens.assign(tokens, tokens + N);
  t.parents.assign(parents, parents + N);
  t.depth.assign(depth, depth + N);
  t.build_children();
  return t;
}

int wcref_verify_tree_greedy(const int* am, const int* tokens, const int* parents, const int* depth, int N, int* path,
                             int* path_len, int* next) {
  GUARD({
    Verdict v = verify_tree_greedy(std::vector<int>(am, am + N), make_tree(tokens, parents, depth, N));
    *path_len = int(v.path.size());
    for (size_t i = 0; i < v.path.size(); ++i) path[i] = v.path[i];
    *next = v.next;
  })
}

int wcref_tree_mask(const int* tokens, const int* parents, const int* depth, int N, int prefix, uint8_t* m) {
  GUARD({
    auto r = tree_mask(make_tree(tokens, parents, depth, N), prefix);
    std::memcpy(m, r.data(), r.size());
  })
}

// causal_mask / default_positions (model.h:28-30)
int wcref_causal_mask(int prefix, int L, int window, uint8_t* m) {
  GUARD({
    auto r = causal_mask(prefix, L, window);
    std::memcpy(m, r.data(), r.size());
  })
}

// ------------------------------------------------------------------ ops (ops.h:9-24)

int wcref_rmsnorm(const float* x, float* y, int rows, int d, const float* w, float eps) {
  GUARD(ops::rmsnorm(x, y, rows, d, w, eps))
}
int wcref_rope(float* x, int L, int heads, int D, const int* positions, float base) {
  GUARD(ops::rope(x, L, heads, D, positions, base))
}
int wcref_softmax(float* x, int n) { GUARD(ops::softmax(x, n)) }
// linear over an fp32 weight [out][in] held in a Tensor (weights.h:14-24)
int wcref_linear(const float* x, int L, int in, const float* W, int out, float* y, int accumulate) {
  GUARD({
    Tensor t;
    t.shape = {out, in};
    t.data.assign(W, W + int64_t(out) * in);
    ops::linear(x, L, in, t, y, accumulate != 0);
  })
}
int wcref_silu_mul(float* gate, const float* up, int64_t n) { GUARD(ops::silu_mul(gate, up, n)) }
int wcref_attention(const float* q, int L, int H, int Hk, int D, const float* K, const float* V, int T,
                    const uint8_t* mask, float* out, float scale) {
  GUARD(ops::attention(q, L, H, Hk, D, K, V, T, mask, out, scale))
}

}  // extern "C"
