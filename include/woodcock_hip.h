/*
 * woodcock_hip.h -- C ABI of the MI355X (gfx950) backend for Woodcock's
 * per-round speculative-decoding hot path.
 *
 * Conventions
 *   - Every pointer argument named *_dev or typed as a device buffer is device
 *     memory owned by the caller (PyTorch-ROCm tensors in the Python host).
 *     The library allocates nothing per call.
 *   - Every call is stream-ordered on `stream` (a hipStream_t; NULL = the
 *     null stream) and never synchronises the host.
 *   - Return value: WC_OK (0) or a WC_E_* status; wc_last_error() returns the
 *     calling thread's message for the last failure.  Exceptions never cross
 *     this boundary.
 *   - Integers that change from round to round (offsets, accepted lengths,
 *     keep lists) are read from device memory, so a captured HIP graph of a
 *     round stays valid across replays.
 *   - `workspace` is device memory of at least the size the matching
 *     *_workspace_bytes() query returns, zero-filled once with
 *     wc_workspace_init(); kernels leave their counters at zero on exit.  One
 *     workspace must not be used by two streams at once.
 *
 * Each entry point cites the reference interface it stands in for (paths
 * relative to the reference repository).
 */
#ifndef WOODCOCK_HIP_H
#define WOODCOCK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* wc_stream_t; /* == hipStream_t */

#define WC_ABI_VERSION 2
#define WC_MAX_NODES 64   /* verify rows per round: chain k+1 or tree nodes */
#define WC_MAX_LAYERS 64  /* KV compaction: layers per call */

enum {
  WC_OK = 0,
  WC_E_INVALID = 1,     /* bad shape, pointer, alignment or value */
  WC_E_HIP = 2,         /* HIP runtime error (launch, attribute query) */
  WC_E_UNSUPPORTED = 3  /* valid request this backend does not implement */
};

enum { WC_F32 = 0, WC_BF16 = 1 };

/* Result of one verification, written to device memory by the verify kernels
 * (python/woodcock/sampling.py:60-177 return values; include/woodcock/sampling.h:35-38 Verdict). */
typedef struct wc_verdict {
  int32_t n_accepted;  /* chain: accepted draft tokens a; tree: accepted path length */
  int32_t next;        /* target token after the accepted prefix / path */
  int32_t n_keep;      /* n_accepted + 1: verify-block entries the KV compaction keeps */
  int32_t n_uniforms;  /* uniforms consumed (stochastic rules), 0 for greedy */
  int32_t status;      /* 0; WC_E_INVALID when the device saw an invalid input; WC_E_HIP when a bounded wait gave up */
  int32_t reserved[3];
  int32_t tokens[WC_MAX_NODES + 1]; /* accepted tokens then `next` (n_keep entries) */
  int32_t keep[WC_MAX_NODES + 1];   /* verify-block rows kept: 0 then the accepted nodes */
} wc_verdict;

/* ------------------------------------------------------------------ library */

int wc_version(void);                 /* WC_ABI_VERSION */
const char* wc_last_error(void);      /* message of the calling thread's last failure */
size_t wc_workspace_bytes(void);      /* workspace needed by the verify kernels */
/* zero-fill `bytes` of device memory with a kernel (no hipMemset node, so it is graph-safe) */
int wc_workspace_init(void* workspace, size_t bytes, wc_stream_t stream);

/* ------------------------------------------------------------------ greedy verification */

/* Row-wise argmax (lowest index wins a tie) of logits [rows][vocab] with row
 * stride `ld` floats.  Replaces mx.argmax(o.logits[0], axis=-1)
 * (python/woodcock/spec.py:355) and argmax (src/sampling/sampling.cpp:47). */
int wc_argmax_rows(const float* logits, int rows, int vocab, int64_t ld, int32_t* out_dev, void* workspace,
                   wc_stream_t stream);

/* Greedy chain verification fused with the target argmax: rows = k+1 logits at
 * [x_n, d_1..d_k], draft_tokens_dev [k].  Writes n_accepted, next, tokens and
 * keep = 0..a.  Replaces verify_chain_greedy (python/woodcock/sampling.py:60-66) and
 * the inline accept loop of the fused round (python/woodcock/spec.py:355-361). */
int wc_verify_chain_greedy(const float* logits, int rows, int vocab, int64_t ld, const int32_t* draft_tokens_dev,
                           wc_verdict* verdict_dev, void* workspace, wc_stream_t stream);

/* wc_verify_chain_greedy without a caller workspace and without any allocation:
 * its scratch (argmax slots for up to WC_MAX_NODES rows and the kernel's
 * counters, 8,832 bytes) is a static device array of the library, one per GPU,
 * kept until the process ends; each call clears it with a kernel first.
 * rows > WC_MAX_NODES is rejected (WC_E_INVALID).  Every call on one GPU
 * shares that GPU's array, so calls that overlap on one GPU (two streams at
 * once) race; calls ordered on one stream are safe.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int wc_verify_chain_greedy_static(const float* logits, int rows, int vocab, int64_t ld,
                                  const int32_t* draft_tokens_dev, wc_verdict* verdict_dev, wc_stream_t stream);

/* Greedy tree verification fused with the target argmax: N = rows flattened
 * nodes, node 0 the root; tree_tokens_dev/tree_parents_dev [N] (parents[0] = -1,
 * children in ascending node order = draw order).  Writes the accepted path,
 * next, tokens and keep = [0] + path.  Replaces verify_tree_greedy
 * (python/woodcock/sampling.py:131-140; src/sampling/sampling.cpp:95-106). */
int wc_verify_tree_greedy(const float* logits, int rows, int vocab, int64_t ld, const int32_t* tree_tokens_dev,
                          const int32_t* tree_parents_dev, wc_verdict* verdict_dev, void* workspace,
                          wc_stream_t stream);

/* ------------------------------------------------------------------ stochastic verification */

/* Counter-based uniforms: value j of a round is Philox4x64-10 (Salmon et al.,
 * SC'11) with counter (j/4, *round_dev, purpose, 0) and key (seed, 0), word j%4,
 * top 53 bits / 2^53.  Stands in for the np.random.Generator the reference
 * threads through the verification rules (python/woodcock/sampling.py:69-82,143-193). */
typedef struct wc_uniforms {
  uint64_t seed;
  const int32_t* round_dev;
  int32_t purpose;
} wc_uniforms;

/* The warped sampling distribution, fp32, for r < rows (width n, row strides
 * ld / ld_out floats; rows <= WC_MAX_NODES): x = logits[r] / max(T, 1e-6); with
 * 0 < top_k < n every x below the top_k-th largest x drops out (ties with it
 * stay); out[r] = softmax(x); with top_p < 1 only the entries of the
 * descending order whose exclusive cumulative mass is below top_p stay (the
 * first always; among equal values the lower index first), renormalised by
 * the kept mass in fp64.  top_k = 0 and top_p = 1 switch the warps off;
 * top_p must lie in (0, 1].  Replaces probs_from_logits
 * (python/woodcock/sampling.py:39-55; src/sampling/sampling.cpp:9-45) and the
 * draft distribution of SpeculativeDecoder._draft_dist (python/woodcock/spec.py:113-125). */
int wc_probs_from_logits(const float* logits, int rows, int n, int64_t ld, float temperature, int top_k, float top_p,
                         float* out, int64_t ld_out, void* workspace, wc_stream_t stream);

/* Stochastic chain verification (Leviathan et al. 2023 / Chen et al. 2023) with
 * fp64 decisions: p [rows][ld_p] target probabilities at [x_n, d_1..d_K]
 * (rows = K+1), q [K][ld_q] the draft distributions the drafts were drawn from,
 * over the head rows (head_rows wide), d2t_dev [head_rows] the ascending target
 * id of each head row (NULL = identity), draft_rows_dev [K] the drafts' head
 * rows (NULL = looked up in d2t).  q is scattered to the vocabulary and
 * renormalised in fp64; q(d_i) <= 0 rejects without a uniform, else
 * u < min(1, p(d_i)/q(d_i)) accepts; the next token is drawn from
 * norm(max(p - q, 0)) at the first rejection (p when that mass is <= 1e-12), or
 * from p_K.  Writes n_accepted, next, tokens, keep = 0..a and n_uniforms;
 * status = WC_E_INVALID for a draft outside the vocabulary or a d2t that is not
 * strictly ascending.  Replaces verify_chain_stochastic
 * (python/woodcock/sampling.py:69-82, 182-193) as the engine runs it
 * (verify_tree_stochastic on a chain, python/woodcock/spec.py:316-324,
 * sampling.py:143-177; src/sampling/sampling.cpp:116-141). */
int wc_verify_chain_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, int head_rows,
                               int64_t ld_q, const int32_t* d2t_dev, const int32_t* draft_tokens_dev,
                               const int32_t* draft_rows_dev, const wc_uniforms* rng, wc_verdict* verdict_dev,
                               void* workspace, wc_stream_t stream);

/* wc_probs_from_logits at temperature T followed by wc_verify_chain_stochastic,
 * with p never written: logits [rows][ld] are the target logits at
 * [x_n, d_1..d_K]; p_i = softmax(logits_i / max(T, 1e-6)) is formed in place
 * with the same arithmetic (so the decisions and draws equal the two-call
 * path's bit for bit).  rows <= 8 (and chunk blocks that fit on the GPU at
 * once): one launch whose blocks hand results over through mailboxes in the
 * workspace -- a call that gave up waiting (after ~4 s) leaves status
 * WC_E_HIP and the workspace must be initialised again (wc_workspace_init;
 * until then every call on it fails fast with WC_E_HIP); longer chains: two
 * launches (softmax partials, draft masses and the accept tests; then the
 * draw).  Replaces the verify step of the engine's stochastic chain path
 * (python/woodcock/spec.py:316-324: probs_from_logits + verify_tree_stochastic
 * at width 1). */
int wc_verify_chain_stochastic_logits(const float* logits, int rows, int vocab, int64_t ld, float temperature,
                                      const float* q, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                                      const int32_t* draft_tokens_dev, const int32_t* draft_rows_dev,
                                      const wc_uniforms* rng, wc_verdict* verdict_dev, void* workspace,
                                      wc_stream_t stream);

/* Bounded waits of the one-launch stochastic chain kernel: a waiting block
 * gives up after `polls` polls (polls < 0 restores the default, ~4 s), leaving
 * WC_E_HIP in the verdict and a sticky failure flag in the workspace; every
 * later call on that workspace fails fast with WC_E_HIP until
 * wc_workspace_init zero-fills it again.  A test hook (process-wide; takes
 * effect at the next launch) for forcing that path from the host without a
 * kernel that never ends.  No reference counterpart. */
int wc_set_spin_limit(int polls);

/* Stochastic tree verification, fp64 decisions: N = rows flattened nodes (node 0
 * the root, parents[0] = -1, 0 <= parents[i] < i, children in ascending node
 * order = draw order), p [N][ld_p] the target probabilities at every node,
 * q [N][ld_q] the draft distribution each node's children were drawn from
 * without replacement, over the head rows (rows of leaves unused), d2t_dev as
 * above.  At each node the children are tested in draw order: q(x) <= 0
 * rejects without a uniform, else u < min(1, p(x)/q(x)) accepts and the walk
 * descends; a rejection sets p <- norm(max(p - q, 0)) (p / sum p when that mass
 * is <= 1e-12), zeroes q(x) and renormalises q, stopping when q has no mass
 * left; the next token is drawn from the current p where the walk stops.
 * Writes the accepted path (keep = [0] + path), tokens, next and n_uniforms;
 * status = WC_E_INVALID for an invalid tree, token or d2t.  Replaces
 * verify_tree_stochastic (python/woodcock/sampling.py:143-193;
 * src/sampling/sampling.cpp:116-141) as the engine calls it
 * (python/woodcock/spec.py:316-324). */
int wc_verify_tree_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, int head_rows,
                              int64_t ld_q, const int32_t* d2t_dev, const int32_t* tree_tokens_dev,
                              const int32_t* tree_parents_dev, const wc_uniforms* rng, wc_verdict* verdict_dev,
                              void* workspace, wc_stream_t stream);

/* wc_verify_tree_stochastic for a tree drafted on the device, whose size is
 * known only there: the node count is *count_dev (1 <= count <= rows; rows
 * bounds p and the tree arrays), and node v's draft distribution is row
 * q_rows_dev[v] of q [q_count][ld_q] (0 <= q_rows_dev[v] < q_count, else
 * status WC_E_INVALID).  Otherwise the same rule, uniforms and outputs.  The
 * engine's verify step after sampled tree drafting (python/woodcock/spec.py:
 * 321-324, q = kept[v].q). */
int wc_verify_tree_stochastic_indexed(const float* p, int rows, int vocab, int64_t ld_p, const float* q,
                                      int q_count, const int32_t* q_rows_dev, int head_rows, int64_t ld_q,
                                      const int32_t* d2t_dev, const int32_t* tree_tokens_dev,
                                      const int32_t* tree_parents_dev, const int32_t* count_dev,
                                      const wc_uniforms* rng, wc_verdict* verdict_dev, void* workspace,
                                      wc_stream_t stream);

/* ------------------------------------------------------------------ tree helpers */

/* Attention mask of a verify block holding a flattened draft tree: mask_out
 * [n][ld] (ld >= prefix + n) gets 1 for the prefix columns [0, prefix) and for
 * prefix + u when u is an ancestor of the row's node or the node itself, 0
 * elsewhere; parents_dev [n] with parents[0] = -1 and parents[i] < i (the walk
 * stops at a parent that breaks this).  Replaces tree_attention_mask
 * (python/woodcock/sampling.py:118-128; src/sampling/sampling.cpp:85-93). */
int wc_tree_mask(const int32_t* parents_dev, int n, int prefix, uint8_t* mask_out, int64_t ld, wc_stream_t stream);

/* Gumbel-top-k draws without replacement from each of `rows` draft
 * distributions q [rows][ld_q] over the head rows (renormalised in fp64; d2t_dev
 * maps head rows to token ids, NULL = identity): every nonzero entry, in
 * vocabulary order, consumes one uniform u of the stream (row r after the
 * uniforms of rows < r, the first at index uniform_base) and gets the key
 * log q(x) - log(-log u); tokens_out [rows][k_max] receives the min(k_r, nonzero
 * count) largest keys' tokens in descending key order, counts_out [rows] (may be
 * NULL) their number; k_dev [rows] per-row draw counts (NULL = k_max),
 * k_max <= 16.  Replaces sample_without_replacement
 * (python/woodcock/sampling.py:196-203) as tree drafting calls it per frontier
 * node (python/woodcock/spec.py:238-249). */
int wc_sample_without_replacement(const float* q, int rows, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                                  const int32_t* k_dev, int k_max, const wc_uniforms* rng, int64_t uniform_base,
                                  int32_t* tokens_out, int32_t* counts_out, wc_stream_t stream);

/* ------------------------------------------------------------------ greedy tree drafting
 * The drafting loop of SpeculativeDecoder._draft with a StaticPolicy in greedy
 * mode (python/woodcock/spec.py:216-303; policies.py:49-75) without a host
 * round trip per level: a node table (token, parent, depth, phat in fp64,
 * cache slot, feedback row) lives in a caller-owned device state of
 * wc_tree_draft_state_bytes() bytes, zero-initialised once (at most 512
 * nodes, width <= 8; the expansion's counters reset themselves).  The
 * caller runs, per level, the draft head (logits) and wc_tree_draft_expand_logits
 * (or wc_probs_from_logits at T = 1 and wc_tree_draft_expand) over the frontier
 * rows, and unless it is the last
 * level wc_tree_draft_frontier plus wc_drafter_forward with the inputs it
 * wrote; node ids and level ranges follow from the static shape (root 0, then
 * rows * width children per level). */
size_t wc_tree_draft_state_bytes(void);

/* Node 0 = the root token (*root_token_dev); the frontier is the root. */
int wc_tree_draft_begin(void* state, const int32_t* root_token_dev, wc_stream_t stream);

/* Children of the current frontier: for frontier row r (rows of it) the width
 * entries of q [rows][ld_q] with the largest probability (descending; the lower
 * head row first on a tie -- the reference's mx.argpartition leaves this order
 * open) become nodes node_base + r * width + j with token d2t_dev[row] (NULL =
 * identity), parent the frontier node and phat = phat(parent) * q in fp64
 * (spec.py:226-237). */
int wc_tree_draft_expand(void* state, const float* q, int rows, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                         int width, int node_base, wc_stream_t stream);

/* The same expansion from the head logits z [rows][ld] at T = 1, with no
 * probability row written (the greedy branch of spec.py:226-237 on
 * _draft_dist's q = softmax(z), spec.py:113-121): the children are the width
 * largest z (softmax is monotone; same order and tie rule) and each child's
 * q = exp(z - max) / sum exp(z - max) is formed from per-part row statistics.
 * Equal to wc_probs_from_logits (T = 1) + wc_tree_draft_expand up to the
 * association of the row sum (a few ulps of q and phat); one launch. */
int wc_tree_draft_expand_logits(void* state, const float* logits, int rows, int head_rows, int64_t ld,
                                const int32_t* d2t_dev, int width, int node_base, wc_stream_t stream);

/* Next frontier: the min(width, level size) nodes of [level_begin, level_end)
 * with the largest phat, earlier nodes first on a tie (Policy.select_frontier,
 * policies.py:52-53), in that order.  Writes the drafter forward's inputs for
 * frontier row r: tokens_out, feat_rows_out (feedback row of the node's parent;
 * the root's is row 0), positions_out = *offset_dev - 1 + depth, and mask_out
 * [rows][mask_ld] over cache slots: the prefix [lo, *offset_dev) with lo from
 * the sliding window (0 = none), the cache slots of the node's ancestors below
 * the root and its own slot *offset_dev + tree_cache + r (spec.py:281-294).
 * The node's feedback row becomes store_base + r.  level_begin = 0 takes the
 * level that the last wc_tree_draft_expand_sample appended (level_end is then
 * ignored) and fills rows [frontier size, width) of the outputs with padding
 * (the root token on feedback row 0 at position *offset_dev, seeing the prefix
 * and its own slot), so a drafter forward over `width` rows stays valid; the
 * outputs must hold `width` rows. */
int wc_tree_draft_frontier(void* state, int level_begin, int level_end, int width, const int32_t* offset_dev,
                           int tree_cache, int window, int store_base, int32_t* tokens_out, int32_t* feat_rows_out,
                           int32_t* positions_out, uint8_t* mask_out, int64_t mask_ld, wc_stream_t stream);

/* The verified tree (StaticPolicy.select_verify + _to_tree, policies.py:66-75;
 * spec.py:297-303): all n_nodes nodes when n_nodes - 1 <= budget, else the root
 * plus the budget nodes ranked first by (-phat, depth, id), in node order, with
 * parents remapped (-1 for the root).  *count_out receives the node count. */
int wc_tree_draft_select(const void* state, int n_nodes, int budget, int32_t* tokens_out, int32_t* parents_out,
                         int32_t* depth_out, int32_t* count_out, wc_stream_t stream);

/* ------------------------------------------------------------------ sampled tree drafting
 * SpeculativeDecoder._draft at T > 0 (python/woodcock/spec.py:238-249 with
 * Plan.children_for, policies.py:32-36, and StaticPolicy.select_verify keeping
 * every node, policies.py:67-69) on the same state: per level the draft head
 * over the frontier rows, q = wc_probs_from_logits at the temperature (spec.py:
 * 113-125), wc_tree_draft_expand_sample, and unless it is the last level
 * wc_tree_draft_frontier with level_begin = 0 plus a drafter forward over
 * `width` rows; then wc_tree_draft_select_all.  Node counts depend on the
 * draws, so they stay in the state. */

/* Children of the current frontier (the state's frontier rows, at most `rows`):
 * frontier row r draws m_r = min(width, budget left after the rows before it)
 * children -- the number is fixed before drawing; `budget` is the round's
 * draft budget, shared by every level since wc_tree_draft_begin -- without
 * replacement from q row r (q [rows][ld_q] over the head rows, renormalised in
 * fp64; d2t_dev maps head rows to tokens, NULL = identity): the m_r largest
 * keys log q(i) - log(-log u_i) over the nonzero entries, in descending key
 * order (the lower head row first on a tie), where u_i is value
 * v * H4 + i of the Philox stream rng (v the frontier node, H4 = head_rows
 * rounded up to a multiple of 4).  Children get phat = phat(parent) *
 * q(i) / sum(q) in fp64 and are appended in frontier order.  Replaces the
 * per-node sample_without_replacement draws of the drafting loop
 * (python/woodcock/sampling.py:196-203); each entry owns its uniform instead of
 * one sequential generator, so every row and part draws at once. */
int wc_tree_draft_expand_sample(void* state, const float* q, int rows, int head_rows, int64_t ld_q,
                                const int32_t* d2t_dev, int width, int budget, const wc_uniforms* rng,
                                wc_stream_t stream);

/* Every node of the table in node order (tokens, parents with -1 for the root,
 * depth), the row of each node's draft distribution in the caller's q store
 * (its feedback-store row, where the level's q was written; 0 for nodes never
 * expanded), and *count_out = the node count; rows [count, max_nodes) are
 * padding (the root token as a child of the root at depth 1) so a verify block
 * of max_nodes rows is a valid tree. */
int wc_tree_draft_select_all(const void* state, int max_nodes, int32_t* tokens_out, int32_t* parents_out,
                             int32_t* depth_out, int32_t* q_rows_out, int32_t* count_out, wc_stream_t stream);

/* ------------------------------------------------------------------ KV compaction */

/* In-place gather of the accepted entries of the last verify block, in every
 * layer, for K and V, in one launch: for i < n_keep, row start + keep[i] moves
 * to start + i (gather first, then write; nothing moves when keep is the
 * identity), then *offset_dev = start + n_keep.
 *   k_layers/v_layers: host arrays of n_layers device pointers, each
 *     [kv_heads][capacity][row_bytes] (mlx-lm layout [1, Hk, cap, D]).
 *   start_dev, keep_dev [max_keep], n_keep_dev: device ints (e.g. fields of a
 *     wc_verdict); keep must be strictly increasing with start + keep[i] < capacity,
 *     else nothing moves and *status_dev (if not NULL) is set to WC_E_INVALID.
 *   offset_dev may be NULL.
 * Replaces compact_cache (python/woodcock/target.py:159-175) and KVCache::compact
 * (src/cache/kv_cache.cpp:21-31). */
int wc_kv_compact(void* const* k_layers, void* const* v_layers, int n_layers, int kv_heads, int capacity,
                  int row_bytes, const int32_t* start_dev, const int32_t* keep_dev, const int32_t* n_keep_dev,
                  int max_keep, int32_t* offset_dev, int32_t* status_dev, wc_stream_t stream);

/* ------------------------------------------------------------------ drafter step */

#define WC_MAX_DRAFTER_LAYERS 4
#define WC_MAX_FEATURES 3
#define WC_MAX_STEP_ROWS 16 /* rows per drafter launch; longer inputs are tiled by the host */

/* DrafterConfig fields the kernels need (python/woodcock/drafter.py:33-49;
 * include/woodcock/drafter.h:16-24). */
typedef struct wc_drafter_dims {
  int32_t hidden, num_layers, heads, kv_heads, head_dim, inter, target_hidden, num_features, head_rows;
  int32_t vocab; /* embedding rows: token ids read on the device are clamped to [0, vocab) */
  float eps;
  int32_t window; /* 0 = full attention */
} wc_drafter_dims;

/* One decoder layer's device weights, bf16 row-major [out][in] (nn.Linear layout).
 * aux_norm / aux_q / aux_k / aux_v are NULL for layers without the token stream.
 * gate_frag / up_frag (optional, NULL = none): fragment-major copies of gate / up
 * (wc_weights_frag); when both are set, passes over several rows stream them. */
typedef struct wc_layer_weights {
  const void *in_norm, *post_norm, *aux_norm;
  const void *q, *k, *v, *o, *aux_q, *aux_k, *aux_v, *q_norm, *k_norm, *gate, *up, *down;
  const void *gate_frag, *up_frag;
} wc_layer_weights;

typedef struct wc_drafter_weights {
  const void* embed;                          /* [vocab][hidden] */
  const void* fc;                             /* [hidden][num_features * target_hidden] */
  const void* feature_norm[WC_MAX_FEATURES];  /* [target_hidden] each, NULL = feature_norm off */
  const void* final_norm;                     /* [hidden] */
  const void* head;                           /* [head_rows][hidden]: the restricted rows, gathered */
  const int32_t* d2t;                         /* [head_rows] head row -> token id; NULL = identity */
  const float* rope_cos;                      /* [rope_max_pos][head_dim/2] host recipe (wc_rope_table) */
  const float* rope_sin;
  int32_t rope_max_pos;
  wc_layer_weights layers[WC_MAX_DRAFTER_LAYERS];
} wc_drafter_weights;

/* Stochastic drafting: Gumbel-max over the head rows, uniforms from the
 * Philox4x64-10 stream (seed, *round_dev, purpose + row). */
typedef struct wc_gumbel {
  uint64_t seed;
  const int32_t* round_dev;
  int32_t purpose;
  float temperature;
} wc_gumbel;

/* cos/sin table of the rotate-half RoPE with the reference recipe:
 * inv_i = powf(base, -2i/D), angle = (float)pos * inv_i (src/backends/cpu_ops.cpp:61-77).
 * Host memory, [max_pos][D/2] each. */
int wc_rope_table(float* cos_out, float* sin_out, int max_pos, int head_dim, float base);

/* Device workspace for wc_drafter_fuse / wc_drafter_forward / wc_draft_head. */
size_t wc_drafter_workspace_bytes(const wc_drafter_dims* dims);

/* g[r] = fc(concat_f RMS_f(tap_f[row r])) for r < rows (device count *n_rows_dev
 * when not NULL).  taps: num_features device pointers, [.][tap_ld] of tap_dtype;
 * tap_rows_dev (optional) gathers tap rows (e.g. the accepted path, keep): row r
 * reads tap row tap_rows_dev[r], clamped into [0, tap_rows) -- the rows each tap
 * holds (ignored without tap_rows_dev), so stale entries past the device row
 * count never read outside the taps.
 * Replaces Drafter.fuse (python/woodcock/drafter.py:149-153; src/core/drafter.cpp:75-89). */
int wc_drafter_fuse(const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps, int tap_dtype,
                    int64_t tap_ld, const int32_t* tap_rows_dev, int tap_rows, int rows, const int32_t* n_rows_dev,
                    float* g_out, int64_t g_ld, void* workspace, wc_stream_t stream);

/* A chain round's verify and fuse in one launch: wc_verify_chain_greedy over
 * logits [rows][vocab] and the drafts, and wc_drafter_fuse of tap rows
 * 0..rows-1 into g_out (every row, no gather).  A chain keeps the prefix
 * [0..a] of its verify block (python/woodcock/spec.py:362-366) and the fuse is
 * row-wise (python/woodcock/drafter.py:149-153), so the fused rows 0..a are
 * the ones the update pass needs whatever a turns out to be.  Equal to the two
 * calls in sequence, which it makes when the shapes do not fit one launch
 * (one launch: 2..8 rows, three taps of 2048, every tap normed or none,
 * 16-byte logits rows, enough CUs beside the fuse's blocks for the verify's
 * chunks).  No counterpart call in the reference: its round runs the two
 * steps one after the other (python/woodcock/spec.py:356-372). */
int wc_verify_chain_greedy_fuse(const float* logits, int rows, int vocab, int64_t ld,
                                const int32_t* draft_tokens_dev, wc_verdict* verdict_dev, void* verify_workspace,
                                const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps,
                                int tap_dtype, int64_t tap_ld, float* g_out, int64_t g_ld, void* drafter_workspace,
                                wc_stream_t stream);

/* One drafting forward over `rows` tokens appended at cache offset
 * *offset_dev + offset_add: every layer (dual-stream layer 0, GQA attention
 * with q/k RMSNorm and rotate-half RoPE, SwiGLU MLP), then the final RMSNorm.
 *   tokens_dev [rows]; feat [rows][feat_ld] fp32 (feat_row_dev optionally
 *   gathers the feature rows: row r is feat_row_dev[r] + feat_row_add);
 *   k_cache/v_cache: num_layers device pointers [kv_heads][capacity][head_dim]
 *   of kv_dtype; positions_dev [rows] (NULL = offset + r); mask_dev
 *   [rows][mask_ld] uint8 over cache slots (NULL = causal, sliding window
 *   when dims->window > 0); n_rows_dev: device row count (rows <= WC_MAX_STEP_ROWS).
 *   Writes hidden_out / out_out [rows][hidden] fp32 (out_out = NULL leaves the
 *   final RMSNorm to the consumer, e.g. wc_draft_head_norm); when advance_dev
 *   is not NULL, *advance_dev = offset + rows after the last layer.
 * Replaces Drafter.__call__ (python/woodcock/drafter.py:164-191) and
 * Drafter::forward (src/core/drafter.cpp:91-136). */
int wc_drafter_forward(const wc_drafter_dims* dims, const wc_drafter_weights* w, const int32_t* tokens_dev,
                       const float* feat, int64_t feat_ld, const int32_t* feat_row_dev, int feat_row_add, int rows,
                       const int32_t* n_rows_dev, void* const* k_cache, void* const* v_cache, int kv_dtype,
                       int capacity, const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                       const uint8_t* mask_dev, int64_t mask_ld, float* hidden_out, float* out_out,
                       int32_t* advance_dev, void* workspace, wc_stream_t stream);

/* Draft head + argmax + d2t over `rows` output rows: logits z = out . head^T
 * (written when logits_out is not NULL, [rows][head_rows] fp32), token_out[r] =
 * d2t[argmax_r z] (lowest row wins a tie), row_out[r] = the row.  With gumbel,
 * the argmax is of z/T + Gumbel noise (a draw from softmax(z/T)).  With
 * token_out NULL (and logits_out given, no gumbel) only the logits are written:
 * no argmax (the tree drafter's levels choose their children from them).
 * out_row_dev optionally selects input row *out_row_dev + out_row_add (rows = 1).
 * Replaces Drafter.logits + mx.argmax + Drafter.token_ids
 * (python/woodcock/drafter.py:204-215; python/woodcock/spec.py:346). */
int wc_draft_head(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* out_rows, int64_t out_ld,
                  const int32_t* out_row_dev, int out_row_add, int rows, float* logits_out, int64_t logits_ld,
                  int32_t* token_out, int32_t* row_out, const wc_gumbel* gumbel, void* workspace,
                  wc_stream_t stream);

/* ------------------------------------------------------------------ verify-width target layer */

/* Device workspace for wc_target_layer with up to max_rows rows.  Zero-filled
 * once before its first use (wc_workspace_init): blocks of up to 16 rows count
 * their K splits on counters in it, which every call leaves at zero. */
size_t wc_target_workspace_bytes(const wc_drafter_dims* dims, int max_rows);

/* One-time weight layout for the verify-width GEMMs: w [rows][cols] bf16
 * row-major (nn.Linear [out][in]) -> out, the same bytes in fragment-major
 * order: 16-row tile T, 32-column step s, lane l of 64 holds w[16 T + l % 16]
 * [32 s + 8 (l / 16) .. + 8] at ((T cols / 32 + s) 64 + l) 8.  That is the A
 * operand of v_mfma_f32_16x16x32_bf16, so every weight load of the GEMM reads
 * one contiguous kilobyte.  rows a multiple of 16, cols of 32, out not
 * aliasing w.  No reference counterpart (a storage format: the reference keeps
 * nn.Linear weights row-major). */
int wc_weights_frag(const void* w, int rows, int cols, void* out, wc_stream_t stream);

/* One Qwen3 decoder layer over a verify block of `rows` <= 64 tokens, in place
 * on the fp32 residual stream x [rows][hidden]:
 *   h = x + W_o . attn(q_norm(W_q xn), k_norm(W_k xn), W_v xn), xn = RMS_in(x);
 *   x = h + W_down . (silu(W_gate hn) * W_up hn), hn = RMS_post(h);
 * RoPE at positions_dev [rows] (NULL = offset + r) from the cos/sin table
 * (wc_rope_table), mask_dev [rows][mask_ld] uint8 over cache slots (NULL =
 * causal; the tree mask of a draft tree), K/V of the block appended at
 * *offset_dev in k_cache / v_cache [kv_heads][capacity][head_dim] of kv_dtype.
 * The caller advances the offset after the last layer.  dims supplies hidden,
 * heads, kv_heads, head_dim, inter, eps and window; hidden, heads*head_dim and
 * inter must be multiples of 256; the aux fields of L are ignored; the
 * matrices q, k, v, o, gate, up and down are fragment-major (wc_weights_frag),
 * the norm gains plain.
 * Layer chaining: with next_norm (bf16 [hidden], the next layer's in_norm or
 * the final norm) the layer also leaves next_norm * x_out and the partial row
 * sums of squares of x_out in the workspace, and the next call (or
 * wc_target_head) given input_prepared = 1 and the same workspace starts from
 * them instead of preparing x itself.
 * Replaces _block_forward (python/woodcock/target.py:142-156) as called by
 * Target.__call__ with positions and a mask (target.py:82-116), and the layer
 * loop of Qwen3::forward (src/core/qwen3.cpp:86-111). */
int wc_target_layer(const wc_drafter_dims* dims, const wc_layer_weights* L, const float* rope_cos,
                    const float* rope_sin, int rope_max_pos, float* x, int rows, const int32_t* positions_dev,
                    const uint8_t* mask_dev, int64_t mask_ld, void* k_cache, void* v_cache, int kv_dtype,
                    int capacity, const int32_t* offset_dev, const void* next_norm, int input_prepared,
                    void* workspace, wc_stream_t stream);

/* Embedding rows of the target model for a verify block: out [rows][ld] fp32 =
 * table [vocab][hidden] bf16 at tokens_dev [rows] (ids clamped into the table).
 * Replaces Target.embed (python/woodcock/target.py:70-71). */
int wc_target_embed(const void* table, int vocab, int hidden, const int32_t* tokens_dev, int rows, float* out,
                    int64_t ld, wc_stream_t stream);

/* Target logits of a verify block: logits_out [rows][ld] fp32 =
 * RMSNorm(x; final_norm) . head_w^T, head_w [vocab][hidden] bf16 in
 * fragment-major order (wc_weights_frag of the tied embedding for Qwen3, its
 * rows padded to a multiple of 16), rows <= 64, as a streaming MFMA GEMM with the
 * activations split into bf16 hi + lo (fp32-level products).  Workspace: the
 * target-layer workspace for >= rows rows; input_prepared = 1 when the last
 * wc_target_layer call on it had next_norm = final_norm.  Replaces
 * Target.lm_head(model.norm(h)) (python/woodcock/target.py:73-76,113-114). */
int wc_target_head(const wc_drafter_dims* dims, const void* head_w, const void* final_norm, const float* x, int rows,
                   int vocab, float* logits_out, int64_t ld, int input_prepared, void* workspace,
                   wc_stream_t stream);

/* wc_draft_head for one pre-norm hidden row: the final RMSNorm is applied on the
 * fly (out = RMSNorm(hidden), drafter.py:190) and, when out_norm is not NULL,
 * written to out_norm at the same row index (*row_dev + row_add, or 0) -- the
 * drafter's `out` and, with post_norm, the next step's feedback
 * (drafter.py:193-194).  Lets wc_drafter_forward skip its final norm
 * (out_out = NULL) on the chain's critical path.  hidden_size must be a
 * multiple of 512 when out_norm is given.  Replaces Drafter.norm +
 * Drafter.logits + mx.argmax + Drafter.token_ids (drafter.py:190,204-215;
 * spec.py:346). */
int wc_draft_head_norm(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* hidden_rows,
                       int64_t hidden_ld, const int32_t* row_dev, int row_add, float* out_norm, int64_t out_ld,
                       float* logits_out, int64_t logits_ld, int32_t* token_out, int32_t* row_out,
                       const wc_gumbel* gumbel, void* workspace, wc_stream_t stream);

/* The chain step with the head's argmax hand-over moved out of the head launch.
 * wc_draft_head_norm_pending: wc_draft_head_norm for one row whose argmax is
 * left pending in the workspace (every block's maximum key, no token written),
 * so the head launch ends without a last-block reduction.
 * wc_drafter_forward_pending: wc_drafter_forward for one row whose token is that
 * pending argmax: its first QKV launch resolves it (the d2t-mapped token of the
 * largest key) as the token-embedding row, writes the token to token_out[0] and
 * the head row to row_out[0] (row_out may be NULL), and the attention launch after
 * it clears the keys for the next head.  The pair must run in this order on one
 * workspace and stream with nothing else on that workspace between them;
 * the result equals wc_draft_head_norm followed by wc_drafter_forward on its
 * token.  Needs hidden_size a multiple of 512 (at most 10240) and a first layer
 * with the token stream (EAGLE-3).  Same reference interfaces as the two calls
 * it replaces (drafter.py:190,204-215; spec.py:346-352). */
int wc_draft_head_norm_pending(const wc_drafter_dims* dims, const wc_drafter_weights* w, const float* hidden_rows,
                               int64_t hidden_ld, const int32_t* row_dev, int row_add, float* out_norm, int64_t out_ld,
                               float* logits_out, int64_t logits_ld, const wc_gumbel* gumbel, void* workspace,
                               wc_stream_t stream);
int wc_drafter_forward_pending(const wc_drafter_dims* dims, const wc_drafter_weights* w, int32_t* token_out,
                               int32_t* row_out, const float* feat, int64_t feat_ld, const int32_t* feat_row_dev,
                               int feat_row_add, void* const* k_cache, void* const* v_cache, int kv_dtype,
                               int capacity, const int32_t* offset_dev, int offset_add, const int32_t* positions_dev,
                               float* hidden_out, float* out_out, int32_t* advance_dev, void* workspace,
                               wc_stream_t stream);

/* ------------------------------------------------------------------ backend operations
 * The reference runtime's backend interface (include/woodcock/ops.h:9-24,
 * implemented on the CPU by src/backends/cpu_ops.cpp:45-115) on device fp32
 * buffers, for a backend under the reference's own C++ runtime
 * (Drafter::forward, src/core/drafter.cpp:106-133; Qwen3::forward,
 * src/core/qwen3.cpp:86-111).  Same argument meaning and layouts: activations
 * [rows][cols] row-major, attention K / V as KVCache rows [T][Hk][D].  Weights
 * are bf16 or fp32 (w_dtype).  The fused entry points above are the hot path;
 * these are single operations. */

/* y[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * w for r < rows, row length d,
 * the mean from an fp64 sum; x and y may alias.  Replaces ops::rmsnorm
 * (include/woodcock/ops.h:13; src/backends/cpu_ops.cpp:50-59). */
int wc_rmsnorm(const float* x, float* y, int rows, int d, const void* w, int w_dtype, float eps,
               wc_stream_t stream);

/* y[L][out] (+)= x[L][in] . W[out][in]^T (accumulate != 0 adds to y).
 * Replaces ops::linear (include/woodcock/ops.h:11; src/backends/cpu_ops.cpp:45-48). */
int wc_linear(const float* x, int L, int in, const void* W, int w_dtype, int out, float* y, int accumulate,
              wc_stream_t stream);

/* Rotate-half RoPE in place on x[L][heads][head_dim] at positions_dev[L]:
 * inv_i = powf(base, -2i/D) (formed on the host), angle = (float)pos * inv_i.
 * cos_table / sin_table [max_pos][D/2] (optional, from wc_rope_table) supply
 * cos / sin for positions below max_pos; otherwise the device computes them.
 * Replaces ops::rope (include/woodcock/ops.h:15; src/backends/cpu_ops.cpp:61-77). */
int wc_rope(float* x, int L, int heads, int head_dim, const int32_t* positions_dev, float base,
            const float* cos_table, const float* sin_table, int max_pos, wc_stream_t stream);

/* gate[i] = silu(gate[i]) * up[i] for i < n.  Replaces ops::silu_mul
 * (include/woodcock/ops.h:17; src/backends/cpu_ops.cpp:79-84). */
int wc_silu_mul(float* gate, const float* up, int64_t n, wc_stream_t stream);

/* softmax(scale * q K^T + mask) V: q [L][H][D], K / V [T][Hk][D] (GQA: head h
 * reads kv head h / (H / Hk)), mask [L][T] uint8 (NULL = all visible),
 * out [L][H][D], D <= 256.  Replaces ops::attention (include/woodcock/ops.h:19-21;
 * src/backends/cpu_ops.cpp:98-115). */
int wc_attention(const float* q, int L, int H, int Hk, int D, const float* K, const float* V, int T,
                 const uint8_t* mask, float* out, float scale, wc_stream_t stream);

/* In-place softmax of `rows` rows of n: exp(x - max) (0 at -inf), fp64 sum,
 * multiplied by (float)(1 / sum).  rows = 1 is ops::softmax
 * (include/woodcock/ops.h:22; src/backends/cpu_ops.cpp:86-96). */
int wc_softmax(float* x, int rows, int n, wc_stream_t stream);

/* KV rows of L tokens, k / v [L][row] fp32 (row = kv_heads * head_dim), copied
 * to rows *offset_dev + l of k_cache / v_cache [capacity][row] (rows outside
 * [0, capacity) are dropped: the caches are allocated up front and never
 * grow); then, when advance_dev is not NULL, *advance_dev = *offset_dev + L
 * clamped into [0, capacity] (advance_dev may be offset_dev), so an offset
 * never counts rows the append dropped.  Replaces KVCache::append +
 * commit (include/woodcock/cache.h:17-19; src/cache/kv_cache.cpp:8-19). */
int wc_kv_append(float* k_cache, float* v_cache, int capacity, int row, const float* k, const float* v, int L,
                 const int32_t* offset_dev, int32_t* advance_dev, wc_stream_t stream);

/* *offset_dev = n, stream-ordered (a kernel, graph-safe): the rollback of a
 * drafting phase.  Replaces KVCache::trim_to (include/woodcock/cache.h:19) and
 * the cache offset assignment of python/woodcock/spec.py:275-276,351-352. */
int wc_kv_set_offset(int32_t* offset_dev, int n, wc_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WOODCOCK_HIP_H */
