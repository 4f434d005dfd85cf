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

#define WC_ABI_VERSION 1
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
  int32_t status;      /* 0, or WC_E_INVALID when the device saw an invalid input */
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

/* Greedy tree verification fused with the target argmax: N = rows flattened
 * nodes, node 0 the root; tree_tokens_dev/tree_parents_dev [N] (parents[0] = -1,
 * children in ascending node order = draw order).  Writes the accepted path,
 * next, tokens and keep = [0] + path.  Replaces verify_tree_greedy
 * (python/woodcock/sampling.py:131-140; src/sampling/sampling.cpp:95-106). */
int wc_verify_tree_greedy(const float* logits, int rows, int vocab, int64_t ld, const int32_t* tree_tokens_dev,
                          const int32_t* tree_parents_dev, wc_verdict* verdict_dev, void* workspace,
                          wc_stream_t stream);

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

#ifdef __cplusplus
}
#endif

#endif /* WOODCOCK_HIP_H */
