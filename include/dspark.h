/*
 * dspark.h -- C ABI of the MI355X (gfx950) DSpark speculative-decode step.
 *
 * Plain C: pointers are device pointers the caller owns (hipMalloc'd or any device allocation), sizes are element
 * counts, fp16 tensors are passed as `const void*` holding IEEE binary16. Every entry point is stream-ordered on the
 * `stream` argument (a hipStream_t, NULL for the default stream), returns 0 on success and a positive code otherwise
 * (DSPARK_E* below for argument errors, a hipError_t value for a failed launch). Nothing throws across the ABI.
 * A context is not thread-safe: callers serialise calls on one context, as the reference's engine does
 * (internal/model/generate.go:63 "callers must serialize").
 *
 * Reference interfaces each entry point replaces are cited as file:line in jwyjohn/lfm3-1.7b-mi50.
 *
 * KV cache format (this library's own, chosen for the matrix cores): per attention layer two page pools of
 * n_pages x KVH x (32 * D) fp16, and an int32 block table mapping logical page (position / 32) to a physical page
 * (NULL = identity). Inside a (page, KV head) block:
 *   K: matrix-core operand order -- for key block b in {0,1} and k-step s < D/32, 64 lanes x 8 halves, lane
 *      (n = lane % 16, g = lane / 16) holding K[key][32 s + 8 g .. +8] with key = 8 (n / 4) + 4 b + n % 4;
 *   V: transposed, [D][32 keys].
 * dspark_kv_write is the one writer of this format (prefill and verify rounds both append through it).
 */
#ifndef DSPARK_H
#define DSPARK_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dspark_stream_t; /* hipStream_t */

enum {
  DSPARK_OK = 0,
  DSPARK_EINVAL = 1001,    /* a shape, pointer or size argument is out of range */
  DSPARK_ENOSPACE = 1002,  /* the workspace is smaller than the size query returned */
  DSPARK_EUNSUPPORTED = 1003,
};

#define DSPARK_PAGE_TOKENS 32
#define DSPARK_MT_MAX 64 /* verify tokens per round the State can hold (reference MT = 9, dspark.hip:65) */

/* ---------------------------------------------------------------- versions and sizes
 * Replaces lfm3_dspark_workspace_floats / layer_bytes / globals_bytes / state_bytes / max_tokens (dspark.hip:2955-2962). */
int dspark_abi_version(void);
int dspark_page_tokens(void);
int dspark_max_tokens(void);
int dspark_state_bytes(void);

/* ---------------------------------------------------------------- round state
 * struct State of dspark.hip:134-158 (Go mirror internal/model/dspark.go:52-77): the same 22 scalars in the same order,
 * then tokens[DSPARK_MT_MAX] (tokens[0] = anchor, tokens[1..M-1] = drafts). */
typedef struct dspark_state {
  int32_t a, anchor, count, rounds_left, limit, budget, eos, M, ctx_new, ctx_pos, ctx_lo, run, force_m, rounds_done,
      accepted, verified, miss, skip, skip_after, skip_rounds, stop_at, ckpt_slot;
  int32_t tokens[DSPARK_MT_MAX];
} dspark_state;

/* ---------------------------------------------------------------- verify attention
 * One layer's verify attention for M tokens at positions a..a+M-1 whose K/V are already in the pages (dspark_kv_write):
 * token t sees key position kpos iff kpos >= start, kpos <= (causal ? a + t : a + M - 1) and, for window > 0,
 * kpos > a + t - window. GQA: query head qh reads KV head qh / (QH / KVH). Output o = softmax(q k^T / sqrt(D)) v,
 * optionally times sigmoid(gate[t][qh]), stored as fp16 (out) and/or fp32 (out_f32).
 * Replaces verify_attention_paged / attention_v2 / attention_v3 / attention_pass + combine_phase
 * (dspark.hip:1070-1412, 1488-2130, 2132-2185; dispatch 2519-2556). */
typedef struct dspark_attn_args {
  const void* q;               /* fp16 [M][QH][D] (normed, rotated) */
  const void* k_pages;         /* fp16 K page pool */
  const void* v_pages;         /* fp16 V page pool (transposed pages) */
  const int32_t* block_table;  /* [ceil((a+M)/32)] logical -> physical page, NULL = identity */
  int64_t kv_pages;            /* pages in each pool (bounds every page access; pool bytes < 2 GiB) */
  void* out;                   /* fp16 [M][QH][D] or NULL */
  float* out_f32;              /* fp32 [M][QH][D] or NULL */
  const float* gate;           /* fp32 [M][QH] pre-sigmoid gate or NULL (target layers gate the output) */
  void* workspace;             /* split partials; size from dspark_verify_attention_workspace */
  size_t workspace_bytes;
  int32_t M, QH, KVH, D;       /* D in {64, 128}; QH % KVH == 0; 1 <= M <= DSPARK_MT_MAX */
  int32_t a, start, window, causal;
  int32_t splits;              /* key-range splits per KV head; 0 = automatic */
} dspark_attn_args;

size_t dspark_verify_attention_workspace(const dspark_attn_args* args);
int dspark_verify_attention(const dspark_attn_args* args, dspark_stream_t stream);
/* The two phases of dspark_verify_attention, for callers that schedule them apart (the reference separates them by a
 * grid barrier: attention phase, then combine_phase, dspark.hip:2519-2556): the key-split pass writes partials into
 * the workspace; the combine merges them (same args, same workspace, same stream order). */
int dspark_verify_attention_splits(const dspark_attn_args* args, dspark_stream_t stream);
int dspark_verify_attention_combine(const dspark_attn_args* args, dspark_stream_t stream);

/* ---------------------------------------------------------------- KV write (append / commit)
 * Writes K/V rows for positions pos0..pos0+n-1 into the pages: k, v fp16 [n][KVH][D] (row stride `row_stride`
 * elements between tokens, >= KVH*D). Verify rounds append the drafted block's K/V before attention; commit is then
 * the length update alone and rollback leaves the rejected rows to be overwritten (the reference copies fresh K/V at
 * commit instead, dspark.hip:2860-2877; prefill's kv_write, kernels/ops.hip:226-251, is the same call with pos0 = 0). */
int dspark_kv_write(const void* k, const void* v, int64_t row_stride, void* k_pages, void* v_pages,
                    const int32_t* block_table, int32_t KVH, int32_t D, int32_t pos0, int32_t n,
                    dspark_stream_t stream);

/* ---------------------------------------------------------------- verify argmax (greedy head)
 * best_keys[t] = max over r < V of key(pv, r), pv the repetition-penalised fp16-rounded logit (seen[] bitmap, plus
 * drafts tokens[1..t] not yet seen), key = ordered float bits << 32 | (0xFFFFFFFF - r). logits fp32 [M][V] or fp16
 * when logits_f16 != 0. best_keys must hold M u64 and is overwritten (no pre-zeroing needed).
 * Replaces head_run<false, M> (dspark.hip:2219-2318, key 967-971) for logits produced elsewhere. */
int dspark_verify_argmax(const void* logits, int32_t logits_f16, int32_t M, int32_t V, const uint32_t* seen,
                         const dspark_state* st, float rep, float inv_rep, uint64_t* best_keys, void* workspace,
                         size_t workspace_bytes, dspark_stream_t stream);
size_t dspark_verify_argmax_workspace(int32_t M, int32_t V);

/* ---------------------------------------------------------------- acceptance + commit
 * On the device State: acc = longest prefix with token(best[i]) == tokens[i+1]; emit drafts[1..acc] and the bonus
 * token(best[acc]) to out_tokens[count..]; mark them in seen; advance a by acc+1; update counters, skip/miss and run
 * exactly as dspark.hip:2848-2913. `skip_now` is the round's skip flag. The KV rows of positions a..a+acc are already
 * in the pages (dspark_kv_write before attention), so the commit moves no K/V. */
int dspark_accept_commit(dspark_state* st, const uint64_t* best_keys, int32_t M, int32_t skip_now, int32_t* out_tokens,
                         uint32_t* seen, dspark_stream_t stream);

/* ---------------------------------------------------------------- int8-weight verify GEMM
 * y[t][r] = scale[r] * sum_k x[t][k] * q[r][k] for t < M (M <= 64), r < N (N % 16 == 0), K % 64 == 0. Weights int8 [N][K] stored
 * biased (q + 128, the reference's weights.Pack byte format, internal/weights/quant.go:66-104) with one fp16 scale per
 * output row. epilogue: 0 = y fp32 [M][N] (y_f32) and/or fp16 (y_f16); 1 = gated SiLU on row pairs (even row gate,
 * odd row up; cmd/pack/main.go:337-345): h[t][r/2] = fp16(silu(g) * u) into y_f16 [M][N/2]; 2 = SiLU: y_f16 = fp16(silu(y)).
 * Replaces gemv_phase / unit_dot_r (dspark.hip:541-716). */
int dspark_gemm_i8(const void* x, int32_t M, int32_t K, const uint8_t* w, const void* scale, int32_t N,
                   int32_t epilogue, float* y_f32, void* y_f16, void* workspace, size_t workspace_bytes,
                   dspark_stream_t stream);
size_t dspark_gemm_i8_workspace(int32_t M, int32_t N, int32_t K); /* split-K partials (0 when not split) */

/* ---------------------------------------------------------------- cropped head + row argmax
 * y[t][r] = sum_k x[t][k] * W[r][k] (fp16 W [N][K], fp16 x [M][K], fp32 accumulation), and best_keys[t] = max key(y, r)
 * (first maximum). M <= 64, N % 16 == 0, K % 64 == 0. y_f32 may be NULL. best_keys is overwritten.
 * Replaces the drafter head GEMV into `base` + the argmax of markov_phase (dspark.hip:2564-2587, 2322-2366). */
int dspark_head_argmax_f16(const void* x, int32_t M, int32_t K, const void* w, int32_t N, float* y_f32,
                           uint64_t* best_keys, void* workspace, size_t workspace_bytes, dspark_stream_t stream);
size_t dspark_head_argmax_workspace(int32_t M, int32_t N);

/* token id of an argmax key */
static inline int32_t dspark_key_token(uint64_t key) { return (int32_t)(0xFFFFFFFFu - (uint32_t)key); }

#ifdef __cplusplus
}
#endif
#endif
