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
 * token t sees a context key kpos < a iff kpos >= start and, for window > 0, kpos > a + t - window, and the block's
 * key a + j iff j <= t (causal) or j < M (not causal): start and window bound the context keys only
 * (dspark.hip:1308-1312, 2006-2012). GQA: query head qh reads KV head qh / (QH / KVH). Output o = softmax(q k^T / sqrt(D)) v,
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
  void* workspace;             /* per-split partials (o, running max, sum); size from
                                  dspark_verify_attention_workspace. Needs no clearing: the key-split pass writes every
                                  partial the merge reads. Stream-ordered calls may share one workspace; calls that
                                  overlap on different streams need separate workspaces. */
  size_t workspace_bytes;
  int32_t M, QH, KVH, D;       /* D in {64, 128}; QH % KVH == 0; 1 <= M <= DSPARK_MT_MAX */
  int32_t a, start, window, causal;
  int32_t splits;              /* key-range splits per KV head; 0 = automatic */
} dspark_attn_args;

size_t dspark_verify_attention_workspace(const dspark_attn_args* args);
int dspark_verify_attention(const dspark_attn_args* args, dspark_stream_t stream);
/* dspark_verify_attention enqueues two kernels on the stream: the key-split pass (each split of a KV head's key range
 * writes an unnormalised partial output, its running max and its sum into the workspace) and the merge (partials
 * combined in split order, normalised, gated, stored). The two phases below are the same kernels called apart, for
 * callers that schedule them separately (the reference separates them by a grid barrier: attention phase, then
 * combine_phase, dspark.hip:2519-2556); same args, same workspace, same stream order. Both ways give bit-identical
 * outputs. */
int dspark_verify_attention_splits(const dspark_attn_args* args, dspark_stream_t stream);
int dspark_verify_attention_combine(const dspark_attn_args* args, dspark_stream_t stream);

/* dspark_verify_attention without a workspace and without allocating anything: no counterpart in the reference; for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid device
 * allocation). Same arguments and outputs as dspark_verify_attention except that args->workspace and
 * args->workspace_bytes are ignored: the split partials go to a static device array of the library,
 * DSPARK_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. Shapes whose partials need more
 * (dspark_verify_attention_workspace > DSPARK_NOALLOC_SCRATCH_BYTES) are refused with DSPARK_ENOSPACE before any
 * launch. The array needs no clearing (the split pass writes every partial the merge reads). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams, other threads) race; stream-ordered
 * calls do not. */
#define DSPARK_NOALLOC_SCRATCH_BYTES (16 << 20)
int dspark_verify_attention_noalloc(const dspark_attn_args* args, dspark_stream_t stream);

/* ---------------------------------------------------------------- KV write (append / commit)
 * Writes K/V rows for positions pos0..pos0+n-1 into the pages: k, v fp16 [n][KVH][D] (row stride `row_stride`
 * elements between tokens, >= KVH*D). Verify rounds append the drafted block's K/V before attention; commit is then
 * the length update alone and rollback leaves the rejected rows to be overwritten (the reference copies fresh K/V at
 * commit instead, dspark.hip:2860-2877; prefill's kv_write, kernels/ops.hip:226-251, is the same call with pos0 = 0). */
int dspark_kv_write(const void* k, const void* v, int64_t row_stride, void* k_pages, void* v_pages,
                    const int32_t* block_table, int64_t kv_pages, int32_t KVH, int32_t D, int32_t pos0, int32_t n,
                    dspark_stream_t stream);
/* kv_pages: pages in each pool. Without a block table, pos0 + n must fit the pools (DSPARK_EINVAL otherwise); with
 * one, a row whose table entry is outside [0, kv_pages) is not written. */

/* ---------------------------------------------------------------- int8 K/V records (the reference's KV format)
 * Per (position, KV head) one record of DSPARK_REC_BYTES = 264 bytes, K int8[128] | f32 k scale | V int8[128] |
 * f32 v scale, in pages of 32 positions laid out [page][slot][KV head][record] (KVBlock = 32 x KVH x 264 bytes), a
 * logical page (position / 32) mapped to a physical page by an int32 block table (NULL = identity). This is the
 * layout the reference's prefill and commit write (internal/model/engine.go:30-32, kernels/ops.hip:226-251,
 * dspark.hip:2860-2877), so a cache filled by the reference's writers is read as it is. */
#define DSPARK_REC_BYTES 264
/* Records of positions pos0 .. pos0+n-1 from fp32 k, v rows [n][row_stride] (head h at h * 128; K already normed and
 * rotated), each quantized as quantize_pair (ops.hip:212-224): scale = max(amax / 127, 1e-6), q = x * (1 / scale)
 * rounded half away from zero, clamped to [-128, 127]. Replaces kv_write (ops.hip:235-251) and the verified rows'
 * records of query_fresh (dspark.hip:1036-1046). Without a block table pos0 + n must fit the pool (DSPARK_EINVAL
 * otherwise); with one, a position whose entry is outside [0, kv_pages) is not written. */
int dspark_kv_write_rec(const float* k, const float* v, int64_t row_stride, void* pages, const int32_t* block_table,
                        int64_t kv_pages, int32_t KVH, int32_t pos0, int32_t n, dspark_stream_t stream);
/* dspark_verify_attention over a record pool: args->k_pages is the pool (kv_pages pages of 32 x KVH x 264 bytes, under
 * 2 GiB), args->v_pages must be NULL, D = 128 and KVH = 4 (the reference geometry), QH / KVH x M <= 64 rows per KV
 * head (16 verify tokens; the reference verifies at most 9). The reference's int8 numerics: Q quantized per 32-dim group (scale = max(amax / 127, 1e-20), q8 =
 * rint(q * rcp(scale))), exact int8 dot products scaled by the group and key scales, P = fp16(p * v scale * 2^k) on
 * int8 V, fp32 accumulation; the result is the softmax attention of those int8 Q/K/V within the reference's own error
 * (benchmarks/verify_attention.txt). Splits and merge as dspark_verify_attention (same workspace contract).
 * Replaces attention_pass / attention_v2 / attention_v3 over the int8 cache (dspark.hip:1070-1412, 1488-2130) and
 * combine_phase (2132-2185). */
size_t dspark_verify_attention_rec_workspace(const dspark_attn_args* args);
int dspark_verify_attention_rec(const dspark_attn_args* args, dspark_stream_t stream);
/* Its two phases called apart, as dspark_verify_attention_splits / _combine (bit-identical to the one call). */
int dspark_verify_attention_rec_splits(const dspark_attn_args* args, dspark_stream_t stream);
int dspark_verify_attention_rec_combine(const dspark_attn_args* args, dspark_stream_t stream);

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
                         int32_t out_cap, uint32_t* seen, dspark_stream_t stream);
/* out_cap: int32 slots in out_tokens (>= M). A commit that would write past it (State.count + acc + 1 > out_cap)
 * writes nothing and stops the run (State.run = 0), as a launch whose output buffer is full must stop. */

/* ---------------------------------------------------------------- int8-weight verify GEMM
 * y[t][r] = scale[r] * sum_k x[t][k] * q[r][k] for t < M (M <= 64), r < N (N % 16 == 0), K % 64 == 0. Weights int8 [N][K] stored
 * biased (q + 128, the reference's weights.Pack byte format, internal/weights/quant.go:66-104) with one fp16 scale per
 * output row. epilogue: 0 = y fp32 [M][N] (y_f32) and/or fp16 (y_f16); 1 = gated SiLU on row pairs (even row gate,
 * odd row up; cmd/pack/main.go:337-345): h[t][r/2] = fp16(silu(g) * u) into y_f16 [M][N/2]; 2 = SiLU: y_f16 = fp16(silu(y)).
 * One kernel launch. Up to 32 tokens a workgroup usually owns whole rows and sums its ranges of K in LDS: no workspace
 * (the size query returns 0). When K is split across workgroups (more tokens, or long K) the workspace holds a fixed
 * region of arrival counters (one per row group, at the same offset for every shape) followed by the split partials;
 * the last split of a group to arrive
 * sums the partials in split order (the same bits every call) and applies the epilogue. Zero-fill the workspace before
 * its first use: every call leaves its counters at zero again, so one workspace serves any number of stream-ordered
 * GEMM calls of any shapes (not calls that overlap, and not other entry points in between). Replaces gemv_phase /
 * unit_dot_r (dspark.hip:541-716). */
int dspark_gemm_i8(const void* x, int32_t M, int32_t K, const uint8_t* w, const void* scale, int32_t N,
                   int32_t epilogue, float* y_f32, void* y_f16, void* workspace, size_t workspace_bytes,
                   dspark_stream_t stream);
size_t dspark_gemm_i8_workspace(int32_t M, int32_t N, int32_t K); /* counters + split-K partials (0: no split) */
/* dspark_gemm_i8 with the reference's per-128-column weight scales (weights.Pack, internal/weights/quant.go:66-104):
 * y[t][r] = sum_g gscale[g][r] * sum_{k in group g} x[t][k] * q[r][k], groups of 128 columns, gscale fp16 [K/128][N]
 * (group-major: dspark_g128_scales converts the packer's [row][quarter][i] layout), weights biased int8 [N][K] as
 * above, fp16 x. M <= 16 (the reference verifies 9 tokens), K % 128 == 0; same epilogues; no workspace. Each
 * 128-column group's products are scaled in fp32 by the group's scale and added in group order. x stays fp16 here,
 * as in the reference's LFM3_F16 build; the reference's default build (LFM3_X8, dspark.hip:24-26, 802-823, which
 * kernels/build.sh uses) quantizes x to int8 per 16 columns first. Replaces gemv_phase / unit_dot_r over packed
 * weights (dspark.hip:541-716). */
int dspark_gemm_i8_g128(const void* x, int32_t M, int32_t K, const uint8_t* w, const void* gscale, int32_t N,
                        int32_t epilogue, float* y_f32, void* y_f16, dspark_stream_t stream);
/* dspark_gemm_i8_g128 with the reference's default activation format (LFM3_X8, kernels/dspark.hip:24-26): x as int8
 * with one fp32 scale per 16 columns. y[t][r] = sum over 16-column pieces p of fp32(gscale[p / 8][r] * s[t][p]) *
 * (sum_{k in p} q[r][k] * c[t][k]), the integer dots exact (unit_dot_r, dspark.hip:541-566). xscale NULL: x is fp16
 * [M][K] and is quantized per piece as it is loaded, s = max(max|x| / 127, 1e-20), c = rint(x * rcp(s)) (x_fill,
 * 883-904; rcp is the hardware reciprocal, as in the reference); xscale given: x holds the codes c as integer-valued
 * fp16 [M][K] and xscale the scales fp32 [M][K / 16] (the norm's output, norm_compute 802-823). Same shapes, epilogues
 * and no workspace as dspark_gemm_i8_g128. */
int dspark_gemm_i8_g128_x8(const void* x, const float* xscale, int32_t M, int32_t K, const uint8_t* w,
                           const void* gscale, int32_t N, int32_t epilogue, float* y_f32, void* y_f16,
                           dspark_stream_t stream);
/* Host helper: the packer's scale rows ([N][SRow] fp16, SRow = 16 for K = 2048 and 64 otherwise, entry (quarter, i) =
 * group 4 i + quarter at quarter * SRow / 4 + i; quant.go:13-29, 66-104) -> gscale [K/128][N]. No device memory. */
int dspark_g128_scales(const uint16_t* packed, int32_t N, int32_t K, uint16_t* out);
/* K must be a multiple of 512: weights.Pack stores group g's scale only while g / 4 < K / 512 (quant.go:96-99), so
 * another K leaves trailing groups with no stored scale (DSPARK_EINVAL). */

/* ---------------------------------------------------------------- cropped head + row argmax
 * y[t][r] = sum_k x[t][k] * W[r][k] (fp16 W [N][K], fp16 x [M][K], fp32 accumulation), and best_keys[t] = max key(y, r)
 * (first maximum). M <= 64, N % 16 == 0, K % 64 == 0. y_f32 may be NULL. best_keys is overwritten.
 * Replaces the drafter head GEMV into `base` + the argmax of markov_phase (dspark.hip:2564-2587, 2322-2366). */
int dspark_head_argmax_f16(const void* x, int32_t M, int32_t K, const void* w, int32_t N, float* y_f32,
                           uint64_t* best_keys, void* workspace, size_t workspace_bytes, dspark_stream_t stream);
size_t dspark_head_argmax_workspace(int32_t M, int32_t N);

/* ---------------------------------------------------------------- the full DSpark step (engine)
 * An engine owns one model (target + drafter weights, int8 GEMM weights as biased u8 with one fp16 scale per output
 * row) and the runtime buffers of one request, all in device memory of the device current at creation. A round is a
 * fixed launch sequence driven by the device State: context projection of the last round's committed tokens into the
 * drafter's KV ring, the drafter block [anchor, mask x (block-1)] through the drafter layers, the cropped head and the
 * Markov/confidence steps (drafts), the verify pass of the target layers over the whole block with the greedy head,
 * then acceptance + commit. Every kernel reads positions from the State and does nothing once State.run is 0, so
 * rounds are enqueued back to back with no host round trip (the reference runs up to 32 rounds in one persistent
 * launch, dspark.hip:2379-2950). Replaces Engine.draftLaunch + dspark_kernel (internal/model/dspark.go:537-621). */
#define DSPARK_MAX_LAYERS 64
#define DSPARK_MAX_TAPS 8

typedef struct dspark_model_desc {
  int32_t hidden;          /* H (multiple of 256) */
  int32_t ffn;             /* target FFN width I: w13 has 2 I rows (gate, up interleaved) */
  int32_t vocab;           /* V (multiple of 16) */
  int32_t n_layers;        /* target layers */
  int32_t layer_kind[DSPARK_MAX_LAYERS]; /* 0 gated short conv, 1 full attention, 2 sliding attention */
  int32_t q_heads, kv_heads, head_dim;   /* attention geometry (head_dim 64 or 128) */
  int32_t conv_kernel;     /* short-conv taps (<= 8) */
  int32_t window;          /* sliding-window length of kind-2 layers */
  float rope_base;         /* RoPE base; rope_pairs rotating pairs per head (<= head_dim / 2) */
  int32_t rope_pairs;
  int32_t draft_layers;    /* drafter attention layers */
  int32_t draft_ffn;       /* drafter FFN width */
  int32_t block;           /* drafter block = max verified tokens per round (<= 64) */
  int32_t max_drafts;      /* drafts per round (<= block - 1) */
  int32_t crop_rows;       /* N rows of the cropped head (multiple of 16); row N is the confidence row */
  int32_t markov_rank;     /* rank of the Markov head (multiple of 16) */
  int32_t n_taps;          /* tapped target layers feeding the drafter */
  int32_t tap_layer[DSPARK_MAX_TAPS];
  int32_t draft_window;    /* drafter attention window over its context ring */
  int32_t ring_positions;  /* drafter context ring (multiple of 32, > draft_window + block) */
  int32_t mask_token;
  float conf_bias, conf_thr;
  float eps;               /* RMS-norm epsilon */
  /* RoPE of the sliding-window layers (kind 2), when it differs from the table above (which serves full attention
   * and the drafter): the reference builds base 1e6 with 32 pairs for full layers and the drafter, base 1e4 with 64
   * pairs for sliding layers (internal/model/engine.go:333-338). rope_base_swa <= 0: sliding layers use the first. */
  float rope_base_swa;
  int32_t rope_pairs_swa;
  int32_t conv_slots;      /* conv-state slots per conv layer, slot 0 the running state (engine.go:122, 138); >= 1 */
  /* K/V format of the target's attention layers and the drafter ring: 0 fp16 pages in matrix-core order (above), 1 the
   * reference's int8 records (DSPARK_REC_BYTES per position and KV head, quantize_pair; engine.go:30-32), which needs
   * head_dim 128, kv_heads 4 and q_heads / kv_heads x block <= 64. Tensors "kv.L<i>.rec" / "ring.D<j>.rec" then hold
   * the record pages instead of "kv.L<i>.k|v" / "ring.D<j>.k|v". */
  int32_t kv_format;
  /* Scales of the int8 weights ("<name>.s"): 0 one fp16 scale per output row ([N]); 1 the reference's per-128-column
   * group scales (weights.Pack, internal/weights/quant.go:66-104) as fp16 [K/128][N] (dspark_g128_scales converts the
   * packer's layout), which needs block <= 16. */
  int32_t weight_format;
  /* Activations of the int8 GEMMs: 0 fp16; 1 the reference's default build (LFM3_X8, kernels/dspark.hip:24-26):
   * every GEMM input quantized to int8 with one fp32 scale per 16 columns -- by the norm kernel from its fp32 output
   * (norm_compute, 802-823), as it is loaded from fp16 sources (x_fill, 883-904) -- and multiplied int8 by int8
   * (unit_dot_r, 541-566). Needs weight_format 1. */
  int32_t x_format;
} dspark_model_desc;

typedef struct dspark_engine dspark_engine;

/* RoPE table of `positions` rows: out[p][i] = fp16(cos f), out[p][D/2 + i] = fp16(sin f) for i < D/2, with
 * f = (double)((float)p * inv[i]), inv[i] = 1 / (float)pow(base, (float)(2 i) / D) for i < pairs and 0 beyond (a pair
 * that does not rotate), fp16 by round-to-nearest-even. Host code, no device memory; the engine builds its tables with
 * it. Replaces Engine.buildRope (internal/model/engine.go:428-461). */
int dspark_rope_table(float base, int32_t pairs, int32_t head_dim, int32_t positions, uint16_t* out);

/* Allocate weights (uninitialised) and runtime buffers for contexts up to max_context positions. DSPARK_EINVAL for a
 * description outside the documented ranges, or a max_context whose per-layer K/V page pool would reach 2 GiB (the
 * attention kernels address a pool with 32-bit byte offsets). */
int dspark_engine_create(const dspark_model_desc* desc, int32_t max_context, dspark_engine** out);
void dspark_engine_destroy(dspark_engine* e);
/* Random-initialise every weight on the device from `seed` (synthetic benchmarks; no host copy of the weights). */
int dspark_engine_init_random(dspark_engine* e, uint64_t seed, dspark_stream_t stream);
/* Device pointer and size of a named tensor -- weights ("embed", "head.w", "L3.mix.w", "D0.w13.s", ...), caches
 * ("kv.L2.k", "ring.D1.v", "conv.L0") and runtime state ("state", "seen", "out_tokens", "logits", "base", ...); the
 * full list is dspark_engine_tensor_name(e, i) for i < dspark_engine_tensor_count(e). */
int dspark_engine_tensor(dspark_engine* e, const char* name, void** ptr, size_t* bytes);
int dspark_engine_tensor_count(dspark_engine* e);
const char* dspark_engine_tensor_name(dspark_engine* e, int32_t i);
/* Build what the round reads derived from the weights: a tile-major copy of every int8 GEMM weight (each wave's
 * weight load one contiguous 1 KB) and the drafter's Markov transition table (crop_rows <= 16384), T[c][r] =
 * w1q[crop_ids[c]] . w2q[r], from which every draft step after the first reads one row instead of the whole w2q. What
 * may be stale is rebuilt by itself before the next round: everything after dspark_engine_init_random, a GEMM
 * weight's copy after a dspark_engine_tensor lookup of that weight, the table after a lookup of "markov.w1q",
 * "markov.w1s", "markov.w2q", "conf_c2" or "crop_ids". A caller that writes weights through pointers obtained
 * earlier calls this (it rebuilds everything) before its next round. No counterpart in the reference, whose kernel
 * reads its own packed weights directly (dspark.go:635-659) and takes the Markov dots at every step (markov_phase,
 * dspark.hip:2322-2366). */
int dspark_engine_prepare(dspark_engine* e, dspark_stream_t stream);
/* Enqueue one round on `stream`. The verify pass is 1 + max_drafts rows wide (at least force_m). force_m > 0 skips
 * the drafter and verifies tokens[0..force_m) of the State as they are (the reference's force_m debug mode,
 * dspark.hip:147, 2442-2451). force_m = -1 runs the drafter, then replaces
 * its drafts by the engine tensor "plant" (int32 by position: draft j of a round at anchor position a is plant[a + j])
 * -- benchmarks of a set acceptance rate on random-init models; this mode has no counterpart in the reference. The first call for a (force_m, plan) records
 * the round as a HIP graph; later calls replay it. `plan_a` is the position the attention plan is tuned for (any
 * run-time a is correct; the plan is re-recorded when plan_a moves to another 4096-position bucket). */
int dspark_engine_round(dspark_engine* e, int32_t force_m, int32_t plan_a, dspark_stream_t stream);

/* Set the repetition-penalty mask to exactly the given tokens (ids outside the vocabulary are ignored) and the
 * penalty the next rounds use (0 = 1). Replaces Engine.InitSeen (internal/model/engine.go:617-629), which Generate
 * calls once per request with the prompt (generate.go:105); rounds then add every token they emit. */
int dspark_engine_init_seen(dspark_engine* e, const int32_t* tokens, int32_t n, float rep, dspark_stream_t stream);

/* Drafter context seeding at prefill. capture_tap: rows of the hidden state h (fp16, row stride `row_stride` elements)
 * of positions context .. context + tokens - 1, taken after the tapped target layer `slot`, are RMS-normed with
 * tap_norms[slot] into the engine's capture buffer from position max(context, tap_from) on (tap_from = the first
 * position the request captures; the buffer holds draft_window positions from it). Replaces captureTap
 * (internal/model/dspark.go:439-459). project_prompt: the captured positions [first, end) (first = tap_from,
 * end - first <= draft_window) through fc, the hidden norm and ckv, then per drafter layer the k norm, RoPE and the K/V
 * rows into the drafter's ring at their positions. Replaces projectPrompt (dspark.go:461-492); beginDraft's
 * bookkeeping (dspark.go:494-515) is the caller's: the next launch takes ctx_new = 0, ctx_pos = a, ctx_lo = first. */
int dspark_engine_capture_tap(dspark_engine* e, int32_t slot, const void* h, int64_t row_stride, int32_t context,
                              int32_t tokens, int32_t tap_from, dspark_stream_t stream);
int dspark_engine_project_prompt(dspark_engine* e, int32_t first, int32_t end, dspark_stream_t stream);

/* Copy conv-state slot src to slot dst in every conv layer (tensors "conv_state.L<i>", [conv_slots][H][conv_kernel-1]
 * fp16, element (c, k) at c * (conv_kernel - 1) + k, the reference's layout, engine.go:546-547). Replaces
 * Engine.CopyConvSlot (internal/model/prefill.go:596-606). */
int dspark_engine_conv_copy(dspark_engine* e, int32_t src, int32_t dst, dspark_stream_t stream);

/* draftLaunch: run rounds from the sequence's last token to the next 32-position block boundary (the State fields
 * a, anchor, limit, budget, eos, stop_at, ctx_*, miss, skip, ckpt_slot are set from the arguments as
 * internal/model/dspark.go:543-566 does: stop_at = min(next multiple of 32 after a, max_context), limit =
 * min(stop_at + block, max_context)), then copy the State and the emitted tokens back. Synchronous on `stream`.
 * Rounds run until the State stops (run == 0, dspark.hip:2438-2440) or `rounds` have run: the host keeps on the
 * stream only rounds that the books of the last finished round prove necessary (each round mirrors its books into
 * host memory, which the calling thread polls while later rounds run, as the reference's host spins on its mailbox),
 * so a launch enqueues no round that would find run == 0 (an eos can leave the rounds already in flight idle).
 * Each round verifies 1 + the launch's draft cap tokens (the reference verifies 1 + drafts, dspark.hip:2657): a
 * 3-draft launch verifies 4. The first `skip` rounds are skip rounds (dspark.hip:2441-2451): the context projection,
 * then the anchor alone verified without drafting, State.skip decremented; skip_after stays 0 (draftLaunch never
 * sets it), so no round starts skipping again. After the launch, rounds outside a launch (dspark_engine_round) use
 * the model's max_drafts and the penalty of the last dspark_engine_init_seen again.
 * With conv_slot >= 0 the launch first loads the conv history of positions a - (conv_kernel - 1) .. a - 1 from that
 * conv-state slot into the engine's position ring, and at its end writes the running state (the history before the
 * final a) back to the slot and, when ckpt_slot >= 0 and the launch reached stop_at, the history before stop_at to
 * ckpt_slot (dspark.hip:2415-2431, 2921-2947). conv_slot = -1 keeps the ring as the previous launch left it. */
typedef struct dspark_launch_args {
  int32_t a;               /* position of the anchor (= len(tokens) - 1), < max_context */
  int32_t anchor;          /* token at position a */
  int32_t budget;          /* tokens this launch may emit (capped at 512) */
  int32_t eos;             /* stop token or -1 */
  float rep;               /* repetition penalty (1 = none) */
  int32_t rounds;          /* rounds per launch (the reference uses 32) */
  int32_t ctx_new, ctx_pos, ctx_lo;  /* drafter context bookkeeping carried between launches */
  int32_t force_m;         /* > 0: verify-only rounds of the State's tokens (the tokens array below); -1: planted
                              drafts (see dspark_engine_round) */
  int32_t tokens[DSPARK_MT_MAX];
  int32_t max_drafts;      /* drafts per round this launch (<= 0: the model's max_drafts); the reference's policy is
                              7, or 3 for a request whose decode starts at position >= 57344 (dspark.go:568-571) */
  int32_t miss, skip;      /* acceptance-miss / skip counters carried from the previous launch (dspark.go:560, 615) */
  int32_t conv_slot;       /* running conv-state slot (the reference's step conv slot, engine.go:548), or -1 */
  int32_t ckpt_slot;       /* conv checkpoint slot for stop_at (cache.allocConv, dspark.go:550), or -1 */
} dspark_launch_args;

typedef struct dspark_launch_result {
  int32_t count;           /* tokens emitted */
  int32_t rounds, accepted, verified;
  int32_t boundary;        /* the block boundary the launch ran to */
  int32_t ckpt_written;    /* 1: the launch reached the boundary and ckpt_slot holds the conv state there */
  dspark_state state;      /* State after the launch (ctx_new, ctx_pos, miss, skip carry to the next launch) */
  int32_t rounds_enqueued; /* rounds the launch put on the stream (equals rounds unless an eos stopped it early) */
} dspark_launch_result;

int dspark_engine_launch(dspark_engine* e, const dspark_launch_args* args, int32_t* out_tokens, int32_t max_out,
                         dspark_launch_result* result, dspark_stream_t stream);

/* Phase tracing. With tracing on, every round records a mark after each of its phases (the round's HIP graph gains a
 * one-thread kernel per mark that stores the GPU's constant-rate clock; marks cost about a kernel launch each, so
 * traced rounds run a little slower). dspark_engine_trace_read copies the marks recorded since tracing was turned on:
 * out[2 i] = phase (DSPARK_TRACE_* below; verify layer L is DSPARK_TRACE_VERIFY_LAYER + L) | round << 32, out[2 i + 1]
 * = the clock in nanoseconds; *n = the number of marks (at most DSPARK_TRACE_MAX_MARKS are kept). The difference of
 * consecutive marks is the time of a phase. Replaces the reference's trace buffer (trace_mark, dspark.hip:384-391;
 * LFM3_DS_TRACE, internal/model/dstrace.go). */
enum {
  DSPARK_TRACE_BEGIN = 0,        /* round started (State checked, keys cleared) */
  DSPARK_TRACE_CONTEXT = 1,      /* context projection into the drafter ring */
  DSPARK_TRACE_DRAFTER = 2,      /* drafter layers */
  DSPARK_TRACE_CROP_HEAD = 3,    /* cropped head */
  DSPARK_TRACE_MARKOV = 4,       /* Markov / confidence drafts */
  DSPARK_TRACE_LM_HEAD = 5,      /* final norm + LM head */
  DSPARK_TRACE_COMMIT = 6,       /* argmax + acceptance + commit */
  DSPARK_TRACE_VERIFY_LAYER = 16 /* + L: target layer L of the verify pass */
};
#define DSPARK_TRACE_MAX_MARKS 65536
int dspark_engine_trace(dspark_engine* e, int32_t enable, dspark_stream_t stream);
int dspark_engine_trace_read(dspark_engine* e, uint64_t* out, int32_t cap, int32_t* n);

/* Layer-boundary dumps (a debug aid, as the reference's raw dbg_logits dump, dspark.hip:186, 2285). With dumps on,
 * every round records, before each drafter layer j and before the draft norm, and before each target layer i and
 * before the final norm, the residual stream h and the value the next norm adds to it (the previous layer's FFN
 * output, its K bands summed in band order; zeros before the first layer) into the tensor "debug_layers":
 * fp32 [draft_layers + 1 + n_layers + 1][2][block][hidden], slot j (drafter j, block rows), slot draft_layers (before
 * the draft norm), slot draft_layers + 1 + i (target layer i, the verify rows), slot draft_layers + 1 + n_layers
 * (before the final norm); [0] = h, [1] = the added value. Rounds with dumps on are recorded as their own graphs and
 * run one small kernel more per layer. */
int dspark_engine_debug_layers(dspark_engine* e, int32_t enable);

/* token id of an argmax key */
static inline int32_t dspark_key_token(uint64_t key) { return (int32_t)(0xFFFFFFFFu - (uint32_t)key); }

#ifdef __cplusplus
}
#endif
#endif
