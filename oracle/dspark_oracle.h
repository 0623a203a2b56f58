/*
 * CPU oracle for the DSpark speculative-decode step -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's algorithm (jwyjohn/lfm3-1.7b-mi50), used only by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as the checker, never as the
 * product path. Every function cites the reference file:line it restates. Arithmetic is fp64 unless the
 * reference fixes a narrower rounding point (fp16 RNE before argmax, fp16 conv/bx stores, ...).
 *
 * Pinning status per function (what checks each one against something other than itself):
 *   fp16 RNE / widen ........ numpy float16 over all 65536 halves and edge floats (tests/test_oracle.py)
 *   generators .............. distribution moments; determinism (self-consistency only by nature)
 *   verify attention ........ numpy fp64 softmax, torch CPU scaled_dot_product_attention, closed forms
 *                             (single key -> V, equal scores -> mean of V), brute force on tiny shapes
 *   split merge ............. log-sum-exp identity vs the direct pass
 *   argmax key + penalty .... reference KATs internal/sample/sample_test.go:9-25 and numpy argmax
 *   accept / commit ......... invariants (0%/100% planting, offsets) + hand-worked cases
 *   int8 GEMM / crop head ... numpy fp64 matmul; quantization KATs internal/weights/quant_test.go:9-55
 *   Markov lane transpose ... reference KAT cmd/pack/main_test.go:8-28
 *   int8 K/V records ........ quantize_pair closed forms (half-away ties, clamp, the 1e-6 floor, exact multiples),
 *                             round-trip bound |x - q s| <= s/2, byte layout; Q group quantization vs numpy rint;
 *                             fp64 attention of dequantized operands vs orc_verify_attention on fp16-valued input
 *   per-128-column GEMM ..... numpy fp64 sum over groups; equal group scales reduce to the per-row GEMM; one group's
 *                             scales zeroed removes exactly its product (tests/test_oracle_g128.py)
 *   weights.Pack restated ... packed then reconstructed within half a code step per weight of the fp16 matrix product;
 *                             scale slots against the packer's index rule (tests/test_oracle_g128.py)
 *   int8 x (LFM3_X8) ........ closed forms: integer pieces with max 127 give scale 1 and the codes themselves, the
 *                             round-trip bound |x - q s| <= s/2, the all-zero piece at the 1e-20 floor, the +-127 code
 *                             at each piece's max; the x8 GEMM equals the group GEMM on codes times the piece scales
 *                             (fp64 numpy) and reduces to it at unit scales (tests/test_oracle_x8.py)
 *   target/drafter layers ... composed of the pinned pieces above + numpy restatements of RMS norm, RoPE,
 *                             short conv (tests/test_oracle.py::test_rms_norm_rope_conv)
 */
#ifndef DSPARK_ORACLE_H
#define DSPARK_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (internal/fp16/fp16.go) */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

/* ---- seeded counter-based generators (SplitMix64 -> Box-Muller -> RNE fp16) */
uint64_t orc_mix64(uint64_t x);
void orc_gen_normal_f16(uint64_t seed, uint64_t offset, int64_t n, float scale, uint16_t* out);
void orc_gen_int8_uniform(uint64_t seed, int64_t n, int8_t* out); /* uniform [-127, 127] */
void orc_gen_uniform_u32(uint64_t seed, int64_t n, uint32_t bound, uint32_t* out);

/* ---- verify attention (dspark.hip:975-978, 1296-1313, 2000-2015; App. A.6 of the step spec)
 * q [M][QH][D] fp16; k, v logical [T][KVH][D] fp16 with T >= a + M: positions < a are the cache,
 * a..a+M-1 the verified tokens' own (fresh) keys. Token t (position a+t) sees key kpos iff
 *   kpos >= start, and
 *   context (kpos < a): window == 0 || kpos > a + t - window
 *   fresh   (kpos = a + j, j < M): causal ? j <= t : 1
 * out [M][QH][D] fp64 = softmax(q k^T / sqrt(D)) v per query head, kv head = qh / (QH / KVH). */
void orc_verify_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                          int a, int start, int window, int causal, double* out);
/* Same over keys [k0, k1) only: base-2 partials m (max of log2-scaled score), l = sum 2^(s - m), acc = sum 2^(s-m) v
 * (combine_phase inputs, dspark.hip:2132-2185). m = -inf and l = 0 when no key is valid. */
void orc_attn_partial(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D, int a,
                      int start, int window, int causal, int k0, int k1, double* m, double* l, double* acc);
/* Merge S partials [S][M*QH] (+ acc [S][M*QH][D]) -> out [M*QH][D] (dspark.hip:2148-2183; 0 if total weight 0). */
void orc_attn_merge(int S, int rows, int D, const double* m, const double* l, const double* acc, double* out);
/* Multi-threaded fp32 variant for the CPU baseline (same masks; threads over (kv head, token)). */
void orc_verify_attention_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                             int a, int start, int window, int causal, double* out, int threads);
void orc_verify_attention_f32_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                                 int a, int start, int window, int causal, float* out, int threads);

/* ---- int8 K/V records (kernels/ops.hip:212-251; internal/model/engine.go:30-32; dspark.hip:1020-1046)
 * Record of (position, KV head): K int8[128] | f32 k scale | V int8[128] | f32 v scale (264 B), pages of 32 positions
 * laid out [page][slot][KV head][record]. */
float orc_rec_quantize(const float* x, int D, int8_t* q);
void orc_kv_write_rec(const float* k, const float* v, int n, int KVH, int pos0, const int32_t* bt, uint8_t* pages);
void orc_rec_quantize_q(const uint16_t* q, int rows, int D, int8_t* q8, float* qs);
void orc_verify_attention_d(const double* q, const double* k, const double* v, int M, int QH, int KVH, int D, int a,
                            int start, int window, int causal, double* out);
void orc_verify_attention_rec(const uint16_t* q, const uint8_t* pages, const int32_t* bt, int M, int QH, int KVH,
                              int a, int start, int window, int causal, double* out);

/* ---- argmax key and penalised verify argmax (dspark.hip:967-971, 2222-2300; internal/sample/sample.go:59-117) */
uint64_t orc_argmax_key(float v, uint32_t idx);
uint32_t orc_key_index(uint64_t key);
/* For t < M: vr = fp16(logit[t][r]); hit = seen[r] || (r == tokens[j] for 1 <= j <= t with tokens[j] unseen);
 * pv = hit ? (vr > 0 ? vr * inv_rep : vr * rep) : vr; best[t] = max key over r. */
void orc_verify_argmax(const float* logits, int M, int V, const uint32_t* seen_bits, const int32_t* tokens, float rep,
                       float inv_rep, uint64_t* best_keys);
/* Reference host Penalize (sample.go:75-90: divide when > 0, multiply otherwise) and Argmax (108-117, first max). */
void orc_penalize_rep(float* lg, int n, const int32_t* seen, int nseen, float rep);
int32_t orc_argmax_first(const float* lg, int n);

/* ---- round state, acceptance and commit (dspark.hip:134-158, 2848-2913; internal/model/dspark.go:52-77) */
#define ORC_MT_MAX 64
typedef struct {
  int32_t a, anchor, count, rounds_left, limit, budget, eos, M, ctx_new, ctx_pos, ctx_lo, run, force_m, rounds_done,
      accepted, verified, miss, skip, skip_after, skip_rounds, stop_at, ckpt_slot;
  int32_t tokens[ORC_MT_MAX];
} orc_state;
/* acc = longest prefix with best[i] == tokens[i+1]; books as dspark.hip:2852-2913. Returns acc.
 * best_tok[M] are token ids (the decoded keys). */
int orc_accept_commit(orc_state* st, const int32_t* best_tok, int m, int skip_now, int32_t* out_tokens, uint32_t* seen);
/* KV commit: for c <= acc, cache[a + c] <- fresh[c] ([T][KVH][D] logical rows of `row` halves). */
void orc_kv_commit(uint16_t* cache, const uint16_t* fresh, int a, int acc, int row);

/* ---- int8 weight formats (internal/weights/quant.go) */
void orc_quantize_rows_int8(const uint16_t* w, int rows, int k, int8_t* q, float* scales); /* quant.go:115-144 */
int orc_pack_srow(int k);                                                                     /* quant.go:24-29 */
void orc_pack_g128(const uint16_t* w, int rows, int k, uint8_t* biased, uint16_t* scales);     /* quant.go:66-104 */
void orc_transpose_lanes(const uint8_t* src, uint8_t* dst, int64_t n);                         /* cmd/pack/main.go:281-293 */

/* ---- verify GEMMs (dspark.hip:541-716 restated for per-output-channel scales) */
/* y[t][r] = scale[r] * sum_k x[t][k] * q[r][k]; w signed int8 [N][K] or biased (q+128) when biased != 0. */
void orc_gemm_i8(const uint16_t* x, const uint8_t* w, int biased, const uint16_t* scale, int M, int N, int K, double* y);
void orc_gemm_g128(const uint16_t* x, const uint8_t* w, const uint16_t* gs, int M, int N, int K, double* y);
/* LFM3_X8 (kernels/dspark.hip:24-26): GEMV inputs as int8 with one fp32 scale per 16 columns. quantize: per piece of
 * 16 values s = max(max|x| / 127, 1e-20) (fp32 division), q = rint(x * (1 / s)) (norm_compute 802-823, x_fill
 * 883-904; the reference takes 1 / s with the hardware reciprocal, here IEEE fp32). gemm: y[t][r] = sum over pieces p
 * of fp32(gs[p / 8][r] * s[t][p]) * (integer dot of the piece), summed in fp64 (unit_dot_r 541-566). */
void orc_quantize_x16(const float* x, int64_t n, int8_t* q, float* s);
void orc_gemm_x8(const int8_t* q, const float* s, const uint8_t* w, const uint16_t* gs, int M, int N, int K, double* y);
void orc_gemm_f16(const uint16_t* x, const uint16_t* w, int M, int N, int K, double* y);
/* First-max row argmax of y [M][N] (fp32 keys, ties -> smallest index). */
void orc_row_argmax(const float* y, int M, int N, int32_t* idx);

/* ---- layer pieces (dspark.hip:722-843, 2191-2214; kernels/ops.hip:193-224; internal/model/engine.go:428-461) */
/* RMS norm of n floats: y = x / sqrt(mean(x^2) + eps) * w (fp16 w). */
void orc_rms_norm(const float* x, const uint16_t* w, int n, float eps, float* y);
/* RoPE on pairs (i, i + D/2) for i < rot, angle pos * base^(-2i/D). */
void orc_rope(float* x, int D, int rot, double base, int pos);
/* Gated short conv (one channel, kernel K): bx = fp16(B*X); conv = w[K-1]*bx + sum_{k<K-1} w[k]*hist[k];
 * y = fp16(C*conv); hist shifts in bx. Returns y; hist updated in place. */
float orc_conv_step(float B, float C, float X, const float* w, int K, float* hist);
float orc_silu(float x);

#ifdef __cplusplus
}
#endif
#endif
