// Internal launch descriptors shared between the kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

struct dspark_state;

namespace dspark {

typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int CONV_RING = 128;  // conv history positions kept per layer (>= max verify tokens + kernel - 1)

struct AttnParams {
  const struct ::dspark_state* st;  // when set: a (and the drafter's ctx_lo) come from the State at run time
  int drafter;                      // with st: start = max(ctx_lo, a - window), no per-token window
  const _Float16* q;
  const _Float16* kp;
  const _Float16* vp;
  const int32_t* bt;
  uint32_t k_bytes, v_bytes;  // page pool sizes (range of the buffer loads; < 2 GiB)
  float* part_acc;   // [KVH][RG][R][S][D] (row-major: one row's splits contiguous for the merge)
  f32x2_t* part_ml;  // [KVH][RG][R][S] (max, sum); max = -inf when the split saw no key of the row
  _Float16* out16;            // [M][QH][D], or operand order (xop_elem, column qh D + d) when out_op > 0
  float* out32;
  // LFM3_X8: out16 receives the int8 codes of the fp16 outputs (integer-valued halves: what the next GEMM would make of
  // them as it loads them) and out_sc their scales, piece c / 16 of output column c = qh D + d at t out_sc_row + c / 16
  float* out_sc;
  int out_sc_row;
  const float* gate;
  int out_op;                 // > 0: out16 in the verify GEMM's X operand order with out_op token blocks
  int M, QH, KVH, G;
  int a, start, window, causal;
  int page0, npages, pps, S;  // logical page range and its split
  int RG, QB, R, OCC;         // row groups, 16-row blocks per wave, rows per group, workgroups per CU
  int lds, nrb, pl, ppl, lpw; // LDS-ring kernel: row blocks, page lanes, pages per lane per step, loads per wave per step
  int qb, nrg;                // LDS-ring kernel: row blocks per wave, row groups (waves per page lane, nrg * qb >= nrb)
  int full_lo, full_hi;       // pages inside [full_lo, full_hi] need no mask
  float c;                    // log2(e) / sqrt(D)
  int gate_stride;            // > 0: gate of (t, qh) at gate[t * gate_stride + qh] (else t * QH + qh)
  // Fresh block (mix set; the LDS kernel with D = 64, one row block per wave and M <= waves): Q and the block's own
  // K/V (positions a .. a + M - 1) from the attention-mix GEMM's rows instead of q and the pages -- per token
  // `mix_row` floats, q heads at 0, k heads at QH D, v heads at (QH + KVH) D; the q/k RMS norm (q_norm / k_norm, eps)
  // and RoPE (rope [positions][D]: cos | sin, pairs (i, i + D / 2) for i < rot) done here, as the q/k norm + RoPE
  // kernel does. The split holding a fresh position patches its LDS copy of that page and writes the K/V rows into
  // the pages for later rounds.
  const float* mix;
  int mix_row, rot;
  const _Float16* q_norm;
  const _Float16* k_norm;
  const _Float16* rope;
  float eps;
};

void attn_plan(AttnParams& p, int D, int cus);
// attn_range (attn_range.h): the same plan evaluated on the device from the State's a.

struct ResNormParams {
  const struct ::dspark_state* st;
  const float* h_old;           // [groups][M][H] or nullptr (zero)
  const float* v;               // bands of [M][H], v_band_stride apart, or nullptr
  int bands;
  size_t v_band_stride;
  const _Float16* post_w;       // [H] or nullptr (1)
  const _Float16* norm_w;       // [groups][H]
  size_t norm_w_stride;
  int sandwich;
  float eps;
  float* dst;                   // h_new [groups][M][H] or nullptr
  float* tap;                   // [M][H] or nullptr
  _Float16* x16;                // [groups][M][x_row], or operand order (xop_elem, column g x_group_stride + i) when xop
  size_t group_stride, x_group_stride;
  int x_row;
  int H;
  int xop;                      // > 0: x16 in the verify GEMM's X operand order with xop token blocks
  // LFM3_X8: x16 receives int8 codes (integer-valued halves) and xsc their fp32 scales, one per 16 columns, piece
  // c / 16 of token t at t xsc_row + c / 16 (c the x column); nullptr: fp16 x
  float* xsc;
  int xsc_row;
  // h_old from the embedding table instead (the first layer of a pass, embed_kernel's rows; h_old must be null): row
  // t is embed[token(t)], token(t) = st->tokens[t] (embed_mode 0) or t == 0 ? st->anchor : mask_token (1); tokens
  // outside the vocabulary read row 0
  const _Float16* embed;
  int embed_mode, mask_token, vocab;
};

struct QkRopeParams {
  const struct ::dspark_state* st;
  const float* mix;             // per token: q [QH*D] | k [KVH*D] | v [KVH*D] | gate [QH]   (q absent when !q16)
  int row;                      // floats per token row
  int M, QH, KVH, D, rot;
  const _Float16* q_norm;
  const _Float16* k_norm;
  const _Float16* rope;         // [positions][D]: cos | sin
  float eps;
  _Float16* q16;                // [M][QH][D] or nullptr (context projection: K/V only)
  float* gate;                  // [M][QH] or nullptr
  int gate_in_mix;
  _Float16* kp;                 // K/V page pools and block table
  _Float16* vp;
  uint8_t* rec;                 // or (D = 128): the int8 record pool ([page][slot][KVH][264]), written instead
  const int32_t* bt;
  int pos_from_ctx, count_from_ctx;  // positions st->ctx_pos + t, tokens t < st->ctx_new (context projection)
};

constexpr int QKROPE_BATCH = 8;
struct QkRopeBatch {
  QkRopeParams l[QKROPE_BATCH];  // same M, QH, KVH
  int n;
};
int qkrope_batch_launch(const QkRopeBatch& b, hipStream_t s);

struct MarkovParams {
  struct ::dspark_state* st;
  const float* base;            // [block][stride] crop-head outputs; column N is the confidence term
  int stride, N, rank, block, max_drafts;
  const int8_t* w2q;            // [N][rank]
  const float* w2s;             // [N]
  const int8_t* w1q;            // [vocab][rank]
  const float* w1s;             // [vocab]
  const float* c2;              // [vocab]
  const int32_t* crop_ids;      // [N]
  uint64_t* best;               // [block] argmax keys (cleared by round_begin)
  const int32_t* max_drafts_dev;  // when set: the launch's draft cap (min with max_drafts), read at run time
  float conf_bias, conf_thr;
  const float* table;           // [N][N] w1q[crop_ids[c]] . w2q[r] (markov_table_launch), or nullptr: steps dot w2q
  const float* c2c;             // [N] c2[crop_ids[c]]
  const float* s1c;             // [N] w1s[crop_ids[c]]
  // Planted drafts (benchmarks of a set acceptance rate on random-init models), or nullptr: after the drafter's own
  // drafts, tokens[1 .. cap] = plant[a + 1 .. a + cap] and M = 1 + cap (the cap markov_kernel applies)
  const int32_t* plant;
};

int embed_launch(const void* embed, const struct ::dspark_state* st, int mode, int mask_token, int M, int H, int V, float* h,
                 hipStream_t s);
int resnorm_launch(const ResNormParams& p, int rows, int groups, hipStream_t s);
int qkrope_launch(const QkRopeParams& p, hipStream_t s);
int markov_launch(const MarkovParams& p, hipStream_t s);
// Transition table of the drafter's Markov head for crop_rows N <= 16384 (steps after the first read one row of it).
int markov_table_launch(const int8_t* w1q, const float* w1s, const float* c2, const int8_t* w2q, const int32_t* crop_ids,
                        int N, int rank, int vocab, float* T, float* c2c, float* s1c, hipStream_t s);
int round_begin_launch(struct ::dspark_state* st, uint64_t* keys, int nkeys, uint32_t* seen, int block, int max_pos,
                       int vocab, int out_cap, hipStream_t s);
int force_m_launch(struct ::dspark_state* st, int m, hipStream_t s);
// Layer-boundary dump of a debug round: h [rows][H] and the band sum of v ([bands][rows][H], band stride rows x H)
// into dst[0] and dst[1] (each block x H floats).
int layer_dump_launch(float* dst, const float* h, const float* v, int bands, int rows, int H, int block, hipStream_t s);
// Phase trace mark: buf = [count, round << 1 | active, (phase | round << 32, clock) ...]; `begin` marks open a round
// (counted only when the State runs), later marks of an inactive round record nothing.
int trace_mark_launch(uint64_t* buf, const struct ::dspark_state* st, int phase, int begin, int max_marks, hipStream_t s);
int plant_launch(struct ::dspark_state* st, const int32_t* plant, int block, int max_drafts, const int32_t* max_drafts_dev,
                 hipStream_t s);

// Conv state <-> the engine's position ring of conv history (CONV_RING positions x H per conv layer). The state of a
// slot is [H][conv_k - 1] fp16 (channel-major, the reference's layout); history k of it is the position p - (conv_k - 1)
// + k before position p. load: the ring positions before st->a from slot `slot`; store: the positions before st->a to
// slot `slot` and, when st->ckpt_slot >= 0 and st->a >= st->stop_at, those before st->stop_at to st->ckpt_slot;
// copy: slot src -> slot dst.
constexpr int CONV_MAX_LAYERS = 64;
struct ConvStateArgs {
  _Float16* ring[CONV_MAX_LAYERS];
  _Float16* state[CONV_MAX_LAYERS];  // [slots][H][conv_k - 1]
  int n, H, km1, slots;
};
int conv_load_launch(const ConvStateArgs& a, const struct ::dspark_state* st, int slot, hipStream_t s);
int conv_store_launch(const ConvStateArgs& a, const struct ::dspark_state* st, int slot, hipStream_t s);
int conv_copy_launch(const ConvStateArgs& a, int src, int dst, hipStream_t s);
// rows of fp16 h (row stride in elements) -> fp16(x * rsqrt(mean(x^2) + eps) * w) at out + row * out_stride
int rms_rows_launch(const _Float16* h, int64_t h_stride, const _Float16* w, float eps, int H, _Float16* out,
                    int64_t out_stride, int rows, hipStream_t s);
size_t attn_workspace_bytes(const AttnParams& p, int D);
// Carves the split partials out of a workspace of attn_workspace_bytes (256-byte aligned pieces).
void attn_bind_workspace(AttnParams& p, int D, void* ws);
// phases: 1 split pass (partials into the workspace), 2 merge of those partials, 3 both
int attn_launch(AttnParams& p, int D, int phases, hipStream_t s);
int kv_write_launch(const void* k, const void* v, int64_t row_stride, void* kp, void* vp, const int32_t* bt,
                    int64_t kv_pages, int KVH, int D, int pos0, int n, hipStream_t s);

// Verify attention over int8 K/V records (attn_rec.hip): D = 128, 4 KV heads, one workgroup per key split of all heads,
// up to ATTN_REC_MAX_SPLITS splits (the merge takes any split count); same partial format and merge as the fp16 path
// (the workspace size is attn_workspace_bytes(p, 128) of the planned p).
constexpr int ATTN_REC_MAX_SPLITS = 256;
void attn_rec_plan(AttnParams& p, int cus);
int attn_rec_launch(AttnParams& p, int phases, hipStream_t s);
// quantize_pair records of positions pos0 .. pos0 + n - 1 from fp32 k, v rows ([n][row_stride], head h at h * 128).
int kv_write_rec_launch(const float* k, const float* v, int64_t row_stride, void* pages, const int32_t* bt,
                        int64_t kv_pages, int KVH, int pos0, int n, hipStream_t s);

// The State's run flag read with a vector load (issued in order with the kernel's data loads, so a kernel can put it
// first and test it after its loads are in flight, instead of a scalar load the compiler waits for at the next use of
// any kernel argument). 1 when there is no State. Test with run_flag_set().
__device__ __forceinline__ int run_flag_load(const dspark_state* st) {
  if (!st) return 1;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)st, (short)0, (int)sizeof(dspark_state), 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)offsetof(dspark_state, run), 0, 0);
}
__device__ __forceinline__ bool run_flag_set(int v) { return __builtin_amdgcn_readfirstlane(v) != 0; }
// Any State word by the same kind of load (byte offset `off`; st must not be null).
__device__ __forceinline__ int state_word_load(const dspark_state* st, int off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)st, (short)0, (int)sizeof(dspark_state), 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// fp16 of the exact product a b, rounded once (what fp16(a b) computed in float64 gives): the fp32 product rounded to
// odd -- the nearest-even product moved one step toward the exact one when it is inexact and even (the residual from
// an fma) -- then rounded to nearest-even fp16; rounding to odd at 24 bits before rounding at 11 is exact rounding.
// Written out so that every epilogue rounds the same way, whether or not the compiler would fuse the product into
// the conversion.
__device__ __forceinline__ _Float16 f16_product(float a, float b) {
  const float p = a * b;
  const float e = fmaf(a, b, -p);
  uint32_t u = __builtin_bit_cast(uint32_t, p);
  if ((e > 0.f || e < 0.f) && !(u & 1u) && (p > 0.f || p < 0.f)) u += (e > 0.f) == (p > 0.f) ? 1u : 0xffffffffu;
  return (_Float16)__builtin_bit_cast(float, u);
}

// ---------------------------------------------------------------- LFM3_X8 pieces of fp16 values
// The scale of a 16-value piece whose largest magnitude is the finite fp16 value m (x_fill, kernels/dspark.hip:883-904):
// max(m / 127, 1e-20), with m / 127 taken as q0 = fl(m r), r = fl(1 / 127), corrected by one residual step,
// fl(q0 + fl(m - q0 127) r) -- equal to the IEEE quotient for every finite fp16 m.
__device__ __forceinline__ float x8_piece_scale(float m) {
  const float r127 = 1.f / 127.f;
  const float q0 = m * r127;
  return fmaxf(fmaf(fmaf(-q0, 127.f, m), r127, q0), 1e-20f);
}
// |h| of an fp16 value as its bit pattern (for non-negative halves the unsigned order of the patterns is the order of
// the values, so maxima can be taken on integers).
__device__ __forceinline__ uint32_t x8_mag_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h) & 0x7fffu; }
__device__ __forceinline__ float x8_mag_value(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
// x's code at inv = rcp(its piece's scale): rint(x * inv), an integer in [-127, 127], as a half.
__device__ __forceinline__ _Float16 x8_code(_Float16 x, float inv) { return (_Float16)rintf((float)x * inv); }

struct GemmParams {
  const struct ::dspark_state* st;  // when set, a stopped round (run == 0) skips the launch's work
  const _Float16* x;        // [M][K]
  const void* w;            // [N][K] biased int8 or fp16
  const _Float16* scale;    // [N] or nullptr
  const _Float16* gscale;   // or [K / 128][N]: one fp16 scale per (128-column group, row), the reference's per-128
                            // format (internal/weights/quant.go:66-104); K-sliced plans with one token block only
  float* y32;               // [M][N]
  _Float16* y16;            // [M][N] ([M][N/2] for the gated epilogue)
  float* part;              // split-K partials [ksplit][M][N]
  uint64_t* best_part;      // row-argmax keys per strip [M][N/16] (head) or nullptr
  uint64_t* best;           // [M]
  int M, N, K, ksplit, epilogue;
  uint32_t* counters;       // split-K arrival counter per group (zero between calls); nullptr: separate reduce kernel
  int wpg;                  // waves (16-row strips) per workgroup (gemm_plan)
  int cpb;                  // 64-column chunks per weight-load batch: 4 or 8 (gemm_plan)
  int kw;                   // > 0: K-sliced plan, workgroups of wpg strips x kw ranges of K (ksplit 1, gemm_plan)
  int xd;                   // K-sliced, int8, one token block: each wave loads its own range of X (no LDS staging)
  int bands;                // K-sliced, > 1: K in `bands` shares over as many workgroups, band b's scaled sums to
                            // y32 + b M N (epilogue 0, y32 only): the caller adds the bands (the norm kernel does)
  int xop;                  // > 0: x in operand order (xop_elem) with xop >= ceil(M / 16) token blocks; 0: row-major
  int yop;                  // > 0: the fp16 output y16 in operand order with yop token blocks (for the next GEMM's X)
  int tiled;                // int8 weights tile-major: [N / 16][K / 64][1 KB tile], lane l's 16 B at 16 l
  // Fused row-group epilogue (the group's scaled products go through LDS; y32 is not written):
  //   GEMM_FUSE_CONV: each group is 16 channels [B, C, X] of the conv mix (48 rows): gated short conv, y16 [M][N/3]
  //     and the conv history ring at st->a + t (conv_wave)
  int fuse;
  // LFM3_X8 (with gscale only): 1 x is fp16, quantized per 16-column piece as it is loaded; 2 x holds int8 codes as
  // integer-valued halves and xsc their fp32 scales, [token][xsc_row] with piece k / 16 of token t at t xsc_row + k / 16
  int x8;
  const float* xsc;
  int xsc_row;
  // LFM3_X8 output (gated epilogue 1 of a K-sliced plan with an even number of strips per workgroup and one band, or
  // GEMM_FUSE_CONV; group scales only): y16 receives the int8 codes of the fp16 outputs and ysc their scales,
  // [token][ysc_row] with output column c's piece at t ysc_row + c / 16 (the next GEMM reads them with x8 = 2)
  float* ysc;
  int ysc_row;
  const _Float16* conv_w;   // [N/3][conv_k]
  _Float16* conv_ring;      // [CONV_RING][N/3]
  int conv_k;
};
constexpr int GEMM_FUSE_CONV = 2;

struct GemmPlan {
  int ksplit = 1, wpg = 1, cpb = 4, kw = 0, xd = 0, bands = 1;
};
// wpg_req > 0 fixes the strips per workgroup (a fused epilogue's group: 3 for GEMM_FUSE_CONV);
// xop: X comes in operand order (GemmParams::xop); max_bands > 1: the caller adds up to that many output bands
// (GemmParams::bands).
void gemm_plan(int M, int N, int K, bool i8, bool split, GemmPlan* pl, int wpg_req = 0, bool xop = false,
               int max_bands = 1, bool gs = false);
// Split-K workspace: GEMM_COUNTER_BYTES of arrival counters (one u32 per row group, at the same offset for every shape),
// then the partials. Zero-filled once; every call leaves its counters at zero.
constexpr int GEMM_COUNTER_SLOTS = 8192;
constexpr size_t GEMM_COUNTER_BYTES = GEMM_COUNTER_SLOTS * sizeof(uint32_t);
size_t gemm_ws_bytes(const GemmPlan& pl, int M, int N);
size_t gemm_ws_bytes(int M, int N, int K, int wpg_req = 0, bool xop = false);  // for the plan of an int8 GEMM
int gemm_groups(const GemmPlan& pl, int N);                  // row groups (<= GEMM_COUNTER_SLOTS for a split plan)
uint32_t* gemm_ws_counters(void* ws);
float* gemm_ws_partials(void* ws);
int gemm_launch(GemmParams& p, bool i8, hipStream_t s);
// Tile-major copy of an int8 weight [N][K] (the layout GemmParams::tiled reads), N % 16 == 0, K % 64 == 0; x8: the
// order of the int8-x products (LFM3_X8), piece-major within a lane's 16 bytes.
int gemm_tile_launch(const void* src, void* dst, int N, int K, hipStream_t s, int x8 = 0);

size_t verify_argmax_ws(int M, int V);

// fold = false: the partial keys [M][verify_argmax_chunks(V)] stay in ws for accept_commit_fold_launch to fold.
int verify_argmax_launch(const void* logits, int f16, int M, int V, const uint32_t* seen, const dspark_state* st,
                         float rep, float inv_rep, uint64_t* best, void* ws, hipStream_t s, const float* rep_dev = nullptr,
                         bool fold = true);
int verify_argmax_chunks(int V);
int accept_commit_launch(dspark_state* st, const uint64_t* best, int m, int skip_now, int32_t* out_tokens, int out_cap,
                         uint32_t* seen, hipStream_t s);
// The verify argmax's partial keys folded into best[M] (as fold_keys would), then accept + commit of State->M tokens.
// skip_now: the round is a skip round (State.skip is decremented instead of the miss count kept). mirror (optional):
// host memory that receives the State's run, a, count, rounds_left, skip, miss, accepted, verified after the books
// (words 1-8) between two copies of rounds_done (word 15 first, word 0 last).
int accept_commit_fold_launch(dspark_state* st, const uint64_t* part, int nchunks, int M, uint64_t* best,
                              int32_t* out_tokens, int out_cap, uint32_t* seen, int skip_now, int32_t* mirror,
                              hipStream_t s);

}  // namespace dspark
