// The DSpark engine: model + request buffers in device memory, one round as a fixed launch sequence recorded into a
// HIP graph, and the draftLaunch protocol over it.
//
// Round (reference dspark_kernel sections, dspark.hip:2438-2919):
//   begin      clear the round's argmax keys, mark the anchor seen
//   context    last round's committed positions: tap norms -> fc (all taps in one K = taps*H GEMM) -> hidden norm
//              -> ckv GEMM -> per drafter layer k norm + RoPE, K/V into the drafter ring        (sec 0, 2487-2518)
//   drafter    embed [anchor, mask x (B-1)] -> layers (norm, q|k|v, RoPE + ring write, block attention over the
//              ring, out, norm, gated FFN) -> final norm -> cropped head into `base`            (sec 1)
//   drafts     Markov/confidence steps (markov_kernel x (B-1), finalize)                        (2633-2664)
//   verify     embed tokens -> target layers (sandwich norms, mix GEMM, gated conv | q/k norm + RoPE + K/V append +
//              verify attention + gated combine, out GEMM, gated FFN) -> final norm -> LM head -> penalised argmax
//   commit     acceptance + books; K/V of the accepted positions are already in the pages          (2848-2913)
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

using namespace dspark;

namespace {

struct Tensor {
  void* ptr;
  size_t bytes;
};

struct LayerW {
  int kind = 0;  // 0 conv, 1 full attention, 2 sliding attention, 3 drafter attention
  _Float16 *op_norm = nullptr, *ffn_norm = nullptr, *post_op_norm = nullptr, *post_ffn_norm = nullptr;
  uint8_t* mix_w = nullptr;
  _Float16* mix_s = nullptr;
  int mix_rows = 0;
  uint8_t *out_w = nullptr, *w13_w = nullptr, *w2_w = nullptr;
  _Float16 *out_s = nullptr, *w13_s = nullptr, *w2_s = nullptr;
  int ffn = 0;
  _Float16 *conv_w = nullptr, *conv_ring = nullptr;
  _Float16 *q_norm = nullptr, *k_norm = nullptr;
  _Float16 *kv_k = nullptr, *kv_v = nullptr;
  uint8_t* kv_rec = nullptr;  // int8 record pages (kv_format 1) instead of kv_k / kv_v
  int64_t kv_pages = 0;
  const int32_t* bt = nullptr;  // drafter ring table (target layers: identity)
  int tap_slot = -1;
};

int align16(int x) { return (x + 15) / 16 * 16; }

constexpr int ROUND_PLAN_BUCKET = 4096;

}  // namespace

struct dspark_engine {
  dspark_model_desc d;
  int max_context = 0, B = 0;
  std::vector<std::string> names;
  std::map<std::string, Tensor> tensors;
  std::vector<LayerW> L, DL;
  _Float16 *embed = nullptr, *final_norm = nullptr, *draft_norm = nullptr, *tap_norms = nullptr, *hidden_norm = nullptr;
  uint8_t *head_w = nullptr, *crop_w = nullptr, *fc_w = nullptr, *ckv_w = nullptr;
  _Float16 *head_s = nullptr, *crop_s = nullptr, *fc_s = nullptr, *ckv_s = nullptr;
  int32_t* crop_ids = nullptr;
  int8_t *w2q = nullptr, *w1q = nullptr;
  float *w2s = nullptr, *w1s = nullptr, *c2 = nullptr;
  // Markov transition table [crop_rows][crop_rows] with c2 and w1s gathered by crop index (markov_table_launch);
  // rebuilt before the next round whenever a weight it depends on may have been written
  float *mtab = nullptr, *mc2c = nullptr, *ms1c = nullptr;
  bool mtab_dirty = true;
  // Tile-major copies of the int8 GEMM weights (what the round's GEMMs read), rebuilt by dspark_engine_prepare from
  // the row-major tensors whenever one may have been written
  struct TiledW {
    const uint8_t* src;
    uint8_t* dst;
    int N, K;
    bool dirty;
  };
  std::vector<TiledW> tiles;
  std::map<const void*, size_t> tile_of;       // row-major weight -> its tile entry
  std::map<std::string, size_t> tile_by_name;  // tensor name -> its tile entry
  bool tiles_dirty = true;
  _Float16* rope = nullptr;      // full attention and drafter layers: [positions + 1][D] cos | sin
  _Float16* rope_swa = nullptr;  // sliding layers (== rope when the description gives them no table of their own)
  int rot_swa = 0;
  int32_t* ring_bt = nullptr;
  int ring_pages = 0;
  int64_t kv_pages = 0;
  // request state
  dspark_state* st = nullptr;
  dspark_state* ast = nullptr;  // the State the kernels being enqueued read (st, or a prompt-projection chunk's)
  uint32_t* seen = nullptr;
  int32_t* out_tokens = nullptr;
  int32_t* plant = nullptr;  // planted drafts by position (force_m = -1 rounds)
  float* rep = nullptr;  // launch parameters read by the kernels: rep, 1/rep (floats 0, 1), draft cap (int32 at 2)
  // conv state slots of every conv layer ("conv_state.L<i>") and the rings they load into / store from
  ConvStateArgs conv = {};
  // drafter context seeding: normed taps of captured prompt positions [tap_rows][n_taps * H] from tap_from, and one
  // State per projection chunk (ctx_pos, ctx_new of the chunk)
  _Float16* tapx = nullptr;
  int tap_rows = 0, tap_from = -1;
  dspark_state* seed_st = nullptr;
  int seed_chunks = 0;
  std::vector<dspark_state> host_seed;
  std::vector<uint32_t> host_seen;
  // activations
  float *h[2] = {nullptr, nullptr}, *mix = nullptr, *vout = nullptr, *w2out = nullptr, *ctxv = nullptr, *ckvout = nullptr,
        *taps = nullptr, *logits = nullptr, *base = nullptr, *gate = nullptr;
  _Float16 *x16 = nullptr, *q16 = nullptr, *y16 = nullptr, *a16 = nullptr;
  // x_format 1: the int8 codes' scales of the norm outputs in x16; every scale buffer is [16 tbs][x_cols / 16]
  float* xsc = nullptr;
  // x_format 1: the scales of the codes the attention merge, the conv epilogue and the gated epilogue write into y16
  // or a16 (each read by the next GEMM before the other is written)
  float* ysc = nullptr;
  // the context projection's own norm outputs (tap norms, then the hidden norm) and their int8-x scales
  _Float16* xc16 = nullptr;
  float* xcsc = nullptr;
  // whether those producers write codes (else the out and w2 GEMMs quantize y16 / a16 as they load them: the same codes
  // and scales, so bit-identical rounds; DSPARK_X8_PRODUCER_CODES=0 at engine creation selects that form)
  bool y_codes = false;
  uint64_t* keys = nullptr;  // [B] verify best, then [B] Markov best
  void* ws_attn = nullptr;
  size_t ws_attn_bytes = 0;
  void* ws_gemm = nullptr;
  size_t ws_gemm_bytes = 0;
  void* ws_argmax = nullptr;
  size_t ws_argmax_bytes = 0;
  int x_cols = 0, mix_cols = 0, crop_n = 0;
  int tbs = 1;  // 16-token blocks of the round: x16, y16 and a16 hold 16 tbs token rows in the GEMMs' X operand order
  int cus = 256;
  dspark_state host_st;  // launch-time uploads stay alive until the stream has consumed them
  float host_lp[4] = {1.f, 1.f, 0.f, 0.f};
  float seen_rep = 1.f;  // the penalty of the last dspark_engine_init_seen (what rounds outside a launch use)
  float host_lp_idle[4] = {1.f, 1.f, 0.f, 0.f};  // the values restored at the end of a launch
  // host memory the commit kernel mirrors the State's books into after every round (accept_commit_fold_launch), read
  // by the launch loop while later rounds run
  int32_t* mirror = nullptr;
  // recorded rounds: key (force_m, tracing, verify width, skip, plan bucket) -> graph
  std::map<std::vector<int>, hipGraphExec_t> graphs;
  // phase tracing: marks [2 + 2 DSPARK_TRACE_MAX_MARKS] u64 (count, round | active, then (phase, clock) pairs)
  uint64_t* trace = nullptr;
  bool trace_on = false;
  // layer-boundary dumps of debug rounds: [draft_layers + 1 + n_layers + 1][2][B][H] fp32 (dspark_engine_debug_layers)
  float* dump = nullptr;
  bool dump_on = false;
  std::vector<void*> allocs;
  // whether attention layers that can take their block fresh from the mix rows do (attn_fresh_ok); DSPARK_FRESH=0 at
  // engine creation runs the q/k norm + RoPE kernel before every attention instead (for comparisons)
  bool fresh = true;
  int fresh_rec_pps = 8;  // the record kernel's least pages per split for a fresh block (DSPARK_FRESH_REC_PPS)

  ~dspark_engine() {
    for (auto& g : graphs) (void)hipGraphExecDestroy(g.second);
    for (void* p : allocs) (void)hipFree(p);
    if (mirror) (void)hipHostFree(mirror);
  }

  void* alloc(const std::string& name, size_t bytes, int* err) {
    if (*err) return nullptr;
    void* p = nullptr;
    const size_t nb = bytes ? bytes : 16;
#ifdef DSPARK_ALLOC_ROUND
    const size_t ab = (nb + (DSPARK_ALLOC_ROUND) - 1) / (DSPARK_ALLOC_ROUND) * (DSPARK_ALLOC_ROUND);
#else
    const size_t ab = nb;
#endif
    if (hipMalloc(&p, ab) != hipSuccess || hipMemset(p, 0, nb) != hipSuccess) {
      *err = DSPARK_ENOSPACE;
      return nullptr;
    }
    allocs.push_back(p);
    if (!name.empty()) {
      names.push_back(name);
      tensors[name] = Tensor{p, nb};
    }
    return p;
  }
};

namespace {

// ---------------------------------------------------------------- random init (synthetic benchmarks)
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// kind 0: biased int8 (q + 128), q uniform in [-127, 127]; 1: fp16 uniform [a, b); 2: fp16 N(a, b^2);
// 3: fp32 uniform [a, b); 4: signed int8 uniform [-127, 127]; 5: fp16 per-row GEMM scale u / sqrt(K) with u uniform
// in [a, b) (b holds K).
__global__ void rand_fill_kernel(void* dst, size_t n, int kind, float a, float b, uint64_t seed) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const uint64_t r = mix64(seed ^ mix64(i));
    const float u = (float)(r >> 40) * (1.f / 16777216.f);
    switch (kind) {
      case 0: reinterpret_cast<uint8_t*>(dst)[i] = (uint8_t)((int)(r % 255u) - 127 + 128); break;
      case 1: reinterpret_cast<_Float16*>(dst)[i] = (_Float16)(a + (b - a) * u); break;
      case 2: {
        const float u2 = (float)((r >> 16) & 0xffffff) * (1.f / 16777216.f);
        const float z = sqrtf(-2.f * logf(fmaxf(u, 1e-7f))) * cosf(6.2831853f * u2);
        reinterpret_cast<_Float16*>(dst)[i] = (_Float16)(a + b * z);
        break;
      }
      case 3: reinterpret_cast<float*>(dst)[i] = a + (b - a) * u; break;
      case 4: reinterpret_cast<int8_t*>(dst)[i] = (int8_t)((int)(r % 255u) - 127); break;
      default: reinterpret_cast<_Float16*>(dst)[i] = (_Float16)((0.75f + 0.5f * u) * a / sqrtf(b)); break;
    }
  }
}

int rand_fill(void* dst, size_t n, int kind, float a, float b, uint64_t seed, hipStream_t s) {
  if (!n) return 0;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(rand_fill_kernel, dim3(blocks), dim3(256), 0, s, dst, n, kind, a, b, seed);
  return (int)hipGetLastError();
}

// crop_ids[r] = (r * 40503 + 7) mod V: distinct for odd multipliers coprime to V (V a multiple of 16 and not of 40503).
__global__ void crop_ids_kernel(int32_t* ids, int n, int V) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r < n) ids[r] = (int32_t)(((int64_t)r * 40503 + 7) % V);
}

// `fuse` (optional) selects the fused row-group epilogue (GEMM_FUSE_CONV) and carries its parameters.
// `bands` (optional): in, the most output bands the caller adds (y32 holds that many [M][N] blocks); out, the bands
// the plan wrote.
// `xop` false: x is row-major [M][K] (prompt projection) instead of the round's operand order.
// int8 x (x_format 1): x16 holds the norm kernel's codes (scales in xsc); `xsc_in`: x holds codes with these scales
// (y16 / a16 from their producers, xc16 from the context's norms); any other x is fp16, quantized as it is loaded.
// `y_codes` (optional): in, whether the fp16 output y16 should be written as codes + ysc scales; out, whether it was
// (the gated epilogue needs strip pairs inside a workgroup, the conv epilogue always can).
int gemm(dspark_engine* e, const _Float16* x, int M, int K, const uint8_t* w, const _Float16* s, int N, int epilogue,
         float* y32, _Float16* y16, hipStream_t st, const GemmParams* fuse = nullptr, int* bands = nullptr,
         bool xop = true, const float* xsc_in = nullptr, bool* y_codes = nullptr) {
  GemmParams p = {};
  p.st = e->ast;
  p.x = x;
  p.w = w;
  const bool gs = e->d.weight_format == 1;  // per-128-column group scales [K/128][N]
  p.scale = gs ? nullptr : s;
  p.gscale = gs ? s : nullptr;
  p.y32 = epilogue == 0 ? y32 : nullptr;
  p.y16 = y16;
  p.M = M;
  p.N = N;
  p.K = K;
  p.epilogue = epilogue;
  p.xop = xop ? e->tbs : 0;  // every GEMM of the round reads x16, y16 or a16
  p.yop = e->tbs;
  if (e->d.x_format == 1) {
    const bool norm_codes = x == e->x16 && xop;
    p.x8 = norm_codes || xsc_in ? 2 : 1;
    p.xsc = xsc_in ? xsc_in : e->xsc;
    p.xsc_row = e->x_cols / 16;
  }
  int wpg_req = 0;
  if (fuse) {
    p.fuse = fuse->fuse;
    p.conv_w = fuse->conv_w;
    p.conv_ring = fuse->conv_ring;
    p.conv_k = fuse->conv_k;
    p.y32 = nullptr;
    wpg_req = 3;
  }
  GemmPlan pl;
  gemm_plan(M, N, K, true, true, &pl, wpg_req, xop, bands ? *bands : 1, gs);
  if (bands) *bands = pl.bands;
  if (y_codes) {
    const bool can = e->y_codes && y16 &&
                     (fuse ? fuse->fuse == GEMM_FUSE_CONV
                           : epilogue == 1 && pl.kw > 0 && pl.wpg % 2 == 0 && pl.bands == 1 && N % 32 == 0);
    *y_codes = *y_codes && can;
    if (*y_codes) {
      p.ysc = e->ysc;
      p.ysc_row = e->x_cols / 16;
    }
  }
  p.bands = pl.bands;
  p.ksplit = pl.ksplit;
  p.wpg = pl.wpg;
  p.cpb = pl.cpb;
  p.kw = pl.kw;
  p.xd = pl.xd;
  auto it = e->tile_of.find(w);
  if (it != e->tile_of.end()) {
    p.w = e->tiles[it->second].dst;
    p.tiled = 1;
  }
  if (p.ksplit > 1) {
    if (gemm_ws_bytes(pl, M, N) > e->ws_gemm_bytes || gemm_groups(pl, N) > GEMM_COUNTER_SLOTS) return DSPARK_ENOSPACE;
    p.part = gemm_ws_partials(e->ws_gemm);
    p.counters = gemm_ws_counters(e->ws_gemm);  // zeroed at allocation, left at zero by every call
  }
  return gemm_launch(p, true, st);
}

// Residual + RMS norm of M block rows (the bands of v are [M][H] each, as the GEMM of M rows wrote them).
// embed_mode >= 0: h_old is the embedding of the pass's tokens (0: the State's tokens, 1: the drafter block's
// anchor + mask tokens; h_old must be null). x16 / xsc: the outputs (default the round's x16 and its scales).
int resnorm(dspark_engine* e, int M, const float* h_old, const float* v, int bands, const _Float16* post_w,
            const _Float16* norm_w, int sandwich, float* dst, float* tap, hipStream_t s, int embed_mode = -1,
            _Float16* x16 = nullptr, float* xsc = nullptr) {
  ResNormParams p = {};
  p.st = e->ast;
  p.h_old = h_old;
  if (embed_mode >= 0) {
    p.embed = e->embed;
    p.embed_mode = embed_mode;
    p.mask_token = e->d.mask_token;
    p.vocab = e->d.vocab;
  }
  p.v = v;
  p.bands = bands;
  p.v_band_stride = (size_t)M * e->d.hidden;
  p.post_w = post_w;
  p.norm_w = norm_w;
  p.sandwich = sandwich;
  p.eps = e->d.eps;
  p.dst = dst;
  p.tap = tap;
  p.x16 = x16 ? x16 : e->x16;
  p.x_row = e->d.hidden;
  p.H = e->d.hidden;
  p.xop = e->tbs;
  p.xsc = xsc ? xsc : e->xsc;
  p.xsc_row = e->x_cols / 16;
  return resnorm_launch(p, M, 1, s);
}

// The attention launch parameters of layer Lw over M block rows, planned for position plan_a (workspace unbound).
AttnParams attn_setup(dspark_engine* e, const LayerW& Lw, int drafter, int plan_a, const float* gate, int M) {
  const dspark_model_desc& d = e->d;
  AttnParams p = {};
  p.st = e->ast;
  p.drafter = drafter;
  p.q = e->q16;
  p.kp = Lw.kv_rec ? reinterpret_cast<const _Float16*>(Lw.kv_rec) : Lw.kv_k;
  p.vp = Lw.kv_v;
  p.bt = Lw.bt;
  p.k_bytes = p.v_bytes = (uint32_t)(Lw.kv_rec ? Lw.kv_pages * PAGE * d.kv_heads * DSPARK_REC_BYTES
                                               : Lw.kv_pages * d.kv_heads * PAGE * d.head_dim * 2);
  p.out16 = e->y16;
  p.out_op = e->tbs;
  if (e->y_codes) {  // int8 x: the merge writes codes + scales for the out projection
    p.out_sc = e->ysc;
    p.out_sc_row = e->x_cols / 16;
  }
  p.gate = gate;
  p.M = M;
  p.QH = d.q_heads;
  p.KVH = d.kv_heads;
  p.G = d.q_heads / d.kv_heads;
  p.a = plan_a;
  p.causal = drafter ? 0 : 1;
  if (drafter) {
    p.window = d.draft_window;
    p.start = std::max(0, plan_a - d.draft_window);
  } else if (Lw.kind == 2) {
    p.window = d.window;
    p.start = std::max(0, plan_a - d.window + 1);
  }
  p.S = 0;
  if (Lw.kv_rec)
    attn_rec_plan(p, e->cus);
  else
    attn_plan(p, d.head_dim, e->cus);
  if (drafter) p.window = d.draft_window;  // attn_range (device) derives start and drops the per-token window
  return p;
}

// Whether the attention kernel takes the block fresh from the mix rows -- Q and the block's K/V normed and rotated in
// the kernel, no q/k norm + RoPE launch before it: the LDS kernel over fp16 pages at D = 64 with one row block per
// wave and at most one block token per wave, or the record kernel with up to 3 row groups and splits of 8 pages or
// more (its in-kernel Q and record work delays a split's first page by ~1-2 us: reference-build rounds measured
// 1.645 -> 1.672 ms at 1k and 1.699 -> 1.713 at 32k with every record layer fused, 1.787 -> 1.769 at 128k).
bool attn_fresh_ok(dspark_engine* e, const LayerW& Lw, const AttnParams& p) {
  if (!e->fresh || p.qb != 1) return false;
  if (Lw.kv_rec) return p.nrg <= 3 && p.M <= 4 * p.nrg && p.pps >= e->fresh_rec_pps;
  return e->d.head_dim == 64 && p.lds == 1 && p.M <= p.nrg * p.pl;
}

// Layer Lw's verify attention (attn_setup's parameters); fresh: the block from the mix rows (attn_fresh_ok).
int attention(dspark_engine* e, const LayerW& Lw, AttnParams p, bool fresh, hipStream_t s) {
  const dspark_model_desc& d = e->d;
  if (fresh) {
    p.mix = e->mix;
    p.mix_row = Lw.mix_rows;
    p.rot = Lw.kind == 2 ? e->rot_swa : d.rope_pairs;
    p.q_norm = Lw.q_norm;
    p.k_norm = Lw.k_norm;
    p.rope = Lw.kind == 2 ? e->rope_swa : e->rope;
    p.eps = d.eps;
    if (p.gate) {  // the gate straight from the mix rows
      p.gate = e->mix + (size_t)(d.q_heads + 2 * d.kv_heads) * d.head_dim;
      p.gate_stride = Lw.mix_rows;
    }
  }
  if (attn_workspace_bytes(p, d.head_dim) > e->ws_attn_bytes) return DSPARK_ENOSPACE;
  attn_bind_workspace(p, d.head_dim, e->ws_attn);
  return Lw.kv_rec ? attn_rec_launch(p, 3, s) : attn_launch(p, d.head_dim, 3, s);
}

QkRopeParams qk_params(dspark_engine* e, const LayerW& Lw, const float* mix, int row, bool with_q, bool ctx_mode,
                       int M) {
  const dspark_model_desc& d = e->d;
  QkRopeParams p = {};
  p.st = e->ast;
  p.mix = mix;
  p.row = row;
  p.M = M;
  p.QH = d.q_heads;
  p.KVH = d.kv_heads;
  p.D = d.head_dim;
  // sliding layers rotate with their own table (base, pairs); full attention and the drafter with the first
  p.rot = Lw.kind == 2 ? e->rot_swa : d.rope_pairs;
  p.q_norm = Lw.q_norm;
  p.k_norm = Lw.k_norm;
  p.rope = Lw.kind == 2 ? e->rope_swa : e->rope;
  p.eps = d.eps;
  p.q16 = with_q ? e->q16 : nullptr;
  p.gate = (with_q && Lw.kind != 3) ? e->gate : nullptr;
  p.gate_in_mix = p.gate ? 1 : 0;
  p.kp = Lw.kv_k;
  p.vp = Lw.kv_v;
  p.rec = Lw.kv_rec;
  p.bt = Lw.bt;
  p.pos_from_ctx = ctx_mode;
  p.count_from_ctx = ctx_mode;
  return p;
}

// The attention mix GEMM, then the q/k norm + RoPE + K/V page write (qkrope). A fused epilogue needs one head per
// workgroup: 49 workgroups for the C4 mix (10.6 us against 5.1 + 4.7 unfused) and 25 for the reference geometry's
// 128-dim heads (14.5 us), so the two kernels are faster (measured on MI355X).
// qk false: the attention takes the block fresh from the mix rows (attn_fresh_ok), no qkrope launch.
int gemm_mix_qk(dspark_engine* e, const LayerW& W, int M, hipStream_t s, bool qk = true) {
  int rc = gemm(e, e->x16, M, e->d.hidden, W.mix_w, W.mix_s, W.mix_rows, 0, e->mix, nullptr, s);
  if (rc || !qk) return rc;
  return qkrope_launch(qk_params(e, W, e->mix, W.mix_rows, true, false, M), s);
}

// The conv mix GEMM with the gated short conv fused into its epilogue (16 channels per group); output y16.
int gemm_mix_conv(dspark_engine* e, const LayerW& W, int M, hipStream_t s) {
  GemmParams f = {};
  f.fuse = GEMM_FUSE_CONV;
  f.conv_w = W.conv_w;
  f.conv_ring = W.conv_ring;
  f.conv_k = e->d.conv_kernel;
  bool codes = e->y_codes;  // int8 x: codes + scales for the out projection
  return gemm(e, e->x16, M, e->d.hidden, W.mix_w, W.mix_s, W.mix_rows, 0, nullptr, e->y16, s, &f, nullptr, true,
              nullptr, &codes);
}

// Output bands the round's norm kernels add (the w2, out and fc GEMMs may split K over that many workgroups).
constexpr int ENGINE_BANDS = 2;

#define CK(x)                \
  do {                       \
    int _rc = (x);           \
    if (_rc) return _rc;     \
  } while (0)

// A layer-boundary dump (debug rounds only) into slot `slot`: the residual h and the summed bands of v.
int dump(dspark_engine* e, int slot, const float* h, const float* v, int bands, int rows, hipStream_t s) {
  if (!e->dump_on) return 0;
  const size_t per = (size_t)2 * e->B * e->d.hidden;
  return layer_dump_launch(e->dump + slot * per, h, v, bands, rows, e->d.hidden, e->B, s);
}

// A trace mark after a phase (tracing rounds only): one thread stores (phase | round << 32, clock).
int mark(dspark_engine* e, int phase, hipStream_t s) {
  if (!e->trace_on) return 0;
  return trace_mark_launch(e->trace, e->st, phase, phase == DSPARK_TRACE_BEGIN, DSPARK_TRACE_MAX_MARKS, s);
}

// The context projection from its fc GEMM on (dspark.hip:2682-2705, 2487-2518; dspark.go:461-492): x_fc (the normed
// taps of B positions, [B][n_taps * H]: the round's xc16 in operand order, or row-major prompt taps) -> fc -> hidden
// norm -> ckv -> per drafter layer k norm + RoPE, K/V rows into the drafter ring at positions State.ctx_pos + t for
// t < State.ctx_new (of the active State). Its norm outputs go to xc16 (and, int8 x, xcsc), apart from the round's x16.
int enqueue_context(dspark_engine* e, const _Float16* x_fc, bool x_op, hipStream_t s) {
  const dspark_model_desc& d = e->d;
  const int B = e->B, H = d.hidden;
  const bool x8 = d.x_format == 1;
  int nb = ENGINE_BANDS;
  CK(gemm(e, x_fc, B, d.n_taps * H, e->fc_w, e->fc_s, H, 0, e->ctxv, nullptr, s, nullptr, &nb, x_op,
          x8 && x_op ? e->xcsc : nullptr));
  CK(resnorm(e, B, nullptr, e->ctxv, nb, nullptr, e->hidden_norm, 0, nullptr, nullptr, s, -1, e->xc16, e->xcsc));
  const int kvrow = 2 * d.kv_heads * d.head_dim;
  CK(gemm(e, e->xc16, B, H, e->ckv_w, e->ckv_s, d.draft_layers * kvrow, 0, e->ckvout, nullptr, s, nullptr, nullptr,
          true, x8 ? e->xcsc : nullptr));
  for (int j0 = 0; j0 < d.draft_layers; j0 += QKROPE_BATCH) {  // one launch for up to 8 drafter layers
    QkRopeBatch b = {};
    b.n = std::min(QKROPE_BATCH, d.draft_layers - j0);
    for (int j = 0; j < b.n; ++j)
      b.l[j] = qk_params(e, e->DL[j0 + j], e->ckvout + (size_t)(j0 + j) * kvrow, d.draft_layers * kvrow, false, true, B);
    CK(qkrope_batch_launch(b, s));
  }
  return 0;
}

// The round's launch sequence (see the file header). mv: verify width, the token rows of the verify pass (the
// round's drafts are capped below it, so 1 + drafts <= mv; the drafter block stays B wide). skip: a skip round
// (dspark.hip:2441-2451): the context projection, then the anchor alone verified (no drafter), State.skip decremented.
int enqueue_round(dspark_engine* e, int force_m, int plan_a, int mv, bool skip, hipStream_t s) {
  const dspark_model_desc& d = e->d;
  const int B = e->B, H = d.hidden, MV = mv;
  // int8 x: the attention merge and the conv epilogue write y16 as codes with these scales
  float* const ysc = e->y_codes ? e->ysc : nullptr;
  const bool x8 = e->y_codes;
  uint64_t* vbest = e->keys;
  uint64_t* mbest = e->keys + B;
  e->ast = e->st;
  CK(round_begin_launch(e->st, e->keys, 2 * B, e->seen, B, e->max_context + B, d.vocab, e->max_context + 2 * B, s));
  CK(mark(e, DSPARK_TRACE_BEGIN, s));
  // the embedding folded into each pass's first norm (one launch fewer per pass), unless the layer dumps read it
  const bool fold = !e->dump_on;
  if (force_m > 0) {
    CK(force_m_launch(e->st, force_m, s));
  } else {
    // ---- context projection of the last round's committed positions (skipped rows: t >= ctx_new)
    {
      ResNormParams p = {};
      p.st = e->st;
      p.h_old = e->taps;
      p.group_stride = (size_t)B * H;
      p.norm_w = e->tap_norms;
      p.norm_w_stride = H;
      p.eps = d.eps;
      p.x16 = e->xc16;
      p.x_row = d.n_taps * H;
      p.x_group_stride = H;
      p.H = H;
      p.xop = e->tbs;
      p.xsc = e->xcsc;
      p.xsc_row = e->x_cols / 16;
      CK(resnorm_launch(p, B, d.n_taps, s));
    }
    CK(enqueue_context(e, e->xc16, true, s));
    CK(mark(e, DSPARK_TRACE_CONTEXT, s));
  }
  if (skip) {
    CK(force_m_launch(e->st, 1, s));
  } else if (force_m <= 0) {
    // ---- drafter block
    if (!fold) CK(embed_launch(e->embed, e->st, 1, d.mask_token, B, H, d.vocab, e->h[0], s));
    int cur = 0, w2b = 0;  // w2b: bands of the last w2 output
    for (int j = 0; j < d.draft_layers; ++j) {
      const LayerW& W = e->DL[j];
      CK(dump(e, j, e->h[cur], j ? e->w2out : nullptr, w2b, B, s));
      if (j == 0 && fold)
        CK(resnorm(e, B, nullptr, nullptr, 0, nullptr, W.op_norm, 0, e->h[cur ^ 1], nullptr, s, 1));
      else
        CK(resnorm(e, B, e->h[cur], j ? e->w2out : nullptr, w2b, nullptr, W.op_norm, 0, e->h[cur ^ 1], nullptr, s));
      cur ^= 1;
      const AttnParams ap = attn_setup(e, W, 1, plan_a, nullptr, B);
      const bool fr = attn_fresh_ok(e, W, ap);
      CK(gemm_mix_qk(e, W, B, s, !fr));
      CK(attention(e, W, ap, fr, s));
      int ob = ENGINE_BANDS;
      CK(gemm(e, e->y16, B, H, W.out_w, W.out_s, H, 0, e->vout, nullptr, s, nullptr, &ob, true, ysc));
      CK(resnorm(e, B, e->h[cur], e->vout, ob, nullptr, W.ffn_norm, 0, e->h[cur ^ 1], nullptr, s));
      cur ^= 1;
      bool acodes = x8;
      CK(gemm(e, e->x16, B, H, W.w13_w, W.w13_s, 2 * W.ffn, 1, nullptr, e->a16, s, nullptr, nullptr, true, nullptr,
              &acodes));
      w2b = ENGINE_BANDS;
      CK(gemm(e, e->a16, B, W.ffn, W.w2_w, W.w2_s, H, 0, e->w2out, nullptr, s, nullptr, &w2b, true,
              acodes ? e->ysc : nullptr));
    }
    CK(mark(e, DSPARK_TRACE_DRAFTER, s));
    CK(dump(e, d.draft_layers, e->h[cur], e->w2out, w2b, B, s));
    CK(resnorm(e, B, e->h[cur], e->w2out, w2b, nullptr, e->draft_norm, 0, nullptr, nullptr, s));
    CK(gemm(e, e->x16, B, H, e->crop_w, e->crop_s, e->crop_n, 0, e->base, nullptr, s));
    CK(mark(e, DSPARK_TRACE_CROP_HEAD, s));
    MarkovParams mp = {};
    mp.st = e->st;
    mp.base = e->base;
    mp.stride = e->crop_n;
    mp.N = d.crop_rows;
    mp.rank = d.markov_rank;
    mp.block = B;
    mp.max_drafts = d.max_drafts;
    mp.w2q = e->w2q;
    mp.w2s = e->w2s;
    mp.w1q = e->w1q;
    mp.w1s = e->w1s;
    mp.c2 = e->c2;
    mp.crop_ids = e->crop_ids;
    mp.best = mbest;
    mp.max_drafts_dev = reinterpret_cast<const int32_t*>(e->rep + 2);
    mp.conf_bias = d.conf_bias;
    mp.conf_thr = d.conf_thr;
    mp.table = e->mtab;
    mp.c2c = e->mc2c;
    mp.s1c = e->ms1c;
    mp.plant = force_m < 0 ? e->plant : nullptr;  // planted rounds: the Markov launch applies the plant
    CK(markov_launch(mp, s));
    CK(mark(e, DSPARK_TRACE_MARKOV, s));
  }
  // ---- verify (MV rows; rows past the State's M are computed and never committed)
  if (!fold) CK(embed_launch(e->embed, e->st, 0, 0, MV, H, d.vocab, e->h[0], s));
  int cur = 0, w2b = 0;  // w2b: bands of the last w2 output
  for (int i = 0; i < d.n_layers; ++i) {
    const LayerW& W = e->L[i];
    const LayerW* P = i ? &e->L[i - 1] : nullptr;
    float* tap = (P && P->tap_slot >= 0) ? e->taps + (size_t)P->tap_slot * B * H : nullptr;
    CK(dump(e, d.draft_layers + 1 + i, e->h[cur], i ? e->w2out : nullptr, w2b, MV, s));
    if (i == 0 && fold)
      CK(resnorm(e, MV, nullptr, nullptr, 0, nullptr, W.op_norm, 1, e->h[cur ^ 1], nullptr, s, 0));
    else
      CK(resnorm(e, MV, e->h[cur], i ? e->w2out : nullptr, w2b, P ? P->post_ffn_norm : nullptr, W.op_norm, 1,
                 e->h[cur ^ 1], tap, s));
    cur ^= 1;
    if (W.kind == 0) {
      CK(gemm_mix_conv(e, W, MV, s));
    } else {
      const AttnParams ap = attn_setup(e, W, 0, plan_a, e->gate, MV);
      const bool fr = attn_fresh_ok(e, W, ap);
      CK(gemm_mix_qk(e, W, MV, s, !fr));
      CK(attention(e, W, ap, fr, s));
    }
    int ob = ENGINE_BANDS;
    CK(gemm(e, e->y16, MV, H, W.out_w, W.out_s, H, 0, e->vout, nullptr, s, nullptr, &ob, true, ysc));
    CK(resnorm(e, MV, e->h[cur], e->vout, ob, W.post_op_norm, W.ffn_norm, 1, e->h[cur ^ 1], nullptr, s));
    cur ^= 1;
    bool acodes = x8;
    CK(gemm(e, e->x16, MV, H, W.w13_w, W.w13_s, 2 * W.ffn, 1, nullptr, e->a16, s, nullptr, nullptr, true, nullptr,
            &acodes));
    w2b = ENGINE_BANDS;
    CK(gemm(e, e->a16, MV, W.ffn, W.w2_w, W.w2_s, H, 0, e->w2out, nullptr, s, nullptr, &w2b, true,
            acodes ? e->ysc : nullptr));
    CK(mark(e, DSPARK_TRACE_VERIFY_LAYER + i, s));
  }
  {
    const LayerW& P = e->L[d.n_layers - 1];
    float* tap = P.tap_slot >= 0 ? e->taps + (size_t)P.tap_slot * B * H : nullptr;
    CK(dump(e, d.draft_layers + 1 + d.n_layers, e->h[cur], e->w2out, w2b, MV, s));
    CK(resnorm(e, MV, e->h[cur], e->w2out, w2b, P.post_ffn_norm, e->final_norm, 1, nullptr, tap, s));
  }
  CK(gemm(e, e->x16, MV, H, e->head_w, e->head_s, d.vocab, 0, e->logits, nullptr, s));
  CK(mark(e, DSPARK_TRACE_LM_HEAD, s));
  CK(verify_argmax_launch(e->logits, 0, MV, d.vocab, e->seen, e->st, 1.f, 1.f, vbest, e->ws_argmax, s, e->rep, false));
  CK(accept_commit_fold_launch(e->st, static_cast<const uint64_t*>(e->ws_argmax), verify_argmax_chunks(d.vocab), MV,
                               vbest, e->out_tokens, e->max_context + 2 * B, e->seen, skip ? 1 : 0, e->mirror, s));
  CK(mark(e, DSPARK_TRACE_COMMIT, s));
  return 0;
}

int64_t kv_pages_for(const dspark_model_desc& d, int max_context) {
  const int64_t positions = (int64_t)max_context + d.block;
  return (positions + PAGE - 1) / PAGE + 1;
}
int64_t kv_pool_bytes(const dspark_model_desc& d, int max_context) {
  return kv_pages_for(d, max_context) * d.kv_heads * PAGE * (d.kv_format ? DSPARK_REC_BYTES : d.head_dim * 2);
}

bool desc_ok(const dspark_model_desc* d, int max_context) {
  if (!d || d->hidden < 256 || d->hidden % 256 || d->hidden > 8192) return false;
  if (d->ffn < 64 || d->ffn % 64 || d->draft_ffn < 64 || d->draft_ffn % 64) return false;
  if (d->vocab < 16 || d->vocab % 16) return false;
  if (d->n_layers < 1 || d->n_layers > DSPARK_MAX_LAYERS) return false;
  if (d->head_dim != 64 && d->head_dim != 128) return false;
  if (d->kv_heads < 1 || d->q_heads % d->kv_heads || d->q_heads * d->head_dim != d->hidden) return false;
  if (d->conv_kernel < 1 || d->conv_kernel > 8) return false;
  if (d->rope_pairs < 0 || d->rope_pairs > d->head_dim / 2) return false;
  if (!(d->rope_base > 0.f)) return false;
  if (d->rope_base_swa > 0.f && (d->rope_pairs_swa < 0 || d->rope_pairs_swa > d->head_dim / 2)) return false;
  if (d->conv_slots < 0 || d->conv_slots > 65536) return false;
  // int8 records: the record attention kernel's geometry (D 128, 4 KV heads, up to 64 rows per KV head)
  if (d->kv_format < 0 || d->kv_format > 1) return false;
  // group scales: the K-sliced kernel with one token block, whole 128-column groups
  if (d->weight_format < 0 || d->weight_format > 1) return false;
  if (d->weight_format == 1 && (d->block > 16 || d->hidden % 128 || d->ffn % 128 || d->draft_ffn % 128)) return false;
  // int8 x (LFM3_X8): with group scales only
  if (d->x_format < 0 || d->x_format > 1 || (d->x_format == 1 && d->weight_format != 1)) return false;
  if (d->kv_format == 1 && (d->head_dim != 128 || d->kv_heads != 4 || d->q_heads / d->kv_heads * d->block > 64))
    return false;
  if (d->draft_layers < 1 || d->block < 2 || d->block > 64 || d->max_drafts < 0 || d->max_drafts > d->block - 1) return false;
  if (d->crop_rows < 16 || d->crop_rows % 16 || d->markov_rank < 16 || d->markov_rank % 16) return false;
  if (d->crop_rows > d->vocab) return false;
  if (d->n_taps < 1 || d->n_taps > DSPARK_MAX_TAPS) return false;
  for (int i = 0; i < d->n_taps; ++i)
    if (d->tap_layer[i] < 0 || d->tap_layer[i] >= d->n_layers) return false;
  if (d->ring_positions % PAGE || d->ring_positions < d->draft_window + d->block + PAGE) return false;
  if (d->mask_token < 0 || d->mask_token >= d->vocab) return false;
  if (max_context < d->block || max_context > (1 << 24)) return false;
  // every K/V page pool below 2 GiB: the attention kernels address a pool with 32-bit byte offsets
  if (kv_pool_bytes(*d, max_context) >= ((int64_t)1 << 31)) return false;
  int n_attn = 0;
  for (int i = 0; i < d->n_layers; ++i) {
    if (d->layer_kind[i] < 0 || d->layer_kind[i] > 2) return false;
    n_attn += d->layer_kind[i] != 0;
  }
  (void)n_attn;
  return true;
}

}  // namespace

extern "C" {

int dspark_engine_create(const dspark_model_desc* desc, int32_t max_context, dspark_engine** out) {
  if (!out || !desc_ok(desc, max_context)) return DSPARK_EINVAL;
  dspark_engine* e = new dspark_engine();
  e->d = *desc;
  const dspark_model_desc& d = e->d;
  e->max_context = max_context;
  e->B = d.block;
  const int B = e->B, H = d.hidden, D = d.head_dim, QH = d.q_heads, KVH = d.kv_heads;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) e->cus = n;
  }
  int err = 0;
  auto h16 = [&](const std::string& n, size_t count) { return static_cast<_Float16*>(e->alloc(n, count * 2, &err)); };
  // scales of an int8 [N][K] weight: [N] per row, or [K/128][N] per 128-column group (weight_format 1)
  auto sc = [&](const std::string& n, int N, int K) { return h16(n, d.weight_format ? (size_t)(K / 128) * N : (size_t)N); };
  // an int8 GEMM weight [N][K] and its tile-major copy
  auto u8 = [&](const std::string& n, int N, int K) {
    uint8_t* w = static_cast<uint8_t*>(e->alloc(n, (size_t)N * K, &err));
    uint8_t* t = static_cast<uint8_t*>(e->alloc("", (size_t)N * K, &err));
    if (!err) {
      e->tile_of[w] = e->tiles.size();
      e->tile_by_name[n] = e->tiles.size();
      e->tiles.push_back({w, t, N, K, true});
    }
    return w;
  };
  const int64_t positions = (int64_t)max_context + B;
  e->kv_pages = kv_pages_for(d, max_context);
  e->ring_pages = d.ring_positions / PAGE;
  e->embed = h16("embed", (size_t)d.vocab * H);
  e->final_norm = h16("final_norm", H);
  e->head_w = u8("head.w", d.vocab, H);
  e->head_s = sc("head.s", d.vocab, H);
  int tap_slot[DSPARK_MAX_LAYERS];
  for (int i = 0; i < DSPARK_MAX_LAYERS; ++i) tap_slot[i] = -1;
  for (int i = 0; i < d.n_taps; ++i) tap_slot[d.tap_layer[i]] = i;
  e->L.resize(d.n_layers);
  for (int i = 0; i < d.n_layers; ++i) {
    LayerW& W = e->L[i];
    const std::string pre = "L" + std::to_string(i) + ".";
    W.kind = d.layer_kind[i];
    W.tap_slot = tap_slot[i];
    W.op_norm = h16(pre + "op_norm", H);
    W.ffn_norm = h16(pre + "ffn_norm", H);
    W.post_op_norm = h16(pre + "post_op_norm", H);
    W.post_ffn_norm = h16(pre + "post_ffn_norm", H);
    W.mix_rows = W.kind == 0 ? 3 * H : align16(QH * D + 2 * KVH * D + QH);
    W.mix_w = u8(pre + "mix.w", W.mix_rows, H);
    W.mix_s = sc(pre + "mix.s", W.mix_rows, H);
    W.out_w = u8(pre + "out.w", H, H);
    W.out_s = sc(pre + "out.s", H, H);
    W.ffn = d.ffn;
    W.w13_w = u8(pre + "w13.w", 2 * d.ffn, H);
    W.w13_s = sc(pre + "w13.s", 2 * d.ffn, H);
    W.w2_w = u8(pre + "w2.w", H, d.ffn);
    W.w2_s = sc(pre + "w2.s", H, d.ffn);
    if (W.kind == 0) {
      W.conv_w = h16(pre + "conv.w", (size_t)H * d.conv_kernel);
      W.conv_ring = h16("conv.L" + std::to_string(i), (size_t)CONV_RING * H);
      const int km1 = std::max(1, d.conv_kernel - 1);
      _Float16* cs = h16("conv_state.L" + std::to_string(i), (size_t)std::max(1, d.conv_slots) * H * km1);
      if (e->conv.n < CONV_MAX_LAYERS) {
        e->conv.ring[e->conv.n] = W.conv_ring;
        e->conv.state[e->conv.n] = cs;
        e->conv.n++;
      }
    } else {
      W.q_norm = h16(pre + "q_norm", D);
      W.k_norm = h16(pre + "k_norm", D);
      W.kv_pages = e->kv_pages;
      if (d.kv_format) {
        W.kv_rec = static_cast<uint8_t*>(
            e->alloc("kv.L" + std::to_string(i) + ".rec", (size_t)e->kv_pages * PAGE * KVH * DSPARK_REC_BYTES, &err));
      } else {
        W.kv_k = h16("kv.L" + std::to_string(i) + ".k", (size_t)e->kv_pages * KVH * PAGE * D);
        W.kv_v = h16("kv.L" + std::to_string(i) + ".v", (size_t)e->kv_pages * KVH * PAGE * D);
      }
    }
  }
  const int64_t bt_entries = (positions + PAGE - 1) / PAGE + 1;
  e->ring_bt = static_cast<int32_t*>(e->alloc("ring_table", bt_entries * 4, &err));
  e->DL.resize(d.draft_layers);
  for (int j = 0; j < d.draft_layers; ++j) {
    LayerW& W = e->DL[j];
    const std::string pre = "D" + std::to_string(j) + ".";
    W.kind = 3;
    W.op_norm = h16(pre + "op_norm", H);
    W.ffn_norm = h16(pre + "ffn_norm", H);
    W.mix_rows = align16(QH * D + 2 * KVH * D);
    W.mix_w = u8(pre + "mix.w", W.mix_rows, H);
    W.mix_s = sc(pre + "mix.s", W.mix_rows, H);
    W.out_w = u8(pre + "out.w", H, H);
    W.out_s = sc(pre + "out.s", H, H);
    W.ffn = d.draft_ffn;
    W.w13_w = u8(pre + "w13.w", 2 * d.draft_ffn, H);
    W.w13_s = sc(pre + "w13.s", 2 * d.draft_ffn, H);
    W.w2_w = u8(pre + "w2.w", H, d.draft_ffn);
    W.w2_s = sc(pre + "w2.s", H, d.draft_ffn);
    W.q_norm = h16(pre + "q_norm", D);
    W.k_norm = h16(pre + "k_norm", D);
    W.kv_pages = e->ring_pages;
    if (d.kv_format) {
      W.kv_rec = static_cast<uint8_t*>(
          e->alloc("ring.D" + std::to_string(j) + ".rec", (size_t)e->ring_pages * PAGE * KVH * DSPARK_REC_BYTES, &err));
    } else {
      W.kv_k = h16("ring.D" + std::to_string(j) + ".k", (size_t)e->ring_pages * KVH * PAGE * D);
      W.kv_v = h16("ring.D" + std::to_string(j) + ".v", (size_t)e->ring_pages * KVH * PAGE * D);
    }
    W.bt = e->ring_bt;
  }
  e->draft_norm = h16("draft_norm", H);
  e->crop_n = align16(d.crop_rows + 1);
  e->crop_w = u8("crop.w", e->crop_n, H);
  e->crop_s = sc("crop.s", e->crop_n, H);
  e->crop_ids = static_cast<int32_t*>(e->alloc("crop_ids", (size_t)d.crop_rows * 4, &err));
  e->w2q = static_cast<int8_t*>(e->alloc("markov.w2q", (size_t)d.crop_rows * d.markov_rank, &err));
  e->w2s = static_cast<float*>(e->alloc("markov.w2s", (size_t)d.crop_rows * 4, &err));
  e->w1q = static_cast<int8_t*>(e->alloc("markov.w1q", (size_t)d.vocab * d.markov_rank, &err));
  e->w1s = static_cast<float*>(e->alloc("markov.w1s", (size_t)d.vocab * 4, &err));
  e->c2 = static_cast<float*>(e->alloc("conf_c2", (size_t)d.vocab * 4, &err));
  if (d.crop_rows <= 16384) {
    e->mtab = static_cast<float*>(e->alloc("", (size_t)d.crop_rows * d.crop_rows * 4, &err));
    e->mc2c = static_cast<float*>(e->alloc("", (size_t)d.crop_rows * 4, &err));
    e->ms1c = static_cast<float*>(e->alloc("", (size_t)d.crop_rows * 4, &err));
  }
  e->tap_norms = h16("tap_norms", (size_t)d.n_taps * H);
  e->fc_w = u8("fc.w", H, d.n_taps * H);
  e->fc_s = sc("fc.s", H, d.n_taps * H);
  e->hidden_norm = h16("hidden_norm", H);
  const int ckv_rows = d.draft_layers * 2 * KVH * D;
  e->ckv_w = u8("ckv.w", ckv_rows, H);
  e->ckv_s = sc("ckv.s", ckv_rows, H);
  e->rope = h16("rope", (size_t)(positions + 1) * D);
  const bool own_swa = d.rope_base_swa > 0.f;
  e->rope_swa = own_swa ? h16("rope_swa", (size_t)(positions + 1) * D) : e->rope;
  e->rot_swa = own_swa ? d.rope_pairs_swa : d.rope_pairs;
  e->conv.H = H;
  e->conv.km1 = d.conv_kernel - 1;
  e->conv.slots = std::max(1, d.conv_slots);
  // prompt projection: captured taps of up to draft_window positions (+ one block of padding rows the last chunk's
  // GEMM reads), one State per chunk of B positions
  e->tap_rows = (d.draft_window + B - 1) / B * B + B;
  e->tapx = h16("tap_x", (size_t)e->tap_rows * d.n_taps * H);
  e->seed_chunks = e->tap_rows / B;
  e->seed_st = static_cast<dspark_state*>(e->alloc("", (size_t)e->seed_chunks * sizeof(dspark_state), &err));
  // request state and activations
  e->st = static_cast<dspark_state*>(e->alloc("state", sizeof(dspark_state), &err));
  e->seen = static_cast<uint32_t*>(e->alloc("seen", (size_t)(d.vocab + 31) / 32 * 4, &err));
  // tokens emitted since the State was set: a round commits at most M <= limit - a tokens and limit <= max_context,
  // so the count stays below max_context
  e->out_tokens = static_cast<int32_t*>(e->alloc("out_tokens", (size_t)(max_context + 2 * B) * 4, &err));
  e->plant = static_cast<int32_t*>(e->alloc("plant", (size_t)(positions + B + 1) * 4, &err));
  e->rep = static_cast<float*>(e->alloc("rep", 16, &err));
  if (!err && hipHostMalloc((void**)&e->mirror, 16 * sizeof(int32_t), hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) {
    e->mirror = nullptr;
    err = DSPARK_ENOSPACE;
  }
  if (e->mirror) std::memset(e->mirror, 0, 16 * sizeof(int32_t));
  {
    const char* fv = std::getenv("DSPARK_FRESH");
    e->fresh = !(fv && fv[0] == '0');
    const char* fr = std::getenv("DSPARK_FRESH_REC_PPS");
    if (fr) e->fresh_rec_pps = std::max(1, std::atoi(fr));
  }
  e->trace = static_cast<uint64_t*>(e->alloc("trace", (size_t)(2 + 2 * DSPARK_TRACE_MAX_MARKS) * 8, &err));
  e->dump = static_cast<float*>(
      e->alloc("debug_layers", (size_t)(d.draft_layers + d.n_layers + 2) * 2 * B * H * sizeof(float), &err));
  e->x_cols = std::max(std::max(H, d.n_taps * H), std::max(d.ffn, d.draft_ffn));
  e->mix_cols = std::max(std::max(3 * H, align16(QH * D + 2 * KVH * D + QH)), ckv_rows);
  e->h[0] = static_cast<float*>(e->alloc("h0", (size_t)B * H * 4, &err));
  e->h[1] = static_cast<float*>(e->alloc("h1", (size_t)B * H * 4, &err));
  e->tbs = (B + 15) / 16;
  e->x16 = h16("x16", (size_t)16 * e->tbs * e->x_cols);
  e->xc16 = h16("xc16", (size_t)16 * e->tbs * d.n_taps * H);
  {
    const char* v = std::getenv("DSPARK_X8_PRODUCER_CODES");
    e->y_codes = d.x_format == 1 && !(v && v[0] == '0');
  }
  if (d.x_format == 1) {
    e->xsc = static_cast<float*>(e->alloc("x_scales", (size_t)16 * e->tbs * (e->x_cols / 16) * sizeof(float), &err));
    e->ysc = static_cast<float*>(e->alloc("y_scales", (size_t)16 * e->tbs * (e->x_cols / 16) * sizeof(float), &err));
    e->xcsc = static_cast<float*>(e->alloc("xc_scales", (size_t)16 * e->tbs * (e->x_cols / 16) * sizeof(float), &err));
  }
  e->mix = static_cast<float*>(e->alloc("mix", (size_t)B * e->mix_cols * 4, &err));
  e->q16 = h16("q16", (size_t)B * QH * D);
  e->gate = static_cast<float*>(e->alloc("gate", (size_t)B * QH * 4, &err));
  e->y16 = h16("y16", (size_t)16 * e->tbs * H);
  e->vout = static_cast<float*>(e->alloc("vout", (size_t)ENGINE_BANDS * B * H * 4, &err));
  e->a16 = h16("a16", (size_t)16 * e->tbs * std::max(d.ffn, d.draft_ffn));
  e->w2out = static_cast<float*>(e->alloc("w2out", (size_t)ENGINE_BANDS * B * H * 4, &err));
  e->ctxv = static_cast<float*>(e->alloc("ctx", (size_t)ENGINE_BANDS * B * H * 4, &err));
  e->ckvout = static_cast<float*>(e->alloc("ckv_out", (size_t)B * ckv_rows * 4, &err));
  e->taps = static_cast<float*>(e->alloc("taps", (size_t)d.n_taps * B * H * 4, &err));
  e->logits = static_cast<float*>(e->alloc("logits", (size_t)B * d.vocab * 4, &err));
  e->base = static_cast<float*>(e->alloc("base", (size_t)B * e->crop_n * 4, &err));
  e->keys = static_cast<uint64_t*>(e->alloc("keys", (size_t)2 * B * 8, &err));
  // workspaces: the largest split-K partials, attention partials (<= 64 splits x all rows), argmax chunks
  size_t gws = 0;
  const int Ks[] = {H, d.n_taps * H, d.ffn, d.draft_ffn};
  const int Ns[] = {H,        3 * H,    2 * d.ffn, 2 * d.draft_ffn, d.vocab, e->crop_n, ckv_rows,
                    align16(QH * D + 2 * KVH * D + QH), QH * D + 2 * KVH * D};
  // every verify width 1 .. B (a round's verify pass is sized to its draft cap)
  for (int m = 1; m <= B; ++m)
    for (int K : Ks)
      for (int N : Ns)
        for (int wpg_req : {0, 3}) gws = std::max(gws, gemm_ws_bytes(m, N, K, wpg_req, true));
  gws = std::max(gws, gemm_ws_bytes(B, H, d.n_taps * H, 0, false));  // the prompt projection's fc (row-major taps)
  e->ws_gemm_bytes = gws + 256;
  e->ws_gemm = e->alloc("ws_gemm", e->ws_gemm_bytes, &err);
  const int G = QH / KVH;
  const size_t rows_pad = (size_t)(G * B + 16 * 8);
  e->ws_attn_bytes = (size_t)KVH * (d.kv_format ? ATTN_REC_MAX_SPLITS : 64) * rows_pad * (D * 4 + 8) +
                     (size_t)KVH * 64 * 4 + 4096;
  e->ws_attn = e->alloc("ws_attn", e->ws_attn_bytes, &err);
  e->ws_argmax_bytes = verify_argmax_ws(B, d.vocab);
  e->ws_argmax = e->alloc("ws_argmax", e->ws_argmax_bytes, &err);
  if (err) {
    delete e;
    return err;
  }
  // drafter ring table (logical page -> ring page) and the RoPE tables (dspark_rope_table)
  std::vector<int32_t> bt(bt_entries);
  for (int64_t i = 0; i < bt_entries; ++i) bt[i] = (int32_t)(i % e->ring_pages);
  std::vector<uint16_t> rope((size_t)(positions + 1) * D), rope_swa;
  dspark_rope_table(d.rope_base, d.rope_pairs, D, (int32_t)(positions + 1), rope.data());
  if (own_swa) {
    rope_swa.resize(rope.size());
    dspark_rope_table(d.rope_base_swa, d.rope_pairs_swa, D, (int32_t)(positions + 1), rope_swa.data());
  }
  e->host_lp[0] = e->host_lp[1] = 1.f;
  std::memcpy(&e->host_lp[2], &d.max_drafts, 4);
  if (hipMemcpy(e->ring_bt, bt.data(), bt.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(e->rope, rope.data(), rope.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
      (own_swa && hipMemcpy(e->rope_swa, rope_swa.data(), rope_swa.size() * 2, hipMemcpyHostToDevice) != hipSuccess) ||
      hipMemcpy(e->rep, e->host_lp, sizeof(e->host_lp), hipMemcpyHostToDevice) != hipSuccess) {
    delete e;
    return DSPARK_ENOSPACE;
  }
  *out = e;
  return 0;
}

void dspark_engine_destroy(dspark_engine* e) { delete e; }

int dspark_engine_tensor(dspark_engine* e, const char* name, void** ptr, size_t* bytes) {
  if (!e || !name) return DSPARK_EINVAL;
  auto it = e->tensors.find(name);
  if (it == e->tensors.end()) return DSPARK_EINVAL;
  // a pointer to a weight the Markov table is built from may be written through: rebuild before the next round
  static const char* const table_inputs[] = {"markov.w1q", "markov.w1s", "markov.w2q", "conf_c2", "crop_ids"};
  for (const char* n : table_inputs)
    if (std::strcmp(name, n) == 0) e->mtab_dirty = true;
  auto tw = e->tile_by_name.find(name);
  if (tw != e->tile_by_name.end()) {
    e->tiles[tw->second].dirty = true;
    e->tiles_dirty = true;
  }
  if (ptr) *ptr = it->second.ptr;
  if (bytes) *bytes = it->second.bytes;
  return 0;
}

int dspark_engine_tensor_count(dspark_engine* e) { return e ? (int)e->names.size() : 0; }

const char* dspark_engine_tensor_name(dspark_engine* e, int32_t i) {
  if (!e || i < 0 || i >= (int)e->names.size()) return nullptr;
  return e->names[i].c_str();
}

int dspark_engine_init_random(dspark_engine* e, uint64_t seed, dspark_stream_t stream) {
  if (!e) return DSPARK_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dspark_model_desc& d = e->d;
  const int H = d.hidden;
  uint64_t k = seed * 1000003ull;
  int rc = 0;
  auto fill = [&](const std::string& name, int kind, float a, float b) {
    if (rc) return;
    auto it = e->tensors.find(name);
    if (it == e->tensors.end()) {
      rc = DSPARK_EINVAL;
      return;
    }
    const size_t n = kind == 0 || kind == 4 ? it->second.bytes : (kind == 3 ? it->second.bytes / 4 : it->second.bytes / 2);
    rc = rand_fill(it->second.ptr, n, kind, a, b, ++k, s);
  };
  // one fp16 scale per output row: |y| ~ |x| for inputs of unit RMS (int8 uniform has std 73.3)
  auto gemm_w = [&](const std::string& pre, int K) {
    fill(pre + ".w", 0, 0.f, 0.f);
    fill(pre + ".s", 5, 1.f / 73.3f, (float)K);
  };
  fill("embed", 2, 0.f, 1.f);
  fill("final_norm", 1, 0.8f, 1.2f);
  gemm_w("head", H);
  for (int i = 0; i < d.n_layers; ++i) {
    const std::string pre = "L" + std::to_string(i) + ".";
    for (const char* n : {"op_norm", "ffn_norm", "post_op_norm", "post_ffn_norm"}) fill(pre + n, 1, 0.8f, 1.2f);
    gemm_w(pre + "mix", H);
    gemm_w(pre + "out", H);
    gemm_w(pre + "w13", H);
    gemm_w(pre + "w2", d.ffn);
    if (d.layer_kind[i] == 0) {
      fill(pre + "conv.w", 2, 0.f, 1.f / std::sqrt((float)d.conv_kernel));
    } else {
      fill(pre + "q_norm", 1, 0.8f, 1.2f);
      fill(pre + "k_norm", 1, 0.8f, 1.2f);
    }
  }
  for (int j = 0; j < d.draft_layers; ++j) {
    const std::string pre = "D" + std::to_string(j) + ".";
    fill(pre + "op_norm", 1, 0.8f, 1.2f);
    fill(pre + "ffn_norm", 1, 0.8f, 1.2f);
    gemm_w(pre + "mix", H);
    gemm_w(pre + "out", H);
    gemm_w(pre + "w13", H);
    gemm_w(pre + "w2", d.draft_ffn);
    fill(pre + "q_norm", 1, 0.8f, 1.2f);
    fill(pre + "k_norm", 1, 0.8f, 1.2f);
  }
  fill("draft_norm", 1, 0.8f, 1.2f);
  gemm_w("crop", H);
  fill("markov.w2q", 4, 0.f, 0.f);
  fill("markov.w2s", 3, 0.5f / (73.3f * 16.f), 1.5f / (73.3f * 16.f));
  fill("markov.w1q", 4, 0.f, 0.f);
  fill("markov.w1s", 3, 1.f / 73.3f, 1.f / 73.3f);
  fill("conf_c2", 3, -0.1f, 0.1f);
  fill("tap_norms", 1, 0.8f, 1.2f);
  gemm_w("fc", d.n_taps * H);
  fill("hidden_norm", 1, 0.8f, 1.2f);
  gemm_w("ckv", H);
  if (rc) return rc;
  hipLaunchKernelGGL(crop_ids_kernel, dim3((d.crop_rows + 255) / 256), dim3(256), 0, s, e->crop_ids, d.crop_rows, d.vocab);
  e->mtab_dirty = true;
  for (auto& t : e->tiles) t.dirty = true;
  e->tiles_dirty = true;
  return (int)hipGetLastError();
}

namespace {
// Rebuild what is derived from the weights: everything (all) or what may have changed since the last build.
int prepare(dspark_engine* e, hipStream_t s, bool all) {
  for (auto& t : e->tiles) {
    if (!t.dirty && !all) continue;
    const int rc = gemm_tile_launch(t.src, t.dst, t.N, t.K, s, e->d.x_format == 1 ? 1 : 0);
    if (rc) return rc;
    t.dirty = false;
  }
  e->tiles_dirty = false;
  if (!e->mtab || (!e->mtab_dirty && !all)) return 0;
  const dspark_model_desc& d = e->d;
  const int rc = markov_table_launch(e->w1q, e->w1s, e->c2, e->w2q, e->crop_ids, d.crop_rows, d.markov_rank, d.vocab,
                                     e->mtab, e->mc2c, e->ms1c, s);
  if (!rc) e->mtab_dirty = false;
  return rc;
}
}  // namespace

namespace {
// One round at verify width mv (skip: a skip round), recorded as a HIP graph the first time its key is met, then
// replayed on s.
int round_enqueue(dspark_engine* e, int force_m, int plan_a, int mv, bool skip, hipStream_t s) {
  if (mv < 1 || mv > e->B || (force_m > 0 && !skip && mv < force_m)) return DSPARK_EINVAL;
  if (e->mtab_dirty || e->tiles_dirty) {
    const int rc = prepare(e, s, false);
    if (rc) return rc;
  }
  const int bucket = plan_a / ROUND_PLAN_BUCKET;
  const std::vector<int> key = {force_m, (e->trace_on ? 1 : 0) | (e->dump_on ? 2 : 0), mv, skip ? 1 : 0, bucket};
  auto it = e->graphs.find(key);
  if (it == e->graphs.end()) {
    // Record the round on a private stream (capture needs a non-default stream), then replay it on `s`.
    hipStream_t cap;
    if (hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) != hipSuccess) return DSPARK_ENOSPACE;
    hipGraph_t g = nullptr;
    int rc = (int)hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal);
    if (!rc) {
      const int plan = bucket * ROUND_PLAN_BUCKET + ROUND_PLAN_BUCKET / 2;
      rc = enqueue_round(e, force_m, plan, mv, skip, cap);
      const int rc2 = (int)hipStreamEndCapture(cap, &g);
      if (!rc) rc = rc2;
    }
    hipGraphExec_t ex = nullptr;
    if (!rc) rc = (int)hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(cap);
    if (rc) return rc;
    it = e->graphs.emplace(key, ex).first;
  }
  return (int)hipGraphLaunch(it->second, s);
}
}  // namespace

int dspark_engine_prepare(dspark_engine* e, dspark_stream_t stream) {
  if (!e) return DSPARK_EINVAL;
  return prepare(e, reinterpret_cast<hipStream_t>(stream), true);
}

int dspark_engine_round(dspark_engine* e, int32_t force_m, int32_t plan_a, dspark_stream_t stream) {
  if (!e || force_m < -1 || force_m > e->B || plan_a < 0) return DSPARK_EINVAL;
  // outside a launch the device's draft cap is the model's: drafts <= max_drafts, so 1 + max_drafts verify rows
  const int mv = std::max(force_m, 1 + e->d.max_drafts);
  return round_enqueue(e, force_m, plan_a, mv, false, reinterpret_cast<hipStream_t>(stream));
}

int dspark_engine_init_seen(dspark_engine* e, const int32_t* tokens, int32_t n, float rep, dspark_stream_t stream) {
  if (!e || n < 0 || (n > 0 && !tokens)) return DSPARK_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int V = e->d.vocab;
  e->host_seen.assign((size_t)(V + 31) / 32, 0u);
  for (int32_t i = 0; i < n; ++i) {
    const int32_t t = tokens[i];
    if (t >= 0 && t < V) e->host_seen[t >> 5] |= 1u << (t & 31);
  }
  if (rep == 0.f) rep = 1.f;
  e->seen_rep = rep;
  e->host_lp[0] = rep;
  e->host_lp[1] = 1.f / rep;
  if (hipMemcpyAsync(e->seen, e->host_seen.data(), e->host_seen.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(e->rep, e->host_lp, 8, hipMemcpyHostToDevice, s) != hipSuccess)
    return DSPARK_EINVAL;
  return hipStreamSynchronize(s) == hipSuccess ? 0 : DSPARK_EINVAL;  // the host buffers are reused by the next call
}

int dspark_engine_capture_tap(dspark_engine* e, int32_t slot, const void* h, int64_t row_stride, int32_t context,
                              int32_t tokens, int32_t tap_from, dspark_stream_t stream) {
  if (!e || !h || slot < 0 || slot >= e->d.n_taps || context < 0 || tokens < 0 || tap_from < 0) return DSPARK_EINVAL;
  const int H = e->d.hidden;
  if (row_stride < H || row_stride % 4 || reinterpret_cast<uintptr_t>(h) % 8) return DSPARK_EINVAL;
  const int first = std::max(context, tap_from);
  const int rows = context + tokens - first;
  if (rows <= 0) return 0;
  if (first - tap_from + rows > e->d.draft_window) return DSPARK_EINVAL;  // beyond the capture buffer
  e->tap_from = tap_from;
  const _Float16* src = static_cast<const _Float16*>(h) + (size_t)(first - context) * row_stride;
  _Float16* dst = e->tapx + (size_t)(first - tap_from) * e->d.n_taps * H + (size_t)slot * H;
  return rms_rows_launch(src, row_stride, e->tap_norms + (size_t)slot * H, e->d.eps, H, dst, (int64_t)e->d.n_taps * H,
                         rows, reinterpret_cast<hipStream_t>(stream));
}

int dspark_engine_project_prompt(dspark_engine* e, int32_t first, int32_t end, dspark_stream_t stream) {
  if (!e || first < 0 || end < first || end - first > e->d.draft_window || end > e->max_context) return DSPARK_EINVAL;
  if (end == first) return 0;
  if (first != e->tap_from) return DSPARK_EINVAL;  // the capture buffer holds positions from tap_from
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (e->mtab_dirty || e->tiles_dirty) {
    const int rc = prepare(e, s, false);
    if (rc) return rc;
  }
  const int B = e->B, nch = (end - first + B - 1) / B;
  if (nch > e->seed_chunks) return DSPARK_EINVAL;
  e->host_seed.assign(nch, dspark_state{});
  for (int c = 0; c < nch; ++c) {
    dspark_state& t = e->host_seed[c];
    t.run = 1;
    t.ctx_pos = first + c * B;
    t.ctx_new = std::min(B, end - t.ctx_pos);
  }
  if (hipMemcpyAsync(e->seed_st, e->host_seed.data(), nch * sizeof(dspark_state), hipMemcpyHostToDevice, s) != hipSuccess)
    return DSPARK_EINVAL;
  const size_t row = (size_t)e->d.n_taps * e->d.hidden;
  int rc = 0;
  for (int c = 0; c < nch && !rc; ++c) {
    e->ast = e->seed_st + c;
    rc = enqueue_context(e, e->tapx + (size_t)c * B * row, false, s);
  }
  e->ast = e->st;
  if (rc) return rc;
  return hipStreamSynchronize(s) == hipSuccess ? 0 : DSPARK_EINVAL;  // host_seed stays in use until the copy is done
}

int dspark_engine_conv_copy(dspark_engine* e, int32_t src, int32_t dst, dspark_stream_t stream) {
  if (!e || src < 0 || dst < 0 || src >= e->conv.slots || dst >= e->conv.slots) return DSPARK_EINVAL;
  if (src == dst) return 0;
  return conv_copy_launch(e->conv, src, dst, reinterpret_cast<hipStream_t>(stream));
}

int dspark_engine_trace(dspark_engine* e, int32_t enable, dspark_stream_t stream) {
  if (!e) return DSPARK_EINVAL;
  e->trace_on = enable != 0;
  if (!e->trace_on) return 0;
  // a fresh trace: count and round counter to zero (outside any graph)
  return (int)hipMemsetAsync(e->trace, 0, 16, reinterpret_cast<hipStream_t>(stream));
}

int dspark_engine_debug_layers(dspark_engine* e, int32_t enable) {
  if (!e) return DSPARK_EINVAL;
  e->dump_on = enable != 0;
  return 0;
}

int dspark_engine_trace_read(dspark_engine* e, uint64_t* out, int32_t cap, int32_t* n) {
  if (!e || !n || cap < 0 || (cap > 0 && !out)) return DSPARK_EINVAL;
  if (hipDeviceSynchronize() != hipSuccess) return DSPARK_EINVAL;
  uint64_t head[2];
  if (hipMemcpy(head, e->trace, 16, hipMemcpyDeviceToHost) != hipSuccess) return DSPARK_EINVAL;
  const int total = (int)std::min<uint64_t>(head[0], DSPARK_TRACE_MAX_MARKS);
  *n = total;
  const int k = std::min(total, cap);
  if (k > 0 && hipMemcpy(out, e->trace + 2, (size_t)k * 16, hipMemcpyDeviceToHost) != hipSuccess) return DSPARK_EINVAL;
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
      khz <= 0)
    return DSPARK_EUNSUPPORTED;
  for (int i = 0; i < k; ++i) out[2 * i + 1] = (uint64_t)((double)out[2 * i + 1] * 1e6 / khz);  // ticks -> ns
  return 0;
}

int dspark_engine_launch(dspark_engine* e, const dspark_launch_args* a, int32_t* out_tokens, int32_t max_out,
                         dspark_launch_result* res, dspark_stream_t stream) {
  if (!e || !a || !res || a->a < 0 || a->a >= e->max_context || a->rounds < 1 || a->force_m < -1 || a->force_m > e->B)
    return DSPARK_EINVAL;
  if (a->anchor < 0 || a->anchor >= e->d.vocab || a->budget < 1) return DSPARK_EINVAL;
  if (a->conv_slot < -1 || a->conv_slot >= e->conv.slots || a->ckpt_slot < -1 || a->ckpt_slot >= e->conv.slots)
    return DSPARK_EINVAL;
  if (a->ckpt_slot >= 0 && a->conv_slot < 0) return DSPARK_EINVAL;  // a checkpoint needs the conv state's slots
  if (a->ctx_new < 0 || a->ctx_new > e->B || a->ctx_lo < 0 || a->skip < 0) return DSPARK_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int block_tokens = 32;  // the prefix cache's block (internal/model/engine.go:30)
  const int stop = std::min((a->a / block_tokens + 1) * block_tokens, e->max_context);
  const int limit = std::min(stop + e->B, e->max_context);
  dspark_state& st = e->host_st;
  st = dspark_state{};
  st.a = a->a;
  st.anchor = a->anchor;
  st.rounds_left = a->rounds;
  st.limit = limit;
  st.budget = std::min(a->budget, 512);
  st.eos = a->eos;
  st.ctx_new = a->ctx_new;
  st.ctx_pos = a->ctx_pos;
  st.ctx_lo = a->ctx_lo;
  st.run = 1;
  st.force_m = a->force_m;
  st.miss = a->miss;
  st.skip = a->skip;
  st.skip_rounds = 1;
  st.stop_at = stop;
  st.ckpt_slot = a->ckpt_slot;
  std::memcpy(st.tokens, a->tokens, sizeof(st.tokens));
  st.tokens[0] = a->anchor;
  const float rep = a->rep == 0.f ? 1.f : a->rep;
  const int32_t md = a->max_drafts > 0 ? std::min(a->max_drafts, e->d.max_drafts) : e->d.max_drafts;
  e->host_lp[0] = rep;
  e->host_lp[1] = 1.f / rep;
  std::memcpy(&e->host_lp[2], &md, 4);
  if (hipMemcpyAsync(e->st, &st, sizeof(st), hipMemcpyHostToDevice, s) != hipSuccess) return DSPARK_EINVAL;
  if (hipMemcpyAsync(e->rep, e->host_lp, sizeof(e->host_lp), hipMemcpyHostToDevice, s) != hipSuccess)
    return DSPARK_EINVAL;
  int rc = 0;
  if (a->conv_slot >= 0) rc = conv_load_launch(e->conv, e->st, a->conv_slot, s);
  // Rounds until the State stops (dspark.hip:2438-2440), without enqueueing rounds that would find run == 0: the host
  // keeps in flight only rounds the last round it has seen proves necessary (each commits at most mv tokens, a skip
  // round exactly one), reading the books each round mirrors into host memory while the next rounds run.
  // Verify width: the launch's draft cap (the reference verifies 1 + drafts, dspark.hip:2657); skip rounds verify the
  // anchor alone (dspark.hip:2441-2444); force_m rounds verify force_m tokens.
  const int mv = a->force_m > 0 ? std::max(a->force_m, 1 + md) : 1 + md;
  const int m_max = a->force_m > 0 ? a->force_m : mv;
  const int skip0 = a->skip;  // skip rounds come first (State.skip_after is 0: no round sets skip again)
  // rounds enqueued before this call (dspark_engine_round) mirror their own books: let them finish first
  if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = DSPARK_EINVAL;
  volatile int32_t* mir = e->mirror;
  for (int i = 0; i < 16; ++i) mir[i] = -1;
  int done = 0, enq = 0;  // rounds completed (seen in the mirror) and enqueued
  int cur_a = st.a, cur_count = 0, cur_run = 1;
  auto needed = [&]() {  // rounds the books of the last round seen prove necessary from there
    if (!cur_run) return 0;
    int left = std::max(1, std::min(stop - cur_a, st.budget - cur_count));
    int need = 0;
    const int sk = std::max(0, skip0 - done);  // skip rounds still ahead commit one token each
    const int k1 = std::min(sk, left);
    need += k1;
    left -= k1;
    if (left > 0) need += (left + m_max - 1) / m_max;
    return std::min(need, a->rounds - done);
  };
  while (!rc) {
    const int need = needed();
    while (!rc && enq - done < need) {
      rc = round_enqueue(e, a->force_m, a->a, enq < skip0 ? 1 : mv, enq < skip0, s);
      ++enq;
    }
    if (rc || enq == done) break;  // nothing in flight: the State has stopped (or every round has run)
    // Wait for the next round's books in the mirror. The stream going idle without them means the rounds in flight
    // stopped without a commit (round_begin's bounds check, a full output buffer): the launch is over.
    const int want = done + 1;  // the State starts with rounds_done = 0
    bool got = false, idle = false;
    for (long spin = 0;; ++spin) {
      const int end = mir[0];
      if (end >= want) {
        std::atomic_thread_fence(std::memory_order_acquire);
        const int run = mir[1], a_now = mir[2], count = mir[3];
        std::atomic_thread_fence(std::memory_order_acquire);
        if (mir[15] == end) {  // one round's values (the next commit had not begun rewriting them)
          done = end;
          cur_run = run;
          cur_a = a_now;
          cur_count = count;
          got = true;
          break;
        }
        continue;
      }
      if (idle) break;  // the mirror was read once more after the stream went idle
      if ((spin & 1023) == 1023) {
        const hipError_t q = hipStreamQuery(s);
        if (q == hipSuccess) {
          idle = true;
        } else if (q != hipErrorNotReady) {
          rc = (int)q;
          break;
        }
      }
    }
    if (!got) break;
  }
  if (!rc && a->conv_slot >= 0) rc = conv_store_launch(e->conv, e->st, a->conv_slot, s);
  // rounds outside a launch use the model's draft cap and the request's penalty again
  e->host_lp_idle[0] = e->seen_rep;
  e->host_lp_idle[1] = 1.f / e->seen_rep;
  std::memcpy(&e->host_lp_idle[2], &e->d.max_drafts, 4);
  if (hipMemcpyAsync(e->rep, e->host_lp_idle, sizeof(e->host_lp_idle), hipMemcpyHostToDevice, s) != hipSuccess && !rc)
    rc = DSPARK_EINVAL;
  if (rc) {
    (void)hipStreamSynchronize(s);  // the host copies above stay in use until the stream has consumed them
    return rc;
  }
  if (hipMemcpyAsync(&res->state, e->st, sizeof(dspark_state), hipMemcpyDeviceToHost, s) != hipSuccess)
    return DSPARK_EINVAL;
  if (hipStreamSynchronize(s) != hipSuccess) return DSPARK_EINVAL;
  const int n = res->state.count;
  const int max_n = std::min(limit - a->a, st.budget);
  if (n < 1 || n > max_n) return DSPARK_EINVAL;  // the reference's "speculative decode: %d tokens" check
  if (out_tokens) {
    if (n > max_out) return DSPARK_ENOSPACE;
    if (hipMemcpy(out_tokens, e->out_tokens, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess) return DSPARK_EINVAL;
  }
  res->count = n;
  res->rounds = res->state.rounds_done;
  res->accepted = res->state.accepted;
  res->verified = res->state.verified;
  res->boundary = stop;
  res->ckpt_written = (a->ckpt_slot >= 0 && res->state.a >= stop) ? 1 : 0;
  res->rounds_enqueued = enq;
  return 0;
}

}  // extern "C"
