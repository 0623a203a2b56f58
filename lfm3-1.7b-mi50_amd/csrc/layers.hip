// Elementwise and small kernels of the DSpark round: embedding, residual + RMS norms, q/k norm + RoPE + K/V page write
// (the context projection's, and the verify and drafter blocks' where the attention kernel does not take the block
// fresh from the mix rows), the drafter's Markov/confidence steps and the round's bookkeeping. Every kernel reads the
// positions it needs (a, ctx_pos, ...) from the device State and returns at once when State.run is 0, so a whole
// round is a fixed launch sequence that can be replayed without the host reading anything back.
// Reference: norm_compute (dspark.hip:722-843), query_fresh + norm_rope (999-1061, 946-951),
// embed (2463-2486), markov_phase + draft loop (2322-2366, 2633-2664), context ring write (2487-2518).
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

__device__ __forceinline__ bool stopped(const dspark_state* st) { return st && ldg(&st->run) == 0; }

// Drafts a round may propose (dspark.hip:2633-2640): the model's (or the launch's, when md_dev is set) draft cap, the
// block, the context limit and the budget.
__device__ __forceinline__ int draft_cap(const dspark_state* st, int max_drafts, const int32_t* md_dev, int block) {
  const int md = md_dev ? min(max_drafts, ldg(md_dev)) : max_drafts;
  return min(min(md, block - 1), min(st->limit - st->a, st->budget - st->count) - 1);
}

// ---------------------------------------------------------------- embedding
// h[t][:] = embed[token(t)][:] (fp16 -> fp32). mode 0: token(t) = st->tokens[t]; mode 1 (drafter block):
// t == 0 ? st->anchor : mask_token. Tokens outside the vocabulary read row 0.
// The run flag and the token come from one round trip (vector loads issued together); the row (H % 8 == 0, H <= 8192)
// is read as 16 bytes per thread per 2048 columns, every load issued before the first store (clamped to a valid
// column; the stores are guarded).
__global__ __launch_bounds__(256) void embed_kernel(const _Float16* embed, const dspark_state* st, int mode, int mask_token,
                                                    int M, int H, int V, float* h) {
  const int t = blockIdx.x;
  const int run = run_flag_load(st);
  const int tok_v = state_word_load(st, mode == 0 ? (int)offsetof(dspark_state, tokens) + 4 * t
                                                  : (int)offsetof(dspark_state, anchor));
  if (!run_flag_set(run)) return;
  int tok = __builtin_amdgcn_readfirstlane(tok_v);
  if (mode != 0 && t != 0) tok = mask_token;
  if (tok < 0 || tok >= V) tok = 0;
  const _Float16* row = embed + (size_t)tok * H;
  constexpr int G = 4;
  half8 v[G];
#pragma unroll
  for (int g = 0; g < G; ++g) v[g] = ldg(reinterpret_cast<const half8*>(row + min(2048 * g + 8 * (int)threadIdx.x, H - 8)));
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i = 2048 * g + 8 * (int)threadIdx.x;
    if (i < H) {
      f32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = (float)v[g][j];
        hi[j] = (float)v[g][4 + j];
      }
      *reinterpret_cast<f32x4*>(h + (size_t)t * H + i) = lo;
      *reinterpret_cast<f32x4*>(h + (size_t)t * H + i + 4) = hi;
    }
  }
}

// ---------------------------------------------------------------- residual + RMS norm (norm_compute)
// v = sum of `bands` inputs in band order; a = bands == 0 ? 0 : (sandwich ? rsqrt(mean(v^2) + eps) : 1);
// h_new = h_old + a * v * post_w; x = fp16(h_new * rsqrt(mean(h_new^2) + eps) * norm_w).
// One block per (row, group): blockIdx.y selects a group with its own inputs (the drafter's tap norms).
// EMB: h_old is row token(t) of the embedding table (a pass's first layer, embed_kernel folded in).
template <int NK, bool HAS_H, bool EMB = false>
__global__ __launch_bounds__(256) void resnorm_kernel(ResNormParams p) {
  const int run = run_flag_load(p.st);  // tested after every load is in flight
  const int t = blockIdx.x, gi = blockIdx.y;
  const int H = p.H;
  const float* hold = HAS_H ? p.h_old + (size_t)gi * p.group_stride + (size_t)t * H : nullptr;
  const _Float16* erow = nullptr;
  if constexpr (EMB) {
    // the token from the State (a vector load issued with the run flag), then its row
    const int tok_v = state_word_load(p.st, p.embed_mode == 0 ? (int)offsetof(dspark_state, tokens) + 4 * t
                                                              : (int)offsetof(dspark_state, anchor));
    int tok = __builtin_amdgcn_readfirstlane(tok_v);
    if (p.embed_mode != 0 && t != 0) tok = p.mask_token;
    if (tok < 0 || tok >= p.vocab) tok = 0;
    erow = p.embed + (size_t)tok * H;
  }
  const _Float16* nw = p.norm_w + (size_t)gi * p.norm_w_stride;
  const _Float16* pw = p.post_w ? p.post_w : nw;  // no post_w: loaded from nw and replaced by 1 below
  // Four consecutive columns per thread per 1024 (NK = ceil(H / 1024) groups). Loads go to clamped, valid columns
  // with no branches, so every load of the kernel is in flight before the first is used; columns past H are masked.
  int col[NK];
  bool ok[NK];
  f32x4 hv[NK], vv[NK];
  half4 wn[NK], wp[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = 1024 * k + 4 * (int)threadIdx.x;
    ok[k] = i < H;
    col[k] = min(i, H - 4);
    if constexpr (EMB) {
      const half4 e4 = ldg(reinterpret_cast<const half4*>(erow + col[k]));
      hv[k] = f32x4{(float)e4[0], (float)e4[1], (float)e4[2], (float)e4[3]};
    } else {
      hv[k] = HAS_H ? ldg(reinterpret_cast<const f32x4*>(hold + col[k])) : f32x4{0, 0, 0, 0};
    }
    wn[k] = ldg(reinterpret_cast<const half4*>(nw + col[k]));
    wp[k] = ldg(reinterpret_cast<const half4*>(pw + col[k]));
    vv[k] = f32x4{0, 0, 0, 0};
  }
  // Bands BB at a time (all of a batch's loads in flight before the first add; the adds stay in band order). The
  // first batch is outside the loop: at a loop head the compiler's wait for the previous iteration's loads would also
  // hold the first band loads back until the loads above had arrived.
  constexpr int BB = 2;  // the round's GEMMs write at most 2 bands
  auto band_batch = [&](int b0) {
    f32x4 lb[BB][NK];
#pragma unroll
    for (int bb = 0; bb < BB; ++bb) {
      const float* vb = p.v + (size_t)min(b0 + bb, p.bands - 1) * p.v_band_stride + (size_t)t * H;
#pragma unroll
      for (int k = 0; k < NK; ++k) lb[bb][k] = ldg(reinterpret_cast<const f32x4*>(vb + col[k]));
    }
    // every load issued before the first add waits; a select, not a branch: under a branch the compiler sinks the
    // second band's loads into it, behind the wait for the first band's values
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int bb = 0; bb < BB; ++bb) {
      const bool use = b0 + bb < p.bands;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const f32x4 sum = vv[k] + lb[bb][k];
        vv[k] = use ? sum : vv[k];
      }
    }
  };
  if (p.bands > 0) band_batch(0);
  for (int b0 = BB; b0 < p.bands; b0 += BB) band_batch(b0);
  // the stop flag is tested once every load is in flight (a test before the band loads would hold them back by the
  // flag's latency); a stopped round waits for the loads and writes nothing
  if (!run_flag_set(run)) {
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const half4 one = {1, 1, 1, 1};
  const f32x4 zero = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (!p.post_w) wp[k] = one;
    if (!ok[k]) hv[k] = vv[k] = zero;
  }
  float s_vv = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) s_vv += vv[k][j] * vv[k][j];
  // one LDS slot set per sum (the kernel takes two), so a sum needs one barrier, not one more to guard a reused set
  __shared__ float red[2][4];
  auto block_sum = [&](int k, float x) -> float {
    x = wave_sum(x);
    if ((threadIdx.x & 63) == 0) red[k][threadIdx.x >> 6] = x;
    __syncthreads();
    return (red[k][0] + red[k][1]) + (red[k][2] + red[k][3]);
  };
  float a = 0.f;
  if (p.bands > 0) a = p.sandwich ? rsqrtf(block_sum(0, s_vv) / H + p.eps) : 1.f;
  float s_hh = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hv[k][j] = fmaf(vv[k][j] * a, (float)wp[k][j], hv[k][j]);
      s_hh += hv[k][j] * hv[k][j];
    }
  const float inv = rsqrtf(block_sum(1, s_hh) / H + p.eps);
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = 1024 * k + 4 * (int)threadIdx.x;
    float xf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xf[j] = hv[k][j] * inv * (float)wn[k][j];
    half4 x;
    float xsc = 0.f;
    if (p.xsc) {
      // LFM3_X8 (norm_compute, dspark.hip:802-823): the fp32 value as int8 codes with one scale per 16 columns, the 4
      // threads of a quad holding a piece (columns past H are zero, whole pieces: H % 16 == 0)
      float m = fmaxf(fmaxf(fabsf(xf[0]), fabsf(xf[1])), fmaxf(fabsf(xf[2]), fabsf(xf[3])));
      m = fmaxf(m, __shfl_xor(m, 1));
      m = fmaxf(m, __shfl_xor(m, 2));
      xsc = fmaxf(__fdiv_rn(m, 127.f), 1e-20f);
      const float r = __builtin_amdgcn_rcpf(xsc);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = (_Float16)rintf(xf[j] * r);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = (_Float16)xf[j];
    }
    if (ok[k]) {
      const size_t o = (size_t)gi * p.group_stride + (size_t)t * H + i;
      if (p.dst) *reinterpret_cast<f32x4*>(p.dst + o) = hv[k];
      if (p.tap) *reinterpret_cast<f32x4*>(p.tap + (size_t)t * H + i) = hv[k];
      const int xcol = gi * (int)p.x_group_stride + i;
      const size_t xo = p.xop ? xop_elem(t, xcol, p.xop) : (size_t)gi * p.x_group_stride + (size_t)t * p.x_row + i;
      *reinterpret_cast<half4*>(p.x16 + xo) = x;
      if (p.xsc && (threadIdx.x & 3) == 0) p.xsc[(size_t)t * p.xsc_row + xcol / 16] = xsc;
    }
  }
}

// ---------------------------------------------------------------- q/k norm + RoPE + K/V page write (query_fresh)
// One wave per (token, head) over heads [0, QH) for q and [QH, QH + KVH) for k (v rides with k). Row layout of `mix`
// per token: q [QH*D] | k [KVH*D] | v [KVH*D] | gate [QH] (gate optional), `row` floats apart. Position of token t:
// base + t with base = st->a (verify, drafter block) or st->ctx_pos (context projection); tokens t >= count
// (count = M, or st->ctx_new) are skipped.
// D (64 or 128, p.D) as a template argument: the per-lane dims loops unroll, so the row loads go out together (with
// D a run-time value, each pass of the loads loop waited for the previous one's: four round trips at D = 128).
template <int D>
__device__ __forceinline__ void qkrope_body(const QkRopeParams& p) {
  // The parameters' three 64-byte lines (fields at 0, 64 and 132 bytes span any placement of the 136-byte struct) in
  // one round trip: read where they are first used, behind the early-exit tests, they were four dependent misses.
  asm volatile("" ::"s"(p.st), "s"(p.eps), "s"(p.count_from_ctx));
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = p.QH + p.KVH;
  if (task >= p.M * heads) return;
  const int t = task / heads, hh = task % heads;
  const bool isq = hh < p.QH;
  if (isq && !p.q16) return;
  // Two rounds of loads: first the row, V, the norm weights and the State words (run flag, position base, token count;
  // vector loads, tested and used once everything is in flight), then the RoPE row and the block-table entry of the
  // position. (Loaded where they are used, they had formed a chain of five dependent load latencies.)
  const int run = run_flag_load(p.st);
  const int base_v = state_word_load(p.st, p.pos_from_ctx ? (int)offsetof(dspark_state, ctx_pos)
                                                           : (int)offsetof(dspark_state, a));
  const int count_v = p.count_from_ctx ? state_word_load(p.st, (int)offsetof(dspark_state, ctx_new)) : p.M;
  constexpr int half = D / 2;
  const float* row = p.mix + (size_t)t * p.row;
  const float* src = isq ? row + (size_t)hh * D : row + (size_t)p.QH * D * (p.q16 ? 1 : 0) + (size_t)(hh - p.QH) * D;
  const _Float16* nw = isq ? p.q_norm : p.k_norm;
  const int kvh = hh - p.QH;
  const float* vsrc = row + (size_t)p.QH * D * (p.q16 ? 1 : 0) + (size_t)p.KVH * D + (size_t)kvh * D;
  // lane l holds dims l and l + 32 (D = 64) or l, l+32, l+64, l+96 (D = 128): pairs (i, i + D/2) share a lane
  constexpr int ne = D / 32;  // 2 or 4
  float v[ne], vv[ne], wn[ne];
#pragma unroll
  for (int e = 0; e < ne; ++e) {
    const int d = (lane & 31) + 32 * e;
    v[e] = src[d];
    wn[e] = (float)nw[d];
    vv[e] = isq ? 0.f : vsrc[d];
  }
  if (!run_flag_set(run)) {  // a stopped round writes nothing
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const int count = __builtin_amdgcn_readfirstlane(count_v);
  if (t >= count) return;
  const int pos = __builtin_amdgcn_readfirstlane(base_v) + t;
  // RoPE: pair (i, i + half) for i < rot, cos/sin from the table row of `pos` (cos | sin, D halves)
  const _Float16* rt = p.rope + (size_t)pos * D;
  float cs[ne / 2], sn[ne / 2];
#pragma unroll
  for (int e = 0; e < ne / 2; ++e) {
    const int i = (lane & 31) + 32 * e;  // i < half
    cs[e] = (float)rt[i];
    sn[e] = (float)rt[half + i];
  }
  const int lp = pos / PAGE, slot = pos % PAGE;
  const int phys = isq ? 0 : (p.bt ? p.bt[lp] : lp);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < ne; ++e) ss += v[e] * v[e];
  // lanes 32..63 duplicate lanes 0..31; sum over the first 32 lanes
  ss = (lane < 32) ? ss : 0.f;
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / D + p.eps);
#pragma unroll
  for (int e = 0; e < ne; ++e) v[e] = v[e] * inv * wn[e];
  float r[ne];
#pragma unroll
  for (int e = 0; e < ne; ++e) r[e] = v[e];
#pragma unroll
  for (int e = 0; e < ne / 2; ++e) {
    const int i = (lane & 31) + 32 * e;  // i < half
    if (i < p.rot) {
      const float c = cs[e], s = sn[e];
      const float x0 = v[e], x1 = v[e + ne / 2];
      r[e] = x0 * c - x1 * s;
      r[e + ne / 2] = x1 * c + x0 * s;
    }
  }
  if (!isq && p.rec) {
    // int8 record of (pos, kvh) (D = 128: lanes 0..31 hold dims l, l + 32, l + 64, l + 96; lanes 32..63 repeat
    // them): quantize_pair of K (normed, rotated, fp32) and of V (fp32), kernels/ops.hip:212-251
    float ak = 0.f, av = 0.f;
#pragma unroll
    for (int e = 0; e < ne; ++e) {
      ak = fmaxf(ak, fabsf(r[e]));
      av = fmaxf(av, fabsf(vv[e]));
    }
    ak = wave_max(ak);
    av = wave_max(av);
    if (lane >= 32) return;
    uint8_t* rb = p.rec + (size_t)phys * ((size_t)PAGE * p.KVH * 264) + ((size_t)slot * p.KVH + kvh) * 264;
    const float ks = rec_scale(ak), vs = rec_scale(av);
    const float ki = __fdiv_rn(1.f, ks), vi = __fdiv_rn(1.f, vs);
#pragma unroll
    for (int e = 0; e < ne; ++e) {
      const int d = (lane & 31) + 32 * e;
      rb[d] = (uint8_t)rec_code(r[e], ki);
      rb[D + 4 + d] = (uint8_t)rec_code(vv[e], vi);
    }
    if (lane == 0) {
      *reinterpret_cast<float*>(rb + D) = ks;
      *reinterpret_cast<float*>(rb + 2 * D + 4) = vs;
    }
    return;
  }
  if (lane >= 32) return;
  if (isq) {
    _Float16* q = p.q16 + ((size_t)t * p.QH + hh) * D;
#pragma unroll
    for (int e = 0; e < ne; ++e) q[(lane & 31) + 32 * e] = (_Float16)r[e];
    if (p.gate && p.gate_in_mix) {
      if (lane == 0) p.gate[(size_t)t * p.QH + hh] = row[(size_t)(p.QH + 2 * p.KVH) * D + hh];
    }
    return;
  }
  // K (normed, rotated) and V (as is) into the pages at `pos`
  _Float16* kb = p.kp + ((size_t)phys * p.KVH + kvh) * (PAGE * D);
  _Float16* vb = p.vp + ((size_t)phys * p.KVH + kvh) * (D * PAGE);
#pragma unroll
  for (int e = 0; e < ne; ++e) {
    const int d = (lane & 31) + 32 * e;
    kb[k_page_elem(slot, d, D)] = (_Float16)r[e];
    vb[v_page_elem(slot, d)] = (_Float16)vv[e];
  }
}

template <int D>
__global__ __launch_bounds__(256) void qkrope_kernel(QkRopeParams p) { qkrope_body<D>(p); }

// Several layers of the same shape in one launch (the context projection's drafter layers): layer blockIdx.y.
template <int D>
__global__ __launch_bounds__(256) void qkrope_batch_kernel(QkRopeBatch b) { qkrope_body<D>(b.l[blockIdx.y]); }

// ---------------------------------------------------------------- drafter: Markov + confidence (markov_phase)
// Step j (0-based) proposes draft j+1 from prev = (j == 0 ? anchor : the token of step j-1's argmax key):
//   cap = min(max_drafts, block - 1, min(limit - a, budget - count) - 1); steps j >= cap do nothing;
//   conf = base[j][N] + c2[prev] + conf_bias; conf < thr stops drafting (st->M = j + 1);
//   z[r] = base[j][r] + (sum_k w2q[r][k] * w1q[prev][k]) * w2s[r] * w1s[prev]; best[j] = max key(z[r], r);
//   st->tokens[j] = prev (for j >= 1). A stop recorded by an earlier step turns the later ones into no-ops.
// Launched as block - 1 steps, then markov_finalize writes the last token and st->M.
__global__ __launch_bounds__(256) void markov_kernel(MarkovParams p, int j) {
  // rows: one per thread, 256 rows per block; w2q stored row-major [N][rank]. Everything that does not depend on the
  // previous draft (this row's first 256 w2 bytes, its scale, its base term, the confidence term) is loaded before
  // the State and the previous step's key are read, so a step waits on one chain: key -> crop id -> w1 row.
  constexpr int RC = 16;  // 16-byte chunks of w2 held in registers (rank <= 256 in one pass)
  const int r = blockIdx.x * 256 + threadIdx.x;
  const bool live = r < p.N;
  const int rr = live ? r : p.N - 1;
  const int8_t* w2 = p.w2q + (size_t)rr * p.rank;
  const int rc0 = min(RC, p.rank / 16);
  u32x4 a4[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c)
    if (c < rc0) a4[c] = ldg(reinterpret_cast<const u32x4*>(w2 + 16 * c));
  const float bz = ldg(p.base + (size_t)j * p.stride + rr);
  const float s2 = ldg(p.w2s + rr);
  const float bconf = ldg(p.base + (size_t)j * p.stride + p.N);

  dspark_state* st = p.st;
  if (stopped(st)) return;
  if (ldg(&st->M) != 0) return;  // drafting already stopped (M is set by the stop or the finalize)
  const int cap = draft_cap(st, p.max_drafts, p.max_drafts_dev, p.block);
  if (j >= cap) return;
  int prev;
  if (j == 0) {
    prev = st->anchor;
  } else {
    const uint64_t key = __hip_atomic_load(p.best + (j - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = p.crop_ids[0xffffffffu - (uint32_t)key];
  }
  const int8_t* w1 = p.w1q + (size_t)prev * p.rank;
  u32x4 b4[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c)
    if (c < rc0) b4[c] = ldg(reinterpret_cast<const u32x4*>(w1 + 16 * c));
  const float c2 = ldg(p.c2 + prev), s1 = ldg(p.w1s + prev);
  const float conf = bconf + c2 + p.conf_bias;
  if (!(conf >= p.conf_thr)) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      if (j >= 1) st->tokens[j] = prev;
      st->M = j + 1;
    }
    return;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0 && j >= 1) st->tokens[j] = prev;
  int acc = 0;
#pragma unroll
  for (int c = 0; c < RC; ++c)
    if (c < rc0) {
      acc = __builtin_amdgcn_sdot4(a4[c][0], b4[c][0], acc, false);
      acc = __builtin_amdgcn_sdot4(a4[c][1], b4[c][1], acc, false);
      acc = __builtin_amdgcn_sdot4(a4[c][2], b4[c][2], acc, false);
      acc = __builtin_amdgcn_sdot4(a4[c][3], b4[c][3], acc, false);
    }
  for (int k = 16 * RC; k < p.rank; k += 16) {  // ranks above 256
    const u32x4 x = ldg(reinterpret_cast<const u32x4*>(w2 + k));
    const u32x4 y = ldg(reinterpret_cast<const u32x4*>(w1 + k));
    acc = __builtin_amdgcn_sdot4(x[0], y[0], acc, false);
    acc = __builtin_amdgcn_sdot4(x[1], y[1], acc, false);
    acc = __builtin_amdgcn_sdot4(x[2], y[2], acc, false);
    acc = __builtin_amdgcn_sdot4(x[3], y[3], acc, false);
  }
  uint64_t best = 0;
  if (live) best = argmax_key(fmaf((float)acc, s2 * s1, bz), (uint32_t)r);
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0 && best)
    __hip_atomic_fetch_max(p.best + j, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After the steps: if drafting ran to its cap, the last draft comes from the last step's key and M = 1 + drafts.
__global__ void markov_finalize(MarkovParams p) {
  dspark_state* st = p.st;
  if (stopped(st) || threadIdx.x != 0) return;
  st->tokens[0] = st->anchor;
  if (st->M != 0) return;  // stopped by confidence: tokens and M already written
  const int cap = draft_cap(st, p.max_drafts, p.max_drafts_dev, p.block);
  const int drafts = max(cap, 0);
  if (drafts >= 1) {
    const uint64_t key = p.best[drafts - 1];
    st->tokens[drafts] = p.crop_ids[0xffffffffu - (uint32_t)key];
  }
  st->M = drafts + 1;
}

// ---------------------------------------------------------------- drafter: the Markov chain from a transition table
// T[c][r] = (float) (w1q[crop_ids[c]] . w2q[r]) for crop indices c, r < N: the integer dot of every step after the
// first (whose previous token is always a crop token) depends on the weights only, so it is computed once per model
// (exact in fp32: |dot| <= rank * 127 * 127 < 2^24). c2c[c] = c2[crop_ids[c]], s1c[c] = w1s[crop_ids[c]]. 64 x 64
// tiles, 256 threads with 4 x 4 outputs each, rank in 256-byte slices through LDS. Crop ids outside the vocabulary
// read row 0 (the table is built before any round checks them).
__global__ __launch_bounds__(256) void markov_table_kernel(const int8_t* w1q, const float* w1s, const float* c2,
                                                           const int8_t* w2q, const int32_t* crop_ids, int N, int rank,
                                                           int vocab, float* T, float* c2c, float* s1c) {
  constexpr int KS = 256, ROWB = KS + 16;  // rank slice and padded LDS row
  __shared__ __attribute__((aligned(16))) int8_t As[64 * ROWB], Bs[64 * ROWB];
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const int c0 = blockIdx.y * 64, q0 = blockIdx.x * 64;
  if (blockIdx.x == 0 && tid < 64 && c0 + tid < N) {
    int id = crop_ids[c0 + tid];
    if (id < 0 || id >= vocab) id = 0;
    c2c[c0 + tid] = c2[id];
    s1c[c0 + tid] = w1s[id];
  }
  int acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0;
  for (int k0 = 0; k0 < rank; k0 += KS) {
    const int pieces = min(KS, rank - k0) / 16;
    for (int idx = tid; idx < 64 * pieces; idx += 256) {
      const int row = idx / pieces, pc = idx % pieces;
      int id = crop_ids[min(c0 + row, N - 1)];
      if (id < 0 || id >= vocab) id = 0;
      const int r = min(q0 + row, N - 1);
      *reinterpret_cast<u32x4*>(As + row * ROWB + 16 * pc) =
          ldg(reinterpret_cast<const u32x4*>(w1q + (size_t)id * rank + k0 + 16 * pc));
      *reinterpret_cast<u32x4*>(Bs + row * ROWB + 16 * pc) =
          ldg(reinterpret_cast<const u32x4*>(w2q + (size_t)r * rank + k0 + 16 * pc));
    }
    __syncthreads();
    for (int pc = 0; pc < pieces; ++pc) {
      u32x4 av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = *reinterpret_cast<const u32x4*>(As + (4 * ty + i) * ROWB + 16 * pc);
        bv[i] = *reinterpret_cast<const u32x4*>(Bs + (4 * tx + i) * ROWB + 16 * pc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j] = __builtin_amdgcn_sdot4(av[i][e], bv[j][e], acc[i][j], false);
    }
    __syncthreads();
  }
  const int q = q0 + 4 * tx;
  if (q >= N) return;  // N % 16 == 0: the 4 columns are all inside or all outside
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + 4 * ty + i;
    if (c < N)
      *reinterpret_cast<f32x4*>(T + (size_t)c * N + q) =
          f32x4{(float)acc[i][0], (float)acc[i][1], (float)acc[i][2], (float)acc[i][3]};
  }
}

// Draft steps 1 .. block - 2 and the finalize in one workgroup. Step j's previous token is the crop token of step
// j - 1's key, so its dots are row ci of the table and its values fmaf(T[ci][r], w2s[r] * s1c[ci], base[j][r]) are
// markov_kernel's bit for bit; the confidence test and the writes of tokens, M and the per-step keys are
// markov_kernel's and markov_finalize's. Step 0 (previous token = the anchor, any vocabulary id) stays with
// markov_kernel. Thread t owns rows 16 t .. 16 t + 15 (N <= 16384), so a step is one table row read with all its
// loads in flight, then a workgroup argmax.
constexpr int CHAIN_THREADS = 1024, CHAIN_ROWS = 16, CHAIN_MAX_N = CHAIN_THREADS * CHAIN_ROWS;
__global__ __launch_bounds__(1024) void markov_chain_kernel(MarkovParams p) {
  __shared__ uint64_t red[2][CHAIN_THREADS / 64];  // double-buffered by step parity: one barrier per step
  dspark_state* st = p.st;
  if (stopped(st)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = p.N, r0 = CHAIN_ROWS * tid;
  const bool live = r0 < N;  // N % 16 == 0: a thread's rows are all inside or all outside
  f32x4 s2[CHAIN_ROWS / 4];
#pragma unroll
  for (int i = 0; i < CHAIN_ROWS / 4; ++i)
    s2[i] = live ? ldg(reinterpret_cast<const f32x4*>(p.w2s + r0) + i) : f32x4{0, 0, 0, 0};
  const int cap = draft_cap(st, p.max_drafts, p.max_drafts_dev, p.block);
  int M = st->M;  // nonzero when step 0's confidence test stopped drafting
  uint64_t key = 0;
  if (M == 0 && cap >= 1) key = __hip_atomic_load(p.best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // A step's base row and confidence word do not depend on the previous step's argmax: each is loaded one step ahead
  // (with the current step's table row), so only the table row's latency lies on the chain.
  f32x4 bv[CHAIN_ROWS / 4];
  float bconf = 0.f;
  auto base_row = [&](int j, f32x4 (&b)[CHAIN_ROWS / 4], float& c) {
    const float* brow = p.base + (size_t)j * p.stride;
    if (live) {
#pragma unroll
      for (int i = 0; i < CHAIN_ROWS / 4; ++i) b[i] = ldg(reinterpret_cast<const f32x4*>(brow + r0) + i);
    }
    c = ldg(brow + N);
  };
  if (M == 0 && cap >= 2) base_row(1, bv, bconf);
  for (int j = 1; j < cap && M == 0; ++j) {
    const uint32_t ci = 0xffffffffu - (uint32_t)key;
    f32x4 tv[CHAIN_ROWS / 4];
    if (live) {
      const f32x4* trow = reinterpret_cast<const f32x4*>(p.table + (size_t)ci * N + r0);
#pragma unroll
      for (int i = 0; i < CHAIN_ROWS / 4; ++i) tv[i] = ldg(trow + i);
    }
    const int prev = ldg(p.crop_ids + ci);
    const float s1 = ldg(p.s1c + ci);
    const float conf = bconf + ldg(p.c2c + ci) + p.conf_bias;
    f32x4 bn[CHAIN_ROWS / 4];
    float bnconf = 0.f;
    base_row(min(j + 1, cap - 1), bn, bnconf);  // the last step reloads its own row (unused)
    if (!(conf >= p.conf_thr)) {
      if (tid == 0) {
        st->tokens[j] = prev;
        st->M = j + 1;
      }
      M = j + 1;
      break;
    }
    if (tid == 0) st->tokens[j] = prev;
    uint64_t best = 0;
    if (live) {
#pragma unroll
      for (int i = 0; i < CHAIN_ROWS / 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t k = argmax_key(fmaf(tv[i][e], s2[i][e] * s1, bv[i][e]), (uint32_t)(r0 + 4 * i + e));
          best = k > best ? k : best;
        }
    }
    best = wave_max_u64(best);
    // red[j & 1] was last read in step j - 2, before every thread passed step j - 1's barrier
    if (lane == 0) red[j & 1][wave] = best;
    __syncthreads();
    key = red[j & 1][0];
#pragma unroll
    for (int w = 1; w < CHAIN_THREADS / 64; ++w) key = red[j & 1][w] > key ? red[j & 1][w] : key;
    if (tid == 0) p.best[j] = key;
#pragma unroll
    for (int i = 0; i < CHAIN_ROWS / 4; ++i) bv[i] = bn[i];
    bconf = bnconf;
  }
  if (p.plant) {
    // Planted drafts replace the chain's (the plant kernel's books, one launch fewer): after a barrier that orders them
    // behind thread 0's chain stores, lane j of wave 0 loads plant[a + j] and stores tokens[j] (one load and one store
    // each, instead of a load-store chain on one thread), lane 0 the anchor and M.
    __syncthreads();
    if (wave != 0) return;
    const int a = st->a, drafts = max(cap, 0);
    if (lane >= 1 && lane <= drafts) st->tokens[lane] = ldg(p.plant + a + lane);
    if (lane == 0) {
      st->tokens[0] = st->anchor;
      st->M = drafts + 1;
    }
    return;
  }
  if (tid != 0) return;
  st->tokens[0] = st->anchor;
  if (M != 0) return;  // stopped by confidence: tokens and M already written
  const int drafts = max(cap, 0);
  if (drafts >= 1) st->tokens[drafts] = p.crop_ids[0xffffffffu - (uint32_t)key];
  st->M = drafts + 1;
}

// ---------------------------------------------------------------- round start
// Clears the per-round scratch the kernels fold into (argmax keys) and the draft count, marks the anchor seen
// (dspark.hip:2432-2435). A State the buffers cannot hold -- anchor position a with a + block > max_pos, an anchor
// outside the vocabulary, or an emitted count with no room for a block more in out_tokens -- stops the run instead
// (every later kernel of the round returns on run == 0).
__global__ void round_begin_kernel(dspark_state* st, uint64_t* keys, int nkeys, uint32_t* seen, int block, int max_pos,
                                   int vocab, int out_cap) {
  if (stopped(st)) return;
  const int a = st->a, anchor = st->anchor, count = st->count;
  if (a < 0 || a + block > max_pos || anchor < 0 || anchor >= vocab || count < 0 || count + block > out_cap) {
    if (threadIdx.x == 0) st->run = 0;
    return;
  }
  for (int i = threadIdx.x; i < nkeys; i += blockDim.x) keys[i] = 0;
  if (threadIdx.x == 0) {
    st->M = 0;
    const int t = st->anchor;
    if (seen && t >= 0) seen[t >> 5] |= 1u << (t & 31);
  }
}

// Verify-only rounds (force_m: verify the tokens already in the State, no drafter; dspark.hip:147, 2442-2451).
__global__ void force_m_kernel(dspark_state* st, int m) {
  if (stopped(st) || threadIdx.x != 0) return;
  st->tokens[0] = st->anchor;
  st->M = m;
}

// Phase trace mark (one thread; stream order makes the marks of a round sequential, so no atomics): the clock is the
// constant-rate wall clock, read first. buf[1] = rounds opened << 1 | whether the current round runs.
__global__ void trace_mark_kernel(uint64_t* buf, const dspark_state* st, int phase, int begin, int max_marks) {
  if (threadIdx.x != 0) return;
  const uint64_t clk = wall_clock64();
  if (begin) {
    const uint64_t active = st->run != 0 ? 1 : 0;
    buf[1] = (((buf[1] >> 1) + active) << 1) | active;
    if (!active) return;
  } else if (!(buf[1] & 1)) {
    return;
  }
  const uint64_t round = (buf[1] >> 1) - 1, i = buf[0];
  if (i < (uint64_t)max_marks) {
    buf[2 + 2 * i] = (uint64_t)(uint32_t)phase | (round << 32);
    buf[3 + 2 * i] = clk;
  }
  buf[0] = i + 1;
}

int trace_mark_launch(uint64_t* buf, const dspark_state* st, int phase, int begin, int max_marks, hipStream_t s) {
  hipLaunchKernelGGL(trace_mark_kernel, dim3(1), dim3(64), 0, s, buf, st, phase, begin, max_marks);
  return (int)hipGetLastError();
}

// Planted drafts (benchmarks of a set acceptance rate on random-init models): after the drafter has run, its drafts
// are replaced by plant[a + 1 .. a + M - 1], with M = 1 + the drafter's cap on drafts this round (the same cap
// markov_kernel applies, so limit and budget still bound the round).
__global__ void plant_kernel(dspark_state* st, const int32_t* plant, int block, int max_drafts,
                             const int32_t* max_drafts_dev) {
  if (stopped(st) || threadIdx.x != 0) return;
  const int a = st->a;
  const int cap = draft_cap(st, max_drafts, max_drafts_dev, block);
  const int drafts = max(cap, 0);
  st->tokens[0] = st->anchor;
  for (int j = 1; j <= drafts; ++j) st->tokens[j] = plant[a + j];
  st->M = drafts + 1;
}

// ---------------------------------------------------------------- host launchers
int embed_launch(const void* embed, const dspark_state* st, int mode, int mask_token, int M, int H, int V, float* h,
                 hipStream_t s) {
  if (!st || H < 8 || H % 8 || H > 8192) return DSPARK_EINVAL;
  hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, s, (const _Float16*)embed, st, mode, mask_token, M, H, V, h);
  return (int)hipGetLastError();
}
template <int NK>
static void resnorm_launch_nk(const ResNormParams& p, dim3 grid, hipStream_t s) {
  if (p.embed)
    hipLaunchKernelGGL((resnorm_kernel<NK, false, true>), grid, dim3(256), 0, s, p);
  else if (p.h_old)
    hipLaunchKernelGGL((resnorm_kernel<NK, true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((resnorm_kernel<NK, false>), grid, dim3(256), 0, s, p);
}

int resnorm_launch(const ResNormParams& p, int rows, int groups, hipStream_t s) {
  if (p.H < 4 || p.H % 4 || p.H > 8192) return DSPARK_EINVAL;
  if (p.embed && (p.h_old || !p.st || groups != 1 || p.vocab < 1)) return DSPARK_EINVAL;
  const dim3 grid(rows, groups);
  switch ((p.H + 1023) / 1024) {
    case 1: resnorm_launch_nk<1>(p, grid, s); break;
    case 2: resnorm_launch_nk<2>(p, grid, s); break;
    case 3: resnorm_launch_nk<3>(p, grid, s); break;
    case 4: resnorm_launch_nk<4>(p, grid, s); break;
    case 5: resnorm_launch_nk<5>(p, grid, s); break;
    case 6: resnorm_launch_nk<6>(p, grid, s); break;
    case 7: resnorm_launch_nk<7>(p, grid, s); break;
    default: resnorm_launch_nk<8>(p, grid, s); break;
  }
  return (int)hipGetLastError();
}
int qkrope_launch(const QkRopeParams& p, hipStream_t s) {
  if (p.D != 64 && p.D != 128) return DSPARK_EINVAL;
  const int tasks = p.M * (p.QH + p.KVH);
  if (p.D == 64)
    hipLaunchKernelGGL(qkrope_kernel<64>, dim3((tasks + 3) / 4), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(qkrope_kernel<128>, dim3((tasks + 3) / 4), dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

int qkrope_batch_launch(const QkRopeBatch& b, hipStream_t s) {
  if (b.n < 1 || b.n > QKROPE_BATCH) return DSPARK_EINVAL;
  const QkRopeParams& p = b.l[0];
  for (int j = 1; j < b.n; ++j)
    if (b.l[j].M != p.M || b.l[j].QH != p.QH || b.l[j].KVH != p.KVH) return DSPARK_EINVAL;
  if (p.D != 64 && p.D != 128) return DSPARK_EINVAL;
  for (int j = 1; j < b.n; ++j)
    if (b.l[j].D != p.D) return DSPARK_EINVAL;
  const int tasks = p.M * (p.QH + p.KVH);
  if (p.D == 64)
    hipLaunchKernelGGL(qkrope_batch_kernel<64>, dim3((tasks + 3) / 4, b.n), dim3(256), 0, s, b);
  else
    hipLaunchKernelGGL(qkrope_batch_kernel<128>, dim3((tasks + 3) / 4, b.n), dim3(256), 0, s, b);
  return (int)hipGetLastError();
}
int markov_launch(const MarkovParams& p, hipStream_t s) {
  const int blocks = (p.N + 255) / 256;
  if (p.table && p.N <= CHAIN_MAX_N) {
    if (p.block >= 2) hipLaunchKernelGGL(markov_kernel, dim3(blocks), dim3(256), 0, s, p, 0);
    hipLaunchKernelGGL(markov_chain_kernel, dim3(1), dim3(CHAIN_THREADS), 0, s, p);  // (applies p.plant itself)
    return (int)hipGetLastError();
  }
  for (int j = 0; j < p.block - 1; ++j) hipLaunchKernelGGL(markov_kernel, dim3(blocks), dim3(256), 0, s, p, j);
  hipLaunchKernelGGL(markov_finalize, dim3(1), dim3(64), 0, s, p);
  if (p.plant) return plant_launch(p.st, p.plant, p.block, p.max_drafts, p.max_drafts_dev, s);
  return (int)hipGetLastError();
}
int markov_table_launch(const int8_t* w1q, const float* w1s, const float* c2, const int8_t* w2q, const int32_t* crop_ids,
                        int N, int rank, int vocab, float* T, float* c2c, float* s1c, hipStream_t s) {
  if (N < 16 || N % 16 || N > CHAIN_MAX_N || rank < 16 || rank % 16) return DSPARK_EINVAL;
  hipLaunchKernelGGL(markov_table_kernel, dim3((N + 63) / 64, (N + 63) / 64), dim3(256), 0, s, w1q, w1s, c2, w2q, crop_ids,
                     N, rank, vocab, T, c2c, s1c);
  return (int)hipGetLastError();
}
int round_begin_launch(dspark_state* st, uint64_t* keys, int nkeys, uint32_t* seen, int block, int max_pos, int vocab,
                       int out_cap, hipStream_t s) {
  hipLaunchKernelGGL(round_begin_kernel, dim3(1), dim3(256), 0, s, st, keys, nkeys, seen, block, max_pos, vocab, out_cap);
  return (int)hipGetLastError();
}
int plant_launch(dspark_state* st, const int32_t* plant, int block, int max_drafts, const int32_t* max_drafts_dev,
                 hipStream_t s) {
  hipLaunchKernelGGL(plant_kernel, dim3(1), dim3(64), 0, s, st, plant, block, max_drafts, max_drafts_dev);
  return (int)hipGetLastError();
}
int force_m_launch(dspark_state* st, int m, hipStream_t s) {
  hipLaunchKernelGGL(force_m_kernel, dim3(1), dim3(64), 0, s, st, m);
  return (int)hipGetLastError();
}

// Layer-boundary dump (debug rounds): dst[0][t][c] = h[t][c], dst[1][t][c] = the sum of the `bands` inputs v in band
// order (the value the next norm kernel adds; 0 without bands), for t < rows.
__global__ void layer_dump_kernel(float* dst, const float* h, const float* v, int bands, size_t band_stride, int rows,
                                  int H, size_t half) {
  const size_t n = (size_t)rows * H;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    dst[i] = h[i];
    float acc = 0.f;
    for (int b = 0; b < bands; ++b) acc += v[b * band_stride + i];
    dst[half + i] = acc;
  }
}

int layer_dump_launch(float* dst, const float* h, const float* v, int bands, int rows, int H, int block,
                      hipStream_t s) {
  const size_t n = (size_t)rows * H;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(layer_dump_kernel, dim3(blocks), dim3(256), 0, s, dst, h, v, v ? bands : 0, n, rows, H,
                     (size_t)block * H);
  return (int)hipGetLastError();
}

}  // namespace dspark
