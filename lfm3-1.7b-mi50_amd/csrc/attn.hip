// Verify attention for gfx950: one pass over each KV head's pages for all verified tokens and all query heads of the
// GQA group, on the matrix cores.
//
// Work split. A workgroup owns one (KV head, row group, key split); its four waves take the split's 32-key pages in
// turn, so every K/V byte travels from HBM into exactly one wave's registers and no LDS staging is needed. A wave
// holds all QB*16 query rows (token t, group member j -> row t*G + j) of its row group:
//   S^T[keys][rows] = K[keys][D] * Q^T[D][rows]           (A = K rows, 16-byte loads straight from a K page)
//   O^T[D][rows]   += V^T[D][keys] * P^T[keys][rows]      (A = V^T rows, 16-byte loads from a transposed V page)
//   l[rows]        += ones[16][keys] * P^T[keys][rows]    (the softmax row sum rides the matrix cores too)
// In the 16x16x32 layout a lane holds one query row (lane % 16) in both S^T and O^T, so the online-softmax state of
// a row is lane-local apart from the 4-lane max exchange when the running max moves. The running max moves lazily:
// only when a score exceeds it by more than TAU (P stays <= 2^TAU, exact in fp16), so the common tile costs one
// max3 tree, one compare and a ballot per 8 scores.
//
// The K rows of key block b of a page are permuted (row m <- key 8*(m/4) + 4*b + m%4) so that the P^T values a lane
// ends up with are keys 8*(lane/16)..+7 of the page -- exactly the contiguous 16 bytes its V^T load holds. K pages are
// stored in that operand order, so both K and V loads read whole contiguous kilobytes.
//
// Splits write unnormalised partials (acc, max, sum); attn_combine merges them in a fixed order (deterministic, no
// float atomics), applies the optional sigmoid gate and stores fp16/fp32. Reference: dspark.hip:1070-1412
// (attention_pass), 1488-2120 (attention_v2/v3), 2132-2185 (combine_phase); masks 975-978, 1308-1312, 2006-2012.
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

constexpr float TAU = 8.f;        // lazy-rescale slack in log2 units
constexpr float M_INIT = -1e30f;  // running max of a row that has not seen a key yet

template <int D>
struct Tile {
  half8 k[2][D / 32];  // key block b, k-step s
  half8 v[D / 16];     // d block c
};

// K pages are stored in matrix-core operand order: for key block b and k-step s, 64 lanes x 16 bytes, lane (n, g)
// holding K[key(n, b)][32 s + 8 g .. + 8] with key(n, b) = 8 (n / 4) + 4 b + n % 4. Every K load instruction then reads
// 1 KB of contiguous memory. V pages are stored transposed ([d][32 keys]): V load c reads rows 16 c .. 16 c + 15, also
// 1 KB contiguous. Page loads are non-temporal (the cache policy of a one-pass stream).
constexpr int NT = 2;  // buffer-load cache-policy bits: nt

template <int D>
__device__ __forceinline__ void load_tile(const AttnParams& p, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int h,
                                          int lpage, bool valid, Tile<D>& tl, uint32_t lane16, uint32_t voff) {
  // `valid` false (a page past the split) turns every load into an out-of-range buffer access: zeros, no memory
  // traffic, and no branch for the load counter to merge around.
  uint32_t base = 0x80000000u;  // beyond any pool (pools are < 2 GiB)
  if (valid) {
    const int phys = p.bt ? p.bt[lpage] : lpage;
    base = (uint32_t)(phys * p.KVH + h) * (uint32_t)(PAGE * D * 2);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      tl.k[b][s] = as_half8(__builtin_amdgcn_raw_buffer_load_b128(rk, base + lane16 + (uint32_t)((b * (D / 32) + s) * 1024), 0, NT));
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    tl.v[c] = as_half8(__builtin_amdgcn_raw_buffer_load_b128(rv, base + voff + (uint32_t)(c * 16 * PAGE * 2), 0, NT));
}

// Q operands: registers, or (QLDS, for many row blocks) an LDS copy in operand order [QB][D/32][64 lanes].
template <int D, int QB, bool QLDS>
struct QOps {
  half8 r[QLDS ? 1 : QB][D / 32];
  const half8* lds;
  __device__ __forceinline__ half8 get(int qb, int s, int lane) const {
    if constexpr (QLDS) return lds[(qb * (D / 32) + s) * 64 + lane];
    else return r[qb][s];
  }
};

// One page for every row block. Q operands carry log2(e)/sqrt(D), and the score MFMA starts from C = -m (the row's
// running max, log2 units), so its output is already s*log2(e)/sqrt(D) - m: the softmax costs one exp2 per score,
// a max3 tree, one compare against TAU and a ballot (no rescale in the common tile).
template <int D, int QB, bool QLDS>
__device__ __forceinline__ void tile_step(const AttnParams& p, const Tile<D>& tl, int lpage, const QOps<D, QB, QLDS>& qf,
                                          int row0, float (&mrun)[QB], f32x4 (&o)[QB][D / 16], f32x4 (&ls)[QB], int g,
                                          int lane) {
  const int base = lpage * PAGE;
  const bool edge = base < p.full_lo || base + PAGE - 1 > p.full_hi;
  const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    // A row that has not seen a key yet (mrun == M_INIT) starts from C = 0 and adopts its first page's maximum.
    const bool fresh = mrun[qb] == M_INIT;
    const float nm = fresh ? 0.f : -mrun[qb];
    f32x4 s0 = {nm, nm, nm, nm}, s1 = s0;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const half8 qs = qf.get(qb, s, lane);
      s0 = mfma16x16x32(tl.k[0][s], qs, s0);
      s1 = mfma16x16x32(tl.k[1][s], qs, s1);
    }
    if (edge) {
      // Visible keys of the lane's row (token t = row / G; padding rows act as the last token).
      const int t = min((row0 + 16 * qb + (lane & 15)) / p.G, p.M - 1);
      const int lo = max(p.start, p.window > 0 ? p.a + t - p.window + 1 : 0);
      const int hi = p.causal ? p.a + t : p.a + p.M - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k0 = base + 8 * g + i, k1 = k0 + 4;
        s0[i] = (k0 >= lo && k0 <= hi) ? s0[i] : -INFINITY;
        s1[i] = (k1 >= lo && k1 <= hi) ? s1[i] : -INFINITY;
      }
    }
    const float tmax = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])), fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
    if (__builtin_amdgcn_ballot_w64(fresh ? tmax > -INFINITY : tmax > TAU) != 0) {
      // Some row passed its running max by more than TAU (or saw its first key): move that row's max up to its page
      // maximum. fresh and rm are the same on the four lanes of a row.
      float rm = fmaxf(tmax, __shfl_xor(tmax, 16));
      rm = fmaxf(rm, __shfl_xor(rm, 32));
      if (fresh ? rm > -INFINITY : rm > TAU) {
        const float alpha = fresh ? 0.f : fast_exp2(-rm);
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] *= alpha;
        ls[qb] *= alpha;
        mrun[qb] = fresh ? rm : mrun[qb] + rm;
        s0 -= rm;
        s1 -= rm;
      }
    }
    half8 pp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pp[i] = (_Float16)fast_exp2(s0[i]);
      pp[4 + i] = (_Float16)fast_exp2(s1[i]);
    }
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] = mfma16x16x32(tl.v[cc], pp, o[qb][cc]);
    ls[qb] = mfma16x16x32(ones, pp, ls[qb]);
    // With many blocks, keep one block's scores live at a time (the scheduler would otherwise hoist every block's
    // score products ahead of the softmax and run out of registers).
    if constexpr (QLDS) __builtin_amdgcn_sched_barrier(0);
  }
}

// Page range, pages per split and unmasked range from a (the host plan evaluated with the State's a at run time).
__device__ void attn_range(AttnParams& p) {
  const int a = p.st->a;
  p.a = a;
  if (p.drafter) {
    // drafter ring: context [max(ctx_lo, a - window), a) for every block token, block keys in both directions
    p.start = max(p.st->ctx_lo, a - p.window);
    p.window = 0;
    p.causal = 0;
  } else if (p.window > 0) {
    p.start = max(0, a - p.window + 1);
  }
  const int lo0 = max(p.start, p.window > 0 ? a - p.window + 1 : 0);
  const int lo_last = max(p.start, p.window > 0 ? a + p.M - p.window : 0);
  const int hi_last = a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  p.pps = (p.npages + p.S - 1) / p.S;
}

template <int D, int QB, int PF, int OCC, bool QLDS>
__global__ __launch_bounds__(256, OCC) void verify_attn_kernel(AttnParams p) {
  if (p.st) {
    if (p.st->run == 0) return;
    attn_range(p);
  }
  constexpr int R = 16 * QB;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: page indices stay scalar
  const int n = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin (id % 8). Row groups of one (head, split) read the same pages, so
  // they take ids 8 apart inside a chunk of 8*RG: same XCD (shared L2), dispatched together.
  const int bid = blockIdx.x;
  const int chunk = bid / (8 * p.RG), within = bid % (8 * p.RG);
  const int rg = within / 8;
  const int unit = chunk * 8 + within % 8;
  if (unit >= p.KVH * p.S) return;
  const int h = unit / p.S, split = unit % p.S;

  QOps<D, QB, QLDS> qf;
  __shared__ half8 q_lds[QLDS ? QB * (D / 32) * 64 : 1];
  // Operand (qb, s) of lane (n, g): Q[t][qh][32 s + 8 g .. + 8] for row r = 16 qb + n of this row group.
  auto q_operand = [&](int qb, int s, int ln) -> half8 {
    const int r = rg * R + 16 * qb + (ln & 15);
    u32x4 u = {0, 0, 0, 0};
    if (r < p.G * p.M) {
      const int t = r / p.G, qh = h * p.G + r % p.G;
      u = ldg(reinterpret_cast<const u32x4*>(p.q + ((size_t)t * p.QH + qh) * D + 32 * s + 8 * (ln >> 4)));
    }
    half8 q = as_half8(u);
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = (_Float16)((float)q[j] * p.c);  // scores in log2 units
    return q;
  };
  if constexpr (QLDS) {
    for (int e = threadIdx.x; e < QB * (D / 32) * 64; e += 256) q_lds[e] = q_operand(e / ((D / 32) * 64), (e / 64) % (D / 32), e % 64);
    qf.lds = q_lds;
    __syncthreads();
  } else {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) qf.r[qb][s] = q_operand(qb, s, lane);
  }

  f32x4 o[QB][D / 16];
  f32x4 ls[QB];
  float mrun[QB];  // running max of the lane's row (log2 units); the score MFMA starts from -mrun
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] = f32x4{0, 0, 0, 0};
    ls[qb] = f32x4{0, 0, 0, 0};
    mrun[qb] = M_INIT;
  }

  // PF pages in flight per wave while one is computed: a ring of PF + 1 register tiles, unrolled so every index is
  // static. A wave's pages are pb + wave, pb + wave + 4, ...
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)p.kp, (short)0, (int)p.k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)p.vp, (short)0, (int)p.v_bytes, 0x00020000);
  const uint32_t koff = (uint32_t)lane * 16u, voff = (uint32_t)((n * PAGE + 8 * g) * 2);
  const int pb = p.page0 + split * p.pps;
  const int pe = min(pb + p.pps, p.page0 + p.npages);
  constexpr int NBUF = PF + 1;
  Tile<D> buf[NBUF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load_tile<D>(p, rk, rv, h, pb + wave + 4 * i, pb + wave + 4 * i < pe, buf[i], koff, voff);
  int pg = pb + wave;
  while (pg < pe) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      load_tile<D>(p, rk, rv, h, pg + 4 * PF, pg + 4 * PF < pe, buf[(j + PF) % NBUF], koff, voff);
      if (pg < pe) tile_step<D, QB, QLDS>(p, buf[j], pg, qf, rg * R, mrun, o, ls, g, lane);
      pg += 4;
    }
  }

  // Merge the four waves in a fixed order -- (w1 + w0) + (w3 + w2), each scaled to the common max -- through two LDS
  // row buffers, then write this split's partial.
  __shared__ float sm_m[4][R], sm_l[4][R];
  __shared__ f32x4 sm_o[2][R][D / 4 + 1];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
    if (g == 0) {
      sm_m[wave][16 * qb + n] = mrun[qb];
      sm_l[wave][16 * qb + n] = ls[qb][0];
    }
  __syncthreads();
  float fw[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = 16 * qb + n;
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    fw[qb] = fast_exp2(mrun[qb] - mx);
  }
  if (wave & 1) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) sm_o[wave >> 1][16 * qb + n][4 * cc + g] = o[qb][cc] * fw[qb];
  }
  __syncthreads();
  if (!(wave & 1)) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        f32x4& dst = sm_o[wave >> 1][16 * qb + n][4 * cc + g];
        dst = dst + o[qb][cc] * fw[qb];
      }
  }
  __syncthreads();
  const size_t slot = ((size_t)h * p.RG + rg) * p.S + split;
  f32x4* dst = reinterpret_cast<f32x4*>(p.part_acc + slot * R * D);
  for (int e = threadIdx.x; e < R * D / 4; e += 256) {
    const int r = e / (D / 4), c4 = e % (D / 4);
    dst[e] = sm_o[0][r][c4] + sm_o[1][r][c4];
  }
  for (int r = threadIdx.x; r < R; r += 256) {
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    const float L = (fast_exp2(sm_m[1][r] - mx) * sm_l[1][r] + fast_exp2(sm_m[0][r] - mx) * sm_l[0][r]) +
                    (fast_exp2(sm_m[3][r] - mx) * sm_l[3][r] + fast_exp2(sm_m[2][r] - mx) * sm_l[2][r]);
    p.part_ml[slot * R + r] = f32x2{L > 0.f ? mx : -INFINITY, L};
  }
}

// One wave per output row (KV head h, row r = t*G + j); lanes over D. Splits merge in index order.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
  if (p.st && p.st->run == 0) return;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rows = p.G * p.M;
  const int task = blockIdx.x * 4 + wave;
  if (task >= p.KVH * rows) return;
  const int h = task / rows, r = task % rows;
  const int R = p.R, rg = r / R, rr = r % R;
  const int t = r / p.G, qh = h * p.G + r % p.G;
  const size_t slot0 = ((size_t)h * p.RG + rg) * p.S;
  float ms = -INFINITY, lsv = 0.f;
  if (lane < p.S) {
    const f32x2 ml = p.part_ml[(slot0 + lane) * R + rr];
    ms = ml[0];
    lsv = ml[1];
  }
  const float mx = wave_max(ms);
  const float f = (ms == -INFINITY) ? 0.f : fast_exp2(ms - mx);
  const float L = wave_sum(f * lsv);
  constexpr int DL = D / 64;
  float acc[DL];
#pragma unroll
  for (int k = 0; k < DL; ++k) acc[k] = 0.f;
  const float* src = p.part_acc + (slot0 * R + rr) * D + lane;
  const size_t sstride = (size_t)R * D;
  float v[64][DL];
#pragma unroll
  for (int j = 0; j < 64; ++j)
#pragma unroll
    for (int k = 0; k < DL; ++k) v[j][k] = (j < p.S) ? ldg(src + j * sstride + 64 * k) : 0.f;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    const float fj = __shfl(f, j);
#pragma unroll
    for (int k = 0; k < DL; ++k) acc[k] = fmaf(fj, v[j][k], acc[k]);
  }
  float scale = L > 0.f ? 1.f / L : 0.f;
  if (p.gate) scale *= 1.f / (1.f + expf(-ldg(p.gate + (size_t)t * p.QH + qh)));
#pragma unroll
  for (int k = 0; k < DL; ++k) {
    const float val = acc[k] * scale;
    const size_t idx = ((size_t)t * p.QH + qh) * D + lane + 64 * k;
    if (p.out16) p.out16[idx] = (_Float16)val;
    if (p.out32) p.out32[idx] = val;
  }
}

// K/V rows of positions pos0..pos0+n-1 into the pages: one thread per (token, head, 8 dims).
__global__ __launch_bounds__(256) void kv_write_kernel(const _Float16* k, const _Float16* v, int64_t row_stride,
                                                       _Float16* kp, _Float16* vp, const int32_t* bt, int KVH, int D,
                                                       int pos0, int n) {
  const int d8n = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)n * KVH * d8n) return;
  const int tok = (int)(idx / (KVH * d8n));
  const int rem = (int)(idx % (KVH * d8n));
  const int h = rem / d8n, d8 = rem % d8n;
  const int pos = pos0 + tok, lp = pos / PAGE, slot = pos % PAGE;
  const int phys = bt ? bt[lp] : lp;
  const _Float16* ks = k + tok * row_stride + h * D + 8 * d8;
  const _Float16* vs = v + tok * row_stride + h * D + 8 * d8;
  // K in operand order: key `slot` is row n = 4 (slot / 8) + slot % 4 of key block b = (slot / 4) % 2; its 8 dims
  // 8 d8 .. belong to k-step s = d8 / 4 and lane n + 16 (d8 % 4).
  const int b = (slot >> 2) & 1, nrow = 4 * (slot >> 3) + (slot & 3), s = d8 >> 2, lanek = nrow + 16 * (d8 & 3);
  _Float16* kd = kp + ((size_t)phys * KVH + h) * (PAGE * D) + ((size_t)(b * (D / 32) + s) * 64 + lanek) * 8;
  *reinterpret_cast<u32x4*>(kd) = *reinterpret_cast<const u32x4*>(ks);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(vs);
  _Float16 hv[8];
  __builtin_memcpy(hv, &vv, 16);
  _Float16* vd = vp + (((size_t)phys * KVH + h) * D + 8 * d8) * PAGE + slot;
#pragma unroll
  for (int i = 0; i < 8; ++i) vd[i * PAGE] = hv[i];
}

// ---------------------------------------------------------------- host launchers
// Two launch shapes. OCC = 1: one 4-wave workgroup per CU, a wave may hold up to 512 VGPR + AGPR -- every query row of
// its KV head (up to 7 blocks of 16 rows at D = 64, 2 at D = 128) and a ring of PF pages in flight; no page is read
// twice, which long contexts need. OCC = 2: two workgroups per CU, 256 registers per wave, so at most 2 blocks per
// wave and row groups of one split share pages through the XCD's L2; twice the waves hide the launch's ramp and
// drain better, which short splits (few pages per wave) need.
#ifndef DSPARK_ATTN_PF
#define DSPARK_ATTN_PF 2
#endif
#ifndef DSPARK_ATTN_OCC2_MAX_PAGES
#define DSPARK_ATTN_OCC2_MAX_PAGES 12  // pages per wave (at one workgroup per CU) below which OCC = 2 is used
#endif
// The largest blocks per wave at OCC = 1. Up to 9 blocks fit with the Q operands in LDS (QLDS), but with one page in
// flight such a wave is latency-bound: two row groups of <= 6 blocks are faster on MI355X (measured at M = 33).
constexpr int QB_MAX_64 = 6, QB_MAX_128 = 2;
constexpr int QB_MAX_OCC2 = 2;

template <int D, int QB, int OCC>
static void launch_attn(const AttnParams& p, hipStream_t s) {
  constexpr bool QLDS = QB > 6;
  constexpr int PF = QLDS ? 1 : (OCC == 2 ? 2 : ((QB * D <= 4 * 64) ? DSPARK_ATTN_PF : 2));
  const int units = p.KVH * p.S;
  hipLaunchKernelGGL((verify_attn_kernel<D, QB, PF, OCC, QLDS>), dim3((units + 7) / 8 * 8 * p.RG), dim3(256), 0, s, p);
}

void attn_plan(AttnParams& p, int D, int cus) {
  const int rows = p.G * p.M;
  const int nblk = (rows + 15) / 16;
  const int lo0 = std::max(p.start, p.window > 0 ? p.a - p.window + 1 : 0);
  const int lo_last = std::max(p.start, p.window > 0 ? p.a + p.M - 1 - p.window + 1 : 0);
  const int hi_last = p.a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? p.a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  // Launch shape: one workgroup per CU unless the pages per wave are few and the rows fit OCC = 2.
  const int qb_max1 = D == 64 ? QB_MAX_64 : QB_MAX_128;
  const int rg1 = (nblk + qb_max1 - 1) / qb_max1;
  const double pages_per_wave = (double)p.npages * p.KVH * rg1 / (4.0 * cus);
  p.OCC = (D == 64 && pages_per_wave < DSPARK_ATTN_OCC2_MAX_PAGES) ? 2 : 1;
  const int qb_max = p.OCC == 2 ? QB_MAX_OCC2 : qb_max1;
  p.RG = (nblk + qb_max - 1) / qb_max;
  p.QB = (nblk + p.RG - 1) / p.RG;
  p.R = 16 * p.QB;
  int S = p.S;
  if (S <= 0) {
    const int groups = p.KVH * p.RG;
    const int target_wgs = cus * p.OCC;
    S = (target_wgs + groups - 1) / groups;
    S = std::min(S, (p.npages + 3) / 4);  // at least one page per wave
  }
  S = std::max(1, std::min(S, std::min(64, p.npages)));
  p.pps = (p.npages + S - 1) / S;
  p.S = (p.npages + p.pps - 1) / p.pps;
  p.c = (float)(1.4426950408889634 / std::sqrt((double)D));
}

size_t attn_workspace_bytes(const AttnParams& p, int D) {
  const size_t slots = (size_t)p.KVH * p.RG * p.S;
  return slots * p.R * D * sizeof(float) + slots * p.R * sizeof(f32x2) + 256;
}

int attn_launch(AttnParams& p, int D, int phases, hipStream_t s) {
  if (!(phases & 1)) {
  } else if (D == 64 && p.OCC == 2) {
    if (p.QB == 1) launch_attn<64, 1, 2>(p, s);
    else launch_attn<64, 2, 2>(p, s);
  } else if (D == 64) {
    switch (p.QB) {
      case 1: launch_attn<64, 1, 1>(p, s); break;
      case 2: launch_attn<64, 2, 1>(p, s); break;
      case 3: launch_attn<64, 3, 1>(p, s); break;
      case 4: launch_attn<64, 4, 1>(p, s); break;
      case 5: launch_attn<64, 5, 1>(p, s); break;
      default: launch_attn<64, 6, 1>(p, s); break;
    }
  } else {
    if (p.QB == 1) launch_attn<128, 1, 1>(p, s);
    else launch_attn<128, 2, 1>(p, s);
  }
  const int tasks = p.KVH * p.G * p.M;
  if (!(phases & 2)) {
  } else if (D == 64)
    hipLaunchKernelGGL(attn_combine_kernel<64>, dim3((tasks + 3) / 4), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_combine_kernel<128>, dim3((tasks + 3) / 4), dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

int kv_write_launch(const void* k, const void* v, int64_t row_stride, void* kp, void* vp, const int32_t* bt, int KVH,
                    int D, int pos0, int n, hipStream_t s) {
  const int64_t threads = (int64_t)n * KVH * (D / 8);
  if (threads == 0) return 0;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     (const _Float16*)k, (const _Float16*)v, row_stride, (_Float16*)kp, (_Float16*)vp, bt, KVH, D, pos0,
                     n);
  return (int)hipGetLastError();
}

}  // namespace dspark
