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
// The K rows loaded for key block b of a page are permuted (row m <- key 8*(m/4) + 4*b + m%4) so that the P^T values a
// lane ends up with are keys 8*(lane/16)..+7 of the page -- exactly the contiguous 16 bytes its V^T load holds.
//
// Splits write unnormalised partials (acc, max, sum); attn_combine merges them in a fixed order (deterministic, no
// float atomics), applies the optional sigmoid gate and stores fp16/fp32. Reference: dspark.hip:1070-1412
// (attention_pass), 1488-2120 (attention_v2/v3), 2132-2185 (combine_phase); masks 975-978, 1308-1312, 2006-2012.
#include "common.h"
#include "dspark_internal.h"

namespace dspark {

constexpr float TAU = 8.f;        // lazy-rescale slack in log2 units
constexpr float M_INIT = -1e30f;  // finite "no key yet": exp2(M_INIT - m) == 0 for any real m

template <int D>
struct Tile {
  half8 k[2][D / 32];  // key block b, k-step s
  half8 v[D / 16];     // d block c
};

template <int D>
__device__ __forceinline__ void load_tile(const AttnParams& p, int h, int lpage, Tile<D>& tl, int n, int g) {
  const int phys = p.bt ? ldg(p.bt + lpage) : lpage;
  const _Float16* kb = p.kp + ((size_t)phys * p.KVH + h) * (PAGE * D);
  const _Float16* vb = p.vp + ((size_t)phys * p.KVH + h) * (D * PAGE);
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int key = 8 * (n >> 2) + 4 * b + (n & 3);
#pragma unroll
    for (int s = 0; s < D / 32; ++s) tl.k[b][s] = as_half8(ldg(reinterpret_cast<const u32x4*>(kb + key * D + 32 * s + 8 * g)));
  }
#pragma unroll
  for (int c = 0; c < D / 16; ++c) tl.v[c] = as_half8(ldg(reinterpret_cast<const u32x4*>(vb + (16 * c + n) * PAGE + 8 * g)));
}

template <int D, int QB>
__device__ __forceinline__ void tile_step(const AttnParams& p, const Tile<D>& tl, int lpage, const half8 (&qf)[QB][D / 32],
                                          const int (&lo)[QB], const int (&hi)[QB], float (&mrun)[QB],
                                          f32x4 (&o)[QB][D / 16], f32x4 (&ls)[QB], int g) {
  const int base = lpage * PAGE;
  const bool edge = base < p.full_lo || base + PAGE - 1 > p.full_hi;
  const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
  const float c = p.c;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    f32x4 s0 = {0, 0, 0, 0}, s1 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      s0 = mfma16x16x32(tl.k[0][s], qf[qb][s], s0);
      s1 = mfma16x16x32(tl.k[1][s], qf[qb][s], s1);
    }
    if (edge) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k0 = base + 8 * g + i, k1 = k0 + 4;
        s0[i] = (k0 >= lo[qb] && k0 <= hi[qb]) ? s0[i] : -INFINITY;
        s1[i] = (k1 >= lo[qb] && k1 <= hi[qb]) ? s1[i] : -INFINITY;
      }
    }
    const float tmax = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])), fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
    if (__builtin_amdgcn_ballot_w64(tmax * c > mrun[qb] + TAU) != 0) {
      float rm = fmaxf(tmax, __shfl_xor(tmax, 16));
      rm = fmaxf(rm, __shfl_xor(rm, 32));
      const float cand = rm * c;
      if (cand > mrun[qb] + TAU) {
        const float alpha = fast_exp2(mrun[qb] - cand);
        mrun[qb] = cand;
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] *= alpha;
        ls[qb] *= alpha;
      }
    }
    const float m = mrun[qb];
    half8 pp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pp[i] = (_Float16)fast_exp2(fmaf(s0[i], c, -m));
      pp[4 + i] = (_Float16)fast_exp2(fmaf(s1[i], c, -m));
    }
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] = mfma16x16x32(tl.v[cc], pp, o[qb][cc]);
    ls[qb] = mfma16x16x32(ones, pp, ls[qb]);
  }
}

template <int D, int QB>
__global__ __launch_bounds__(256, 2) void verify_attn_kernel(AttnParams p) {
  constexpr int R = 16 * QB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin (id % 8). Row groups of one (head, split) read the same pages, so
  // they take ids 8 apart inside a chunk of 8*RG: same XCD (shared L2), dispatched together.
  const int bid = blockIdx.x;
  const int chunk = bid / (8 * p.RG), within = bid % (8 * p.RG);
  const int rg = within / 8;
  const int unit = chunk * 8 + within % 8;
  if (unit >= p.KVH * p.S) return;
  const int h = unit / p.S, split = unit % p.S;

  half8 qf[QB][D / 32];
  int lo[QB], hi[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = rg * R + 16 * qb + n;
    const bool real = r < p.G * p.M;
    const int t = real ? r / p.G : p.M - 1;
    const int qh = h * p.G + (real ? r % p.G : 0);
    lo[qb] = max(p.start, p.window > 0 ? p.a + t - p.window + 1 : 0);
    hi[qb] = p.causal ? p.a + t : p.a + p.M - 1;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      u32x4 u = {0, 0, 0, 0};
      if (real) u = ldg(reinterpret_cast<const u32x4*>(p.q + ((size_t)t * p.QH + qh) * D + 32 * s + 8 * g));
      qf[qb][s] = as_half8(u);
    }
  }

  f32x4 o[QB][D / 16];
  f32x4 ls[QB];
  float mrun[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) o[qb][cc] = f32x4{0, 0, 0, 0};
    ls[qb] = f32x4{0, 0, 0, 0};
    mrun[qb] = M_INIT;
  }

  const int pb = p.page0 + split * p.pps;
  const int pe = min(pb + p.pps, p.page0 + p.npages);
  int pg = pb + wave;
  Tile<D> ta, tb;
  if (pg < pe) load_tile<D>(p, h, pg, ta, n, g);
  while (pg < pe) {
    if (pg + 4 < pe) load_tile<D>(p, h, pg + 4, tb, n, g);
    tile_step<D, QB>(p, ta, pg, qf, lo, hi, mrun, o, ls, g);
    pg += 4;
    if (pg >= pe) break;
    if (pg + 4 < pe) load_tile<D>(p, h, pg + 4, ta, n, g);
    tile_step<D, QB>(p, tb, pg, qf, lo, hi, mrun, o, ls, g);
    pg += 4;
  }

  // Merge the four waves (fixed order), then write this split's partial.
  __shared__ float sm_m[4][R], sm_l[4][R];
  __shared__ f32x4 sm_o[4][R][D / 4 + 1];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
    if (g == 0) {
      sm_m[wave][16 * qb + n] = mrun[qb];
      sm_l[wave][16 * qb + n] = ls[qb][0];
    }
  __syncthreads();
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = 16 * qb + n;
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    const float f = fast_exp2(mrun[qb] - mx);
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) sm_o[wave][r][4 * cc + g] = o[qb][cc] * f;
  }
  __syncthreads();
  const size_t slot = ((size_t)h * p.RG + rg) * p.S + split;
  f32x4* dst = reinterpret_cast<f32x4*>(p.part_acc + slot * R * D);
  for (int e = threadIdx.x; e < R * D / 4; e += 256) {
    const int r = e / (D / 4), c4 = e % (D / 4);
    dst[e] = ((sm_o[0][r][c4] + sm_o[1][r][c4]) + sm_o[2][r][c4]) + sm_o[3][r][c4];
  }
  for (int r = threadIdx.x; r < R; r += 256) {
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) L += fast_exp2(sm_m[w][r] - mx) * sm_l[w][r];
    p.part_ml[slot * R + r] = f32x2{L > 0.f ? mx : -INFINITY, L};
  }
}

// One wave per output row (KV head h, row r = t*G + j); lanes over D. Splits merge in index order.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  for (int s0 = 0; s0 < p.S; s0 += 8) {
    float v[8][DL];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < DL; ++k) v[j][k] = (s0 + j < p.S) ? ldg(src + (s0 + j) * sstride + 64 * k) : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float fj = __shfl(f, s0 + j);
#pragma unroll
      for (int k = 0; k < DL; ++k) acc[k] = fmaf(fj, v[j][k], acc[k]);
    }
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
  *reinterpret_cast<u32x4*>(kp + (((size_t)phys * KVH + h) * PAGE + slot) * D + 8 * d8) = *reinterpret_cast<const u32x4*>(ks);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(vs);
  _Float16 hv[8];
  __builtin_memcpy(hv, &vv, 16);
  _Float16* vd = vp + (((size_t)phys * KVH + h) * D + 8 * d8) * PAGE + slot;
#pragma unroll
  for (int i = 0; i < 8; ++i) vd[i * PAGE] = hv[i];
}

// ---------------------------------------------------------------- host launchers
template <int D, int QB>
static void launch_attn(const AttnParams& p, hipStream_t s) {
  const int units = p.KVH * p.S;
  hipLaunchKernelGGL((verify_attn_kernel<D, QB>), dim3((units + 7) / 8 * 8 * p.RG), dim3(256), 0, s, p);
}

void attn_plan(AttnParams& p, int D, int target_wgs) {
  const int rows = p.G * p.M;
  const int nblk = (rows + 15) / 16;
  const int qb_max = D == 64 ? 3 : 1;
  p.RG = (nblk + qb_max - 1) / qb_max;
  p.QB = (nblk + p.RG - 1) / p.RG;
  p.R = 16 * p.QB;
  const int lo0 = std::max(p.start, p.window > 0 ? p.a - p.window + 1 : 0);
  const int lo_last = std::max(p.start, p.window > 0 ? p.a + p.M - 1 - p.window + 1 : 0);
  const int hi_last = p.a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? p.a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  int S = p.S;
  if (S <= 0) {
    const int groups = p.KVH * p.RG;
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

int attn_launch(AttnParams& p, int D, hipStream_t s) {
  if (D == 64) {
    switch (p.QB) {
      case 1: launch_attn<64, 1>(p, s); break;
      case 2: launch_attn<64, 2>(p, s); break;
      default: launch_attn<64, 3>(p, s); break;
    }
  } else {
    launch_attn<128, 1>(p, s);
  }
  const int tasks = p.KVH * p.G * p.M;
  if (D == 64)
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
