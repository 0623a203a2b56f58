// Verify attention for gfx950: each KV head's pages are read once for all verified tokens and all query heads of the
// GQA group, on the matrix cores.
//
// Tile math (both kernels). In the 16x16x32 MFMA layout a lane holds one query row (lane % 16):
//   S^T[keys][rows] = K[keys][D] * Q^T[D][rows]           (A = K rows from a page, B = Q)
//   O^T[D][rows]   += V^T[D][keys] * P^T[keys][rows]      (A = V^T rows from a transposed page)
//   l[rows]        += ones[16][keys] * P^T[keys][rows]    (the softmax row sum rides the matrix cores too)
// so the online-softmax state of a row is lane-local apart from the 4-lane max exchange when the running max moves.
// The running max moves lazily: only when a score exceeds it by more than TAU (P stays <= 2^TAU, exact in fp16).
// The K rows of key block b of a page are permuted (row m <- key 8*(m/4) + 4*b + m%4) so that the P^T values a lane
// ends up with are keys 8*(lane/16)..+7 of the page -- exactly the 16 bytes its V^T operand holds. K pages are stored
// in that operand order, so K and V reads are whole contiguous kilobytes.
//
// Work split. verify_attn_lds_kernel: a workgroup per (KV head, key split) holds every query row of the head, one
// wave per 16-row block and page lane, and streams the split's pages through an LDS ring (each page read from HBM
// once). verify_attn_kernel (shapes the LDS kernel does not cover): a workgroup per (KV head, row group, key split),
// its four waves take pages in turn into registers.
//
// Splits write unnormalised partials (acc, max, sum); attn_combine_kernel merges them in a fixed order
// (deterministic, no float atomics), applies the optional sigmoid gate and stores fp16/fp32. Reference:
// dspark.hip:1070-1412 (attention_pass), 1488-2120 (attention_v2/v3), 2132-2185 (combine_phase); masks 975-978,
// 1308-1312, 2006-2012.
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"
#include "attn_range.h"

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
// 1 KB contiguous. Page loads use the default cache policy: when row groups of one split read the same pages (their
// workgroups sit on one XCD), the second reader hits L2. (Non-temporal loads measured 14.2 us against 11.0 us for a
// 64 MiB two-reader page stream on MI355X: the second reader missed L2.)
#ifndef DSPARK_ATTN_CPOL
#define DSPARK_ATTN_CPOL 0
#endif
constexpr int CPOL = DSPARK_ATTN_CPOL;  // buffer-load cache-policy bits

template <int D>
__device__ __forceinline__ void load_tile(const AttnParams& p, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int h,
                                          int lpage, bool valid, Tile<D>& tl, uint32_t lane16, uint32_t voff) {
  // `valid` false (a page past the split) turns every load into an out-of-range buffer access: zeros, no memory
  // traffic, and no branch for the load counter to merge around.
  uint32_t base = 0x80000000u;  // beyond any pool (pools are < 2 GiB)
  if (valid) {
    // The page is wave-uniform: a scalar load of the table entry waits on lgkmcnt only. (A vector load here makes
    // the compiler wait for vmcnt(0) -- every page still in flight -- before the next page's loads are issued.)
    const int lp = __builtin_amdgcn_readfirstlane(lpage);
    const int phys = p.bt ? p.bt[lp] : lp;
    base = (uint32_t)(phys * p.KVH + h) * (uint32_t)(PAGE * D * 2);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      tl.k[b][s] = as_half8(__builtin_amdgcn_raw_buffer_load_b128(rk, base + lane16 + (uint32_t)((b * (D / 32) + s) * 1024), 0, CPOL));
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    tl.v[c] = as_half8(__builtin_amdgcn_raw_buffer_load_b128(rv, base + voff + (uint32_t)(c * 16 * PAGE * 2), 0, CPOL));
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

// Online-softmax state of the rows a wave holds (in the 16x16 MFMA layout a lane owns one row of each 16-row block).
// Q operands carry log2(e)/sqrt(D) and the score MFMA starts from C = c = -m (the row's running max, log2 units), so
// its output is already s*log2(e)/sqrt(D) - m: a page costs one exp2 per score, a max3 tree, one compare against TAU
// and a ballot. The running max moves lazily, only when a score passes it by more than TAU (P stays <= 2^TAU, exact
// in fp16), so the common page has no rescale.
template <int D, int QB>
struct RowState {
  f32x4 o[QB][D / 16];  // O^T accumulators
  f32x4 ls[QB];         // row sums (the same value in the 4 lanes of a row)
  float m[QB];          // running max; M_INIT before the row's first visible key
  f32x4 c[QB];          // score accumulator start: -m (0 while m is M_INIT)
};

// Scores of one page for every row block: s[qb][b] = K_b Q^T + c.
template <int D, int QB, bool QLDS>
__device__ __forceinline__ void page_scores(const Tile<D>& tl, const QOps<D, QB, QLDS>& qf, const f32x4 (&c)[QB],
                                            f32x4 (&s)[QB][2], int lane) {
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    f32x4 s0 = c[qb], s1 = c[qb];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      const half8 qs = qf.get(qb, ks, lane);
      s0 = mfma16x16x32(tl.k[0][ks], qs, s0);
      s1 = mfma16x16x32(tl.k[1][ks], qs, s1);
    }
    s[qb][0] = s0;
    s[qb][1] = s1;
  }
}

// Masks (pages at the edges of the visible range only) and the lazy running-max update of one page.
template <int D, int QB>
__device__ __forceinline__ void page_prep(const AttnParams& p, int lpage, int row0, RowState<D, QB>& rs,
                                          f32x4 (&s)[QB][2], int g, int lane) {
  const int base = lpage * PAGE;
  if (base < p.full_lo || base + PAGE - 1 > p.full_hi) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      // Visible keys of the lane's row (token t = row / G; padding rows act as the last token): start and the window
      // bound the context keys only (dspark.hip:1308-1312, 2006-2012), the block's own keys are visible up to t.
      const int t = min((row0 + 16 * qb + (lane & 15)) / p.G, p.M - 1);
      const int lo = min(p.a, max(p.start, p.window > 0 ? p.a + t - p.window + 1 : 0));
      const int hi = p.causal ? p.a + t : p.a + p.M - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k0 = base + 8 * g + i, k1 = k0 + 4;
        s[qb][0][i] = (k0 >= lo && k0 <= hi) ? s[qb][0][i] : -INFINITY;
        s[qb][1][i] = (k1 >= lo && k1 <= hi) ? s[qb][1][i] : -INFINITY;
      }
    }
  }
  float tmax[QB];
  bool need = false;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const f32x4 a = s[qb][0], b = s[qb][1];
    tmax[qb] = fmaxf(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])), fmaxf(fmaxf(b[0], b[1]), fmaxf(b[2], b[3])));
    // bitwise, not ||: a short-circuit here compiles to exec-mask branches on every page
    const float thr = rs.m[qb] == M_INIT ? -INFINITY : TAU;
    need = need | (tmax[qb] > thr);
  }
  if (__builtin_amdgcn_ballot_w64(need) != 0) {
    // Some row passed its running max by more than TAU (or saw its first key): move that row's max up to its page
    // maximum. m and the row maximum are the same on the four lanes of a row.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const bool fresh = rs.m[qb] == M_INIT;
      float rm = fmaxf(tmax[qb], __shfl_xor(tmax[qb], 16));
      rm = fmaxf(rm, __shfl_xor(rm, 32));
      if (fresh ? rm > -INFINITY : rm > TAU) {
        const float alpha = fresh ? 0.f : fast_exp2(-rm);
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) rs.o[qb][cc] *= alpha;
        rs.ls[qb] *= alpha;
        rs.m[qb] = fresh ? rm : rs.m[qb] + rm;
        rs.c[qb] = f32x4{-rs.m[qb], -rs.m[qb], -rs.m[qb], -rs.m[qb]};
        s[qb][0] -= rm;
        s[qb][1] -= rm;
      }
    }
  }
}

// P = exp2(scores) in fp16, then O^T += V^T P^T and the row sums ride the matrix cores too (ones x P^T).
template <int D, int QB>
__device__ __forceinline__ void page_accumulate(const Tile<D>& tl, RowState<D, QB>& rs, const f32x4 (&s)[QB][2]) {
  const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    half8 pp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pp[i] = (_Float16)fast_exp2(s[qb][0][i]);
      pp[4 + i] = (_Float16)fast_exp2(s[qb][1][i]);
    }
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) rs.o[qb][cc] = mfma16x16x32(tl.v[cc], pp, rs.o[qb][cc]);
    rs.ls[qb] = mfma16x16x32(ones, pp, rs.ls[qb]);
  }
}

template <int D, int QB, int PF, int OCC, bool QLDS>
__global__ __launch_bounds__(256, OCC) void verify_attn_kernel(AttnParams p) {
  if (p.st && !attn_state_range(p)) return;
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

  RowState<D, QB> rs;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) rs.o[qb][cc] = f32x4{0, 0, 0, 0};
    rs.ls[qb] = f32x4{0, 0, 0, 0};
    rs.m[qb] = M_INIT;
    rs.c[qb] = f32x4{0, 0, 0, 0};
  }

  // A wave's pages are pb + wave, pb + wave + 4, ...; a ring of PF + 1 register tiles keeps the next PF pages in
  // flight, unrolled so every index is static. Software pipeline: in the iteration of page j the score products of
  // page j + 1 are issued next to the exp2 / PV work of page j (independent, so the matrix cores and the VALU
  // overlap); the rare running-max update of page j comes first, so page j + 1's scores already use the new max.
  // Pages past the split load as zeros (out-of-range buffer loads) and their scores are never used.
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)p.kp, (short)0, (int)p.k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)p.vp, (short)0, (int)p.v_bytes, 0x00020000);
  const uint32_t koff = (uint32_t)lane * 16u, voff = (uint32_t)((n * PAGE + 8 * g) * 2);
  const int pb = p.page0 + split * p.pps;
  const int pe = min(pb + p.pps, p.page0 + p.npages);
  constexpr int NBUF = PF + 1;
  Tile<D> buf[NBUF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load_tile<D>(p, rk, rv, h, pb + wave + 4 * i, pb + wave + 4 * i < pe, buf[i], koff, voff);
  f32x4 sc[QB][2];
  page_scores<D, QB, QLDS>(buf[0], qf, rs.c, sc, lane);
  int pg = pb + wave;
  while (pg < pe) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      load_tile<D>(p, rk, rv, h, pg + 4 * PF, pg + 4 * PF < pe, buf[(j + PF) % NBUF], koff, voff);
      if (pg < pe) {
        page_prep<D, QB>(p, pg, rg * R, rs, sc, g, lane);
        f32x4 sn[QB][2];
        page_scores<D, QB, QLDS>(buf[(j + 1) % NBUF], qf, rs.c, sn, lane);
        page_accumulate<D, QB>(buf[j], rs, sc);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          sc[qb][0] = sn[qb][0];
          sc[qb][1] = sn[qb][1];
        }
      }
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
      sm_m[wave][16 * qb + n] = rs.m[qb];
      sm_l[wave][16 * qb + n] = rs.ls[qb][0];
    }
  __syncthreads();
  float fw[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = 16 * qb + n;
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    fw[qb] = fast_exp2(rs.m[qb] - mx);
  }
  if (wave & 1) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) sm_o[wave >> 1][16 * qb + n][4 * cc + g] = rs.o[qb][cc] * fw[qb];
  }
  __syncthreads();
  if (!(wave & 1)) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        f32x4& dst = sm_o[wave >> 1][16 * qb + n][4 * cc + g];
        dst = dst + rs.o[qb][cc] * fw[qb];
      }
  }
  __syncthreads();
  // row-major partials: row r of this split at ((hr R + r) S + split)
  const size_t row0 = ((size_t)h * p.RG + rg) * R * p.S + split;
  f32x4* dst = reinterpret_cast<f32x4*>(p.part_acc) + row0 * (D / 4);
  for (int e = threadIdx.x; e < R * D / 4; e += 256) {
    const int r = e / (D / 4), c4 = e % (D / 4);
    dst[(size_t)r * p.S * (D / 4) + c4] = sm_o[0][r][c4] + sm_o[1][r][c4];
  }
  for (int r = threadIdx.x; r < R; r += 256) {
    const float mx = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
    const float L = (fast_exp2(sm_m[1][r] - mx) * sm_l[1][r] + fast_exp2(sm_m[0][r] - mx) * sm_l[0][r]) +
                    (fast_exp2(sm_m[3][r] - mx) * sm_l[3][r] + fast_exp2(sm_m[2][r] - mx) * sm_l[2][r]);
    p.part_ml[row0 + (size_t)r * p.S] = f32x2{L > 0.f ? mx : -INFINITY, L};
  }
}

// ---------------------------------------------------------------- LDS-staged verify attention
// A workgroup owns one (KV head, key split) and every query row of the head: NW = NRB x PL waves, wave w holds row
// block rb = w % NRB (16 rows: token t, group member j -> row t*G + j) for page lane pl = w / NRB. A step of the split
// is PPS = PL x PPL pages (32 KB of K+V whatever the lane count); step k covers pages pb + k*PPS + j*PL + pl
// (j < PPL) for page lane pl. The workgroup brings a step's pages from HBM into one slot of a RING-slot LDS ring with
// direct-to-LDS buffer loads -- every page byte crosses HBM once -- and each wave reads its page lane's PPL pages from
// LDS for its rows. RING - 1 steps (64 KB per CU) are in flight while one is computed:
//   step k:  s_waitcnt (this wave's loads of step k done) ; s_barrier (everyone's) ; issue step k + RING - 1 into the
//            slot of step k - 1 (free: every wave finished step k - 1 before the barrier) ; compute step k.
// The ring slots are separate LDS arrays selected by static index (the loop is unrolled by RING), which lets the
// compiler see that reads of slot k never alias the loads in flight into the other slots, so it keeps the counted
// wait above instead of draining every load before each read. (3 slots measured 16.2 against 16.5 us for 4 slots per
// C2 layer on MI355X.)
// LDS page layout: 1 KB chunks in lane order -- K chunk (b, s) holds lane l's 16-byte operand at l*16 (the global
// layout), V^T chunk c holds lane (n, g)'s keys 8g..8g+7 of row 16c + n at (n + 16g)*16 (permuted by the loads'
// source offsets), so every ds_read_b128 of the compute is a conflict-free lane-order read.
// At the end the PL page lanes of each row block merge in order pl = 0, 1, ... through LDS and page lane 0 writes the
// workgroup's partial (all rows of the head).
#ifndef DSPARK_ATTN_RING
#define DSPARK_ATTN_RING 3
#endif
constexpr int RING = DSPARK_ATTN_RING;  // LDS ring slots (3 or 4): RING - 1 steps in flight
static_assert(RING == 3 || RING == 4, "ring of 3 or 4 slots");
// Each page has exactly one reader here, so its loads are non-temporal (15.4 against 16.4 us per C2 layer measured).
#ifndef DSPARK_ATTN_LDS_CPOL
#define DSPARK_ATTN_LDS_CPOL 2
#endif
constexpr int LDS_CPOL = DSPARK_ATTN_LDS_CPOL;
constexpr int LDS_BT_MAX = 2048;  // pages per split the LDS kernel accepts
constexpr int LDS_STEP_BYTES = 32768;  // K+V bytes of one ring step (4 pages at D = 64, 2 at D = 128)
constexpr int ATTN_CPOL_COHERENT = 16;  // buffer-store cache policy SC1: device-scope coherent


#define DSPARK_LDSP(x) ((__attribute__((address_space(3))) void*)(x))

// QB row blocks per wave: wave w is row group rg = w % NRG (row blocks rg QB .. rg QB + QB - 1, past NRB padding) of
// page lane pl = w / NRG. With QB > 1 fewer waves share each page (LDS reads per step fall by QB) and the waves can be
// a multiple of four (one share per SIMD: 9 row blocks as 3 groups of 3 x 4 page lanes = 12 waves, where 9 waves of
// one block each left one SIMD a third more work than the others).
// FR: the instantiation that takes a fresh block from the mix rows (p.mix; D = 64, QB = 1); the others are free of
// that code, so the plain kernel's registers and load order stay its own.
template <int D, int QB, int PL, int PPL, int LPW, int MAXW, bool FR = false>
__global__ __launch_bounds__(MAXW * 64) void verify_attn_lds_kernel(AttnParams p) {
  constexpr int PAGEB = 4 * PAGE * D;  // K + V bytes of one (page, KV head)
  constexpr int CPG = PAGEB / 1024;    // 1 KB chunks per page: K chunks first, then V^T chunks
  constexpr int PPS = PL * PPL;        // pages per step
  __shared__ __attribute__((aligned(16))) char ring0[PPS * PAGEB], ring1[PPS * PAGEB], ring2[PPS * PAGEB];
  __shared__ __attribute__((aligned(16))) char ring3[RING > 3 ? PPS * PAGEB : 16];
  __shared__ __attribute__((aligned(16))) char trash[1024];  // destination of the padding loads
  __shared__ int32_t sm_bt[LDS_BT_MAX];                       // the split's block-table entries
  // Q operands of up to MAXW / PL row groups: staged in the last ring slot (not written before step 0, and every wave
  // has read its Q before step 0's barrier) when they fit it.
  constexpr int QBYTES = (MAXW / PL) * QB * (D / 32) * 1024;
  constexpr bool QRING = QBYTES <= PPS * PAGEB;
  __shared__ __attribute__((aligned(16))) char q_own[QRING ? 16 : QBYTES];
  char* const q_lds = QRING ? (RING > 3 ? ring3 : ring2) : q_own;
  // The kernel arguments' last line (the fresh block's rope and eps) with the others in the first round trip: loaded
  // later, with the arguments the block-table loads need, its miss would delay them.
  if constexpr (FR) asm volatile("" ::"s"(p.rope));
  if (p.st && !attn_state_range(p)) return;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int NRB = p.nrb, NRG = p.nrg, NW = NRG * PL;
  const int rg = wave % NRG, pl = wave / NRG;
  const int h = blockIdx.x / p.S, split = blockIdx.x % p.S;
  const int R = NRB * 16;

  QOps<D, QB, false> qf;
  RowState<D, QB> rs;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) rs.o[qb][cc] = f32x4{0, 0, 0, 0};
    rs.ls[qb] = f32x4{0, 0, 0, 0};
    rs.m[qb] = M_INIT;
    rs.c[qb] = f32x4{0, 0, 0, 0};
  }

  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)p.kp, (short)0, (int)p.k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)p.vp, (short)0, (int)p.v_bytes, 0x00020000);
  // split bounds are workgroup-uniform: keep them scalar so every step condition is a scalar branch
  const int pb = __builtin_amdgcn_readfirstlane(p.page0 + split * p.pps);
  const int pe = __builtin_amdgcn_readfirstlane(min(pb + p.pps, p.page0 + p.npages));
  const int nsteps = pe > pb ? (pe - pb + PPS - 1) / PPS : 0;
  p.full_lo = __builtin_amdgcn_readfirstlane(p.full_lo);
  p.full_hi = __builtin_amdgcn_readfirstlane(p.full_hi);
  const uint32_t koff = (uint32_t)lane * 16u, voff = (uint32_t)(n * 64 + g * 16);
  // Block-table entries of the split into LDS before any page load: a table read inside the step loop would be a
  // vector load (the direct-to-LDS loads count as possible clobbers), and its wait would drain the pages in flight.
  const bool paged = p.bt != nullptr;
  if (paged) {
    for (int i = threadIdx.x; i < pe - pb; i += NW * 64) sm_bt[i] = ldg(p.bt + pb + i);
    __syncthreads();
  }

  // Fresh block (p.mix): wave w's fresh row is token w's K/V, at position a + w (the host sends M <= waves).
  constexpr int NE = D / 32;  // a fresh K/V row's dims per lane: lanes 0..31 hold dims l + 32 e, 32..63 repeat them
  constexpr bool FRESH_OK = FR && QB == 1 && D == 64;  // (the host sends a fresh block to these shapes only)
  const bool fresh = FRESH_OK && p.mix != nullptr;
  const int fpos = p.a + wave;
  const int fpage = fpos / PAGE;
  const bool fmine = fresh && wave < p.M && fpage >= pb && fpage < pe;  // wave-uniform
  _Float16 fkh[NE], fvh[NE];  // the fresh K / V row's halves of this lane (dims l + 32 e)

  // Step `k`'s chunks into `slot`: chunk c of [0, PPS*CPG) goes to wave c % NW; every wave issues exactly LPW loads
  // (chunks past the step, or of pages past the split, become out-of-range loads into `trash`), so the counted waits
  // are compile-time constants.
  auto issue = [&](int k, char* slot) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int c = wave + i * NW;
      const int pp = c / CPG, cc = c % CPG;
      const int page = pb + k * PPS + pp;
      const bool isv = cc >= CPG / 2;
      char* dst = trash;
      uint32_t off = 0x80000000u;
      if (c < PPS * CPG && page < pe) {
        const int phys = paged ? __builtin_amdgcn_readfirstlane(sm_bt[page - pb]) : page;
        const uint32_t base = (uint32_t)(phys * p.KVH + h) * (uint32_t)(PAGEB / 2);
        off = isv ? base + (uint32_t)(cc - CPG / 2) * 1024u + voff : base + (uint32_t)cc * 1024u + koff;
        dst = slot + pp * PAGEB + cc * 1024;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isv ? rv : rk, DSPARK_LDSP(dst), 16, off, 0, 0, LDS_CPOL);
    }
  };
  auto step = [&](int k, const char* cur, char* nxt) {
    // steps issued after step k that may still be in flight
    const int ahead = min(RING - 2, nsteps - 1 - k);
    if (RING > 3 && ahead >= 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LPW));
    else if (ahead >= 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPW));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    if (k + RING - 1 < nsteps) issue(k + RING - 1, nxt);
    // fresh positions in this step's pages: their K / V rows into the LDS copy (stale in the pool), then a barrier
    if (fresh && p.a + p.M - 1 >= (pb + k * PPS) * PAGE && p.a < min(pe, pb + (k + 1) * PPS) * PAGE) {
      if (fmine && (fpage - pb) / PPS == k && lane < 32) {
        char* pg = const_cast<char*>(cur) + ((fpage - pb) % PPS) * PAGEB;
        const int slot = fpos % PAGE;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          const int d = lane + 32 * e;
          *reinterpret_cast<_Float16*>(pg + 2 * k_page_elem(slot, d, D)) = fkh[e];
          *reinterpret_cast<_Float16*>(pg + (CPG / 2 + d / 16) * 1024 + (16 * (slot / 8) + d % 16) * 16 + 2 * (slot % 8)) =
              fvh[e];
        }
      }
      __builtin_amdgcn_s_waitcnt(LGKMCNT0_IMM);
      __builtin_amdgcn_s_barrier();
    }
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int pp = j * PL + pl;
      const int page = pb + k * PPS + pp;
      if (page < pe) {
        const char* src = cur + pp * PAGEB;
        Tile<D> tl;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          tl.k[c / (D / 32)][c % (D / 32)] = *reinterpret_cast<const half8*>(src + c * 1024 + lane * 16);
          tl.v[c] = *reinterpret_cast<const half8*>(src + (D / 16 + c) * 1024 + lane * 16);
        }
        f32x4 sc[QB][2];
        page_scores<D, QB, false>(tl, qf, rs.c, sc, lane);
        page_prep<D, QB>(p, page, rg * QB * 16, rs, sc, g, lane);
        page_accumulate<D, QB>(tl, rs, sc);
      }
    }
  };
  // The table (when staged) is in LDS before any other load is issued. Q of each row block goes to LDS with the
  // same direct loads (the page-lane-0 wave of the block, before its first page loads: the oldest in its load
  // counter), so the wait for Q below leaves the first steps' pages in flight. Padding rows past G*M read the last
  // row (the merge never stores them).
  if (paged) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  // Fresh block: this wave's rows of Q and its fresh K/V row (token `wave`, when its position falls in this split)
  // loaded from the mix rows first, so they are the oldest loads in the counter and the first step's wait covers them.
  f32x4 fq[QB][D / 32][2];
  half8 fqw[D / 32], fqc[D / 64], fqs[D / 64];
  // (kept in their loaded types until the first barrier: a conversion next to its load would make the compiler wait
  // for these loads, and every older one, before the pages are issued)
  float fk[NE], fv[NE];
  _Float16 fkw[NE], fkc[NE / 2], fks[NE / 2];
  if (fresh) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int r = min((rg * QB + qb) * 16 + n, p.G * p.M - 1);
      const float* qr = p.mix + (size_t)(r / p.G) * p.mix_row + (size_t)(h * p.G + r % p.G) * D + 8 * g;
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        fq[qb][s][0] = ldg(reinterpret_cast<const f32x4*>(qr + 32 * s));
        fq[qb][s][1] = ldg(reinterpret_cast<const f32x4*>(qr + 32 * s + 4));
      }
    }
#pragma unroll
    for (int s = 0; s < D / 32; ++s) fqw[s] = ldg(reinterpret_cast<const half8*>(p.q_norm + 32 * s + 8 * g));
    if (fmine) {
      const float* row = p.mix + (size_t)wave * p.mix_row;
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int d = (lane & 31) + 32 * e;
        fk[e] = row[(size_t)(p.QH + h) * D + d];
        fv[e] = row[(size_t)(p.QH + p.KVH + h) * D + d];
        fkw[e] = p.k_norm[d];
      }
#pragma unroll
      for (int e = 0; e < NE / 2; ++e) {
        const int i = (lane & 31) + 32 * e;
        fkc[e] = p.rope[(size_t)fpos * D + i];
        fks[e] = p.rope[(size_t)fpos * D + D / 2 + i];
      }
    }
  }
  if (fresh) {
    // (the RoPE rows of the wave's tokens: a second round of loads, the token known only per row)
#pragma unroll
    for (int s = 0; s < D / 64; ++s) {
      const int r = min(rg * QB * 16 + n, p.G * p.M - 1);
      const _Float16* rt = p.rope + (size_t)(p.a + r / p.G) * D + 32 * s + 8 * g;
      fqc[s] = ldg(reinterpret_cast<const half8*>(rt));
      fqs[s] = ldg(reinterpret_cast<const half8*>(rt + D / 2));
    }
  }
  if (pl == 0 && !fresh) {
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.q, (short)0, (int)((size_t)p.M * p.QH * D * 2), 0x00020000);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int rb = rg * QB + qb;
      const int r = min(rb * 16 + n, p.G * p.M - 1);
      const int t = r / p.G, qh = h * p.G + r % p.G;
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, DSPARK_LDSP(q_lds + (rb * (D / 32) + s) * 1024), 16,
                                                 (uint32_t)((((size_t)t * p.QH + qh) * D + 32 * s + 8 * g) * 2), 0, 0, 0);
    }
  }
  char* const slots[4] = {ring0, ring1, ring2, ring3};
#pragma unroll
  // (with a fresh block every one of the first RING - 1 steps is issued, steps past the split as out-of-range loads
  // into `trash`: a fixed count of younger loads, so the compiler's own wait for the raw rows above leaves the pages
  // in flight; the counted waits stay right, the extra loads being the youngest)
  for (int u = 0; u < RING - 1; ++u)
    if (FRESH_OK || u < nsteps) issue(u, slots[u]);
  if (nsteps >= RING - 1)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((RING - 1) * LPW));
  else if (nsteps >= 1)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPW));
  else
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __builtin_amdgcn_s_barrier();
  if (fresh) {
    // The raw rows are first used here: an empty asm that rewrites them keeps the compiler from moving any use (a
    // conversion) up next to its load, where it would wait for the loads before the pages were issued.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) asm volatile("" : "+v"(fq[qb][s][0]), "+v"(fq[qb][s][1]));
#pragma unroll
    for (int s = 0; s < D / 32; ++s) asm volatile("" : "+v"(fqw[s]));
#pragma unroll
    for (int s = 0; s < D / 64; ++s) asm volatile("" : "+v"(fqc[s]), "+v"(fqs[s]));
    if (fmine) {
#pragma unroll
      for (int e = 0; e < NE; ++e) asm volatile("" : "+v"(fk[e]), "+v"(fv[e]), "+v"(fkw[e]));
#pragma unroll
      for (int e = 0; e < NE / 2; ++e) asm volatile("" : "+v"(fkc[e]), "+v"(fks[e]));
    }
    // q/k norm + RoPE of the block (the q/k norm + RoPE kernel's arithmetic): row n's dims 32 s + 8 g + j sit in
    // lane (n, g), so a row's sum of squares is four lanes and every RoPE pair (i, i + D / 2) is in one lane
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float x[D / 32][8];
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[s][j] = fq[qb][s][j / 4][j % 4];
          ss += x[s][j] * x[s][j];
        }
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      const float inv = rsqrtf(ss / D + p.eps);
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) x[s][j] = x[s][j] * inv * (float)fqw[s][j];
#pragma unroll
      for (int s = 0; s < D / 64; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (32 * s + 8 * g + j < p.rot) {
            const float c = (float)fqc[s][j], sn = (float)fqs[s][j];
            const float x0 = x[s][j], x1 = x[s + D / 64][j];
            x[s][j] = x0 * c - x1 * sn;
            x[s + D / 64][j] = x1 * c + x0 * sn;
          }
        }
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        half8 q;
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = (_Float16)((float)(_Float16)x[s][j] * p.c);
        qf.r[qb][s] = q;
      }
    }
    if (fmine) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < NE; ++e) ss += fk[e] * fk[e];
      ss = (lane < 32) ? ss : 0.f;
      ss = wave_sum(ss);
      const float inv = rsqrtf(ss / D + p.eps);
      float r[NE];
#pragma unroll
      for (int e = 0; e < NE; ++e) r[e] = fk[e] * inv * (float)fkw[e];
#pragma unroll
      for (int e = 0; e < NE / 2; ++e) {
        if ((lane & 31) + 32 * e < p.rot) {
          const float x0 = r[e], x1 = r[e + NE / 2], c = (float)fkc[e], sn = (float)fks[e];
          r[e] = x0 * c - x1 * sn;
          r[e + NE / 2] = x1 * c + x0 * sn;
        }
      }
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        fkh[e] = (_Float16)r[e];
        fvh[e] = (_Float16)fv[e];
      }
    }
  } else {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        half8 q = *reinterpret_cast<const half8*>(q_lds + ((rg * QB + qb) * (D / 32) + s) * 1024 + lane * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = (_Float16)((float)q[j] * p.c);
        qf.r[qb][s] = q;
      }
  }
  for (int k = 0; k < nsteps; k += RING) {
#pragma unroll
    for (int u = 0; u < RING; ++u)
      if (k + u < nsteps) step(k + u, slots[u], slots[(u + RING - 1) % RING]);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  // the fresh K / V row into the pools, for later rounds (nothing in this launch reads the pools' copy)
  if (fmine && lane < 32) {
    const int phys = paged ? sm_bt[fpage - pb] : fpage;
    const int slot = fpos % PAGE;
    _Float16* kb = const_cast<_Float16*>(p.kp) + ((size_t)phys * p.KVH + h) * (PAGE * D);
    _Float16* vb = const_cast<_Float16*>(p.vp) + ((size_t)phys * p.KVH + h) * (D * PAGE);
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int d = lane + 32 * e;
      kb[k_page_elem(slot, d, D)] = fkh[e];
      vb[d * PAGE + slot] = fvh[e];
    }
  }

  // Page lanes merge through LDS as a tree: at level `half` (PL / 2, ..., 1) lanes half .. 2 half - 1 store their
  // states and lane q < half folds in lane q + half's -- ((0 + 2) + (1 + 3)) for four lanes, a fixed order. The state
  // of row block rb stored by lane q + half goes to area q * NRG QB + rb, area i at (i / RING) AREAF floats into ring
  // slot i % RING: 16 rows of (D + 6) floats, o [16][D + 4], then m [16] and l [16] (the host plan checks that
  // PL / 2 x NRG x QB areas fit the ring).
  if constexpr (PL > 1) {
    constexpr int ROWF = D + 4, AREAF = 16 * (ROWF + 2);
    const int NRGQ = NRG * QB;
    auto area_of = [&](int i) -> float* {
      float* a = nullptr;
#pragma unroll
      for (int k = 0; k < RING; ++k)
        if (i % RING == k) a = reinterpret_cast<float*>(slots[k]) + (i / RING) * AREAF;
      return a;
    };
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int half = PL / 2; half >= 1; half /= 2) {
      if (pl >= half && pl < 2 * half) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          float* area = area_of((pl - half) * NRGQ + rg * QB + qb);
#pragma unroll
          for (int cc = 0; cc < D / 16; ++cc)
            *reinterpret_cast<f32x4*>(area + n * ROWF + 16 * cc + 4 * g) = rs.o[qb][cc];
          if (g == 0) {
            area[16 * ROWF + n] = rs.m[qb];
            area[16 * ROWF + 16 + n] = rs.ls[qb][0];
          }
        }
      }
      __syncthreads();
      if (pl < half) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float* area = area_of(pl * NRGQ + rg * QB + qb);
          f32x4 ob[D / 16];
#pragma unroll
          for (int cc = 0; cc < D / 16; ++cc) ob[cc] = *reinterpret_cast<const f32x4*>(area + n * ROWF + 16 * cc + 4 * g);
          const float mb = area[16 * ROWF + n], lb = area[16 * ROWF + 16 + n];
          const float mx = fmaxf(rs.m[qb], mb);
          const float fa = fast_exp2(rs.m[qb] - mx), fb = fast_exp2(mb - mx);
#pragma unroll
          for (int cc = 0; cc < D / 16; ++cc) rs.o[qb][cc] = rs.o[qb][cc] * fa + ob[cc] * fb;
          rs.ls[qb] = rs.ls[qb] * fa + f32x4{lb, lb, lb, lb} * fb;
          rs.m[qb] = mx;
        }
      }
      __syncthreads();  // the areas are rewritten by the next level
    }
  }
  if (pl != 0) return;
  // The split's partial, stored device-coherent (SC1: written through to memory, so the end of the kernel has no
  // dirty L2 lines to write back; measured 0.4-0.6 us less per C2 layer than default stores).
  // row-major partials ([head][row][split][D]; the head's region is R x S rows of D floats)
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      p.part_acc + (size_t)h * R * p.S * D, (short)0, R * p.S * D * (int)sizeof(float), 0x00020000);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(p.part_ml + (size_t)h * R * p.S, (short)0,
                                                                      R * p.S * (int)sizeof(f32x2), 0x00020000);
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int rb = rg * QB + qb;
    if (rb >= NRB) break;  // padding row blocks of the last group
    const int ri = (rb * 16 + n) * p.S + split;
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, rs.o[qb][cc]), ra,
                                             (uint32_t)((ri * D + 16 * cc + 4 * g) * sizeof(float)), 0,
                                             ATTN_CPOL_COHERENT);
    if (g == 0) {
      const float L = rs.ls[qb][0];
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{L > 0.f ? rs.m[qb] : -INFINITY, L}), rm,
                                            (uint32_t)(ri * sizeof(f32x2)), 0, ATTN_CPOL_COHERENT);
    }
  }
}
#undef DSPARK_LDSP

// ---------------------------------------------------------------- merge of the split partials
// The partials are row-major ([KV head x row group][row][split][D]), so one workgroup merges one output row: thread
// (j, q) takes dims 4 q .. 4 q + 3 of splits j, j + SL, ... with batches of 8 loads in flight (one load of a wave covers
// 64 / (D / 4) whole splits of the row, contiguous), and merges them as a log-sum-exp (m = max, l = sum f_s l_s,
// acc = sum f_s acc_s, f_s = exp2(m_s - m)); the split lanes of a wave then merge pairwise in a fixed xor tree and the
// waves in wave order through LDS, so outputs are bit-identical run to run. o = acc / l (0 when nothing was visible),
// times the optional sigmoid gate, stored fp16 and/or fp32. blockIdx = (row, KV head x row group); rows past G M (padding
// of the last row block, never stored by the split kernels) store nothing. Measured on MI355X, graph-replayed with the
// partials in HBM: 256 splits at D 128 6.8 us (18.7 with the split-major layout and 32 lanes per output quad, whose
// every load touched 32 cache lines), 64 splits 3.6 (4.9), C2's 24 splits at D 64 2.8 with 4 split lanes, one wave
// per row (3.6; 3.3 with 8 lanes; 3.4 before the arguments, flag, gate and partials came in one round trip each);
// 16 split lanes beyond 96 splits, 8 below (4 at D = 64 up to 32 splits). Reference
// combine_phase, dspark.hip:2132-2185 (there the splits are the 60 workgroups' key ranges).
template <int D, int SL>
__global__ __launch_bounds__(SL * D / 4) void attn_combine_kernel(AttnParams p) {
  constexpr int Q = D / 4, NT = SL * Q, W = NT / 64, PER = 8;
  static_assert(NT % 64 == 0 && 64 % Q == 0, "whole waves of whole rows");
  __shared__ f32x4 s_acc[W > 1 ? W - 1 : 1][Q];
  __shared__ f32x2 s_ml[W > 1 ? W - 1 : 1][Q];
  const int hr = blockIdx.y, h = hr / p.RG, rg = hr % p.RG, r = blockIdx.x;
  const int row = rg * p.R + r;
  // Padding rows of the last row group (row >= G M, the same for the whole workgroup) load their partials (inside the
  // workspace) and store nothing: returning before the loads would put the kernel arguments the loads need behind the
  // test's own, one more dependent round trip for every row.
  const bool live = row < p.G * p.M;
  const int run = run_flag_load(p.st);  // tested once the partial loads are in flight
  // The gate word is loaded with the partials (a zero-length buffer when there is no gate: the load returns 0).
  const int rowc = min(row, p.G * p.M - 1);
  const int t = rowc / p.G, qh = h * p.G + rowc % p.G;
  const int gstride = p.gate_stride > 0 ? p.gate_stride : p.QH;
  const __amdgpu_buffer_rsrc_t rgate = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.gate, (short)0, p.gate ? (int)((size_t)p.M * gstride * sizeof(float)) : 0, 0x00020000);
  const float gv = __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(rgate, (int)(((size_t)t * gstride + qh) * sizeof(float)), 0, 0));
  const int q = threadIdx.x % Q, j = threadIdx.x / Q;
  const size_t base = ((size_t)hr * p.R + r) * p.S;
  float m = -INFINITY, l = 0.f;
  f32x4 acc = {0, 0, 0, 0};
  // Batches of SL x PER splits; the first is outside the loop (a loop head's wait, counted for the back edge, would hold
  // its partial loads until the flag and gate words had arrived). Returns false when the workgroup stores nothing.
  auto batch = [&](int b0) -> bool {
    f32x2 ml[PER];
    f32x4 av[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int sp = b0 + j + SL * i;
      const bool ok = sp < p.S;
      ml[i] = ok ? ldg(p.part_ml + base + sp) : f32x2{-INFINITY, 0.f};
      av[i] = ok ? ldg(reinterpret_cast<const f32x4*>(p.part_acc + (base + sp) * D) + q) : f32x4{0, 0, 0, 0};
    }
    if (!run_flag_set(run) || !live) {  // a stopped round or a padding row writes nothing (the whole workgroup)
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
    float mb = m;
#pragma unroll
    for (int i = 0; i < PER; ++i) mb = fmaxf(mb, ml[i][0]);
    if (mb > -INFINITY) {
      const float fr = m == -INFINITY ? 0.f : fast_exp2(m - mb);  // the running state rescaled to the batch max
      l *= fr;
      acc *= fr;
      m = mb;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const float f = ml[i][0] == -INFINITY ? 0.f : fast_exp2(ml[i][0] - m);
        l = fmaf(f, ml[i][1], l);
        acc += f * av[i];
      }
    }
    return true;
  };
  if (!batch(0)) return;  // (S >= 1)
  for (int b0 = SL * PER; b0 < p.S; b0 += SL * PER)
    if (!batch(b0)) return;
  auto fold = [&](float mk, float lk, f32x4 ak) {
    const float mx = fmaxf(m, mk);
    if (mx > -INFINITY) {
      const float fa = m == -INFINITY ? 0.f : fast_exp2(m - mx), fb = mk == -INFINITY ? 0.f : fast_exp2(mk - mx);
      l = l * fa + lk * fb;
      acc = acc * fa + ak * fb;
      m = mx;
    }
  };
#pragma unroll
  for (int off = Q; off < 64; off <<= 1) {
    f32x4 ak;
#pragma unroll
    for (int i = 0; i < 4; ++i) ak[i] = __shfl_xor(acc[i], off);
    fold(__shfl_xor(m, off), __shfl_xor(l, off), ak);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (W > 1) {
    if (wave > 0 && lane < Q) {
      s_acc[wave - 1][q] = acc;
      s_ml[wave - 1][q] = f32x2{m, l};
    }
    __syncthreads();
    if (wave > 0) return;
    for (int w = 0; w < W - 1; ++w) {
      const f32x2 mlw = s_ml[w][q];
      fold(mlw[0], mlw[1], s_acc[w][q]);
    }
  }
  if (lane >= Q) return;
  float scale = l > 0.f ? 1.f / l : 0.f;
  if (p.gate) scale *= 1.f / (1.f + expf(-gv));
  {
#pragma clang fp contract(off)  // the fp16 output is the fp32 output rounded (no product fused into the conversion)
    acc *= scale;
  }
  const size_t idx = ((size_t)t * p.QH + qh) * D + 4 * q;
  if (p.out16) {
    half4 hv;
#pragma unroll
    for (int i = 0; i < 4; ++i) hv[i] = (_Float16)acc[i];
    if (p.out_sc) {
      // LFM3_X8 output: a 16-dim piece is a quad of lanes (q = 4 k .. 4 k + 3; Q is a multiple of 4 and every lane
      // below Q is live)
      uint32_t mb = max(max(x8_mag_bits(hv[0]), x8_mag_bits(hv[1])), max(x8_mag_bits(hv[2]), x8_mag_bits(hv[3])));
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 1));
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 2));
      const float sc = x8_piece_scale(x8_mag_value(mb));
      const float inv = __builtin_amdgcn_rcpf(sc);
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[i] = x8_code(hv[i], inv);
      if ((q & 3) == 0) p.out_sc[(size_t)t * p.out_sc_row + (qh * D + 4 * q) / 16] = sc;
    }
    *reinterpret_cast<half4*>(p.out16 + (p.out_op ? xop_elem(t, qh * D + 4 * q, p.out_op) : idx)) = hv;
  }
  if (p.out32) *reinterpret_cast<f32x4*>(p.out32 + idx) = acc;
}

// K/V rows of positions pos0..pos0+n-1 into the pages: one thread per (token, head, 8 dims).
__global__ __launch_bounds__(256) void kv_write_kernel(const _Float16* k, const _Float16* v, int64_t row_stride,
                                                       _Float16* kp, _Float16* vp, const int32_t* bt, int64_t kv_pages,
                                                       int KVH, int D, int pos0, int n) {
  const int d8n = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)n * KVH * d8n) return;
  const int tok = (int)(idx / (KVH * d8n));
  const int rem = (int)(idx % (KVH * d8n));
  const int h = rem / d8n, d8 = rem % d8n;
  const int pos = pos0 + tok, lp = pos / PAGE, slot = pos % PAGE;
  const int phys = bt ? bt[lp] : lp;
  if (phys < 0 || phys >= kv_pages) return;  // a table entry outside the pools: the row is not written
  const _Float16* ks = k + (int64_t)tok * row_stride + h * D + 8 * d8;
  const _Float16* vs = v + (int64_t)tok * row_stride + h * D + 8 * d8;
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
// Two kernels. The LDS-ring kernel (verify_attn_lds_kernel) reads every page from HBM once for all query rows of its
// KV head; it covers up to 16 row blocks (256 rows: M <= 64 at 4 query heads per KV head). The register kernel
// (verify_attn_kernel) covers the rest: a wave holds QB row blocks and takes pages in turn, row groups of one split
// share pages through the XCD's L2. OCC = 1: one 4-wave workgroup per CU (up to 6 blocks per wave at D = 64);
// OCC = 2: two workgroups per CU, at most 2 blocks per wave.
#ifndef DSPARK_ATTN_PF
#define DSPARK_ATTN_PF 2
#endif
#ifndef DSPARK_ATTN_LDS_FILL
#define DSPARK_ATTN_LDS_FILL 75  // LDS kernel, up to 4 row blocks: key splits x KV heads = this % of the workgroup slots
#endif
#ifndef DSPARK_ATTN_LDS_FILL_WIDE
#define DSPARK_ATTN_LDS_FILL_WIDE 100  // LDS kernel, 5 or more row blocks (compute-bound): the same percentage
#endif
#ifndef DSPARK_ATTN_OCC2_MAX_PAGES
#define DSPARK_ATTN_OCC2_MAX_PAGES 12  // pages per wave (at one workgroup per CU) below which OCC = 2 is used
#endif
#ifndef DSPARK_ATTN_PF2
#define DSPARK_ATTN_PF2 2  // pages in flight per wave at OCC = 2
#endif
#ifndef DSPARK_ATTN_QB_MAX_64
#define DSPARK_ATTN_QB_MAX_64 6
#endif
#ifndef DSPARK_ATTN_QB_MAX_OCC2
#define DSPARK_ATTN_QB_MAX_OCC2 2
#endif
#ifndef DSPARK_ATTN_LDS
#define DSPARK_ATTN_LDS 1  // 0: register kernel only
#endif
constexpr int QB_MAX_64 = DSPARK_ATTN_QB_MAX_64, QB_MAX_128 = 2;
constexpr int QB_MAX_OCC2 = DSPARK_ATTN_QB_MAX_OCC2;

template <int D, int QB, int OCC>
static void launch_attn(const AttnParams& p, hipStream_t s) {
  constexpr bool QLDS = QB > 6;
  constexpr int PF = QLDS ? 1 : (OCC == 2 ? DSPARK_ATTN_PF2 : ((QB * D <= 4 * 64) ? DSPARK_ATTN_PF : 2));
  const int units = p.KVH * p.S;
  hipLaunchKernelGGL((verify_attn_kernel<D, QB, PF, OCC, QLDS>), dim3((units + 7) / 8 * 8 * p.RG), dim3(256), 0, s, p);
}

// MAXW: the most waves a plan of this shape launches (the launch bound, so the register budget is the shape's own).
template <int D, int QB, int PL, int PPL, int LPW, int MAXW>
static int launch_lds(const AttnParams& p, hipStream_t s) {
  if (p.nrg * PL > MAXW) return DSPARK_EUNSUPPORTED;
  if constexpr (QB == 1 && D == 64) {
    if (p.mix) {  // a fresh block: at most one block token per wave
      if (p.M > p.nrg * PL) return DSPARK_EUNSUPPORTED;
      hipLaunchKernelGGL((verify_attn_lds_kernel<D, QB, PL, PPL, LPW, MAXW, true>), dim3(p.KVH * p.S),
                         dim3(p.nrg * PL * 64), 0, s, p);
      return 0;
    }
  }
  if (p.mix) return DSPARK_EUNSUPPORTED;
  hipLaunchKernelGGL((verify_attn_lds_kernel<D, QB, PL, PPL, LPW, MAXW>), dim3(p.KVH * p.S), dim3(p.nrg * PL * 64), 0, s,
                     p);
  return 0;
}

#ifndef DSPARK_ATTN_QB3
#define DSPARK_ATTN_QB3 1  // 0: 9 row blocks as 9 waves of one block (the QB = 1 shape)
#endif

// LDS-ring shape for nblk row blocks: a step is PPS = LDS_STEP_BYTES / page bytes pages; QB row blocks per wave in
// NRG = ceil(nblk / QB) row groups; page lanes PL (NRG * PL <= 16 waves; the page-lane merge's PL / 2 x NRG x QB
// areas fit the ring), PPL = PPS / PL pages per lane per step, and loads per wave per step LPW = ceil(chunks per step /
// waves). QB = 3 for 9 row blocks at D = 64 (33 tokens x 4 query heads: 3 groups x 4 page lanes = 12 waves, three per
// SIMD, each reading one page per step), QB = 1 otherwise. Returns false when the register kernel is needed.
static bool lds_shape(int D, int nblk, int* qb, int* nrg, int* pl, int* ppl, int* lpw) {
  if (!DSPARK_ATTN_LDS || nblk < 1 || nblk > 16) return false;
  const int pageb = 4 * PAGE * D, cpg = pageb / 1024;
  int pps = LDS_STEP_BYTES / pageb;
  const size_t areaf = 16 * (D + 6) * 4, areas_in_ring = (size_t)RING * (LDS_STEP_BYTES / areaf);
  if (DSPARK_ATTN_QB3 && D == 64 && nblk == 9) {
    *qb = 3;
    *nrg = 3;
    *pl = 4;
    *ppl = pps / 4;
    *lpw = (pps * cpg + 11) / 12;
    return (size_t)(4 / 2) * 9 <= areas_in_ring;
  }
  int PL = 1;
  for (int c = pps; c >= 1; c /= 2) {
    if (nblk * c <= 16 && (c == 1 || (size_t)(c / 2) * nblk <= areas_in_ring)) {
      PL = c;
      break;
    }
  }
  // Q staged apart from the ring (it does not fit one slot: D = 128 with one page lane) -> one page per lane per step,
  // so ring + Q stay within the 160 KB of LDS.
  if ((16 / PL) * (D / 32) * 1024 > pps * pageb) pps = PL;
  *qb = 1;
  *nrg = nblk;
  *pl = PL;
  *ppl = pps / PL;
  *lpw = (pps * cpg + nblk * PL - 1) / (nblk * PL);
  return true;
}

void attn_plan(AttnParams& p, int D, int cus) {
  const int rows = p.G * p.M;
  const int nblk = (rows + 15) / 16;
  const int lo0 = std::min(p.a, std::max(p.start, p.window > 0 ? p.a - p.window + 1 : 0));  // the block's keys from a
  const int lo_last = std::max(p.start, p.window > 0 ? p.a + p.M - 1 - p.window + 1 : 0);
  const int hi_last = p.a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? p.a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  p.c = (float)(1.4426950408889634 / std::sqrt((double)D));
  const int S_req = p.S;
  auto finish = [&](int S) {
    S = std::max(1, std::min(S, std::min(64, p.npages)));
    p.pps = (p.npages + S - 1) / S;
    p.S = (p.npages + p.pps - 1) / p.pps;
  };
  int qb = 1, nrg = 0, pl = 0, ppl = 0, lpw = 0;
  // LDS-ring kernel: one workgroup per (KV head, split) holding all rows; enough workgroups for every CU (two per
  // CU for small ones); splits no longer than its LDS block table.
  if (lds_shape(D, nblk, &qb, &nrg, &pl, &ppl, &lpw) && (p.npages + 63) / 64 <= LDS_BT_MAX) {
    p.lds = 1;
    p.nrb = nblk;
    p.qb = qb;
    p.nrg = nrg;
    p.pl = pl;
    p.ppl = ppl;
    p.lpw = lpw;
    p.RG = 1;
    p.QB = 1;
    p.R = 16 * nblk;
    p.OCC = nrg * pl <= 8 ? 2 : 1;
    int S = S_req;
    if (S <= 0) {
      // Up to 4 row blocks a split streams pages at the HBM rate and three quarters of the workgroup slots measured
      // best on MI355X (9 and 16 tokens at 32k and 128k keys: the per-split fixed costs outweigh the last quarter of
      // the CUs). From 5 row blocks on, the per-page matrix-core and exp2 work of the NRB waves is the bound, and
      // every CU is used (24, 33 and 64 tokens: 4-12 % faster at 32k and 128k keys).
      const int fill = nblk <= 4 ? DSPARK_ATTN_LDS_FILL : DSPARK_ATTN_LDS_FILL_WIDE;
      S = (cus * p.OCC * fill / 100 + p.KVH - 1) / p.KVH;
      S = std::min(S, (p.npages + pl * ppl - 1) / (pl * ppl));  // at least one step per split
    }
    S = std::max(S, (p.npages + LDS_BT_MAX - 1) / LDS_BT_MAX);
    finish(S);
    return;
  }
  // Register kernel: one workgroup per CU unless the pages per wave are few and the rows fit OCC = 2.
  p.lds = 0;
  const int qb_max1 = D == 64 ? QB_MAX_64 : QB_MAX_128;
  const int rg1 = (nblk + qb_max1 - 1) / qb_max1;
  const double pages_per_wave = (double)p.npages * p.KVH * rg1 / (4.0 * cus);
  p.OCC = (D == 64 && pages_per_wave < DSPARK_ATTN_OCC2_MAX_PAGES) ? 2 : 1;
  const int qb_max = p.OCC == 2 ? QB_MAX_OCC2 : qb_max1;
  p.RG = (nblk + qb_max - 1) / qb_max;
  p.QB = (nblk + p.RG - 1) / p.RG;
  p.R = 16 * p.QB;
  int S = S_req;
  if (S <= 0) {
    const int groups = p.KVH * p.RG;
    S = (cus * p.OCC + groups - 1) / groups;
    S = std::min(S, (p.npages + 3) / 4);  // at least one page per wave
  }
  finish(S);
}

// Workspace: partial accumulators [KVH][RG][R][S][D] f32 (row-major: one row's splits contiguous), then (max, sum)
// pairs [KVH][RG][R][S].
static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

size_t attn_workspace_bytes(const AttnParams& p, int D) {
  const size_t slots = (size_t)p.KVH * p.RG * p.S;
  return round256(slots * p.R * D * sizeof(float)) + round256(slots * p.R * sizeof(f32x2));
}

void attn_bind_workspace(AttnParams& p, int D, void* ws) {
  const size_t slots = (size_t)p.KVH * p.RG * p.S;
  char* b = static_cast<char*>(ws);
  p.part_acc = reinterpret_cast<float*>(b);
  p.part_ml = reinterpret_cast<f32x2_t*>(b + round256(slots * p.R * D * sizeof(float)));
}

static int launch_split(const AttnParams& p, int D, hipStream_t s) {
  if (p.mix && !p.lds) return DSPARK_EUNSUPPORTED;  // (a fresh block goes to the LDS kernel only)
  if (p.lds) {
    // instantiated shapes (see lds_shape), as (PL, PPL, LPW): D = 64: (4, 1, 8 | 4 | 3 | 2), (2, 2, 4 | 3 | 2),
    // (1, 4, 4 | 3 | 2); D = 128: (2, 1, 16 | 8 | 6 | 4 | 3 | 2), (1, 1, 2 | 1)
    if (p.qb == 3) {
      if (D != 64 || p.nrg != 3 || p.pl != 4 || p.ppl != 1 || p.lpw != 3) return DSPARK_EUNSUPPORTED;
      return launch_lds<64, 3, 4, 1, 3, 12>(p, s);
    }
    if (p.qb != 1) return DSPARK_EUNSUPPORTED;
    const int key = D * 10000 + p.pl * 1000 + p.ppl * 100 + p.lpw;
    switch (key) {
      case 644108: return launch_lds<64, 1, 4, 1, 8, 16>(p, s);
      case 644104: return launch_lds<64, 1, 4, 1, 4, 16>(p, s);
      case 644103: return launch_lds<64, 1, 4, 1, 3, 16>(p, s);
      case 644102: return launch_lds<64, 1, 4, 1, 2, 16>(p, s);
      case 642204: return launch_lds<64, 1, 2, 2, 4, 16>(p, s);
      case 642203: return launch_lds<64, 1, 2, 2, 3, 16>(p, s);
      case 642202: return launch_lds<64, 1, 2, 2, 2, 16>(p, s);
      case 641404: return launch_lds<64, 1, 1, 4, 4, 16>(p, s);
      case 641403: return launch_lds<64, 1, 1, 4, 3, 16>(p, s);
      case 641402: return launch_lds<64, 1, 1, 4, 2, 16>(p, s);
      case 1282116: return launch_lds<128, 1, 2, 1, 16, 4>(p, s);
      case 1282108: return launch_lds<128, 1, 2, 1, 8, 4>(p, s);
      case 1282106: return launch_lds<128, 1, 2, 1, 6, 8>(p, s);
      case 1282104: return launch_lds<128, 1, 2, 1, 4, 12>(p, s);
      case 1282103: return launch_lds<128, 1, 2, 1, 3, 16>(p, s);
      case 1282102: return launch_lds<128, 1, 2, 1, 2, 16>(p, s);
      case 1281102: return launch_lds<128, 1, 1, 1, 2, 16>(p, s);
      case 1281101: return launch_lds<128, 1, 1, 1, 1, 16>(p, s);
      default: return DSPARK_EUNSUPPORTED;
    }
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
  return 0;
}

int attn_launch(AttnParams& p, int D, int phases, hipStream_t s) {
  if (phases & 1) {
    const int rc = launch_split(p, D, s);
    if (rc) return rc;
  }
  if (phases & 2) {
    const bool wide = p.S > 96;  // 16 split lanes per row, else 8 (4 at D = 64 up to 32 splits: one wave per row)
    const dim3 grid(p.R, p.KVH * p.RG);
    if (D == 64 && p.S <= 32)
      hipLaunchKernelGGL((attn_combine_kernel<64, 4>), grid, dim3(4 * 16), 0, s, p);
    else if (D == 64 && !wide)
      hipLaunchKernelGGL((attn_combine_kernel<64, 8>), grid, dim3(8 * 16), 0, s, p);
    else if (D == 64)
      hipLaunchKernelGGL((attn_combine_kernel<64, 16>), grid, dim3(16 * 16), 0, s, p);
    else if (!wide)
      hipLaunchKernelGGL((attn_combine_kernel<128, 8>), grid, dim3(8 * 32), 0, s, p);
    else
      hipLaunchKernelGGL((attn_combine_kernel<128, 16>), grid, dim3(16 * 32), 0, s, p);
  }
  return (int)hipGetLastError();
}

int kv_write_launch(const void* k, const void* v, int64_t row_stride, void* kp, void* vp, const int32_t* bt,
                    int64_t kv_pages, int KVH, int D, int pos0, int n, hipStream_t s) {
  const int64_t threads = (int64_t)n * KVH * (D / 8);
  if (threads == 0) return 0;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     (const _Float16*)k, (const _Float16*)v, row_stride, (_Float16*)kp, (_Float16*)vp, bt, kv_pages, KVH,
                     D, pos0, n);
  return (int)hipGetLastError();
}

}  // namespace dspark
