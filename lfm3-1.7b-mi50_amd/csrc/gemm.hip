// Verify GEMMs for M <= 64 tokens on the matrix cores: int8 weights (biased u8, one fp16 scale per output row) and the
// fp16 cropped head with a fused row argmax.
//
// Layout. C^T[rows][tokens] = W[rows][K] * X^T[K][tokens] with v_mfma_f32_16x16x32_f16: a wave streams a 16-row strip
// of W (lane l: row l%16, 16 contiguous bytes per 64-column chunk), X^T comes from the same 16-byte pieces of the
// token rows. int8 -> fp16 is exact: byte b (= q + 128) placed under 0x64 is the half 1024 + b, minus 1152 gives q
// (v_perm_b32 + v_pk_add_f16 per two weights). Two kernels: the K-sliced kernel (up to 32 tokens) gives a workgroup
// S strips and all of K, its S x KW waves each stream one range of K with every weight load in flight and add the
// ranges in LDS in range order; the split kernel (any M <= 64) gives each workgroup a share of K and lets the last
// workgroup of a row group to arrive add the split partials in split order (or a reduce kernel does). Weights are read
// once per call for all tokens; both are HBM-bound (about 2*M flop per weight byte).
// Reference: gemv_phase / unit_dot_r (dspark.hip:541-716), head_run<true> (2219-2318), markov argmax (2322-2366).
#include <type_traits>

#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

__device__ __forceinline__ half8 i8x8_to_half8(uint32_t w0, uint32_t w1) {
  const uint32_t k64 = 0x64646464u;
  const uint32_t a0 = __builtin_amdgcn_perm(k64, w0, 0x04010400u);
  const uint32_t a1 = __builtin_amdgcn_perm(k64, w0, 0x04030402u);
  const uint32_t a2 = __builtin_amdgcn_perm(k64, w1, 0x04010400u);
  const uint32_t a3 = __builtin_amdgcn_perm(k64, w1, 0x04030402u);
  u32x4 u = {a0, a1, a2, a3};
  half8 h = as_half8(u);
  const half8 bias = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
  return h - bias;
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

// Epilogue for one lane's 4 rows (row0 + 4g + i) of token t.
// The per-row weight scales of rows r .. r + 3 as fp16 bits (1 without scales). The kernels load them with their first
// loads (read in the epilogue, they were a dependent round trip after the main loop) and widen them in the epilogue,
// behind an empty asm: widened where they are loaded, the conversion's wait would hold every weight load back.
__device__ __forceinline__ u32x2 gemm_row_scales(const GemmParams& p, int r) {
  if (!p.scale) return u32x2{0x3C003C00u, 0x3C003C00u};
  return ldg(reinterpret_cast<const u32x2*>(p.scale + r));
}
__device__ __forceinline__ f32x4 gemm_row_scales_f32(u32x2 raw) {
  asm volatile("" : "+v"(raw));
  const half4 h = __builtin_bit_cast(half4, raw);
  return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

// sc: gemm_row_scales of rows row0 + 4 g .. (a product by 1 leaves the value unchanged)
__device__ __forceinline__ void gemm_store(const GemmParams& p, int t, int row0, int g, f32x4 v, f32x4 sc) {
  if (t >= p.M) return;
  const int r = row0 + 4 * g;
  v *= sc;
  if (p.epilogue == 1) {
    // rows (2i, 2i+1) = (gate, up): h[t][r/2 + i] = fp16(silu(gate) * up); r/2 is even, so the pair is contiguous
    _Float16* y = p.y16 + (p.yop ? xop_elem(t, r / 2, p.yop) : (size_t)t * (p.N / 2) + r / 2);
    y[0] = f16_product(silu_f(v[0]), v[1]);
    y[1] = f16_product(silu_f(v[2]), v[3]);
    return;
  }
  if (p.y32) *reinterpret_cast<f32x4*>(p.y32 + (size_t)t * p.N + r) = v;
  if (p.y16) {
    half4 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = (_Float16)(p.epilogue == 2 ? silu_f(v[i]) : v[i]);
    *reinterpret_cast<half4*>(p.y16 + (p.yop ? xop_elem(t, r, p.yop) : (size_t)t * p.N + r)) = h;
  }
}

// X^T of a band staged in LDS by the K-sliced kernel (bytes): every token block at once when that fits, else passes
// of two token blocks, else of one (each token block's X^T is the band's chunks x 2 KB).
constexpr int GEMM_X_LDS = 131072;
__host__ __device__ inline int gemm_pass_tbs(int tb, int band_chunks) {
  if (tb * band_chunks * 2048 <= GEMM_X_LDS) return tb;
  return 2 * band_chunks * 2048 <= GEMM_X_LDS ? 2 : 1;
}

// TB token blocks of 16. I8: weights biased int8, else fp16.
__device__ __forceinline__ bool gemm_stopped(const GemmParams& p) { return p.st && p.st->run == 0; }

constexpr int GEMM_VMCNT0 = 0x0F70;  // s_waitcnt vmcnt(0), other counters left unconstrained

// ---------------------------------------------------------------- fused row-group epilogues
// The workgroup's group of R = 16 * nw rows is complete (unsplit, or summed by the last split): every wave puts its
// scaled products into an LDS tile [token][row] (stride RS = R + 4 floats), then the group's rows are finished there.

// GEMM_FUSE_CONV (conv_wave, dspark.hip:2191-2214): R == 48, so a group is 16 channels c with rows [B, C, X] at 3c ..
// 3c + 2. One thread per (token, channel): bx = fp16(B X); conv = w[K-1] bx + sum_{k<K-1} w[k] hist[pos-K+1+k] with the
// history inside the block recomputed from the tile and before it read from the ring; y = fp16(C conv); ring[pos] = bx.
// Ring slots written (a .. a+M-1) and read (a-K+1 .. a-1) are disjoint for M + K - 1 <= CONV_RING.
// cs: the group's weights and ring history staged in LDS at the kernel's start (conv_stage_issue), or cs.ring null:
// read from the global ring and weights here.
struct ConvStage {
  const _Float16* ring = nullptr;  // LDS [CONV_RING][16]: the group's 16 channels of every ring slot
  const _Float16* w = nullptr;     // LDS [16][K] (+ padding to 128 halves)
  int a = 0;                       // the State's a
};
__device__ void epi_conv(const GemmParams& p, const float* tile, int RS, int grow0, int R, int nthreads, ConvStage cs) {
  const int H = p.N / 3, c0 = grow0 / 3, nch = R / 3, K = p.conv_k;
  const bool staged = cs.ring != nullptr;
  const int a = staged ? cs.a : p.st->a;
  for (int e = threadIdx.x; e < p.M * nch; e += nthreads) {
    const int t = e / nch, cl = e % nch, c = c0 + cl;
    if (c >= H) continue;
    constexpr int KMAX = 8;
    float w[KMAX], bx[KMAX];
    float C = 0.f, bx_t = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      w[k] = 0.f;
      bx[k] = 0.f;
      if (k < K) {
        w[k] = (float)(staged ? cs.w[cl * K + k] : p.conv_w[(size_t)c * K + k]);
        const int tt = t - (K - 1) + k;
        if (tt >= 0) {
          const float* m = tile + tt * RS + 3 * cl;
          bx[k] = (float)f16_product(m[0], m[2]);
          if (k == K - 1) {
            C = m[1];
            bx_t = bx[k];
          }
        } else {
          const int slot = (a + tt) & (CONV_RING - 1);
          bx[k] = (float)(staged ? cs.ring[slot * 16 + cl] : p.conv_ring[(size_t)slot * H + c]);
        }
      }
    }
    float conv = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
      if (k == K - 1) conv = w[k] * bx[k];
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
      if (k < K - 1) conv = fmaf(w[k], bx[k], conv);
    p.conv_ring[(size_t)((a + t) & (CONV_RING - 1)) * H + c] = (_Float16)bx_t;
    _Float16 y = f16_product(C, conv);
    if (p.ysc) {
      // LFM3_X8 output: the group's 16 channels are one piece, held by 16 aligned lanes (nch == 16, the workgroup a
      // multiple of 16 threads: the host checked), all live or all skipped together
      uint32_t mb = x8_mag_bits(y);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o));
      const float sc = x8_piece_scale(x8_mag_value(mb));
      y = x8_code(y, __builtin_amdgcn_rcpf(sc));
      if (cl == 0) p.ysc[(size_t)t * p.ysc_row + c / 16] = sc;
    }
    p.y16[p.yop ? xop_elem(t, c, p.yop) : (size_t)t * H + c] = y;
  }
}

// The conv epilogue's ring history and weights of the group's 16 channels c0 .. c0 + 15 into LDS, issued at the kernel's
// start by direct-to-LDS loads (no registers, no waits; the epilogue waits for them before its first barrier): every
// ring slot, since the slots read depend on the State's a, and the group's 16 x K weights (128 halves loaded). Read in
// the epilogue, they were a dependent round trip after the main loop.
__device__ __forceinline__ void conv_stage_issue(const GemmParams& p, int c0, int wave, int nw, int lane,
                                                 _Float16* ring_lds, _Float16* w_lds) {
  const int H = p.N / 3;
  const __amdgpu_buffer_rsrc_t rr =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.conv_ring, (short)0, CONV_RING * H * 2, 0x00020000);
  for (int i = wave; i < CONV_RING / 8; i += nw)  // 8 slots x 16 channels (32 B each) per instruction
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (__attribute__((address_space(3))) void*)(ring_lds + i * 128), 4,
                                             (uint32_t)(((8 * i + (lane >> 3)) * H + c0) * 2 + (lane & 7) * 4), 0,
                                             0, 0);
  if (wave == nw - 1) {
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.conv_w, (short)0, H * p.conv_k * 2, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)w_lds, 4,
                                             (uint32_t)(c0 * p.conv_k * 2 + lane * 4), 0, 0, 0);
  }
}

// S strips per group; the waves with `holder` set hold strip s's sums (every wave of the workgroup finishes the group).
// sc: the holder's row scales (gemm_row_scales of rows grow0 + r; strips past N hold rows no epilogue reads).
template <int TB>
__device__ void gemm_group_epilogue(const GemmParams& p, const f32x4 (&acc)[TB], int grp, int s, int S, bool holder,
                                    int lane, float* tile, f32x4 sc, ConvStage cs = ConvStage{}) {
  const int R = 16 * S, RS = R + 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int grow0 = grp * R, r = 16 * s + 4 * g;
  if (cs.ring) __builtin_amdgcn_s_waitcnt(GEMM_VMCNT0);  // this wave's staging loads are in LDS (the barrier: all)
  __syncthreads();  // every wave is done with the LDS it used before
  if (holder) {
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = 16 * tb + n;
      if (t < p.M) *reinterpret_cast<f32x4*>(tile + t * RS + r) = acc[tb] * sc;
    }
  }
  __syncthreads();
  (void)wave;
  epi_conv(p, tile, RS, grow0, R, 64 * nw, cs);
}

// Finished sums of one strip (lane (n, g): rows 16 strip + 4 g + i of token 16 tb + n): the strip's row-argmax key
// per token when the call asks for it, then the epilogue store.
template <int TB>
__device__ __forceinline__ void gemm_strip_out(const GemmParams& p, const f32x4 (&acc)[TB], int strip, int lane,
                                               f32x4 sc) {
  const int n = lane & 15, g = lane >> 4, row0 = strip * 16;
  if (p.best_part) {
    // fold the lane's 4 rows, then the 4 row groups
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = 16 * tb + n;
      uint64_t b = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint64_t k = argmax_key(acc[tb][i], (uint32_t)(row0 + 4 * g + i));
        b = k > b ? k : b;
      }
      uint64_t o = shfl_xor_u64(b, 16);
      b = o > b ? o : b;
      o = shfl_xor_u64(b, 32);
      b = o > b ? o : b;
      if (g == 0 && t < p.M) p.best_part[(size_t)t * (p.N / 16) + strip] = b;
    }
  }
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) gemm_store(p, 16 * tb + n, row0, g, acc[tb], sc);
}

constexpr int GEMM_CPOL_COHERENT = 16;  // buffer-op cache policy SC1: device-scope coherent store / load
// s_waitcnt immediate: vmcnt(n) (6 bits, split low 4 / high 2), other counters left unconstrained
#define GEMM_VMCNT(n) ((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)
#define GEMM_LGKMCNT0 0xC07F  // lgkmcnt(0), vmcnt and expcnt unconstrained
constexpr int GEMM_FIXUP_BATCH = 8;     // split partials loaded per batch by the last split

// Weight loads go in batches of CPB chunks (64 columns: 16 B per lane int8, 32 B fp16), two batches in registers.
constexpr int GEMM_PHASE_UNITS = 32;  // X staged per phase: TB x chunks <= 32 (64 KB of LDS)

// Grid: (ceil(strips / waves per group)) groups x ksplit; each wave owns one 16-row strip and the group's K range.
// The group stages its X slice into LDS once per phase (64 KB at most), in operand order [tb][chunk][half][lane]
// (16 B each, so every B-operand read is one contiguous 1 KB row of LDS), and every wave streams its strip's
// weights in batches of gemm_cpb chunks, the next batch in flight while the current one is multiplied. Loads past
// the range are clamped to valid addresses and discarded, so the number of loads in flight is the same on every path
// and the compiler's waits stay counted.
template <int TB, bool I8, int CPB>
__global__ __launch_bounds__(512) void gemm_kernel(GemmParams p) {
  if (gemm_stopped(p)) return;
  extern __shared__ u32x4 xs[];
  constexpr int WV = I8 ? 1 : 2, PH = GEMM_PHASE_UNITS / TB;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int grp = blockIdx.x / p.ksplit, ks = blockIdx.x % p.ksplit;
  const int strips = p.N / 16;
  const int strip_raw = grp * nw + wave;
  const bool live = strip_raw < strips;
  const int strip = live ? strip_raw : strips - 1;
  const int row0 = strip * 16;
  const u32x2 rsc = gemm_row_scales(p, row0 + 4 * g);  // first of the kernel's loads (the epilogue's)
  const int chunks = p.K / 64;
  const int cpk = (chunks + p.ksplit - 1) / p.ksplit;
  const int c0 = ks * cpk, c1 = min(chunks, c0 + cpk);

  f32x4 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) acc[tb] = f32x4{0, 0, 0, 0};

  const bool tiled = I8 && p.tiled;
  const uint8_t* wrow = tiled ? reinterpret_cast<const uint8_t*>(p.w) + (size_t)strip * chunks * 1024 + lane * 16
                              : reinterpret_cast<const uint8_t*>(p.w) + (size_t)(row0 + n) * p.K * (I8 ? 1 : 2) + 16 * g;
  const int cstride = tiled ? 1024 : 64;  // bytes from one 64-column chunk of the lane's row to the next
  // chunks cb .. cb + CPB - 1, clamped to the phase's last chunk ce - 1 (a re-read of a line just fetched)
  auto load = [&](u32x4 (&w)[CPB][WV], int cb, int ce) {
#pragma unroll
    for (int i = 0; i < CPB; ++i) {
      const int c = min(cb + i, ce - 1);
      if (I8) {
        w[i][0] = ldg_nt(reinterpret_cast<const u32x4*>(wrow + (size_t)c * cstride));
      } else {
        const u32x4* wp = reinterpret_cast<const u32x4*>(wrow + 2 * c * 64 + 16 * g);  // fp16: 32 B per lane
        w[i][0] = ldg_nt(wp);
        w[i][WV - 1] = ldg_nt(wp + 1);
      }
    }
  };
  // LDS slot of lane l's X operand in a half-h row: l, or l ^ (4 g + 2 h) when X is staged through registers (the
  // swizzle spreads a full-line read's 16-byte pieces over every bank group; it permutes slots within the row, so the
  // reads stay conflict-free)
  // X goes through registers for the deep-batch plans (phases of 16+ chunks: 32-64 KB of X per workgroup, where
  // full-line reads beat the direct loads' 16-line gathers; measured on MI355X) and by direct loads otherwise.
  constexpr int XRG = 16;  // X loads per wave on the register path (TB * 2 * phase chunks <= 64 = XRG * 4 waves)
  const bool xreg = CPB == 8 && nw >= 4 && !p.xop;
  const int xl0 = xreg ? lane ^ (4 * g) : lane, xl1 = xreg ? lane ^ (4 * g + 2) : lane;
  // chunk cb + i of the phase starting at chunk ph (pc chunks staged). With one token block the batch's X operands
  // are read from LDS before its first MFMA, so their latency is paid once per batch, not once per chunk.
  auto compute = [&](const u32x4 (&w)[CPB][WV], int cb, int ph, int pc) {
    if constexpr (TB == 1) {
      u32x4 xb[CPB][2];
#pragma unroll
      for (int i = 0; i < CPB; ++i) {
        const int j = min(cb + i - ph, pc - 1);
        const u32x4* xp = xs + ((size_t)j * 2) * 64;
        xb[i][0] = xp[xl0];
        xb[i][1] = xp[64 + xl1];
      }
#pragma unroll
      for (int i = 0; i < CPB; ++i) {
        if (cb + i - ph < pc) {
          half8 a[2];
          if (I8) {
            a[0] = i8x8_to_half8(w[i][0][0], w[i][0][1]);
            a[1] = i8x8_to_half8(w[i][0][2], w[i][0][3]);
          } else {
            a[0] = as_half8(w[i][0]);
            a[1] = as_half8(w[i][WV - 1]);
          }
          acc[0] = mfma16x16x32(a[0], as_half8(xb[i][0]), acc[0]);
          acc[0] = mfma16x16x32(a[1], as_half8(xb[i][1]), acc[0]);
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < CPB; ++i) {
      const int j = cb + i - ph;
      if (j < pc) {
        half8 a[2];
        if (I8) {
          a[0] = i8x8_to_half8(w[i][0][0], w[i][0][1]);
          a[1] = i8x8_to_half8(w[i][0][2], w[i][0][3]);
        } else {
          a[0] = as_half8(w[i][0]);
          a[1] = as_half8(w[i][WV - 1]);
        }
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          const u32x4* xb = xs + ((size_t)(tb * pc + j) * 2) * 64;
          acc[tb] = mfma16x16x32(a[0], as_half8(xb[xl0]), acc[tb]);
          acc[tb] = mfma16x16x32(a[1], as_half8(xb[64 + xl1]), acc[tb]);
        }
      }
    }
  };

  // X row r of a phase = [tb][chunk j][half h] (1 KB of LDS, lane l's 16 B at 16 l): token 16 tb + l % 16, columns
  // (ph + j) * 64 + 16 (l / 16) + 8 h .. + 8. Rows go straight from global memory to LDS with direct loads (each lane
  // gathers its 16 B), the waves taking rows in turn.
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.x, (short)0, (int)((size_t)(p.xop ? 16 * p.xop : p.M) * p.K * 2), 0x00020000);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  u32x4 wa[CPB][WV], wb[CPB][WV];
  for (int ph = c0; ph < c1; ph += PH) {
    const int pc = min(PH, c1 - ph), pe = ph + pc;
    if (ph != c0) __syncthreads();  // every wave is done reading the previous phase
    if (xreg) {
      // One load = 8 tokens x one 64-column chunk: lane l reads token 8 (k % 2TB) + l / 8, 16 B at column
      // 64 j + 8 (l % 8) of chunk j = k / 2TB, so a load covers 8 whole 128-byte lines. The wave's X loads (at most
      // XRG with four or more waves) go out before the phase's first two weight batches, so the counted wait for them
      // leaves the weights in flight.
      const int ninstr = TB * 2 * pc;
      u32x4 xr[XRG];
#pragma unroll
      for (int i = 0; i < XRG; ++i) {
        const int k = min(wave_u + i * nw, ninstr - 1);
        const int t = min(8 * (k % (2 * TB)) + (lane >> 3), p.M - 1), j = k / (2 * TB);
        xr[i] = ldg(reinterpret_cast<const u32x4*>(p.x + (size_t)t * p.K + (size_t)(ph + j) * 64 + 8 * (lane & 7)));
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the X loads ahead of the weight loads in issue order
      load(wa, ph, pe);
      load(wb, ph + CPB, pe);  // clamped to the phase: a second batch is always issued, used when it exists
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(GEMM_VMCNT(2 * CPB * WV));
#pragma unroll
      for (int i = 0; i < XRG; ++i) {
        const int k = wave_u + i * nw;
        const int t = 8 * (k % (2 * TB)) + (lane >> 3), j = k / (2 * TB);
        const int q = lane & 7, gq = q >> 1, hq = q & 1;
        if (k < ninstr && t < p.M)
          xs[(((t >> 4) * pc + j) * 2 + hq) * 64 + (((t & 15) + 16 * gq) ^ (4 * gq + 2 * hq))] = xr[i];
      }
      __builtin_amdgcn_s_waitcnt(GEMM_LGKMCNT0);  // this wave's LDS writes (the weights stay in flight)
      __builtin_amdgcn_s_barrier();
    } else {
    // Issue order: this wave's X rows, then the phase's first two weight batches; the counted wait below then covers
    // X (the oldest loads) and leaves the weights in flight.
    for (int r = wave_u; r < TB * pc * 2; r += nw) {
      const int h = r & 1, j = (r >> 1) % pc, tb = (r >> 1) / pc;
      const int t = 16 * tb + n;
      // lanes of token rows past M load nothing: their LDS slots feed only output columns that are never stored
      // (a column of the product depends only on its own token)
      if (t < p.M) {
        const uint32_t off = p.xop ? (uint32_t)(((((size_t)(ph + j) * p.xop + tb) * 2 + h) * 64 + lane) * 16)
                                   : (uint32_t)(((size_t)t * p.K + (ph + j) * 64 + 16 * g + 8 * h) * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(xs + r * 64), 16, off, 0,
                                                 0, 0);
      }
    }
    load(wa, ph, pe);
    if (pc > CPB) {
      load(wb, ph + CPB, pe);
      __builtin_amdgcn_s_waitcnt(GEMM_VMCNT(2 * CPB * WV));
    } else {
      __builtin_amdgcn_s_waitcnt(GEMM_VMCNT(CPB * WV));
    }
    __builtin_amdgcn_s_barrier();
    }
    for (int cb = ph; cb < pe; cb += 2 * CPB) {
      compute(wa, cb, ph, pc);
      if (cb + 2 * CPB < pe) load(wa, cb + 2 * CPB, pe);
      if (cb + CPB < pe) compute(wb, cb + CPB, ph, pc);
      if (cb + 3 * CPB < pe) load(wb, cb + 3 * CPB, pe);
    }
  }
  if (p.ksplit > 1) {
    // Partials [ks][M][N] fp32. With counters, the last split of the group to arrive sums all of them in split order
    // and runs the epilogue: partials are stored and loaded device-coherent (SC1), every store of a split is complete
    // (vmcnt 0, then the workgroup barrier) before its arrival is counted, and the last split's loads are issued only
    // after its own count returned ksplit - 1. It resets the counter for the next call. Without counters the reduce
    // kernel does the sum.
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        p.part, (short)0, (int)((size_t)p.ksplit * p.M * p.N * sizeof(float)), 0x00020000);
    if (live) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const int t = 16 * tb + n;
        if (t < p.M)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, acc[tb]), rp,
              (uint32_t)((((size_t)ks * p.M + t) * p.N + row0 + 4 * g) * sizeof(float)), 0, GEMM_CPOL_COHERENT);
      }
    }
    if (!p.counters) return;
    __builtin_amdgcn_s_waitcnt(GEMM_VMCNT0);
    __syncthreads();
    __shared__ int last_s;
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(p.counters + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_s = old == (uint32_t)(p.ksplit - 1);
      if (last_s) __hip_atomic_store(p.counters + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_s || (!live && !p.fuse)) return;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = min(16 * tb + n, p.M - 1);
      u32x4 v[GEMM_FIXUP_BATCH];
      f32x4 sum = {0, 0, 0, 0};
      for (int k0 = 0; k0 < p.ksplit; k0 += GEMM_FIXUP_BATCH) {
#pragma unroll
        for (int k = 0; k < GEMM_FIXUP_BATCH; ++k)
          v[k] = __builtin_amdgcn_raw_buffer_load_b128(
              rp, (uint32_t)((((size_t)min(k0 + k, p.ksplit - 1) * p.M + t) * p.N + row0 + 4 * g) * sizeof(float)), 0,
              GEMM_CPOL_COHERENT);
#pragma unroll
        for (int k = 0; k < GEMM_FIXUP_BATCH; ++k)
          if (k0 + k < p.ksplit) sum += __builtin_bit_cast(f32x4, v[k]);
      }
      acc[tb] = sum;
    }
  }
  if (p.fuse) {
    gemm_group_epilogue<TB>(p, acc, grp, wave, nw, true, lane, reinterpret_cast<float*>(xs), gemm_row_scales_f32(rsc));
    return;
  }
  if (!live) return;
  gemm_strip_out<TB>(p, acc, strip, lane, gemm_row_scales_f32(rsc));
}

// K-sliced GEMM for one workgroup of S x KW waves (S = wpg strips of 16 rows, KW = kw contiguous ranges of K): wave
// (s, k) = (wave % S, wave / S) streams strip s over range k with every weight load of the range in flight at once, the
// KW sums of a strip are added in LDS in range order by the k = 0 waves, and nothing leaves the workgroup before the
// epilogue (no split partials, no arrival counters). X: XD = false stages X^T of the band in LDS for all waves, every
// token block at once when that is at most 64 KB, else one token block (at most 64 KB) per pass with the range's
// weights held in registers (up to 4 token blocks); XD = true (TB = 1) has every wave load its own range of X straight
// into B operands. Ranges longer than CPW chunks go in batches of CPW. Chunk order inside a range, then range order,
// fixes the summation order, so results do not depend on timing.
// GS (one token block, int8 weights): per-128-column group scales (p.gscale [K/128][N]): the products of a group's two
// 64-column chunks go to a fresh accumulator that is scaled by the group's scales of the lane's 4 rows and added in group
// order (the reference applies the scale per group as well, dspark.hip:553-580). Every range and band starts on an
// even chunk (gemm_launch checks), so a batch's chunk pairs (cb + 2 j, cb + 2 j + 1) are whole groups, the second one
// absent only at the end of a range.
template <int CPW>
__device__ __forceinline__ void gscale_load(const GemmParams& p, u32x2 (&gsr)[CPW / 2], int cb, int c1, int r4) {
#pragma unroll
  for (int j = 0; j < CPW / 2; ++j) {
    const int c = min(cb + 2 * j, c1 - 1);
    gsr[j] = ldg(reinterpret_cast<const u32x2*>(p.gscale + (size_t)(c >> 1) * p.N + r4));
  }
}

// prod(i, t): t plus the products of chunk cb + i
template <int CPW, typename F>
__device__ __forceinline__ void gscale_products(f32x4& acc, const u32x2 (&gsr)[CPW / 2], int cb, int c1, F prod) {
#pragma unroll
  for (int j = 0; j < CPW / 2; ++j) {
    if (cb + 2 * j < c1) {
      f32x4 t = prod(2 * j, f32x4{0, 0, 0, 0});
      if (cb + 2 * j + 1 < c1) t = prod(2 * j + 1, t);
      const half4 sc = __builtin_bit_cast(half4, gsr[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf(t[r], (float)sc[r], acc[r]);
    }
  }
}

// LFM3_X8 (the reference's default build, dspark.hip:24-26; unit_dot_r 541-566): the GEMM input as int8 codes with one
// fp32 scale per 16-column piece, multiplied piece by piece. On v_mfma_f32_16x16x16_f16 (K = 16) one product is one
// piece: lane (g, n) gives row n's / token n's columns 16 p + 4 g .. + 3 of piece p. The weight tiles of an int8-x
// engine are laid out for it (gemm_tile_kernel, x8: byte b of lane (g, n) is column 16 (b / 4) + 4 g + b % 4 of the
// 64-column chunk, so a[p / 2] halves 4 (p % 2) .. + 3 are piece p's four weights); row-major weights (the C ABI) are
// gathered in the same order. Codes are integer-valued halves, so each product is the piece's exact integer dot
// (|dot| <= 16 * 127 * 127 < 2^24). p.x8 = 1: x is fp16 and each piece is quantized by the four lanes that hold it, as
// x_fill does (883-904): s = max(max|x| / 127, 1e-20), codes rint(x * rcp(s)); p.x8 = 2: x holds the codes (the norm
// kernel's output) and p.xsc the scales [token][K / 16].
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16x16x16(half4v a, half4v b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Token n's 4 halves of piece p of chunk c (lane (g, n)): operand-order x at p.x (xop), or row-major.
struct X8Src {
  const _Float16* base;  // this lane's first 4 halves of chunk 0, piece 0
  size_t cstride, pstride;
};
__device__ __forceinline__ X8Src x8_src(const GemmParams& p, int g, int n) {
  if (p.xop) {
    // xop_elem(n, 64 c + 16 p + 4 g + j) = (((c tbs) 2 + g / 2) 64 + 16 p + n) 8 + 4 (g % 2) + j
    return X8Src{p.x + ((size_t)(g >> 1) * 64 + n) * 8 + 4 * (g & 1), (size_t)p.xop * 1024, 128};
  }
  return X8Src{p.x + (size_t)min(n, p.M - 1) * p.K + 4 * g, 64, 16};
}

// Per-half max of two packed pairs of fp16 magnitudes: for non-negative halves the order of the bit patterns as
// unsigned integers is the order of the values.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pmax_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
// Max over the lanes n, n + 16, n + 32, n + 48 of a packed pair, by the two VALU half-wave swaps (no LDS-unit shuffle).
__device__ __forceinline__ uint32_t pmax_u16_lanes(uint32_t v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = pmax_u16(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return pmax_u16(b[0], b[1]);
}

// p.x8 == 1: quantize the lane's 4 pieces (each piece's 16 values sit in the lanes (g', n), g' = 0..3); returns the
// piece scales and turns xq into codes. max|x| is taken on the fp16 bit patterns, two pieces per packed word.
__device__ __forceinline__ f32x4 x8_quantize(u32x2 (&xq)[4]) {
  uint32_t pm[4];
#pragma unroll
  for (int pc = 0; pc < 4; ++pc) pm[pc] = pmax_u16(xq[pc][0] & 0x7fff7fffu, xq[pc][1] & 0x7fff7fffu);
  uint32_t m2[2];  // pieces 2 k (low half) and 2 k + 1 (high half)
#pragma unroll
  for (int k = 0; k < 2; ++k)
    m2[k] = pmax_u16_lanes(pmax_u16(__builtin_amdgcn_perm(pm[2 * k + 1], pm[2 * k], 0x05040100u),
                                    __builtin_amdgcn_perm(pm[2 * k + 1], pm[2 * k], 0x07060302u)));
  f32x4 sc;
#pragma unroll
  for (int pc = 0; pc < 4; ++pc) {
    half4v h = __builtin_bit_cast(half4v, xq[pc]);
    const float s = x8_piece_scale(x8_mag_value((m2[pc >> 1] >> (16 * (pc & 1))) & 0xffffu));
    const float inv = __builtin_amdgcn_rcpf(s);
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = (_Float16)rintf((float)h[j] * inv);
    xq[pc] = __builtin_bit_cast(u32x2, h);
    sc[pc] = s;
  }
  return sc;
}

// One chunk under LFM3_X8: accg[r] += dot_p[r] * xs[p] over its 4 pieces (accg: the 128-column group's sum, scaled by
// the lane's 4 rows' group scales once the group is done -- the reference scales each piece by fp32(ws * xs), one
// rounding apart).
__device__ __forceinline__ void x8_chunk(f32x4& accg, const half8 (&a)[2], const u32x2 (&xq)[4], f32x4 xs4) {
  const f32x4 z4 = {0, 0, 0, 0};
#pragma unroll
  for (int pc = 0; pc < 4; ++pc) {
    const half8 ah = a[pc >> 1];
    const half4v ap = (pc & 1) ? half4v{ah[4], ah[5], ah[6], ah[7]} : half4v{ah[0], ah[1], ah[2], ah[3]};
    const f32x4 t = mfma16x16x16(ap, __builtin_bit_cast(half4v, xq[pc]), z4);
#pragma unroll
    for (int r = 0; r < 4; ++r) accg[r] = fmaf(t[r], xs4[pc], accg[r]);
  }
}

// The gated epilogue (1) with LFM3_X8 output: h = fp16(silu(gate) up) as int8 codes + piece scales. Strip 2 i + e of
// the workgroup's strips holds output columns 16 i + 8 e .. + 7 (its rows are 8 (gate, up) pairs), so piece i is
// strips 2 i and 2 i + 1: each wave takes its 8 columns' max|h| per token, the pair meets in LDS, and each wave then
// stores its codes (strip 2 i also the scale). Every wave of the workgroup calls this (both barriers); `holder`: the
// wave holds strip `strip`'s finished sums (range 0, a live strip). ex: 16 S words of LDS no wave still reads.
__device__ __forceinline__ void gemm_gated_x8_out(const GemmParams& p, f32x4 v, int strip, int s, bool holder, int lane,
                                                  uint32_t* ex) {
  const int n = lane & 15, g = lane >> 4;
  const _Float16 y0 = f16_product(silu_f(v[0]), v[1]), y1 = f16_product(silu_f(v[2]), v[3]);  // gemm_store's values
  const uint32_t mb = pmax_u16_lanes(max(x8_mag_bits(y0), x8_mag_bits(y1)));  // lanes (g', n): token n's 8 columns
  __syncthreads();  // every wave is done with the LDS it used before
  if (holder && g == 0) ex[16 * s + n] = mb;
  __syncthreads();
  if (!holder) return;
  const float sc = x8_piece_scale(x8_mag_value(max(mb, ex[16 * (s ^ 1) + n])));
  const float inv = __builtin_amdgcn_rcpf(sc);
  const int t = n, c = strip * 8 + 2 * g;  // output columns c, c + 1 (c even: the pair is contiguous)
  if (t >= p.M) return;
  _Float16* y = p.y16 + (p.yop ? xop_elem(t, c, p.yop) : (size_t)t * (p.N / 2) + c);
  y[0] = x8_code(y0, inv);
  y[1] = x8_code(y1, inv);
  if ((strip & 1) == 0 && g == 0) p.ysc[(size_t)t * p.ysc_row + strip / 2] = sc;
}

// Token n's 4 piece scales of chunk c (p.x8 == 2).
__device__ __forceinline__ f32x4 x8_scales_load(const GemmParams& p, int n, int c) {
  return ldg(reinterpret_cast<const f32x4*>(p.xsc + (size_t)min(n, p.M - 1) * p.xsc_row + 4 * c));
}

// X8: 0 fp16 x; 1 int8 x quantized as it is loaded (p.x8 == 1); 2 int8 codes + scales given (p.x8 == 2).
// TO (int8 x): tile-major weights only -- with the row-major form also compiled in, whose chunk is four loads against
// one, the compiler cannot count a batch's loads past the layout test and waits for all of them before the first product.
template <int TB, bool I8, int CPW, bool XD, int MAXT = 1024, bool GS = false, int X8 = 0, bool ONEB = false,
          bool TO = false>
__global__ __launch_bounds__(MAXT) void gemm_sliced_kernel(GemmParams p) {
  static_assert(!GS || (TB == 1 && I8 && CPW % 2 == 0), "group scales: one token block, int8 weights, whole groups");
  static_assert(!X8 || GS, "int8 x goes with group scales");
  static_assert(!ONEB || (XD && MAXT > 512), "the one-batch form is the 1024-thread X-per-wave kernel's");
  // The stop flag is loaded first and tested once the data loads are in flight and the products computed (before
  // anything is stored), so its latency overlaps theirs; a stopped round writes nothing.
  const int run = run_flag_load(p.st);
  extern __shared__ u32x4 xs[];
  constexpr int WV = I8 ? 1 : 2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int S = p.wpg, KW = p.kw;
  const int s = wave % S, kq = wave / S;
  const int groups = (p.N / 16 + S - 1) / S;
  const int grp = blockIdx.x % groups, band = blockIdx.x / groups;  // band: a share of K (bands > 1)
  const int strips = p.N / 16;
  const int strip_raw = grp * S + s;
  const bool live = strip_raw < strips;
  const int strip = live ? strip_raw : strips - 1;
  const int row0 = strip * 16;
  const u32x2 rsc = gemm_row_scales(p, row0 + 4 * g);  // first of the kernel's loads (the epilogue's)
  __shared__ __attribute__((aligned(16))) _Float16 conv_ring_lds[CONV_RING * 16];
  __shared__ __attribute__((aligned(16))) _Float16 conv_w_lds[128];
  const bool conv_st = p.fuse == GEMM_FUSE_CONV && p.st;
  int conv_a = 0;  // the State's a, kept unread until the epilogue
  if (conv_st) {
    conv_a = state_word_load(p.st, (int)offsetof(dspark_state, a));
    conv_stage_issue(p, grp * 16, wave, nw, lane, conv_ring_lds, conv_w_lds);
  }
  const int chunks = p.K / 64;
  const int cpb_ = (chunks + p.bands - 1) / p.bands;  // chunks per band
  const int b0 = min(chunks, band * cpb_), b1 = min(chunks, b0 + cpb_);
  const int cpk = (b1 - b0 + KW - 1) / KW;
  const int c0 = min(b1, b0 + kq * cpk), c1 = min(b1, c0 + cpk);

  f32x4 acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) acc[tb] = f32x4{0, 0, 0, 0};

  const bool tiled = I8 && (TO || p.tiled);
  const uint8_t* wrow = tiled ? reinterpret_cast<const uint8_t*>(p.w) + (size_t)strip * chunks * 1024 + lane * 16
                              : reinterpret_cast<const uint8_t*>(p.w) + (size_t)(row0 + n) * p.K * (I8 ? 1 : 2) + 16 * g;
  const int cstride = tiled ? 1024 : 64;
  // chunk cb + i, clamped to the last valid chunk (a re-read of a line just fetched, discarded): the number of loads
  // issued is CPW * WV on every path, so the counted wait for X below stays exact
  auto load = [&](u32x4 (&w)[CPW][WV], int cb) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = min(cb + i, max(c1, 1) - 1);
      if (X8 && !tiled) {
        // row-major weights in the int8-x tile order: byte b = column 16 (b / 4) + 4 g + b % 4 of the chunk
        const uint8_t* rp = reinterpret_cast<const uint8_t*>(p.w) + (size_t)(row0 + n) * p.K + (size_t)c * 64 + 4 * g;
        w[i][0] = u32x4{ldg_nt(reinterpret_cast<const uint32_t*>(rp)), ldg_nt(reinterpret_cast<const uint32_t*>(rp + 16)),
                        ldg_nt(reinterpret_cast<const uint32_t*>(rp + 32)), ldg_nt(reinterpret_cast<const uint32_t*>(rp + 48))};
      } else if (I8) {
        w[i][0] = ldg_nt(reinterpret_cast<const u32x4*>(wrow + (size_t)c * cstride));
      } else {
        const u32x4* wp = reinterpret_cast<const u32x4*>(wrow + 2 * c * 64 + 16 * g);
        w[i][0] = ldg_nt(wp);
        w[i][WV - 1] = ldg_nt(wp + 1);
      }
    }
  };
  auto weights = [&](const u32x4 (&w)[WV], half8 (&a)[2]) {
    if (I8) {
      a[0] = i8x8_to_half8(w[0][0], w[0][1]);
      a[1] = i8x8_to_half8(w[0][2], w[0][3]);
    } else {
      a[0] = as_half8(w[0]);
      a[1] = as_half8(w[WV - 1]);
    }
  };
  u32x4 w[CPW][WV];
  if constexpr (XD) {
    // lane (n, g): token n (min(n, M - 1) row-major: rows past M feed only output columns that are never stored),
    // 16 B at columns 64 c + 16 g and 64 c + 16 g + 8 of chunk c; in operand order those are lane l's 16 B of the two
    // 1 KB blocks of chunk c
    const _Float16* xb0 = p.xop ? p.x + lane * 8 : p.x + (size_t)min(n, p.M - 1) * p.K + 16 * g;
    const size_t xcs = p.xop ? (size_t)p.xop * 1024 : 64, xhs = p.xop ? 512 : 8;  // halves per chunk, per half
    // One batch: its X and weight loads, then its products. The first batch is outside the loop: at a loop head the
    // compiler's wait for the previous iteration's loads would also hold the first batch back behind the flag load.
    // Token block tb of chunk c (operand order, TB > 1 needs it): the next 1 KB block pair, tb * 1024 halves on.
    auto batch = [&](int cb) {
      u32x4 xb[X8 ? 1 : CPW][TB][2];
      u32x2 xq[X8 ? CPW : 1][4];
      u32x2 gsr[GS ? CPW / 2 : 1];
      f32x4 xsl[X8 ? CPW : 1];
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int c = min(cb + i, c1 - 1);
        if constexpr (X8) {
          const X8Src xsrc = x8_src(p, g, n);
#pragma unroll
          for (int pc = 0; pc < 4; ++pc)
            xq[i][pc] = ldg(reinterpret_cast<const u32x2*>(xsrc.base + (size_t)c * xsrc.cstride + pc * xsrc.pstride));
          if (X8 == 2) xsl[i] = x8_scales_load(p, n, c);
        } else {
#pragma unroll
          for (int tb = 0; tb < TB; ++tb) {
            xb[i][tb][0] = ldg(reinterpret_cast<const u32x4*>(xb0 + (size_t)c * xcs + tb * 1024));
            xb[i][tb][1] = ldg(reinterpret_cast<const u32x4*>(xb0 + (size_t)c * xcs + tb * 1024 + xhs));
          }
        }
      }
      if constexpr (GS) gscale_load<CPW>(p, gsr, cb, c1, row0 + 4 * g);
      load(w, cb);
      // every load of the batch issued before its first product (the scheduler would otherwise reuse a consumed
      // chunk's registers for the last loads, a round trip after the first products)
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (X8) {
        f32x4 accg = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
          if (cb + i < c1) {
            half8 a[2];
            weights(w[i], a);
            const f32x4 xs4 = X8 == 2 ? xsl[i] : x8_quantize(xq[i]);
            x8_chunk(accg, a, xq[i], xs4);
          }
          // a 128-column group ends after its second chunk (or the range's last): scale it by the rows' group scales
          if ((i & 1) && cb + i - 1 < c1) {
            const half4 ws = __builtin_bit_cast(half4, gsr[i >> 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[0][r] = fmaf(accg[r], (float)ws[r], acc[0][r]);
            accg = f32x4{0, 0, 0, 0};
          }
        }
      } else if constexpr (GS) {
        gscale_products<CPW>(acc[0], gsr, cb, c1, [&](int i, f32x4 t) {
          half8 a[2];
          weights(w[i], a);
          t = mfma16x16x32(a[0], as_half8(xb[i][0][0]), t);
          return mfma16x16x32(a[1], as_half8(xb[i][0][1]), t);
        });
      } else {
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
          if (cb + i < c1) {
            half8 a[2];
            weights(w[i], a);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              acc[tb] = mfma16x16x32(a[0], as_half8(xb[i][tb][0]), acc[tb]);
              acc[tb] = mfma16x16x32(a[1], as_half8(xb[i][tb][1]), acc[tb]);
            }
          }
        }
      }
    };
    if constexpr (MAXT <= 512) {  // with 128 VGPRs (1024 threads) the peeled copy spills: keep the plain loop there
      if (c0 < c1) batch(c0);
      for (int cb = c0 + CPW; cb < c1; cb += CPW) batch(cb);
    } else if constexpr (ONEB) {
      // one batch per range (the host checked): no loop, so no loop-head waits -- counted for the back edge, they
      // would hold the batch's later weight loads behind the loads issued before it (stop flag, scales, conv staging)
      if (c0 < c1) batch(c0);
    } else {
      for (int cb = c0; cb < c1; cb += CPW) batch(cb);
    }
  } else {
    // X^T rows [tb][chunk][half] of 1 KB (lane l's 16 B at 16 l: token 16 tb + l % 16, columns 64 c + 16 (l / 16) +
    // 8 h), loaded straight into LDS by the waves in turn; then this wave's first weight batch, so the counted wait
    // covers X (the oldest loads) and leaves the weights in flight. At most 64 KB of X^T at a time: when the band's
    // X^T for every token block does not fit, the token blocks come one per pass, and the range's weights (one batch:
    // the plan keeps the range within CPW chunks) stay in registers across the passes.
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.x, (short)0, (int)((size_t)(p.xop ? 16 * p.xop : p.M) * p.K * 2), 0x00020000);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int bc = b1 - b0;  // the band's chunks: X^T rows [tb - t0][chunk - b0][half]
    const int tbp = gemm_pass_tbs(TB, cpb_);  // token blocks per stage (the host sizes LDS the same way)
    const bool all = tbp >= TB;
    auto stage = [&](int t0, int nt) {
      for (int r = wave_u; r < nt * bc * 2; r += nw) {
        const int h = r & 1, j = b0 + (r >> 1) % bc, tb = t0 + (r >> 1) / bc;
        const int t = 16 * tb + n;
        if (t < p.M) {
          const uint32_t off = p.xop ? (uint32_t)(((((size_t)j * p.xop + tb) * 2 + h) * 64 + lane) * 16)
                                     : (uint32_t)(((size_t)t * p.K + j * 64 + 16 * g + 8 * h) * 2);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(xs + r * 64), 16, off,
                                                   0, 0, 0);
        }
      }
    };
    u32x2 gsr[GS ? CPW / 2 : 1];
    // LFM3_X8 codes from the norm (p.x8 == 2): the band's piece scales go to LDS after its X^T, [chunk][token] x 16 B
    // (token t's 4 pieces of the chunk), by the same kind of loads (issued before the weights, so the counted wait
    // below covers them)
    const f32x4* xsc_lds = reinterpret_cast<const f32x4*>(xs + (size_t)(b1 - b0) * 2 * 64);
    if constexpr (X8 == 2) {
      {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.xsc, (short)0, (int)((size_t)p.M * p.xsc_row * 4), 0x00020000);
        const int bcs = b1 - b0;
        for (int r = wave_u; r < (bcs + 3) / 4; r += nw) {
          const int j = b0 + 4 * r + g;  // lane (g, n): token n's scales of chunk j
          if (n < p.M && j < b1)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(xs + (size_t)bcs * 2 * 64 + (size_t)r * 64), 16,
                (uint32_t)(((size_t)n * p.xsc_row + 4 * j) * 4), 0, 0, 0);
        }
      }
    }
    if constexpr (GS) gscale_load<CPW>(p, gsr, c0, c1, row0 + 4 * g);  // older than X: covered by the wait below
    stage(0, min(tbp, TB));
    load(w, c0);
    __builtin_amdgcn_s_waitcnt(GEMM_VMCNT(CPW * WV));
    __builtin_amdgcn_s_barrier();
    if constexpr (X8) {  // one token block, X^T of the band in LDS at once, as below
      for (int cb = c0; cb < c1; cb += CPW) {
        if (cb != c0) {
          gscale_load<CPW>(p, gsr, cb, c1, row0 + 4 * g);
          load(w, cb);
        }
        f32x4 accg = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
          if (cb + i < c1) {
            half8 a[2];
            weights(w[i], a);
            // X^T in operand order: piece p's columns 4 g .. + 3 of token n are half g / 2 of lane 16 p + n's slot,
            // halves 4 (g % 2) .. + 3
            const char* xb = reinterpret_cast<const char*>(xs + ((size_t)(cb + i - b0) * 2) * 64);
            u32x2 xq[4];
#pragma unroll
            for (int pc = 0; pc < 4; ++pc)
              xq[pc] = *reinterpret_cast<const u32x2*>(xb + (((g >> 1) * 64 + 16 * pc + n) * 16 + 8 * (g & 1)));
            // chunk j's scales of token n: 4-chunk rows of 64 lanes, row (j - b0) / 4, lane 16 ((j - b0) % 4) + n
            const int jr = cb + i - b0;
            const f32x4 xs4 = X8 == 2 ? xsc_lds[(jr >> 2) * 64 + 16 * (jr & 3) + n] : x8_quantize(xq);
            x8_chunk(accg, a, xq, xs4);
          }
          if ((i & 1) && cb + i - 1 < c1) {
            const half4 ws = __builtin_bit_cast(half4, gsr[i >> 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[0][r] = fmaf(accg[r], (float)ws[r], acc[0][r]);
            accg = f32x4{0, 0, 0, 0};
          }
        }
      }
    } else if constexpr (GS) {  // one token block, X^T of the band in LDS at once (gemm_launch checked)
      for (int cb = c0; cb < c1; cb += CPW) {
        if (cb != c0) {
          gscale_load<CPW>(p, gsr, cb, c1, row0 + 4 * g);
          load(w, cb);
        }
        gscale_products<CPW>(acc[0], gsr, cb, c1, [&](int i, f32x4 t) {
          half8 a[2];
          weights(w[i], a);
          const u32x4* xb = xs + ((size_t)(cb + i - b0) * 2) * 64;
          t = mfma16x16x32(a[0], as_half8(xb[lane]), t);
          return mfma16x16x32(a[1], as_half8(xb[64 + lane]), t);
        });
      }
    } else if (all || CPW > 8) {  // (16-chunk batches: the plan never takes passes)
      for (int cb = c0; cb < c1; cb += CPW) {
        if (cb != c0) load(w, cb);
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
          if (cb + i < c1) {
            half8 a[2];
            weights(w[i], a);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              const u32x4* xb = xs + ((size_t)(tb * bc + cb + i - b0) * 2) * 64;
              acc[tb] = mfma16x16x32(a[0], as_half8(xb[lane]), acc[tb]);
              acc[tb] = mfma16x16x32(a[1], as_half8(xb[64 + lane]), acc[tb]);
            }
          }
        }
      }
    } else if constexpr (CPW <= 8) {
      // passes of PT token blocks (static indices throughout): PT = 2 when two fit, else 1
      auto passes = [&](auto pt) {
        constexpr int PT = decltype(pt)::value;
#pragma unroll
        for (int t0 = 0; t0 < TB; t0 += PT) {
          if (t0 > 0) {
            __syncthreads();  // every wave is done with the previous pass's X^T
            stage(t0, min(PT, TB - t0));
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_s_barrier();
          }
#pragma unroll
          for (int i = 0; i < CPW; ++i) {
            if (c0 + i < c1) {
              half8 a[2];
              weights(w[i], a);
#pragma unroll
              for (int u = 0; u < PT; ++u) {
                if (t0 + u < TB) {
                  const u32x4* xb = xs + ((size_t)(u * bc + c0 + i - b0) * 2) * 64;
                  acc[t0 + u] = mfma16x16x32(a[0], as_half8(xb[lane]), acc[t0 + u]);
                  acc[t0 + u] = mfma16x16x32(a[1], as_half8(xb[64 + lane]), acc[t0 + u]);
                }
              }
            }
          }
        }
      };
      if (tbp >= 2)
        passes(std::integral_constant<int, 2>{});
      else
        passes(std::integral_constant<int, 1>{});
    }
  }
  if (!run_flag_set(run)) {  // the same for every wave
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  if (KW > 1) {
    // ranges 1 .. KW - 1 of strip s go to LDS (over X, which every wave has finished reading); the range-0 wave adds
    // them to its own sum in range order
    f32x4* red = reinterpret_cast<f32x4*>(xs);
    if (!XD) __syncthreads();
    if (kq > 0) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) red[(((kq - 1) * S + s) * TB + tb) * 64 + lane] = acc[tb];
    }
    __syncthreads();
    if (kq == 0) {
      for (int k = 1; k < KW; ++k) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[tb] += red[(((k - 1) * S + s) * TB + tb) * 64 + lane];
      }
    }
  }
  if (p.fuse) {
    ConvStage cs;  // (fields set one by one: an aggregate of LDS addresses would become a constant initializer)
    cs.ring = nullptr;
    cs.w = nullptr;
    cs.a = 0;
    if (conv_st) {
      cs.ring = conv_ring_lds;
      cs.w = conv_w_lds;
      asm volatile("" : "+v"(conv_a));
      cs.a = __builtin_amdgcn_readfirstlane(conv_a);
    }
    gemm_group_epilogue<TB>(p, acc, grp, s, S, kq == 0, lane, reinterpret_cast<float*>(xs),
                            gemm_row_scales_f32(rsc), cs);
    return;
  }
  if constexpr (GS) {
    if (p.ysc && p.epilogue == 1) {  // the gated epilogue with int8-x output (the same for every wave)
      gemm_gated_x8_out(p, acc[0], strip, s, kq == 0 && live, lane, reinterpret_cast<uint32_t*>(xs));
      return;
    }
  }
  if (kq != 0 || !live) return;
  if (p.bands > 1) {  // band b's scaled sums go to y32 + b M N (the consumer adds the bands in order)
    GemmParams q = p;
    q.y32 = p.y32 + (size_t)band * p.M * p.N;
    gemm_strip_out<TB>(q, acc, strip, lane, gemm_row_scales_f32(rsc));
    return;
  }
  gemm_strip_out<TB>(p, acc, strip, lane, gemm_row_scales_f32(rsc));
}

// Split-K reduce in index order + epilogue: one thread per 4 rows of one token, partial loads in flight in batches.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
  if (gemm_stopped(p)) return;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int groups = p.N / 4;
  if (idx >= p.M * groups) return;
  const int t = idx / groups, r = (idx % groups) * 4;
  const u32x2 rsc = gemm_row_scales(p, r);
  f32x4 v = {0, 0, 0, 0};
  for (int k0 = 0; k0 < p.ksplit; k0 += GEMM_FIXUP_BATCH) {
    f32x4 b[GEMM_FIXUP_BATCH];
#pragma unroll
    for (int k = 0; k < GEMM_FIXUP_BATCH; ++k)
      b[k] = ldg(reinterpret_cast<const f32x4*>(p.part + ((size_t)min(k0 + k, p.ksplit - 1) * p.M + t) * p.N + r));
#pragma unroll
    for (int k = 0; k < GEMM_FIXUP_BATCH; ++k)
      if (k0 + k < p.ksplit) v += b[k];
  }
  // gemm_store expects the lane's 4 rows at row0 + 4g: pass row0 = r, g = 0.
  gemm_store(p, t, r, 0, v, gemm_row_scales_f32(rsc));
}

__global__ __launch_bounds__(64) void fold_strip_keys(const uint64_t* part, int strips, uint64_t* best,
                                                      const dspark_state* st) {
  if (st && st->run == 0) return;
  const int t = blockIdx.x;
  uint64_t b = 0;
  for (int c = threadIdx.x; c < strips; c += 64) {
    const uint64_t k = part[(size_t)t * strips + c];
    b = k > b ? k : b;
  }
  b = wave_max_u64(b);
  if (threadIdx.x == 0) best[t] = b;
}

// Tile-major copy of an int8 weight [N][K]: tile (strip, chunk) = 1 KB with row n, bytes 16 g .. 16 g + 15 of the
// chunk at 16 (n + 16 g), i.e. lane l's operand at 16 l, so a wave's weight load is one contiguous 1 KB.
// x8: the int8-x order (byte b of lane (g, n) = column 16 (b / 4) + 4 g + b % 4 of the chunk: piece-major, for the
// K = 16 products of gemm_sliced_kernel's X8 path); else lane (g, n) holds columns 16 g .. + 15.
__global__ __launch_bounds__(256) void gemm_tile_kernel(const uint8_t* src, uint8_t* dst, int N, int K, int x8) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte piece of the destination
  if (i >= (size_t)N * K / 16) return;
  const int l = (int)(i % 64), n = l % 16, g = l / 16;
  const size_t tile = i / 64;
  const int chunks = K / 64;
  const size_t strip = tile / chunks;
  const int c = (int)(tile % chunks);
  const uint8_t* row = src + (strip * 16 + n) * (size_t)K + c * 64;
  u32x4 v;
  if (x8) {
#pragma unroll
    for (int pc = 0; pc < 4; ++pc) v[pc] = ldg(reinterpret_cast<const uint32_t*>(row + 16 * pc + 4 * g));
  } else {
    v = ldg(reinterpret_cast<const u32x4*>(row + 16 * g));
  }
  *reinterpret_cast<u32x4*>(dst + 16 * i) = v;
}

int gemm_tile_launch(const void* src, void* dst, int N, int K, hipStream_t s, int x8) {
  if (N < 16 || N % 16 || K < 64 || K % 64) return DSPARK_EINVAL;
  const size_t pieces = (size_t)N * K / 16;
  hipLaunchKernelGGL(gemm_tile_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), N, K, x8);
  return (int)hipGetLastError();
}

#ifndef DSPARK_GEMM_TARGET_WGS
#define DSPARK_GEMM_TARGET_WGS 192  // split K until groups x splits reach this many workgroups
#endif
#ifndef DSPARK_GEMM_MIN_CHUNKS
#define DSPARK_GEMM_MIN_CHUNKS 8  // a split keeps at least this many 64-column chunks
#endif

static size_t gemm_lds_bytes(int tb, int K, int ksplit) {
  const int chunks = K / 64, cpk = (chunks + ksplit - 1) / ksplit;
  return (size_t)tb * std::min(cpk, GEMM_PHASE_UNITS / tb) * 2048;
}

template <int TB, bool I8>
static void launch_gemm_tb(const GemmParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (p.cpb >= 8)
    hipLaunchKernelGGL((gemm_kernel<TB, I8, 8>), grid, block, lds, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<TB, I8, 4>), grid, block, lds, s, p);
}

// K-sliced launches where every wave loads its own range of X (the plan's choice; int8, one token block).
// X loaded per wave straight into B operands: one token block (row-major or operand-order X), or 2-4 token blocks in
// operand order within 8 waves
static bool gemm_sliced_xd(const GemmParams& p, bool i8) {
  return i8 && p.xd && (p.M <= 16 || (p.xop && p.M <= 64 && p.wpg * p.kw <= 8 && !p.gscale));
}

// LDS of a K-sliced launch: X^T (unless each wave loads its own), the range sums, the fused epilogue's tile.
static size_t gemm_sliced_lds_bytes(const GemmParams& p, bool i8) {
  const int tb = (p.M + 15) / 16;
  const int bands = std::max(1, p.bands);
  const int bc = (p.K / 64 + bands - 1) / bands;  // X^T of the token blocks of one pass (all of them when they fit)
  size_t x = gemm_sliced_xd(p, i8) ? 0 : (size_t)gemm_pass_tbs(tb, bc) * bc * 2048;
  if (x && p.x8 == 2) x += (size_t)(bc + 3) / 4 * 1024;  // the band's int8-x piece scales after X^T
  const size_t red = (size_t)(p.kw - 1) * p.wpg * tb * 1024;
  const size_t tile = p.fuse ? (size_t)tb * 16 * (16 * p.wpg + 4) * sizeof(float) : 0;
  const size_t ex = p.ysc && p.epilogue == 1 ? (size_t)16 * p.wpg * sizeof(uint32_t) : 0;  // gemm_gated_x8_out
  return std::max(std::max(x, ex), std::max(red, tile));
}

// Dynamic LDS above 64 KB (X^T passes of up to 128 KB): the kernel's limit is raised first (on the current device).
template <typename F>
static void allow_lds(F* kernel, size_t lds) {
  if (lds > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
}

// int8 x with group scales: X per wave (<= 8 waves) or X^T of the band through LDS; TO: tile-major weights only.
template <bool I8, int X8, bool TO>
static void launch_sliced_x8(const GemmParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (gemm_sliced_xd(p, I8)) {
    hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, true, 512, true, X8, false, TO>), grid, block, lds, s, p);
  } else {
    allow_lds(gemm_sliced_kernel<1, I8, 8, false, 1024, true, X8, false, TO>, lds);
    hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, false, 1024, true, X8, false, TO>), grid, block, lds, s, p);
  }
}

template <int TB, bool I8>
static void launch_sliced_tb(const GemmParams& p, hipStream_t s) {
  const int groups = (p.N / 16 + p.wpg - 1) / p.wpg;
  const dim3 grid(groups * p.bands), block(64 * p.wpg * p.kw);
  const size_t lds = gemm_sliced_lds_bytes(p, I8);
  const int cpk = ((p.K / 64 + p.bands - 1) / p.bands + p.kw - 1) / p.kw;  // chunks per range (of the band's)
  if constexpr (I8 && TB == 1) {
    if (p.gscale) {  // group scales: X per wave, or X^T of the band in LDS at once (gemm_launch checked)
      if (p.x8 == 1) {  // int8 x (LFM3_X8), quantized as it is loaded
        if (p.tiled) {
          launch_sliced_x8<I8, 1, true>(p, grid, block, lds, s);
        } else {
          launch_sliced_x8<I8, 1, false>(p, grid, block, lds, s);
        }
        return;
      }
      if (p.x8 == 2) {  // int8 codes + scales from the norm kernel
        if (p.tiled) {
          launch_sliced_x8<I8, 2, true>(p, grid, block, lds, s);
        } else {
          launch_sliced_x8<I8, 2, false>(p, grid, block, lds, s);
        }
        return;
      }
      if (gemm_sliced_xd(p, I8)) {
        hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, true, 512, true>), grid, block, lds, s, p);
      } else {
        allow_lds(gemm_sliced_kernel<1, I8, 8, false, 1024, true>, lds);
        hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, false, 1024, true>), grid, block, lds, s, p);
      }
      return;
    }
  }
  if constexpr (I8 && TB > 1) {
    if (gemm_sliced_xd(p, I8)) {  // X per wave for 2-4 token blocks (operand order): 4-chunk batches, <= 8 waves
      hipLaunchKernelGGL((gemm_sliced_kernel<TB, I8, 4, true, 512>), grid, block, lds, s, p);
      return;
    }
  }
  if constexpr (I8) {
    if (TB == 1 && gemm_sliced_xd(p, I8)) {
      if (block.x <= 512)  // up to 8 waves: twice the registers per wave (no spills with the first batch peeled)
        hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, true, 512>), grid, block, lds, s, p);
      else if (cpk <= 8)  // every range one batch (w13, the conv mix)
        hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, true, 1024, false, 0, true>), grid, block, lds, s, p);
      else
        hipLaunchKernelGGL((gemm_sliced_kernel<1, I8, 8, true>), grid, block, lds, s, p);
      return;
    }
    if constexpr (TB <= 2) {
      if (cpk > 8) {  // 16-chunk batches of int8 weights: 64 VGPRs (the plan keeps 3 or 4 token blocks within 8)
        allow_lds(gemm_sliced_kernel<TB, I8, 16, false>, lds);
        hipLaunchKernelGGL((gemm_sliced_kernel<TB, I8, 16, false>), grid, block, lds, s, p);
        return;
      }
    }
  }
  allow_lds(gemm_sliced_kernel<TB, I8, 8, false>, lds);
  hipLaunchKernelGGL((gemm_sliced_kernel<TB, I8, 8, false>), grid, block, lds, s, p);
}

template <bool I8>
static void launch_gemm(const GemmParams& p, hipStream_t s) {
  const int tb = (p.M + 15) / 16;
  if (p.kw > 0) {
    switch (tb) {
      case 1: launch_sliced_tb<1, I8>(p, s); break;
      case 2: launch_sliced_tb<2, I8>(p, s); break;
      case 3: launch_sliced_tb<3, I8>(p, s); break;
      default: launch_sliced_tb<4, I8>(p, s); break;
    }
    return;
  }
  const int strips = p.N / 16;
  const int groups = (strips + p.wpg - 1) / p.wpg;
  const dim3 grid(groups * p.ksplit), block(64 * p.wpg);
  size_t lds = gemm_lds_bytes(tb, p.K, p.ksplit);
  if (p.fuse) lds = std::max(lds, (size_t)tb * 16 * (16 * p.wpg + 4) * sizeof(float));
  switch (tb) {
    case 1: launch_gemm_tb<1, I8>(p, grid, block, lds, s); break;
    case 2: launch_gemm_tb<2, I8>(p, grid, block, lds, s); break;
    case 3: launch_gemm_tb<3, I8>(p, grid, block, lds, s); break;
    default: launch_gemm_tb<4, I8>(p, grid, block, lds, s); break;
  }
}

// Plan (measured per C4 shape on MI355X, 16 and 9 tokens, in HIP graphs): groups of four 16-row strips (eight for
// very wide heads, whose 512+ unsplit groups fill the CUs twice), split along K until groups x splits reach
// DSPARK_GEMM_TARGET_WGS while each split keeps DSPARK_GEMM_MIN_CHUNKS chunks, and 8-chunk weight batches when a phase
// has 16 or more chunks in groups of at most four (4-chunk batches otherwise: more workgroups per CU). No split when
// `split` is false (the fused head argmax needs whole rows).
#ifndef DSPARK_GEMM_XD_MAX_S
#define DSPARK_GEMM_XD_MAX_S 4  // groups of up to this many strips load X per wave (operand-order X) instead of via LDS
#endif
#ifndef DSPARK_GEMM_SLICED
#define DSPARK_GEMM_SLICED 1  // 0: K-sliced plans off (split-K across workgroups instead)
#endif

// K-sliced plans (measured per shape on MI355X, 16 tokens, graph-replayed): a fused epilogue fixes S and takes
// KW = 16 / S ranges; int8 GEMMs of one token block with at most 512 strips take S = 1, each wave loading its own X:
// with X in operand order 4 to 8 ranges of at least 8 chunks (2048 x 2048: 4.7 us; 2048 x 8192: 9.0 us against 10.9
// split 8 ways), with row-major X (64-byte pieces of 16 token rows per load) four ranges and only up to K = 4096;
// wider GEMMs take S = max(4, strips / 256) strips per group (at most 256 groups: 257 groups on 256 CUs measured
// 14.2 us against 10.2 for 256) and 16 / S ranges, X loaded per wave for S <= 4 with operand-order X (16384 x 2048:
// 9.6 against 10.3 us through LDS; equal at 3104 and 6144 rows, slower for S = 5 and 16), else staged in LDS once (at
// most 64 KB). Two to four token blocks (X through LDS) take the same groups, X^T in passes of two or one token blocks
// of at most 128 KB when all of them do not fit (ranges of at most 8 chunks): 33 tokens, C5 round 2.19 -> 1.95 ms
// against the split-K kernel (2.02 with 64 KB passes of one token block). Group scales (9 tokens, operand-order X) take
// the same plans, with even chunk counts per band and range, and X through LDS where X per wave would need more than 8
// waves: 128000 x 2048 50.0 us (47.6 with row scales; 63.3 with one strip and 4 ranges per workgroup), 15360 x 2048
// 10.2 (9.6), 2048 x 7680 in 2 bands 7.3 (7.0), 3072 x 2048 5.0 (5.0). Returns false when no sliced plan fits (the
// split-K plan is used; never with group scales).
static bool gemm_plan_sliced(int N, int K, int tb, bool i8, int wpg_req, bool xop, int max_bands, GemmPlan* pl,
                             bool gs = false) {
  const int strips = N / 16, chunks = K / 64;
  if ((!DSPARK_GEMM_SLICED && !gs) || tb > 4) return false;
  int S, KW, bands = 1;
  bool xdm = false;  // X per wave for 2-4 token blocks (operand-order X)
  if (wpg_req > 0) {
    S = wpg_req;
    KW = 16 / S;
  } else if (i8 && strips <= 512 && (xop || K <= 4096)) {
    S = 1;
    // fewer than 256 strips: K in bands over more workgroups when the caller adds the bands (at least 8 chunks each)
    while (bands * 2 <= max_bands && strips * bands * 2 <= 256 && chunks / (bands * 2) >= 8) bands *= 2;
    const int bc = chunks / bands;
    // ranges of at most 8 chunks: one batch per wave (row-major X with one token block: four ranges)
    KW = xop || tb > 1 ? std::min(8, std::max(4, (bc + 7) / 8)) : 4;
    if (tb > 1 && !gs) {
      // 2-4 token blocks: two strips per workgroup when that still leaves 128 or more workgroups, else shorter
      // ranges; with operand-order X every wave loads its own X (33 tokens: 6144 x 2048 21.1 us with one strip and X^T
      // staged in LDS -> 11.4 with two strips -> 9.8 with X per wave; 3104 x 2048 11.3 -> 7.3; 2048 x 8192 in two
      // bands 16.7 -> 11.1; 2048 x 2048 in two bands 7.3 -> 5.5)
      if (strips > 256 && bands == 1) {  // (256 strips: one per workgroup, 4096 x 2048 7.5 us against 9.5 with two)
        S = 2;
        KW = 4;
      } else {
        KW = std::max(KW, std::min(8, bc / 4));
      }
      xdm = xop;
    }
  } else {
    S = std::min(16, std::max(4, (strips + 255) / 256));
    KW = std::max(1, 16 / S);
    if (tb >= 3 && xop && !gs && S == 4) {  // 33 tokens, 16384 x 2048: 16.4 -> 15.2 us (17 tokens: staged X^T is better)
      KW = 2;
      xdm = true;
    }
  }
  bool xd = i8 && ((tb == 1 && (S == 1 || (xop && S <= DSPARK_GEMM_XD_MAX_S))) || xdm);
  if (gs) {
    // group scales: every band and range starts on an even chunk (whole 128-column groups); X^T of a band through LDS
    // only when it fits at once, else one strip per workgroup with X per wave
    while (bands > 1 && ((chunks + bands - 1) / bands) % 2) bands /= 2;
    const int gbc = (chunks + bands - 1) / bands;
    const bool fits = (size_t)gbc * 2048 <= GEMM_X_LDS;
    if (xd && S * KW > 8) {  // the X-per-wave kernel with group scales takes at most 8 waves (16 would spill)
      if (fits)
        xd = false;
      else
        KW = std::max(1, 8 / S);
    }
    if (!xd && !fits) {
      S = 1;
      KW = std::min(8, std::max(4, (gbc + 7) / 8));
      xd = true;
    }
    while (KW > 1 && ((gbc + KW - 1) / KW) % 2) --KW;
  }
  // X^T through LDS: all token blocks at once when they fit 64 KB, else one token block per pass, each pass's X^T
  // within 64 KB and each range within one 8-chunk batch (its weights stay in registers)
  const int bc = (chunks + bands - 1) / bands, cpk = (bc + KW - 1) / std::max(1, KW);
  const int tp = gemm_pass_tbs(tb, bc);
  if (!xd && ((size_t)tp * bc * 2048 > GEMM_X_LDS || (tp < tb && cpk > 8) || (tb > 2 && cpk > 8))) return false;
  pl->ksplit = 1;
  pl->bands = bands;
  pl->xd = xd;
  pl->wpg = S;
  pl->kw = std::max(1, std::min(KW, chunks));
  pl->cpb = 8;
  return true;
}

void gemm_plan(int M, int N, int K, bool i8, bool split, GemmPlan* pl, int wpg_req, bool xop, int max_bands, bool gs) {
  const int strips = N / 16, chunks = K / 64, tb = (M + 15) / 16;
  if (gemm_plan_sliced(N, K, tb, i8, wpg_req, xop, max_bands, pl, gs)) return;
  pl->kw = 0;
  pl->bands = 1;
  const int wpg = wpg_req > 0 ? wpg_req : (strips >= 8 * 512 ? 8 : std::min(4, std::max(1, strips)));
  const int groups = (strips + wpg - 1) / wpg;
  int ks = 1;
  if (split)
    while (groups * ks < DSPARK_GEMM_TARGET_WGS && chunks / (2 * ks) >= DSPARK_GEMM_MIN_CHUNKS && ks < 32) ks *= 2;
  const int pc = std::min((chunks + ks - 1) / ks, GEMM_PHASE_UNITS / std::max(1, std::min(4, tb)));
  pl->ksplit = ks;
  pl->wpg = wpg;
  pl->cpb = (pc >= 16 && wpg <= 4) ? 8 : 4;
}

// Split-K workspace: one fixed region of arrival counters first (GEMM_COUNTER_SLOTS u32, one per row group), then the
// partials [ks][M][N] fp32. The counters sit at the same place for every shape, so GEMMs of different shapes that share
// a workspace never write partials over each other's counters; every call leaves the counters it used at zero.
size_t gemm_ws_bytes(const GemmPlan& pl, int M, int N) {
  if (pl.ksplit <= 1) return 0;
  return GEMM_COUNTER_BYTES + (((size_t)pl.ksplit * M * N * sizeof(float) + 255) / 256) * 256;
}

size_t gemm_ws_bytes(int M, int N, int K, int wpg_req, bool xop) {
  GemmPlan pl;
  gemm_plan(M, N, K, true, true, &pl, wpg_req, xop);
  return gemm_ws_bytes(pl, M, N);
}

int gemm_groups(const GemmPlan& pl, int N) { return (N / 16 + pl.wpg - 1) / pl.wpg; }

uint32_t* gemm_ws_counters(void* ws) { return static_cast<uint32_t*>(ws); }

float* gemm_ws_partials(void* ws) { return reinterpret_cast<float*>(static_cast<char*>(ws) + GEMM_COUNTER_BYTES); }

#ifndef DSPARK_GEMM_FIXUP
#define DSPARK_GEMM_FIXUP 1  // 0: split-K partials summed by the reduce kernel even when counters are given
#endif

int gemm_launch(GemmParams& p, bool i8, hipStream_t s) {
  if ((p.xop && p.xop < (p.M + 15) / 16) || (p.yop && p.yop < (p.M + 15) / 16)) return DSPARK_EINVAL;
  // group scales: the K-sliced kernel, one token block, whole 128-column groups in every band and range, X per wave or
  // the band's X^T in LDS at once, no row scales
  if (p.x8 && (!p.gscale || p.x8 > 2 || (p.x8 == 2 && (!p.xsc || p.xsc_row < p.K / 16)))) return DSPARK_EINVAL;
  // int8-x output: the gated epilogue over whole strip pairs of one workgroup (one band), or the conv epilogue's
  // 16-channel groups (one piece each, 15 waves)
  if (p.ysc) {
    const bool gated = p.epilogue == 1 && !p.fuse && p.kw > 0 && p.wpg % 2 == 0 && p.bands <= 1 && p.N % 32 == 0 &&
                       !p.best_part && p.y16;
    const bool conv = p.fuse == GEMM_FUSE_CONV && p.wpg == 3 && p.y16;
    if (!p.gscale || (!gated && !conv) || p.ysc_row < (gated ? p.N / 32 : p.N / 48)) return DSPARK_EINVAL;
  }
  if (p.gscale) {
    if (!i8 || p.kw <= 0 || p.M > 16 || p.K % 128 || p.scale) return DSPARK_EINVAL;
    const int bands = std::max(1, p.bands), bc = (p.K / 64 + bands - 1) / bands, cpk = (bc + p.kw - 1) / p.kw;
    if ((bands > 1 && bc % 2) || cpk % 2 || (!gemm_sliced_xd(p, i8) && (size_t)bc * 2048 > GEMM_X_LDS) ||
        (gemm_sliced_xd(p, i8) && p.wpg * p.kw > 8))
      return DSPARK_EINVAL;
  }
  if (p.kw > 0) {
    // K-sliced: whole K in one workgroup of wpg x kw <= 16 waves; X^T in LDS (<= 64 KB) unless one strip per group
    const int tb = (p.M + 15) / 16;
    if (p.bands < 1) p.bands = 1;
    if (p.ksplit != 1 || p.wpg < 1 || p.wpg * p.kw > 16 || tb > 4 || gemm_sliced_lds_bytes(p, i8) > GEMM_X_LDS)
      return DSPARK_EINVAL;
    // X^T in passes (it does not fit LDS for every token block at once): each range within one batch of weights
    const int bc = (p.K / 64 + p.bands - 1) / p.bands, cpk = (bc + p.kw - 1) / p.kw;
    const int tp = gemm_pass_tbs(tb, bc);
    if (!gemm_sliced_xd(p, i8) && ((size_t)tp * bc * 2048 > GEMM_X_LDS || (tp < tb && cpk > 8) || (tb > 2 && cpk > 8)))
      return DSPARK_EINVAL;
    // bands: plain scaled sums into y32 only (each band its own [M][N]), nothing fused
    if (p.bands > 1 && (p.epilogue != 0 || !p.y32 || p.y16 || p.best_part || p.fuse || p.bands > p.K / 64))
      return DSPARK_EINVAL;
  }
  if (!DSPARK_GEMM_FIXUP) p.counters = nullptr;
  if (p.fuse && p.ksplit > 1 && !p.counters) return DSPARK_EINVAL;  // a fused epilogue needs the in-kernel fixup
  if (i8)
    launch_gemm<true>(p, s);
  else
    launch_gemm<false>(p, s);
  if (p.ksplit > 1 && !p.counters) {
    const int threads = p.M * (p.N / 4);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, p);
  }
  if (p.best_part && p.best)
    hipLaunchKernelGGL(fold_strip_keys, dim3(p.M), dim3(64), 0, s, p.best_part, p.N / 16, p.best, p.st);
  return (int)hipGetLastError();
}

}  // namespace dspark
