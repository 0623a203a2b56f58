// Verify attention over the reference's int8 K/V records, and their writer.
//
// Record format (internal/model/engine.go:30-32, kernels/ops.hip:212-251): per (position, KV head) 264 bytes,
//   K int8[128] | f32 k scale | V int8[128] | f32 v scale,
// pages of 32 positions laid out [page][slot][KV head][record] (KVBlock = 32 x KVH x 264 bytes; kv_head = 264,
// kv_slot = KVH x 264), a logical page mapped to a physical one through the block table. quantize_pair
// (ops.hip:212-224, dspark.hip:933-944): scale = max(amax / 127, 1e-6), q = x * (1 / scale) rounded half away from
// zero, clamped to [-128, 127].
//
// Attention numerics of the reference's int8 path (query_fresh, dspark.hip:1020-1035; attention_pass, 1215-1412):
//   Q int8 per 32-dim group: s_g = max(amax_g / 127, 1e-20), q8 = rint(q * rcp(s_g));
//   score (log2 units) = ks * sum_g idot_g * (s_g * log2(e) / sqrt(128)), each group's int8 dot product exact
//   (the group terms summed in order g = 0..3, where the reference sums pairs (0 + 1) + (2 + 3): an ulp of the score);
//   p = exp2(score - m); l = sum p; P = fp16(p * vs * PSCALE); acc += P * v (int8 V, exact in fp16); o = acc / PSCALE.
// The output is the softmax of those scores over the dequantized V, the reference's fp64 claim (accuracy against an
// fp64 attention of the same int8 Q/K/V, benchmarks/verify_attention.txt).
//
// gfx950 mapping. A workgroup owns one key split of every KV head (the records of a position's heads are
// interleaved, so a page is one contiguous 33 KB read): wave (h, rg) holds QB 16-row blocks of KV head h. Pages
// stream through a 3-slot LDS ring with direct-to-LDS loads; per page the workgroup first expands V into a
// transposed fp16 copy (V^T chunks in the operand order of the PV product) and gathers the page's scales, then each
// wave runs
//   S^T[keys][rows] = K8[keys][128] * Q8^T      on v_mfma_i32_16x16x32_i8, one product per 32-dim group (exact)
//   O^T[128][rows] += V^T[128][keys] * P^T      on v_mfma_f32_16x16x32_f16
// with the lazy running max of the fp16 kernels (a row's max moves only when a score passes it by more than TAU, so
// p <= 2^TAU); P is scaled by PSCALE 2^-TAU, which keeps P below the reference's bound (v scale x 4096) and rounds
// it at the same relative point. Splits write the fp16 kernels' partial format; attn_combine_kernel merges them.
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"
#include "attn_range.h"

namespace dspark {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int REC_D = 128;
constexpr int REC_BYTES = 2 * REC_D + 8;                 // 264
constexpr int REC_KVH = 4;                               // KV heads the attention kernel takes (the reference's)
constexpr int REC_PAGE = PAGE * REC_KVH * REC_BYTES;     // 33792 bytes: 33 chunks of 1 KB
constexpr int REC_CHUNKS = REC_PAGE / 1024;
constexpr int REC_BT_MAX = 1024;                         // pages per split
constexpr float REC_TAU = 8.f;
constexpr float REC_PSCALE = 4096.f / 256.f;             // 4096 x 2^-TAU
constexpr float REC_M_INIT = -1e30f;
constexpr float REC_QK_SCALE = 0.08838834764831845f * 1.4426950408889634f;  // 1/sqrt(128) x log2(e), in fp32
static_assert(REC_PAGE % 1024 == 0, "a record page is whole 1 KB chunks");

#define DSPARK_LDSP(x) ((__attribute__((address_space(3))) void*)(x))

// ---------------------------------------------------------------- record writer
// quantize_pair over one wave: lane l holds x0 = dim 2l, x1 = dim 2l + 1; stores the two int8 values at q + 2l and
// returns the scale.
__device__ __forceinline__ float rec_quantize(float x0, float x1, uint8_t* q, int lane) {
  const float scale = rec_scale(wave_max(fmaxf(fabsf(x0), fabsf(x1))));
  const float inv = __fdiv_rn(1.f, scale);
  *reinterpret_cast<uint16_t*>(q + 2 * lane) = (uint16_t)((rec_code(x0, inv) & 255) | ((rec_code(x1, inv) & 255) << 8));
  return scale;
}

// One wave per (position, KV head) of positions pos0 .. pos0 + n - 1: k, v fp32 rows [n][row_stride] holding head h at
// h * 128. A position whose table entry is outside [0, kv_pages) is not written.
__global__ __launch_bounds__(256) void kv_write_rec_kernel(const float* k, const float* v, int64_t row_stride,
                                                           uint8_t* pages, const int32_t* bt, int64_t kv_pages, int KVH,
                                                           int pos0, int n) {
  const int w = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (w >= n * KVH) return;
  const int tok = w / KVH, h = w % KVH, pos = pos0 + tok;
  const int phys = bt ? ldg(bt + pos / PAGE) : pos / PAGE;
  if (phys < 0 || phys >= kv_pages) return;
  const f32x2 kk = ldg(reinterpret_cast<const f32x2*>(k + (int64_t)tok * row_stride + h * REC_D) + lane);
  const f32x2 vv = ldg(reinterpret_cast<const f32x2*>(v + (int64_t)tok * row_stride + h * REC_D) + lane);
  uint8_t* rec = pages + (size_t)phys * ((size_t)PAGE * KVH * REC_BYTES) + ((size_t)(pos % PAGE) * KVH + h) * REC_BYTES;
  const float ks = rec_quantize(kk[0], kk[1], rec, lane);
  const float vs = rec_quantize(vv[0], vv[1], rec + REC_D + 4, lane);
  if (lane == 0) {
    *reinterpret_cast<float*>(rec + REC_D) = ks;
    *reinterpret_cast<float*>(rec + 2 * REC_D + 4) = vs;
  }
}

// ---------------------------------------------------------------- attention over records
// Q of one 16-row block: lane (n, g) holds row n's dims 32 grp + 8 g .. + 7 of each group grp, quantized per group
// (the group's 32 dims are the four lanes n, n + 16, n + 32, n + 48).
struct RecQ {
  int64_t q8[4];   // 8 int8 per group
  float qsc[4];    // group scale x 1/sqrt(128) x log2(e)
};

__device__ __forceinline__ RecQ rec_quantize_q(const u32x4 (&raw)[4]) {
  RecQ r;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const half8 hv = as_half8(raw[grp]);
    float f[8];
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f[i] = (float)hv[i];
      am = fmaxf(am, fabsf(f[i]));
    }
    am = fmaxf(am, __shfl_xor(am, 16));
    am = fmaxf(am, __shfl_xor(am, 32));
    const float s = fmaxf(__fdiv_rn(am, 127.f), 1e-20f);
    const float rc = __builtin_amdgcn_rcpf(s);
    uint64_t packed = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) packed |= (uint64_t)((uint32_t)(int)rintf(__fmul_rn(f[i], rc)) & 255u) << (8 * i);
    r.q8[grp] = (int64_t)packed;
    r.qsc[grp] = __fmul_rn(s, REC_QK_SCALE);
  }
  return r;
}

// V^T copy of a page: per head 8 chunks (dims 16 c .. + 15) of 64 lane slots of 16 bytes, lane (n, g) holding keys
// 8 g .. + 7 of dim 16 c + n, with 16 bytes of padding after every 8 slots (slot l at (l + l / 8) * 16). The PV operand
// reads stay lane-linear (conflict-free) and the expansion's 16-byte writes fall in distinct banks.
constexpr int VT_CHUNK = 64 * 16 + 8 * 16;  // 1152 bytes
__device__ __forceinline__ int vt_slot(int l) { return (l + (l >> 3)) * 16; }

// V of one page into the V^T copy, and the page's scales. Task (head hh, keys 8 g .. + 7, dims 4 dq .. + 3): eight
// 4-byte reads, an 8x4 byte transpose, widening to fp16 (v ^ 0x80 under the exponent of 1024 is 1152 + v, exact) and
// four 16-byte writes. Task bits: dq & 3, g & 1, dq >> 2, g >> 1, hh (so the 8 tasks of a write pass hit 8 bank groups).
template <int NT>
__device__ __forceinline__ void rec_expand(const char* page, char* vt, float* kvs) {
  const half2v bias = {(_Float16)1152.f, (_Float16)1152.f};
  for (int task = threadIdx.x; task < REC_KVH * 4 * 32; task += NT) {
    const int dq = (task & 3) | (((task >> 3) & 7) << 2), g = ((task >> 2) & 1) | (((task >> 6) & 1) << 1);
    const int hh = task >> 7;
    constexpr int KS = REC_KVH * REC_BYTES;  // one position on
    const char* r0 = page + ((8 * g) * REC_KVH + hh) * REC_BYTES + REC_D + 4 + 4 * dq;
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = *reinterpret_cast<const uint32_t*>(r0 + k * KS) ^ 0x80808080u;
    // dims j of keys 0-3 and 4-7: byte j of each key's word
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t* v = w + 4 * half;
      const uint32_t x01 = __builtin_amdgcn_perm(v[1], v[0], 0x05010400u), y01 = __builtin_amdgcn_perm(v[1], v[0], 0x07030602u);
      const uint32_t x23 = __builtin_amdgcn_perm(v[3], v[2], 0x05010400u), y23 = __builtin_amdgcn_perm(v[3], v[2], 0x07030602u);
      uint32_t* d = half ? hi : lo;
      d[0] = __builtin_amdgcn_perm(x23, x01, 0x05040100u);
      d[1] = __builtin_amdgcn_perm(x23, x01, 0x07060302u);
      d[2] = __builtin_amdgcn_perm(y23, y01, 0x05040100u);
      d[3] = __builtin_amdgcn_perm(y23, y01, 0x07060302u);
    }
    char* base = vt + (hh * 8 + (dq >> 2)) * VT_CHUNK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half2v a = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo[j], 0x04010400u)) - bias;
      const half2v b = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo[j], 0x04030402u)) - bias;
      const half2v c = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi[j], 0x04010400u)) - bias;
      const half2v e = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi[j], 0x04030402u)) - bias;
      const int l = 4 * (dq & 3) + j + 16 * g;
      *reinterpret_cast<u32x4*>(base + vt_slot(l)) =
          u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, c),
                __builtin_bit_cast(uint32_t, e)};
    }
  }
  for (int e = threadIdx.x; e < REC_KVH * PAGE; e += NT) {
    const int hh = e / PAGE, key = e % PAGE;
    const char* rec = page + (key * REC_KVH + hh) * REC_BYTES;
    kvs[(hh * 2) * PAGE + key] = *reinterpret_cast<const float*>(rec + REC_D);
    // v scale x PSCALE (a power of two: fp16(p * (vs * PSCALE)) = fp16(fp32(p * vs) * PSCALE) exactly)
    kvs[(hh * 2 + 1) * PAGE + key] = *reinterpret_cast<const float*>(rec + 2 * REC_D + 4) * REC_PSCALE;
  }
}

// QB row blocks per wave, NRG row groups per KV head: waves = 4 x NRG, wave w = head w / NRG, row group w % NRG
// (instantiated with QB = 1).
template <int QB, int NRG>
__global__ __launch_bounds__(REC_KVH * NRG * 64) void verify_attn_rec_kernel(AttnParams p) {
  constexpr int NW = REC_KVH * NRG, NT = NW * 64;
  constexpr int LPW = (REC_CHUNKS + NW - 1) / NW;  // page chunk loads per wave
  __shared__ __attribute__((aligned(16))) char ring0[REC_PAGE], ring1[REC_PAGE], ring2[REC_PAGE];
  __shared__ __attribute__((aligned(16))) char vt[REC_KVH * 8 * VT_CHUNK];
  __shared__ __attribute__((aligned(16))) float kvs[REC_KVH * 2 * PAGE];
  __shared__ __attribute__((aligned(16))) char trash[1024];
  __shared__ int32_t sm_bt[REC_BT_MAX];
  // Every line of the kernel arguments the prologue reads in the first round trip (the split bounds' line, 0xc0 on,
  // would otherwise be read after the State's, one more dependent miss before the block-table loads).
  asm volatile("" ::"s"(p.mix));
  if (p.st && !attn_state_range(p)) return;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = wave / NRG, rg = wave % NRG;
  const int split = blockIdx.x;
  const int R = p.nrb * 16;
  const int pb = __builtin_amdgcn_readfirstlane(p.page0 + split * p.pps);
  const int pe = __builtin_amdgcn_readfirstlane(min(pb + p.pps, p.page0 + p.npages));
  const int nsteps = pe > pb ? pe - pb : 0;
  p.full_lo = __builtin_amdgcn_readfirstlane(p.full_lo);
  p.full_hi = __builtin_amdgcn_readfirstlane(p.full_hi);
  const bool paged = p.bt != nullptr;
  if (paged) {
    for (int i = threadIdx.x; i < nsteps; i += NT) sm_bt[i] = ldg(p.bt + pb + i);
    __syncthreads();
  }

  // Q of the wave's row blocks (padding rows past G*M read the last row; the store skips them)
  constexpr bool FRESH_OK = QB == 1 && NRG <= 3;  // (the host sends a fresh block to these shapes only: 16 waves spill)
  const bool fresh = FRESH_OK && p.mix != nullptr;  // the block from the mix rows (see below)
  u32x4 qraw[QB][4];
  if (!fresh) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int r = min((rg * QB + qb) * 16 + n, p.G * p.M - 1);
      const int t = r / p.G, qh = h * p.G + r % p.G;
      const _Float16* qr = p.q + ((size_t)t * p.QH + qh) * REC_D + 8 * g;
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) qraw[qb][grp] = ldg(reinterpret_cast<const u32x4*>(qr + 32 * grp));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the Q loads stay ahead of the page loads, so waiting for Q drains no page

  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)p.kp, (short)0, (int)p.k_bytes, 0x00020000);
  // Page k of the split into `slot`: chunk c < 33 of the page goes to wave c % NW; every wave issues exactly LPW loads
  // (chunks past the page become out-of-range loads into `trash`), so the counted waits are compile-time constants.
  auto issue = [&](int k, char* slot) {
    const int phys = paged ? __builtin_amdgcn_readfirstlane(sm_bt[k]) : pb + k;
    const uint32_t base = (uint32_t)phys * (uint32_t)REC_PAGE;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int c = wave + i * NW;
      char* dst = trash;
      uint32_t off = 0x80000000u;
      if (c < REC_CHUNKS) {
        off = base + (uint32_t)c * 1024u + (uint32_t)lane * 16u;
        dst = slot + c * 1024;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, DSPARK_LDSP(dst), 16, off, 0, 0, 2);
    }
  };
  if (nsteps > 0) issue(0, ring0);
  if (nsteps > 1) issue(1, ring1);

  // Fresh block (p.mix): Q and the block's K/V records (positions a .. a + M - 1) from the attention-mix GEMM's rows,
  // the q/k norm + RoPE (+ quantize_pair for the records) done here as the q/k norm + RoPE kernel does. Loaded after
  // the first two pages are in flight (waiting for these loads waits for those pages too, which step 0 needs anyway,
  // and keeps the raw rows out of registers while the pages are issued). Fresh pair i = (token i / 4, head i % 4) of
  // this split's pages goes to wave i % NW; the records sit in registers until their page is in LDS.
  constexpr int FPW = 4;  // fresh pairs per wave at most: 4 M pairs over 4 NRG waves, M <= 4 NRG (the host checks)
  uint32_t fkq[FPW], fvq[FPW];  // lanes 0..31: the record's codes of dims l + 32 e, one byte per e
  float fks[FPW], fvs[FPW];
  int fslot[FPW], fpg[FPW];     // position's slot and page (-1: no pair)
  if (fresh) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int r = min((rg * QB + qb) * 16 + n, p.G * p.M - 1);
      const int t = r / p.G, qh = h * p.G + r % p.G;
      const float* qr = p.mix + (size_t)t * p.mix_row + (size_t)qh * REC_D + 8 * g;
      const _Float16* rt = p.rope + (size_t)(p.a + t) * REC_D + 8 * g;
      float x[4][8];
      float ss = 0.f;
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const f32x4 a0 = ldg(reinterpret_cast<const f32x4*>(qr + 32 * grp));
        const f32x4 a1 = ldg(reinterpret_cast<const f32x4*>(qr + 32 * grp + 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[grp][j] = a0[j];
          x[grp][4 + j] = a1[j];
        }
      }
      half8 w[4], cs[2], sn[2];
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) w[grp] = ldg(reinterpret_cast<const half8*>(p.q_norm + 32 * grp + 8 * g));
#pragma unroll
      for (int grp = 0; grp < 2; ++grp) {
        cs[grp] = ldg(reinterpret_cast<const half8*>(rt + 32 * grp));
        sn[grp] = ldg(reinterpret_cast<const half8*>(rt + REC_D / 2 + 32 * grp));
      }
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[grp][j] * x[grp][j];
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      const float inv = rsqrtf(ss / REC_D + p.eps);
#pragma unroll
      for (int grp = 0; grp < 4; ++grp)
#pragma unroll
        for (int j = 0; j < 8; ++j) x[grp][j] = x[grp][j] * inv * (float)w[grp][j];
#pragma unroll
      for (int grp = 0; grp < 2; ++grp)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (32 * grp + 8 * g + j < p.rot) {
            const float c = (float)cs[grp][j], s_ = (float)sn[grp][j];
            const float x0 = x[grp][j], x1 = x[grp + 2][j];
            x[grp][j] = x0 * c - x1 * s_;
            x[grp + 2][j] = x1 * c + x0 * s_;
          }
        }
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        half8 hq;
#pragma unroll
        for (int j = 0; j < 8; ++j) hq[j] = (_Float16)x[grp][j];
        qraw[qb][grp] = __builtin_bit_cast(u32x4, hq);
      }
    }
    // fresh records of this split's pages (the q/k norm + RoPE kernel's record branch, per pair)
#pragma unroll
    for (int f = 0; f < FPW; ++f) {
      fpg[f] = -1;
      const int i = wave + NW * f;
      const int t = i / REC_KVH, hh = i % REC_KVH;
      const int pos = p.a + t;
      if (t >= p.M || pos / PAGE < pb || pos / PAGE >= pe) continue;  // wave-uniform
      const float* row = p.mix + (size_t)t * p.mix_row;
      float k[4], v[4], kw[4], kc[2], ksn[2];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = (lane & 31) + 32 * e;
        k[e] = row[(size_t)(p.QH + hh) * REC_D + d];
        v[e] = row[(size_t)(p.QH + p.KVH + hh) * REC_D + d];
        kw[e] = (float)p.k_norm[d];
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int ii = (lane & 31) + 32 * e;
        kc[e] = (float)p.rope[(size_t)pos * REC_D + ii];
        ksn[e] = (float)p.rope[(size_t)pos * REC_D + REC_D / 2 + ii];
      }
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += k[e] * k[e];
      ss = (lane < 32) ? ss : 0.f;
      ss = wave_sum(ss);
      const float inv = rsqrtf(ss / REC_D + p.eps);
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = k[e] * inv * kw[e];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        if ((lane & 31) + 32 * e < p.rot) {
          const float x0 = r[e], x1 = r[e + 2];
          r[e] = x0 * kc[e] - x1 * ksn[e];
          r[e + 2] = x1 * kc[e] + x0 * ksn[e];
        }
      }
      float ak = 0.f, av = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ak = fmaxf(ak, fabsf(r[e]));
        av = fmaxf(av, fabsf(v[e]));
      }
      ak = wave_max(ak);
      av = wave_max(av);
      const float ks = rec_scale(ak), vs = rec_scale(av);
      const float ki = __fdiv_rn(1.f, ks), vi = __fdiv_rn(1.f, vs);
      uint32_t kq = 0, vq = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kq |= (uint32_t)(rec_code(r[e], ki) & 255) << (8 * e);
        vq |= (uint32_t)(rec_code(v[e], vi) & 255) << (8 * e);
      }
      fkq[f] = kq;
      fvq[f] = vq;
      fks[f] = ks;
      fvs[f] = vs;
      fslot[f] = (pos % PAGE) * REC_KVH + hh;
      fpg[f] = pos / PAGE;
    }
  }

  RecQ qv[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) qv[qb] = rec_quantize_q(qraw[qb]);
  f32x4 o[QB][8];
  float l[QB], m[QB], mneg[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int c = 0; c < 8; ++c) o[qb][c] = f32x4{0, 0, 0, 0};
    l[qb] = 0.f;
    m[qb] = REC_M_INIT;
    mneg[qb] = 0.f;
  }
  // K operand rows: key block b, row n is key 8 (n / 4) + 4 b + n % 4, so the score lanes end up holding keys
  // 8 g .. 8 g + 7 of their row, the keys of their P^T operand.
  const int kr0 = ((8 * (n >> 2) + (n & 3)) * REC_KVH + h) * REC_BYTES + 8 * g;
  const int kr1 = kr0 + 4 * REC_KVH * REC_BYTES;

  auto step = [&](int k, const char* cur, char* nxt) {
    if (k + 1 < nsteps)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPW));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();  // page k is in LDS; every wave is done with page k - 1 (its slot, vt, kvs)
    if (k + 2 < nsteps) issue(k + 2, nxt);
    // fresh records of page k into its LDS copy (stale in the pool), then a barrier
    if (fresh && p.a + p.M - 1 >= (pb + k) * PAGE && p.a < (pb + k + 1) * PAGE) {
#pragma unroll
      for (int f = 0; f < FPW; ++f) {
        if (fpg[f] == pb + k && lane < 32) {
          char* rec = const_cast<char*>(cur) + fslot[f] * REC_BYTES;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            rec[lane + 32 * e] = (char)((fkq[f] >> (8 * e)) & 255);
            rec[REC_D + 4 + lane + 32 * e] = (char)((fvq[f] >> (8 * e)) & 255);
          }
          if (lane == 0) {
            *reinterpret_cast<float*>(rec + REC_D) = fks[f];
            *reinterpret_cast<float*>(rec + 2 * REC_D + 4) = fvs[f];
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(LGKMCNT0_IMM);
      __builtin_amdgcn_s_barrier();
    }
    rec_expand<NT>(cur, vt, kvs);
    __builtin_amdgcn_s_waitcnt(LGKMCNT0_IMM);
    __builtin_amdgcn_s_barrier();
    const int page = pb + k;
    int64_t ka[2][4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      ka[0][grp] = *reinterpret_cast<const int64_t*>(cur + kr0 + 32 * grp);
      ka[1][grp] = *reinterpret_cast<const int64_t*>(cur + kr1 + 32 * grp);
    }
    const f32x4 ks0 = *reinterpret_cast<const f32x4*>(kvs + (h * 2) * PAGE + 8 * g);
    const f32x4 ks1 = *reinterpret_cast<const f32x4*>(kvs + (h * 2) * PAGE + 8 * g + 4);
    f32x4 sc[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        i32x4 ai[4];
#pragma unroll
        for (int grp = 0; grp < 4; ++grp)
          ai[grp] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka[b][grp], qv[qb].q8[grp], i32x4{0, 0, 0, 0}, 0, 0, 0);
        const f32x4 ks = b ? ks1 : ks0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float d = (float)ai[0][i] * qv[qb].qsc[0];
          d = fmaf((float)ai[1][i], qv[qb].qsc[1], d);
          d = fmaf((float)ai[2][i], qv[qb].qsc[2], d);
          d = fmaf((float)ai[3][i], qv[qb].qsc[3], d);
          sc[qb][b][i] = fmaf(d, ks[i], mneg[qb]);
        }
      }
    }
    // masks at the edges of the visible range (keys 8 g + 4 b + i of the page)
    const int base = page * PAGE;
    if (base < p.full_lo || base + PAGE - 1 > p.full_hi) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int t = min(((rg * QB + qb) * 16 + n) / p.G, p.M - 1);
        // start and the window bound the context keys only (dspark.hip:1308-1312, 2006-2012)
        const int lo = min(p.a, max(p.start, p.window > 0 ? p.a + t - p.window + 1 : 0));
        const int hi = p.causal ? p.a + t : p.a + p.M - 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k0 = base + 8 * g + i, k1 = k0 + 4;
          sc[qb][0][i] = (k0 >= lo && k0 <= hi) ? sc[qb][0][i] : -INFINITY;
          sc[qb][1][i] = (k1 >= lo && k1 <= hi) ? sc[qb][1][i] : -INFINITY;
        }
      }
    }
    // lazy running max
    float tmax[QB];
    bool need = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const f32x4 a = sc[qb][0], b = sc[qb][1];
      tmax[qb] = fmaxf(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])), fmaxf(fmaxf(b[0], b[1]), fmaxf(b[2], b[3])));
      const float thr = m[qb] == REC_M_INIT ? -INFINITY : REC_TAU;
      need = need | (tmax[qb] > thr);
    }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const bool fresh = m[qb] == REC_M_INIT;
        float rm = fmaxf(tmax[qb], __shfl_xor(tmax[qb], 16));
        rm = fmaxf(rm, __shfl_xor(rm, 32));
        if (fresh ? rm > -INFINITY : rm > REC_TAU) {
          const float alpha = fresh ? 0.f : fast_exp2(-rm);
#pragma unroll
          for (int c = 0; c < 8; ++c) o[qb][c] *= alpha;
          l[qb] *= alpha;
          m[qb] = fresh ? rm : m[qb] + rm;
          mneg[qb] = -m[qb];
          sc[qb][0] -= rm;
          sc[qb][1] -= rm;
        }
      }
    }
    const f32x4 vs0 = *reinterpret_cast<const f32x4*>(kvs + (h * 2 + 1) * PAGE + 8 * g);
    const f32x4 vs1 = *reinterpret_cast<const f32x4*>(kvs + (h * 2 + 1) * PAGE + 8 * g + 4);
    half8 pp[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = fast_exp2(sc[qb][0][i]), p1 = fast_exp2(sc[qb][1][i]);
        ps += p0 + p1;
        pp[qb][i] = (_Float16)__fmul_rn(p0, vs0[i]);
        pp[qb][4 + i] = (_Float16)__fmul_rn(p1, vs1[i]);
      }
      l[qb] += ps;
    }
    // one V^T operand at a time, shared by the row blocks
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const half8 vop = *reinterpret_cast<const half8*>(vt + (h * 8 + c) * VT_CHUNK + vt_slot(lane));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) o[qb][c] = mfma16x16x32(vop, pp[qb], o[qb][c]);
    }
  };
  for (int k = 0; k < nsteps; k += 3) {
    step(k, ring0, ring2);
    if (k + 1 < nsteps) step(k + 1, ring1, ring0);
    if (k + 2 < nsteps) step(k + 2, ring2, ring1);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  // the fresh records into the pool, for later rounds (nothing in this launch reads the pool's copy)
  if (fresh) {
#pragma unroll
    for (int f = 0; f < FPW; ++f) {
      if (fpg[f] >= 0 && lane < 32) {
        const int phys = paged ? sm_bt[fpg[f] - pb] : fpg[f];
        uint8_t* rec = reinterpret_cast<uint8_t*>(const_cast<_Float16*>(p.kp)) + (size_t)phys * REC_PAGE +
                       (size_t)fslot[f] * REC_BYTES;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          rec[lane + 32 * e] = (uint8_t)((fkq[f] >> (8 * e)) & 255);
          rec[REC_D + 4 + lane + 32 * e] = (uint8_t)((fvq[f] >> (8 * e)) & 255);
        }
        if (lane == 0) {
          *reinterpret_cast<float*>(rec + REC_D) = fks[f];
          *reinterpret_cast<float*>(rec + 2 * REC_D + 4) = fvs[f];
        }
      }
    }
  }

  // partials of this split: rows of KV head h, (max, sum) and acc / PSCALE
  // row-major partials ([head][row][split][D]; the head's region is R x S rows of D floats)
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      p.part_acc + (size_t)h * R * p.S * REC_D, (short)0, R * p.S * REC_D * (int)sizeof(float), 0x00020000);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(p.part_ml + (size_t)h * R * p.S, (short)0,
                                                                      R * p.S * (int)sizeof(f32x2), 0x00020000);
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int rb = rg * QB + qb;
    float L = l[qb] + __shfl_xor(l[qb], 16);
    L = L + __shfl_xor(L, 32);
    if (rb >= p.nrb) break;
    if (rb * 16 + n >= p.G * p.M) continue;  // padding rows: the merge never reads them
    const int ri = (rb * 16 + n) * p.S + split;
#pragma unroll
    for (int c = 0; c < 8; ++c)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[qb][c] * (1.f / REC_PSCALE)), ra,
                                             (uint32_t)((ri * REC_D + 16 * c + 4 * g) * sizeof(float)), 0, 16);
    if (g == 0)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{L > 0.f ? m[qb] : -INFINITY, L}), rm,
                                            (uint32_t)(ri * sizeof(f32x2)), 0, 16);
  }
}
#undef DSPARK_LDSP

// ---------------------------------------------------------------- host side
// One wave per (KV head, 16-row block): up to 4 row blocks per head (64 rows: 16 tokens at 4 query heads per KV head;
// the reference verifies at most 9). Measured alternatives at 128k keys: two row blocks per wave in 8 waves (the 36 rows
// of 9 tokens padded to 64) 52.0 against 45.1 us; one wave per head with all its row blocks 52.8 us.
void attn_rec_plan(AttnParams& p, int cus) {
  const int rows = p.G * p.M;
  const int nblk = (rows + 15) / 16;
  const int lo0 = std::min(p.a, std::max(p.start, p.window > 0 ? p.a - p.window + 1 : 0));  // the block's keys from a
  const int lo_last = std::max(p.start, p.window > 0 ? p.a + p.M - 1 - p.window + 1 : 0);
  const int hi_last = p.a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? p.a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  p.c = (float)(1.4426950408889634 / std::sqrt((double)REC_D));
  p.lds = 2;
  p.nrb = nblk;
  p.qb = 1;
  p.nrg = nblk;
  p.pl = p.ppl = p.lpw = 1;
  p.RG = 1;
  p.QB = 1;
  p.R = 16 * nblk;
  p.OCC = 1;
  int S = p.S;
  // One workgroup per CU (the LDS ring). A split costs ~8 us before its first page and ~1.9 us per page, so up to 96
  // pages every page gets its own split (the merge keeps its 8-lane form); beyond, two pages or more per split (4096
  // keys: 129 one-page splits took 16.8 us per layer with the merge, 65 two-page splits 16.2; 1024 keys 12.9 against
  // 14.8; reference-geometry rounds 1.448 -> 1.428 ms at 1k).
  if (S <= 0) S = p.npages <= 96 ? p.npages : std::min(cus, (p.npages + 1) / 2);
  S = std::max(S, (p.npages + REC_BT_MAX - 1) / REC_BT_MAX);
  S = std::max(1, std::min(S, std::min(ATTN_REC_MAX_SPLITS, p.npages)));
  p.pps = (p.npages + S - 1) / S;
  p.S = (p.npages + p.pps - 1) / p.pps;
}

int attn_rec_launch(AttnParams& p, int phases, hipStream_t s) {
  if (phases & 1) {
    if (p.KVH != REC_KVH || p.pps > REC_BT_MAX || p.nrb < 1 || p.nrb > 4 || p.qb * p.nrg < p.nrb) return DSPARK_EUNSUPPORTED;
    const dim3 grid(p.S);
    switch (p.qb * 10 + p.nrg) {
      case 11: hipLaunchKernelGGL((verify_attn_rec_kernel<1, 1>), grid, dim3(REC_KVH * 1 * 64), 0, s, p); break;
      case 12: hipLaunchKernelGGL((verify_attn_rec_kernel<1, 2>), grid, dim3(REC_KVH * 2 * 64), 0, s, p); break;
      case 13: hipLaunchKernelGGL((verify_attn_rec_kernel<1, 3>), grid, dim3(REC_KVH * 3 * 64), 0, s, p); break;
      case 14: hipLaunchKernelGGL((verify_attn_rec_kernel<1, 4>), grid, dim3(REC_KVH * 4 * 64), 0, s, p); break;
      default: return DSPARK_EUNSUPPORTED;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (phases & 2) return attn_launch(p, REC_D, 2, s);
  return 0;
}

int kv_write_rec_launch(const float* k, const float* v, int64_t row_stride, void* pages, const int32_t* bt,
                        int64_t kv_pages, int KVH, int pos0, int n, hipStream_t s) {
  const int64_t waves = (int64_t)n * KVH;
  if (waves == 0) return 0;
  hipLaunchKernelGGL(kv_write_rec_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, k, v, row_stride,
                     static_cast<uint8_t*>(pages), bt, kv_pages, KVH, pos0, n);
  return (int)hipGetLastError();
}

}  // namespace dspark
