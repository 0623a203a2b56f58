// extern "C" entry points of libdspark_amd.so (declared in include/dspark.h). Every shape a kernel's grid and
// indexing assume is checked here, on the host, before anything is launched.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "dspark.h"
#include "dspark_internal.h"

using namespace dspark;

namespace {

constexpr int ABI_VERSION = 5;

// Compute units of the current device (queried once per device; 256 on MI355X).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

hipStream_t S(dspark_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// IEEE binary32 -> binary16, round to nearest, ties to even (the host compiler's own _Float16 conversion rounds an exact
// tie away from even, so the tables built on the host use this instead).
uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);  // NaN
  const int e = (int)(ax >> 23);
  const uint32_t mant = ax & 0x7fffffu;
  if (e >= 143) return (uint16_t)(sign | 0x7c00u);          // >= 2^16 (and infinity)
  uint32_t q, r, half;
  if (e >= 113) {                                          // a normal half (or overflow by rounding)
    q = ((uint32_t)(e - 112) << 10) | (mant >> 13);
    r = mant & 0x1fffu;
    half = 0x1000u;
  } else {                                                 // subnormal half: units of 2^-24
    const int shift = 126 - e;
    if (shift > 24) return (uint16_t)sign;
    const uint32_t m = mant | 0x800000u;
    q = m >> shift;
    r = m & ((1u << shift) - 1u);
    half = 1u << (shift - 1);
  }
  if (r > half || (r == half && (q & 1u))) ++q;  // a carry moves into the exponent, up to infinity
  return (uint16_t)(sign | q);
}

bool attn_args_ok(const dspark_attn_args* a) {
  if (!a || !a->q || !a->k_pages || !a->v_pages) return false;
  if (!a->out && !a->out_f32) return false;
  if (a->D != 64 && a->D != 128) return false;
  if (a->KVH < 1 || a->QH < a->KVH || a->QH % a->KVH != 0) return false;
  if (a->M < 1 || a->M > DSPARK_MT_MAX) return false;
  if (a->a < 0 || a->start < 0 || a->window < 0) return false;
  if (a->splits < 0) return false;
  if (a->kv_pages < 1 || a->kv_pages * a->KVH * DSPARK_PAGE_TOKENS * a->D * 2 >= (int64_t)1 << 31) return false;
  if (!a->block_table && a->kv_pages < (a->a + a->M + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS) return false;
  if ((int64_t)a->QH / a->KVH * a->M > 64 * 16) return false;  // rows per KV head
  return true;
}

AttnParams attn_params(const dspark_attn_args* a) {
  AttnParams p = {};
  p.q = static_cast<const _Float16*>(a->q);
  p.kp = static_cast<const _Float16*>(a->k_pages);
  p.vp = static_cast<const _Float16*>(a->v_pages);
  p.bt = a->block_table;
  p.k_bytes = p.v_bytes = (uint32_t)(a->kv_pages * a->KVH * DSPARK_PAGE_TOKENS * a->D * 2);
  p.out16 = static_cast<_Float16*>(a->out);
  p.out32 = a->out_f32;
  p.gate = a->gate;
  p.M = a->M;
  p.QH = a->QH;
  p.KVH = a->KVH;
  p.G = a->QH / a->KVH;
  p.a = a->a;
  p.start = a->start;
  p.window = a->window;
  p.causal = a->causal ? 1 : 0;
  p.S = a->splits;
  attn_plan(p, a->D, device_cus());
  return p;
}

}  // namespace

extern "C" {

int dspark_abi_version(void) { return ABI_VERSION; }

int dspark_rope_table(float base, int32_t pairs, int32_t head_dim, int32_t positions, uint16_t* out) {
  if (!out || !(base > 0.f) || head_dim < 2 || head_dim % 2 || pairs < 0 || pairs > head_dim / 2 || positions < 0)
    return DSPARK_EINVAL;
  const int D = head_dim;
  std::vector<float> inv(D / 2, 0.f);
  for (int i = 0; i < pairs; ++i) {
    const float ex = (float)(2 * i) / (float)D;
    inv[i] = 1.f / (float)std::pow((double)base, (double)ex);
  }
  for (int64_t p = 0; p < positions; ++p) {
    const float t = (float)p;
    for (int i = 0; i < D / 2; ++i) {
      const double f = (double)(t * inv[i]);
      out[(size_t)p * D + i] = f32_to_f16((float)std::cos(f));
      out[(size_t)p * D + D / 2 + i] = f32_to_f16((float)std::sin(f));
    }
  }
  return 0;
}
int dspark_page_tokens(void) { return DSPARK_PAGE_TOKENS; }
int dspark_max_tokens(void) { return DSPARK_MT_MAX; }
int dspark_state_bytes(void) { return (int)sizeof(dspark_state); }

size_t dspark_verify_attention_workspace(const dspark_attn_args* a) {
  if (!a || a->M < 1 || a->M > DSPARK_MT_MAX || a->KVH < 1 || a->QH < a->KVH || (a->D != 64 && a->D != 128)) return 0;
  dspark_attn_args b = *a;
  if (!b.q) b.q = b.k_pages = b.v_pages = b.out = reinterpret_cast<void*>(1);  // size only
  if (b.kv_pages == 0) b.kv_pages = (b.a + b.M + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS;
  if (!attn_args_ok(&b)) return 0;
  AttnParams p = attn_params(&b);
  return attn_workspace_bytes(p, a->D);
}

static int verify_attention_phases(const dspark_attn_args* a, int phases, dspark_stream_t stream) {
  if (!attn_args_ok(a)) return DSPARK_EINVAL;
  AttnParams p = attn_params(a);
  const size_t need = attn_workspace_bytes(p, a->D);
  if (!a->workspace || a->workspace_bytes < need) return DSPARK_ENOSPACE;
  attn_bind_workspace(p, a->D, a->workspace);
  return attn_launch(p, a->D, phases, S(stream));
}

int dspark_verify_attention(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_phases(a, 3, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- verify attention without an allocation
// The split partials of dspark_verify_attention_noalloc live in this file-scope device array (each GPU the library runs
// on holds its own copy until the process ends). Host code never passes the array's name to a kernel: on the host it
// is only a stand-in, not a device address; the device address of each GPU's copy comes from hipGetSymbolAddress,
// looked up once per device (with that device current) and kept below.
static __device__ __align__(256) char scratch[DSPARK_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[NOALLOC_MAX_DEVICES] = {nullptr};

// The current device's copy of `scratch` (nullptr if the lookup failed).
void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}
}  // namespace

extern "C" {

int dspark_verify_attention_noalloc(const dspark_attn_args* a, dspark_stream_t stream) {
  if (!attn_args_ok(a)) return DSPARK_EINVAL;
  AttnParams p = attn_params(a);
  if (attn_workspace_bytes(p, a->D) > (size_t)DSPARK_NOALLOC_SCRATCH_BYTES) return DSPARK_ENOSPACE;
  void* ws = scratch_for_current_device();
  if (!ws) return DSPARK_EUNSUPPORTED;
  attn_bind_workspace(p, a->D, ws);
  return attn_launch(p, a->D, 3, S(stream));
}
int dspark_verify_attention_splits(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_phases(a, 1, stream);
}
int dspark_verify_attention_combine(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_phases(a, 2, stream);
}

int dspark_kv_write(const void* k, const void* v, int64_t row_stride, void* k_pages, void* v_pages,
                    const int32_t* block_table, int64_t kv_pages, int32_t KVH, int32_t D, int32_t pos0, int32_t n,
                    dspark_stream_t stream) {
  if (!k || !v || !k_pages || !v_pages) return DSPARK_EINVAL;
  if ((D != 64 && D != 128) || KVH < 1 || pos0 < 0 || n < 0 || row_stride < (int64_t)KVH * D || row_stride % 8 != 0)
    return DSPARK_EINVAL;
  if (kv_pages < 1 || (int64_t)pos0 + n > ((int64_t)1 << 31) - DSPARK_PAGE_TOKENS) return DSPARK_EINVAL;
  if (!block_table && ((int64_t)pos0 + n + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS > kv_pages) return DSPARK_EINVAL;
  return kv_write_launch(k, v, row_stride, k_pages, v_pages, block_table, kv_pages, KVH, D, pos0, n, S(stream));
}

// ---------------------------------------------------------------- int8 K/V records
static bool rec_args_ok(const dspark_attn_args* a) {
  if (!a || !a->q || !a->k_pages || a->v_pages) return false;
  if (!a->out && !a->out_f32) return false;
  if (a->D != 128 || a->KVH != 4 || a->QH < a->KVH || a->QH % a->KVH != 0) return false;
  if (a->M < 1 || a->M > DSPARK_MT_MAX || (int64_t)a->QH / a->KVH * a->M > 4 * 16) return false;
  if (a->a < 0 || a->start < 0 || a->window < 0) return false;
  if (a->splits < 0) return false;
  if (a->kv_pages < 1 || a->kv_pages * DSPARK_PAGE_TOKENS * a->KVH * DSPARK_REC_BYTES >= (int64_t)1 << 31) return false;
  if (!a->block_table && a->kv_pages < (a->a + a->M + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS) return false;
  return true;
}

static AttnParams rec_params(const dspark_attn_args* a) {
  AttnParams p = {};
  p.q = static_cast<const _Float16*>(a->q);
  p.kp = static_cast<const _Float16*>(a->k_pages);
  p.bt = a->block_table;
  p.k_bytes = (uint32_t)(a->kv_pages * DSPARK_PAGE_TOKENS * a->KVH * DSPARK_REC_BYTES);
  p.out16 = static_cast<_Float16*>(a->out);
  p.out32 = a->out_f32;
  p.gate = a->gate;
  p.M = a->M;
  p.QH = a->QH;
  p.KVH = a->KVH;
  p.G = a->QH / a->KVH;
  p.a = a->a;
  p.start = a->start;
  p.window = a->window;
  p.causal = a->causal ? 1 : 0;
  p.S = a->splits;
  attn_rec_plan(p, device_cus());
  return p;
}

size_t dspark_verify_attention_rec_workspace(const dspark_attn_args* a) {
  if (!a) return 0;
  dspark_attn_args b = *a;
  if (!b.q) {  // size only
    b.q = b.k_pages = b.out = reinterpret_cast<void*>(1);
    b.v_pages = nullptr;
  }
  if (b.kv_pages == 0) b.kv_pages = (b.a + b.M + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS;
  if (!rec_args_ok(&b)) return 0;
  AttnParams p = rec_params(&b);
  return attn_workspace_bytes(p, 128);
}

static int verify_attention_rec_phases(const dspark_attn_args* a, int phases, dspark_stream_t stream) {
  if (!rec_args_ok(a)) return DSPARK_EINVAL;
  AttnParams p = rec_params(a);
  const size_t need = attn_workspace_bytes(p, 128);
  if (!a->workspace || a->workspace_bytes < need) return DSPARK_ENOSPACE;
  attn_bind_workspace(p, 128, a->workspace);
  return attn_rec_launch(p, phases, S(stream));
}

int dspark_verify_attention_rec(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_rec_phases(a, 3, stream);
}
int dspark_verify_attention_rec_splits(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_rec_phases(a, 1, stream);
}
int dspark_verify_attention_rec_combine(const dspark_attn_args* a, dspark_stream_t stream) {
  return verify_attention_rec_phases(a, 2, stream);
}

int dspark_kv_write_rec(const float* k, const float* v, int64_t row_stride, void* pages, const int32_t* block_table,
                        int64_t kv_pages, int32_t KVH, int32_t pos0, int32_t n, dspark_stream_t stream) {
  if (!k || !v || !pages) return DSPARK_EINVAL;
  if (KVH < 1 || pos0 < 0 || n < 0 || row_stride < (int64_t)KVH * 128 || row_stride % 2 != 0) return DSPARK_EINVAL;
  if (kv_pages < 1 || (int64_t)pos0 + n > ((int64_t)1 << 31) - DSPARK_PAGE_TOKENS) return DSPARK_EINVAL;
  if ((int64_t)n * KVH > ((int64_t)1 << 31) - 4) return DSPARK_EINVAL;
  if (!block_table && ((int64_t)pos0 + n + DSPARK_PAGE_TOKENS - 1) / DSPARK_PAGE_TOKENS > kv_pages) return DSPARK_EINVAL;
  return kv_write_rec_launch(k, v, row_stride, pages, block_table, kv_pages, KVH, pos0, n, S(stream));
}

size_t dspark_verify_argmax_workspace(int32_t M, int32_t V) {
  if (M < 1 || M > DSPARK_MT_MAX || V < 1) return 0;
  return verify_argmax_ws(M, V);
}

int dspark_verify_argmax(const void* logits, int32_t logits_f16, int32_t M, int32_t V, const uint32_t* seen,
                         const dspark_state* st, float rep, float inv_rep, uint64_t* best_keys, void* workspace,
                         size_t workspace_bytes, dspark_stream_t stream) {
  if (!logits || !seen || !st || !best_keys || M < 1 || M > DSPARK_MT_MAX || V < 1) return DSPARK_EINVAL;
  if (!workspace || workspace_bytes < verify_argmax_ws(M, V)) return DSPARK_ENOSPACE;
  return verify_argmax_launch(logits, logits_f16, M, V, seen, st, rep, inv_rep, best_keys, workspace, S(stream));
}

int dspark_accept_commit(dspark_state* st, const uint64_t* best_keys, int32_t M, int32_t skip_now, int32_t* out_tokens,
                         int32_t out_cap, uint32_t* seen, dspark_stream_t stream) {
  if (!st || !best_keys || !out_tokens || !seen || M < 1 || M > DSPARK_MT_MAX || out_cap < M) return DSPARK_EINVAL;
  return accept_commit_launch(st, best_keys, M, skip_now, out_tokens, out_cap, seen, S(stream));
}

size_t dspark_gemm_i8_workspace(int32_t M, int32_t N, int32_t K) {
  if (M < 1 || M > 64 || N < 16 || N % 16 || K < 64 || K % 64) return 0;
  return gemm_ws_bytes(M, N, K);
}

int dspark_gemm_i8(const void* x, int32_t M, int32_t K, const uint8_t* w, const void* scale, int32_t N,
                   int32_t epilogue, float* y_f32, void* y_f16, void* workspace, size_t workspace_bytes,
                   dspark_stream_t stream) {
  if (!x || !w || !scale || M < 1 || M > 64 || N < 16 || N % 16 || K < 64 || K % 64) return DSPARK_EINVAL;
  if (epilogue < 0 || epilogue > 2) return DSPARK_EINVAL;
  if (epilogue == 0 && !y_f32 && !y_f16) return DSPARK_EINVAL;
  if (epilogue != 0 && !y_f16) return DSPARK_EINVAL;
  GemmParams p = {};
  p.x = static_cast<const _Float16*>(x);
  p.w = w;
  p.scale = static_cast<const _Float16*>(scale);
  p.y32 = epilogue == 0 ? y_f32 : nullptr;
  p.y16 = static_cast<_Float16*>(y_f16);
  p.M = M;
  p.N = N;
  p.K = K;
  p.epilogue = epilogue;
  GemmPlan pl;
  gemm_plan(M, N, K, true, true, &pl);
  p.ksplit = pl.ksplit;
  p.wpg = pl.wpg;
  p.cpb = pl.cpb;
  p.kw = pl.kw;
  p.xd = pl.xd;
  if (p.ksplit > 1) {
    if (gemm_groups(pl, N) > GEMM_COUNTER_SLOTS) return DSPARK_EINVAL;
    if (!workspace || workspace_bytes < gemm_ws_bytes(pl, M, N)) return DSPARK_ENOSPACE;
    p.part = gemm_ws_partials(workspace);
    p.counters = gemm_ws_counters(workspace);
  }
  return gemm_launch(p, true, S(stream));
}

int dspark_gemm_i8_g128(const void* x, int32_t M, int32_t K, const uint8_t* w, const void* gscale, int32_t N,
                        int32_t epilogue, float* y_f32, void* y_f16, dspark_stream_t stream) {
  if (!x || !w || !gscale || M < 1 || M > 16 || N < 16 || N % 16 || K < 128 || K % 128) return DSPARK_EINVAL;
  if (epilogue < 0 || epilogue > 2) return DSPARK_EINVAL;
  if (epilogue == 0 && !y_f32 && !y_f16) return DSPARK_EINVAL;
  if (epilogue != 0 && !y_f16) return DSPARK_EINVAL;
  GemmParams p = {};
  p.x = static_cast<const _Float16*>(x);
  p.w = w;
  p.gscale = static_cast<const _Float16*>(gscale);
  p.y32 = epilogue == 0 ? y_f32 : nullptr;
  p.y16 = static_cast<_Float16*>(y_f16);
  p.M = M;
  p.N = N;
  p.K = K;
  p.epilogue = epilogue;
  GemmPlan pl;
  gemm_plan(M, N, K, true, false, &pl, 0, false, 1, true);
  p.ksplit = pl.ksplit;
  p.wpg = pl.wpg;
  p.cpb = pl.cpb;
  p.kw = pl.kw;
  p.xd = pl.xd;
  return gemm_launch(p, true, S(stream));
}

int dspark_gemm_i8_g128_x8(const void* x, const float* xscale, int32_t M, int32_t K, const uint8_t* w,
                           const void* gscale, int32_t N, int32_t epilogue, float* y_f32, void* y_f16,
                           dspark_stream_t stream) {
  if (!x || !w || !gscale || M < 1 || M > 16 || N < 16 || N % 16 || K < 128 || K % 128) return DSPARK_EINVAL;
  if (epilogue < 0 || epilogue > 2) return DSPARK_EINVAL;
  if (epilogue == 0 && !y_f32 && !y_f16) return DSPARK_EINVAL;
  if (epilogue != 0 && !y_f16) return DSPARK_EINVAL;
  GemmParams p = {};
  p.x = static_cast<const _Float16*>(x);
  p.w = w;
  p.gscale = static_cast<const _Float16*>(gscale);
  p.y32 = epilogue == 0 ? y_f32 : nullptr;
  p.y16 = static_cast<_Float16*>(y_f16);
  p.M = M;
  p.N = N;
  p.K = K;
  p.epilogue = epilogue;
  p.x8 = xscale ? 2 : 1;
  p.xsc = xscale;
  p.xsc_row = K / 16;
  GemmPlan pl;
  gemm_plan(M, N, K, true, false, &pl, 0, false, 1, true);
  p.ksplit = pl.ksplit;
  p.wpg = pl.wpg;
  p.cpb = pl.cpb;
  p.kw = pl.kw;
  p.xd = pl.xd;
  return gemm_launch(p, true, S(stream));
}

int dspark_g128_scales(const uint16_t* packed, int32_t N, int32_t K, uint16_t* out) {
  // weights.Pack stores group g's scale only while g / 4 < groups / 4 (quant.go:96-99): K % 512 != 0 leaves trailing
  // groups without a stored scale, so such a K has no packed layout to convert
  if (!packed || !out || N < 1 || K < 512 || K % 512) return DSPARK_EINVAL;
  const int groups = K / 128, srow = (K / 512 == 4) ? 16 : 64, sq = srow / 4;
  if ((groups + 3) / 4 > sq) return DSPARK_EINVAL;  // more groups than the packed row holds
  for (int r = 0; r < N; ++r)
    for (int g = 0; g < groups; ++g) out[(size_t)g * N + r] = packed[(size_t)r * srow + (g % 4) * sq + g / 4];
  return 0;
}

size_t dspark_head_argmax_workspace(int32_t M, int32_t N) {
  if (M < 1 || M > 64 || N < 16 || N % 16) return 0;
  return (size_t)M * (N / 16) * sizeof(uint64_t);
}

int dspark_head_argmax_f16(const void* x, int32_t M, int32_t K, const void* w, int32_t N, float* y_f32,
                           uint64_t* best_keys, void* workspace, size_t workspace_bytes, dspark_stream_t stream) {
  if (!x || !w || !best_keys || M < 1 || M > 64 || N < 16 || N % 16 || K < 64 || K % 64) return DSPARK_EINVAL;
  if (!workspace || workspace_bytes < dspark_head_argmax_workspace(M, N)) return DSPARK_ENOSPACE;
  GemmParams p = {};
  p.x = static_cast<const _Float16*>(x);
  p.w = w;
  p.scale = nullptr;
  p.y32 = y_f32;
  p.M = M;
  p.N = N;
  p.K = K;
  GemmPlan pl;
  gemm_plan(M, N, K, false, false, &pl);
  p.ksplit = pl.ksplit;
  p.wpg = pl.wpg;
  p.cpb = pl.cpb;
  p.kw = pl.kw;
  p.xd = pl.xd;
  p.best_part = static_cast<uint64_t*>(workspace);
  p.best = best_keys;
  return gemm_launch(p, false, S(stream));
}

}  // extern "C"
