// Internal launch descriptors shared between the kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

namespace dspark {

typedef float f32x2_t __attribute__((ext_vector_type(2)));

struct AttnParams {
  const _Float16* q;
  const _Float16* kp;
  const _Float16* vp;
  const int32_t* bt;
  uint32_t k_bytes, v_bytes;  // page pool sizes (range of the buffer loads; < 2 GiB)
  float* part_acc;   // [KVH][RG][S][R][D]
  f32x2_t* part_ml;  // [KVH][RG][S][R] (max, sum); max = -inf when the split saw no key of the row
  _Float16* out16;
  float* out32;
  const float* gate;
  int M, QH, KVH, G;
  int a, start, window, causal;
  int page0, npages, pps, S;  // logical page range and its split
  int RG, QB, R, OCC;         // row groups, 16-row blocks per wave, rows per group, workgroups per CU
  int full_lo, full_hi;       // pages inside [full_lo, full_hi] need no mask
  float c;                    // log2(e) / sqrt(D)
};

void attn_plan(AttnParams& p, int D, int cus);
size_t attn_workspace_bytes(const AttnParams& p, int D);
int attn_launch(AttnParams& p, int D, int phases, hipStream_t s);  // phases: 1 split pass, 2 combine, 3 both
int kv_write_launch(const void* k, const void* v, int64_t row_stride, void* kp, void* vp, const int32_t* bt, int KVH,
                    int D, int pos0, int n, hipStream_t s);

struct GemmParams {
  const _Float16* x;        // [M][K]
  const void* w;            // [N][K] biased int8 or fp16
  const _Float16* scale;    // [N] or nullptr
  float* y32;               // [M][N]
  _Float16* y16;            // [M][N] ([M][N/2] for the gated epilogue)
  float* part;              // split-K partials [ksplit][M][N]
  uint64_t* best_part;      // row-argmax keys per strip [M][N/16] (head) or nullptr
  uint64_t* best;           // [M]
  int M, N, K, ksplit, epilogue;
};

int gemm_choose_ksplit(int N, int K, int target_wgs);
size_t gemm_ws_bytes(int M, int N, int K);
int gemm_launch(GemmParams& p, bool i8, hipStream_t s);

size_t verify_argmax_ws(int M, int V);
}  // namespace dspark

struct dspark_state;
namespace dspark {
int verify_argmax_launch(const void* logits, int f16, int M, int V, const uint32_t* seen, const dspark_state* st,
                         float rep, float inv_rep, uint64_t* best, void* ws, hipStream_t s);
int accept_commit_launch(dspark_state* st, const uint64_t* best, int m, int skip_now, int32_t* out_tokens, uint32_t* seen,
                         hipStream_t s);

}  // namespace dspark
