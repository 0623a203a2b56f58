// Conv state of the gated short-conv layers at launch boundaries, and the row norm of prefill's drafter taps.
//
// The round keeps each conv layer's history in a ring of CONV_RING positions (position p at p mod CONV_RING), so a
// rejected draft's history is simply overwritten by the next round. A slot of the conv state holds, per channel c,
// the conv_k - 1 history values before a position: element (c, k) = history of position p - (conv_k - 1) + k, at
// c * (conv_k - 1) + k -- the reference's conv-state layout (internal/model/engine.go:546-547). At launch start the
// running slot is loaded into the ring (dspark.hip:2415-2431); at launch end the ring's history before the final
// position goes back to the running slot, and, when the launch passed its block boundary stop_at and a checkpoint slot
// was given, the history before stop_at goes to that slot (dspark.hip:2921-2947). A launch passes stop_at by less than
// one verify block (<= 64 positions) and the ring holds CONV_RING = 128 positions, so the positions before stop_at are
// still in the ring.
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

__device__ __forceinline__ int ring_row(int pos) { return ((pos % CONV_RING) + CONV_RING) % CONV_RING; }

// grid (layers, ceil(H / 256)); thread = channel
__global__ __launch_bounds__(256) void conv_load_kernel(ConvStateArgs a, const dspark_state* st, int slot) {
  const int li = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
  if (c >= a.H) return;
  const int p0 = st->a - a.km1;
  const _Float16* src = a.state[li] + ((size_t)slot * a.H + c) * a.km1;
  _Float16* ring = a.ring[li];
  for (int k = 0; k < a.km1; ++k) ring[(size_t)ring_row(p0 + k) * a.H + c] = src[k];
}

__global__ __launch_bounds__(256) void conv_store_kernel(ConvStateArgs a, const dspark_state* st, int slot) {
  const int li = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
  if (c >= a.H) return;
  const int a1 = st->a, stop = st->stop_at, ckpt = st->ckpt_slot;
  const _Float16* ring = a.ring[li];
  _Float16* run = a.state[li] + ((size_t)slot * a.H + c) * a.km1;
  for (int k = 0; k < a.km1; ++k) run[k] = ring[(size_t)ring_row(a1 - a.km1 + k) * a.H + c];
  if (ckpt >= 0 && ckpt < a.slots && a1 >= stop) {
    _Float16* ck = a.state[li] + ((size_t)ckpt * a.H + c) * a.km1;
    for (int k = 0; k < a.km1; ++k) ck[k] = ring[(size_t)ring_row(stop - a.km1 + k) * a.H + c];
  }
}

__global__ __launch_bounds__(256) void conv_copy_kernel(ConvStateArgs a, int src, int dst) {
  const int li = blockIdx.x;
  const size_t n = (size_t)a.H * a.km1;
  const size_t i = (size_t)blockIdx.y * 256 + threadIdx.x;
  if (i >= n) return;
  a.state[li][(size_t)dst * n + i] = a.state[li][(size_t)src * n + i];
}

// out[r] = fp16(h[r] * rsqrt(mean(h[r]^2) + eps) * w), one block per row (the reference's rms_norm of prefill taps,
// kernels/ops.hip:89-101). H % 4 == 0, H <= 8192.
__global__ __launch_bounds__(256) void rms_rows_kernel(const _Float16* h, int64_t h_stride, const _Float16* w, float eps,
                                                       int H, _Float16* out, int64_t out_stride) {
  const _Float16* x = h + (size_t)blockIdx.x * h_stride;
  constexpr int NK = 8;  // 4 columns per thread per 1024
  f32x4 v[NK];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = 1024 * k + 4 * (int)threadIdx.x;
    v[k] = f32x4{0, 0, 0, 0};
    if (i < H) {
      const half4 hv = ldg(reinterpret_cast<const half4*>(x + i));
#pragma unroll
      for (int j = 0; j < 4; ++j) v[k][j] = (float)hv[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ss += v[k][j] * v[k][j];
  }
  __shared__ float red[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float inv = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / H + eps);
  _Float16* o = out + (size_t)blockIdx.x * out_stride;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int i = 1024 * k + 4 * (int)threadIdx.x;
    if (i < H) {
      const half4 wv = ldg(reinterpret_cast<const half4*>(w + i));
      half4 y;
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = (_Float16)(v[k][j] * inv * (float)wv[j]);
      *reinterpret_cast<half4*>(o + i) = y;
    }
  }
}

int conv_load_launch(const ConvStateArgs& a, const dspark_state* st, int slot, hipStream_t s) {
  if (a.n < 1 || a.km1 < 1) return 0;
  hipLaunchKernelGGL(conv_load_kernel, dim3(a.n, (a.H + 255) / 256), dim3(256), 0, s, a, st, slot);
  return (int)hipGetLastError();
}

int conv_store_launch(const ConvStateArgs& a, const dspark_state* st, int slot, hipStream_t s) {
  if (a.n < 1 || a.km1 < 1) return 0;
  hipLaunchKernelGGL(conv_store_kernel, dim3(a.n, (a.H + 255) / 256), dim3(256), 0, s, a, st, slot);
  return (int)hipGetLastError();
}

int conv_copy_launch(const ConvStateArgs& a, int src, int dst, hipStream_t s) {
  if (a.n < 1 || a.km1 < 1) return 0;
  const size_t n = (size_t)a.H * a.km1;
  hipLaunchKernelGGL(conv_copy_kernel, dim3(a.n, (unsigned)((n + 255) / 256)), dim3(256), 0, s, a, src, dst);
  return (int)hipGetLastError();
}

int rms_rows_launch(const _Float16* h, int64_t h_stride, const _Float16* w, float eps, int H, _Float16* out,
                    int64_t out_stride, int rows, hipStream_t s) {
  if (H < 4 || H % 4 || H > 8192 || rows < 0) return DSPARK_EINVAL;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(rms_rows_kernel, dim3(rows), dim3(256), 0, s, h, h_stride, w, eps, H, out, out_stride);
  return (int)hipGetLastError();
}

}  // namespace dspark
