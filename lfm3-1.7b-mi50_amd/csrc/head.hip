// Greedy verify argmax over logits and the round's acceptance + commit, on the device State.
//
// verify_argmax: one block per (token, vocab chunk) folds the penalised fp16-rounded logits into the argmax key
// (ordered bits << 32 | 0xFFFFFFFF - index), the second kernel folds the chunks per token. Integer max is order-free,
// so the result is bit-identical run to run. Reference: head_run<false, M> (dspark.hip:2219-2318), argmax_key
// (967-971), penalty sign rule (internal/sample/sample.go:75-90; kernel form multiplies by the host's 1/rep,
// internal/model/dspark.go:575-578).
//
// accept_commit: the books of dspark.hip:2848-2913 on one wave.
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

constexpr int ARGMAX_CHUNK = 4096;  // logits per block

template <bool F16, bool A4>
__global__ __launch_bounds__(256) void verify_argmax_partial(const void* logits, int M, int V, const uint32_t* seen,
                                                             const dspark_state* st, float rep, float inv_rep,
                                                             const float* rep_dev, uint64_t* part, int nchunks) {
  const int run = run_flag_load(st);  // tested once the logit loads are in flight
  const int t = blockIdx.y, chunk = blockIdx.x;
  // Four consecutive logits per thread per 1024 (one seen word covers them). Every load of the chunk is issued before
  // the first is used: addresses are clamped to the last logit (no branches for the compiler to wait at); positions
  // past the chunk are dropped when the keys are formed. A4: V % 4 == 0, rows 16-byte aligned (vector loads).
  constexpr int NK = ARGMAX_CHUNK / 1024;
  const int r0 = chunk * ARGMAX_CHUNK, r1 = min(V, r0 + ARGMAX_CHUNK);
  float lv[NK][4];
  uint32_t sw[NK];
  const float* l32 = reinterpret_cast<const float*>(logits) + (size_t)t * V;
  const _Float16* l16 = reinterpret_cast<const _Float16*>(logits) + (size_t)t * V;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int rb = r0 + 1024 * k + 4 * (int)threadIdx.x;
    sw[k] = ldg(seen + (min(rb, V - 1) >> 5));
    if constexpr (A4) {
      const int rc = min(rb, V - 4);
      if constexpr (F16) {
        const half4 h = ldg(reinterpret_cast<const half4*>(l16 + rc));
#pragma unroll
        for (int i = 0; i < 4; ++i) lv[k][i] = (float)h[i];
      } else {
        const f32x4 f = ldg(reinterpret_cast<const f32x4*>(l32 + rc));
#pragma unroll
        for (int i = 0; i < 4; ++i) lv[k][i] = (float)(_Float16)f[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rc = min(rb + i, V - 1);
        lv[k][i] = F16 ? (float)ldg(l16 + rc) : (float)(_Float16)ldg(l32 + rc);
      }
    }
  }
  if (rep_dev) {  // {rep, 1/rep} in device memory (the reference's g.rep / g.inv_rep, dspark.go:575-578)
    rep = rep_dev[0];
    inv_rep = rep_dev[1];
  }
  // Drafts 1..t that were not seen before this round count as seen for this position (dspark.hip:2226-2232). Lane j
  // of wave 0 looks up draft j; a draft outside the vocabulary matches no logit (and is not looked up in seen).
  __shared__ int dt[DSPARK_MT_MAX];
  __shared__ uint64_t isnew_s;
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    bool fresh = false;
    if (j >= 1 && j <= t && j < M) {
      const int d = st->tokens[j];
      dt[j] = d;
      fresh = d >= 0 && d < V && ((seen[d >> 5] >> (d & 31)) & 1u) == 0;
    }
    const uint64_t bits = __ballot(fresh);
    if (j == 0) isnew_s = bits;
  }
  __syncthreads();
  const uint64_t isnew = isnew_s;
  // the stop flag is tested after the barrier: memory operations do not move across it, so the logit loads above stay
  // ahead of the flag's wait (tested before them, the compiler sinks them below the test); a stopped round writes
  // nothing
  if (!run_flag_set(run)) {
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  uint64_t best = 0;
  // Fresh drafts that fall on this thread's logits: one pass over the drafts (bit 4k + i = logit rb_k + i).
  uint32_t fresh = 0;
  for (uint64_t m = isnew; m; m &= m - 1) {
    const int e = dt[__builtin_ctzll(m)] - r0;
    if (e >= 0 && e < ARGMAX_CHUNK && ((e & 1023) >> 2) == (int)threadIdx.x) fresh |= 1u << (4 * (e >> 10) + (e & 3));
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int rb = r0 + 1024 * k + 4 * (int)threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb + i;
      if (r < r1) {
        const bool hit = (((sw[k] >> (r & 31)) | (fresh >> (4 * k + i))) & 1u) != 0;
        const float vr = lv[k][i];
        const float pv = hit ? (vr > 0.f ? vr * inv_rep : vr * rep) : vr;
        const uint64_t key = argmax_key(pv, (uint32_t)r);
        best = key > best ? key : best;
      }
    }
  }
  best = wave_max_u64(best);
  __shared__ uint64_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int w = 1; w < 4; ++w) b = red[w] > b ? red[w] : b;
    part[(size_t)t * nchunks + chunk] = b;
  }
}

__global__ __launch_bounds__(64) void fold_keys(const uint64_t* part, int nchunks, uint64_t* best, const dspark_state* st) {
  if (st->run == 0) return;
  const int t = blockIdx.x;
  uint64_t b = 0;
  for (int c = threadIdx.x; c < nchunks; c += 64) {
    const uint64_t k = part[(size_t)t * nchunks + c];
    b = k > b ? k : b;
  }
  b = wave_max_u64(b);
  if (threadIdx.x == 0) best[t] = b;
}

__device__ __forceinline__ int key_token(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }

// part (optional): the verify argmax's partial keys [mfold][nchunks], folded here into best[t] first (every thread
// loads its share at once; u64 max in LDS, order-free) instead of by a separate fold_keys launch.
// mirror (optional): host memory the launch loop polls; after the books, words 1.. get the State's run, a, count,
// rounds_left, skip, miss, accepted, verified, and words 0 (last, release) and 15 (first) the State's rounds_done, so
// a reader that finds word 15 == word 0 has read one round's values (system-scope stores: visible to the host).
__global__ __launch_bounds__(64) void accept_commit_kernel(dspark_state* st, uint64_t* best, int m, int skip_now,
                                                           int32_t* out_tokens, int out_cap, uint32_t* seen,
                                                           const uint64_t* part, int nchunks, int mfold,
                                                           int32_t* mirror) {
  // The run word and the first batch of partial keys are requested together, and the keys are folded into LDS before
  // run is tested (an early return ahead of the folding let the compiler move the key loads behind the State's round
  // trip). Buffer loads: 0 -- no key -- past the keys, and for every load when there are none. A stopped round writes
  // nothing.
  const int run = run_flag_load(st);
  const int n = part ? mfold * nchunks : 0;
  constexpr int PB = 8;
  const __amdgpu_buffer_rsrc_t rp =
      __builtin_amdgcn_make_buffer_rsrc((void*)part, (short)0, n * (int)sizeof(uint64_t), 0x00020000);
  u32x2 v0[PB];
#pragma unroll
  for (int i = 0; i < PB; ++i)
    v0[i] = __builtin_amdgcn_raw_buffer_load_b64(rp, (64 * i + (int)threadIdx.x) * (int)sizeof(uint64_t), 0, 0);
  if (part) {
    __shared__ unsigned long long sb[64];
    sb[threadIdx.x] = 0;
    __syncthreads();
    for (int e0 = 0; e0 < n; e0 += 64 * PB) {
      uint64_t v[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i)
        v[i] = e0 == 0 ? __builtin_bit_cast(uint64_t, v0[i]) : ldg(part + min(e0 + 64 * i + (int)threadIdx.x, n - 1));
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int e = e0 + 64 * i + (int)threadIdx.x;
        if (e < n) atomicMax(&sb[e / nchunks], (unsigned long long)v[i]);
      }
    }
    __syncthreads();
    if (threadIdx.x != 0 || !run_flag_set(run)) return;
    for (int t = 0; t < mfold; ++t) best[t] = sb[t];  // the folded keys (thread 0 reads its own writes below)
  }
  if (threadIdx.x != 0 || !run_flag_set(run)) return;
  if (m <= 0) m = st->M;  // rounds that drafted on the device: the verified count is in the State
  int acc = 0;
  for (int t = 0; t < m - 1; ++t) {
    if (key_token(best[t]) != st->tokens[t + 1]) break;
    ++acc;
  }
  const int commit = acc + 1;
  const int bonus = key_token(best[acc]);
  const int aa = st->a;
  int count = st->count;
  if (count < 0 || count + commit > out_cap) {  // no room for the commit: write nothing and stop
    st->run = 0;
    return;
  }
  for (int i = 1; i <= acc; ++i) out_tokens[count++] = st->tokens[i];
  out_tokens[count++] = bonus;
  for (int i = 1; i <= acc; ++i) {
    const int tk = st->tokens[i];
    seen[tk >> 5] |= 1u << (tk & 31);
  }
  seen[bonus >> 5] |= 1u << (bonus & 31);
  bool stop = false;
  if (st->eos >= 0)
    for (int i = count - commit; i < count; ++i) stop = stop || out_tokens[i] == st->eos;
  st->count = count;
  st->ctx_new = commit;
  st->ctx_pos = aa;
  st->a = aa + commit;
  st->anchor = bonus;
  st->accepted += acc;
  st->verified += m;
  if (skip_now > 0) {
    st->skip -= 1;
  } else if (acc == 0) {
    st->miss += 1;
    if (st->skip_after > 0 && st->miss >= st->skip_after) {
      st->skip = st->skip_rounds;
      st->miss = 0;
    }
  } else {
    st->miss = 0;
  }
  st->tokens[0] = bonus;
  st->rounds_done += 1;
  st->rounds_left -= 1;
  st->run = (!stop && st->rounds_left > 0 && st->a < st->stop_at && count < st->budget) ? 1 : 0;
  if (mirror) {
    const int seq = st->rounds_done;
    const int words[8] = {st->run, st->a, st->count, st->rounds_left, st->skip, st->miss, st->accepted, st->verified};
    __hip_atomic_store(mirror + 15, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __atomic_thread_fence(__ATOMIC_RELEASE);  // word 15 before the values
#pragma unroll
    for (int i = 0; i < 8; ++i) __hip_atomic_store(mirror + 1 + i, words[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(mirror, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

size_t verify_argmax_ws(int M, int V) {
  const int nchunks = (V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
  return (size_t)M * nchunks * sizeof(uint64_t);
}

int verify_argmax_launch(const void* logits, int f16, int M, int V, const uint32_t* seen, const dspark_state* st,
                         float rep, float inv_rep, uint64_t* best, void* ws, hipStream_t s, const float* rep_dev,
                         bool fold) {
  const int nchunks = (V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
  uint64_t* part = reinterpret_cast<uint64_t*>(ws);
  if (f16)
    if (V % 4 == 0)
      hipLaunchKernelGGL((verify_argmax_partial<true, true>), dim3(nchunks, M), dim3(256), 0, s, logits, M, V, seen, st,
                         rep, inv_rep, rep_dev, part, nchunks);
    else
      hipLaunchKernelGGL((verify_argmax_partial<true, false>), dim3(nchunks, M), dim3(256), 0, s, logits, M, V, seen, st,
                         rep, inv_rep, rep_dev, part, nchunks);
  else if (V % 4 == 0)
    hipLaunchKernelGGL((verify_argmax_partial<false, true>), dim3(nchunks, M), dim3(256), 0, s, logits, M, V, seen, st,
                       rep, inv_rep, rep_dev, part, nchunks);
  else
    hipLaunchKernelGGL((verify_argmax_partial<false, false>), dim3(nchunks, M), dim3(256), 0, s, logits, M, V, seen, st,
                       rep, inv_rep, rep_dev, part, nchunks);
  if (fold) hipLaunchKernelGGL(fold_keys, dim3(M), dim3(64), 0, s, part, nchunks, best, st);
  return (int)hipGetLastError();
}

int accept_commit_launch(dspark_state* st, const uint64_t* best, int m, int skip_now, int32_t* out_tokens, int out_cap,
                         uint32_t* seen, hipStream_t s) {
  // best is only read when no partial keys are given
  hipLaunchKernelGGL(accept_commit_kernel, dim3(1), dim3(64), 0, s, st, const_cast<uint64_t*>(best), m, skip_now,
                     out_tokens, out_cap, seen, (const uint64_t*)nullptr, 0, 0, (int32_t*)nullptr);
  return (int)hipGetLastError();
}

int verify_argmax_chunks(int V) { return (V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK; }

int accept_commit_fold_launch(dspark_state* st, const uint64_t* part, int nchunks, int M, uint64_t* best,
                              int32_t* out_tokens, int out_cap, uint32_t* seen, int skip_now, int32_t* mirror,
                              hipStream_t s) {
  if (M < 1 || M > 64 || nchunks < 1) return DSPARK_EINVAL;
  hipLaunchKernelGGL(accept_commit_kernel, dim3(1), dim3(64), 0, s, st, best, 0, skip_now, out_tokens, out_cap, seen,
                     part, nchunks, M, mirror);
  return (int)hipGetLastError();
}

}  // namespace dspark
