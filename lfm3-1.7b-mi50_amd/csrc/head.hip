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
//
// The books run on the whole wave: lane l holds the State's header word l, tokens[l], tokens[l + 1] and key l, all
// requested in the kernel's first round with the run flag and the first batch of partial keys. Acceptance is a ballot
// over the lanes (lane t < m - 1 misses when token(key t) != tokens[t + 1]; acc = the first miss, else m - 1); lanes
// 1..acc store the accepted drafts and lane 0 the bonus token, each setting its own seen bit; the header words the
// books change are stored by lane 0 from registers. No value is read back from memory after the first round.
__global__ __launch_bounds__(64) void accept_commit_kernel(dspark_state* st, uint64_t* best, int m, int skip_now,
                                                           int32_t* out_tokens, int out_cap, uint32_t* seen,
                                                           const uint64_t* part, int nchunks, int mfold,
                                                           int32_t* mirror) {
  // Buffer loads return 0 past a buffer's end: past the partial keys, and for every load of best[] when the keys
  // come folded from part (best's buffer is then given length 0). A stopped round writes nothing.
  const int lane = (int)threadIdx.x;
  asm volatile("" ::"s"(mirror));  // the kernarg line past the first: fetched with the first
  constexpr int NH = (int)(offsetof(dspark_state, tokens) / sizeof(int32_t));  // header words
  static_assert(NH <= 64 && DSPARK_MT_MAX == 64, "one header word and one token per lane");
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)st, (short)0, (int)sizeof(dspark_state), 0x00020000);
  const int run = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)offsetof(dspark_state, run), 0, 0);
  const int hw = __builtin_amdgcn_raw_buffer_load_b32(rs, min(lane, NH - 1) * 4, 0, 0);
  const int tk = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)offsetof(dspark_state, tokens) + lane * 4, 0, 0);
  const int tn =
      __builtin_amdgcn_raw_buffer_load_b32(rs, (int)offsetof(dspark_state, tokens) + min(lane + 1, 63) * 4, 0, 0);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)best, (short)0, part ? 0 : max(m, 0) * (int)sizeof(uint64_t), 0x00020000);
  const u32x2 kb = __builtin_amdgcn_raw_buffer_load_b64(rb, lane * (int)sizeof(uint64_t), 0, 0);
  const int n = part ? mfold * nchunks : 0;
  constexpr int PB = 8;
  const __amdgpu_buffer_rsrc_t rp =
      __builtin_amdgcn_make_buffer_rsrc((void*)part, (short)0, n * (int)sizeof(uint64_t), 0x00020000);
  u32x2 v0[PB];
#pragma unroll
  for (int i = 0; i < PB; ++i)
    v0[i] = __builtin_amdgcn_raw_buffer_load_b64(rp, (64 * i + lane) * (int)sizeof(uint64_t), 0, 0);
  __shared__ unsigned long long sb[64];
  if (part) {
    sb[lane] = 0;
    __syncthreads();
    for (int e0 = 0; e0 < n; e0 += 64 * PB) {
      uint64_t v[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i)
        v[i] = e0 == 0 ? __builtin_bit_cast(uint64_t, v0[i]) : ldg(part + min(e0 + 64 * i + lane, n - 1));
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int e = e0 + 64 * i + lane;
        if (e < n) atomicMax(&sb[e / nchunks], (unsigned long long)v[i]);
      }
    }
    __syncthreads();
  }
  if (!run_flag_set(run)) return;
  const uint64_t key = part ? (uint64_t)sb[lane] : __builtin_bit_cast(uint64_t, kb);
  if (part && lane < mfold) best[lane] = key;  // the folded keys
  auto hdr = [&](size_t off) { return __builtin_amdgcn_readlane(hw, (int)(off / sizeof(int32_t))); };
  if (m <= 0) m = hdr(offsetof(dspark_state, M));  // rounds that drafted on the device: the verified count is in the State
  const uint64_t miss = __builtin_amdgcn_ballot_w64(lane < m - 1 && key_token(key) != tn);
  const int acc = miss ? (int)__builtin_ctzll(miss) : max(m - 1, 0);
  const int commit = acc + 1;
  const int bonus = key_token((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, acc));  // the token is the low word
  const int aa = hdr(offsetof(dspark_state, a));
  const int count = hdr(offsetof(dspark_state, count));
  if (count < 0 || count + commit > out_cap) {  // no room for the commit: write nothing and stop
    if (lane == 0) st->run = 0;
    return;
  }
  // lanes 1..acc: the accepted drafts tokens[1..acc] at count..count+acc-1; lane 0: the bonus token after them
  const int val = lane == 0 ? bonus : tk;
  const bool mine = lane <= acc;
  if (mine) {
    out_tokens[lane == 0 ? count + acc : count + lane - 1] = val;
    atomicOr(&seen[val >> 5], 1u << (val & 31));
  }
  const int eos = hdr(offsetof(dspark_state, eos));
  const bool stop = eos >= 0 && __builtin_amdgcn_ballot_w64(mine && val == eos) != 0;
  if (lane != 0) return;
  const int count1 = count + commit, a1 = aa + commit;
  const int accepted = hdr(offsetof(dspark_state, accepted)) + acc;
  const int verified = hdr(offsetof(dspark_state, verified)) + m;
  int skip = hdr(offsetof(dspark_state, skip)), miss_n = hdr(offsetof(dspark_state, miss));
  if (skip_now > 0) {
    skip -= 1;
  } else if (acc == 0) {
    miss_n += 1;
    const int skip_after = hdr(offsetof(dspark_state, skip_after));
    if (skip_after > 0 && miss_n >= skip_after) {
      skip = hdr(offsetof(dspark_state, skip_rounds));
      miss_n = 0;
    }
  } else {
    miss_n = 0;
  }
  const int rounds_done = hdr(offsetof(dspark_state, rounds_done)) + 1;
  const int rounds_left = hdr(offsetof(dspark_state, rounds_left)) - 1;
  const int run1 = (!stop && rounds_left > 0 && a1 < hdr(offsetof(dspark_state, stop_at)) &&
                    count1 < hdr(offsetof(dspark_state, budget)))
                       ? 1
                       : 0;
  st->count = count1;
  st->ctx_new = commit;
  st->ctx_pos = aa;
  st->a = a1;
  st->anchor = bonus;
  st->accepted = accepted;
  st->verified = verified;
  st->skip = skip;
  st->miss = miss_n;
  st->tokens[0] = bonus;
  st->rounds_done = rounds_done;
  st->rounds_left = rounds_left;
  st->run = run1;
  if (mirror) {
    const int words[8] = {run1, a1, count1, rounds_left, skip, miss_n, accepted, verified};
    __hip_atomic_store(mirror + 15, rounds_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __atomic_thread_fence(__ATOMIC_RELEASE);  // word 15 before the values
#pragma unroll
    for (int i = 0; i < 8; ++i) __hip_atomic_store(mirror + 1 + i, words[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(mirror, rounds_done, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
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
