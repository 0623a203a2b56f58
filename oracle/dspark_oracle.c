/*
 * CPU oracle for the DSpark speculative-decode step -- TEST INFRASTRUCTURE ONLY (see dspark_oracle.h).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, as the checker.
 * Citations are file:line in the reference repository jwyjohn/lfm3-1.7b-mi50.
 */
#include "dspark_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

/* Round to nearest half, ties to even: internal/fp16/fp16.go:7-44. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
  const int32_t biased = (int32_t)((b >> 23) & 0xffu);
  uint32_t man = b & 0x7fffffu;
  if (biased == 0xff) return man ? (uint16_t)(sign | 0x7e00u) : (uint16_t)(sign | 0x7c00u);
  const int32_t exp = biased - 127 + 15;
  if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return sign;
    man |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - exp);
    uint32_t m = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
  const uint32_t m = man >> 13;
  const uint32_t rem = man & 0x1fffu;
  uint16_t out = (uint16_t)(sign | ((uint32_t)exp << 10) | m);
  if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) out++; /* a carry into the exponent is the next value */
  return out;
}

/* Exact widening: internal/fp16/fp16.go:46-66. */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      uint32_t e = 127 - 15 + 1;
      while ((man & 0x400u) == 0) {
        man <<= 1;
        e--;
      }
      bits = sign | (e << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | (0xffu << 23) | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

static double h2d(uint16_t h) { return (double)orc_f16_to_f32(h); }

/* ------------------------------------------------------------------ generators */

/* SplitMix64 finaliser (Steele, Lea, Flood 2014). Counter-based: value i of a stream is a pure function of (seed, i). */
uint64_t orc_mix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

static uint64_t ctr(uint64_t seed, uint64_t i) { return orc_mix64(orc_mix64(seed) ^ (i * 0xd1b54a32d192ed03ull)); }

/* N(0, scale^2) by Box-Muller on pairs of counter values, rounded to fp16 (RNE). */
void orc_gen_normal_f16(uint64_t seed, uint64_t offset, int64_t n, float scale, uint16_t* out) {
  for (int64_t j = 0; j < n; ++j) {
    const uint64_t i = offset + (uint64_t)j;
    const uint64_t p = i >> 1;
    const double u1 = ((double)(ctr(seed, 2 * p) >> 11) + 0.5) * 0x1p-53;
    const double u2 = (double)(ctr(seed, 2 * p + 1) >> 11) * 0x1p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double z = (i & 1) ? r * sin(2.0 * M_PI * u2) : r * cos(2.0 * M_PI * u2);
    out[j] = orc_f32_to_f16((float)(z * (double)scale));
  }
}

void orc_gen_int8_uniform(uint64_t seed, int64_t n, int8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (int8_t)((int)(ctr(seed, (uint64_t)i) % 255u) - 127);
}

void orc_gen_uniform_u32(uint64_t seed, int64_t n, uint32_t bound, uint32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint32_t)(ctr(seed, (uint64_t)i) % bound);
}

/* ------------------------------------------------------------------ verify attention */

/* Key validity, dspark.hip:1308-1312 (attention_pass) and 2006-2012 (attention_v3):
 * context keys need start <= kpos < a and (window == 0 || kpos > qpos - window); fresh keys j < M need
 * j <= t when causal (target layers) and nothing else (drafter block keys, causal = false). */
static int key_valid(int kpos, int t, int M, int a, int start, int window, int causal) {
  if (kpos < a) return kpos >= start && (window == 0 || kpos > a + t - window);
  const int j = kpos - a;
  if (j >= M) return 0;
  return causal ? j <= t : 1;
}

void orc_attn_partial(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D, int a,
                      int start, int window, int causal, int k0, int k1, double* m, double* l, double* acc) {
  const int G = QH / KVH;
  const double scale = 1.0 / sqrt((double)D);
  const double log2e = 1.4426950408889634;
  double* s = (double*)malloc(sizeof(double) * (size_t)(k1 > k0 ? k1 - k0 : 1));
  for (int t = 0; t < M; ++t) {
    for (int qh = 0; qh < QH; ++qh) {
      const int h = qh / G;
      const int row = t * QH + qh;
      const uint16_t* qr = q + (size_t)row * D;
      double mx = -INFINITY;
      for (int kp = k0; kp < k1; ++kp) {
        double dot = 0.0;
        if (key_valid(kp, t, M, a, start, window, causal)) {
          const uint16_t* kr = k + ((size_t)kp * KVH + h) * D;
          for (int d = 0; d < D; ++d) dot += h2d(qr[d]) * h2d(kr[d]);
          dot *= scale * log2e;
          if (dot > mx) mx = dot;
        } else {
          dot = -INFINITY;
        }
        s[kp - k0] = dot;
      }
      double sum = 0.0;
      double* o = acc + (size_t)row * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      if (mx != -INFINITY) {
        for (int kp = k0; kp < k1; ++kp) {
          if (s[kp - k0] == -INFINITY) continue;
          const double p = exp2(s[kp - k0] - mx);
          sum += p;
          const uint16_t* vr = v + ((size_t)kp * KVH + h) * D;
          for (int d = 0; d < D; ++d) o[d] += p * h2d(vr[d]);
        }
      }
      m[row] = mx;
      l[row] = sum;
    }
  }
  free(s);
}

/* combine_phase, dspark.hip:2148-2183: f_s = 2^(m_s - max m), o = sum f_s acc_s / sum f_s l_s, 0 if the total is 0. */
void orc_attn_merge(int S, int rows, int D, const double* m, const double* l, const double* acc, double* out) {
  for (int r = 0; r < rows; ++r) {
    double M = -INFINITY;
    for (int s = 0; s < S; ++s)
      if (m[(size_t)s * rows + r] > M) M = m[(size_t)s * rows + r];
    double L = 0.0;
    double* o = out + (size_t)r * D;
    for (int d = 0; d < D; ++d) o[d] = 0.0;
    for (int s = 0; s < S; ++s) {
      const double ms = m[(size_t)s * rows + r];
      if (ms == -INFINITY) continue;
      const double f = exp2(ms - M);
      L += f * l[(size_t)s * rows + r];
      const double* a = acc + ((size_t)s * rows + r) * D;
      for (int d = 0; d < D; ++d) o[d] += f * a[d];
    }
    for (int d = 0; d < D; ++d) o[d] = L > 0 ? o[d] / L : 0.0;
  }
}

void orc_verify_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                          int a, int start, int window, int causal, double* out) {
  const int rows = M * QH;
  double* m = (double*)malloc(sizeof(double) * rows);
  double* l = (double*)malloc(sizeof(double) * rows);
  double* acc = (double*)malloc(sizeof(double) * (size_t)rows * D);
  orc_attn_partial(q, k, v, M, QH, KVH, D, a, start, window, causal, 0, a + M, m, l, acc);
  orc_attn_merge(1, rows, D, m, l, acc, out);
  free(m);
  free(l);
  free(acc);
}

/* The fp64 verify attention above with its (token, query head) rows dealt to threads (each row is computed exactly
 * as orc_verify_attention computes it, so the outputs are the same bits); for long contexts. */
typedef struct {
  const uint16_t *q, *k, *v;
  int M, QH, KVH, D, a, start, window, causal, nthreads, tid;
  double* out;
} attn64_job;

static void* attn64_worker(void* arg) {
  const attn64_job* j = (const attn64_job*)arg;
  const int D = j->D;
  double m, l;
  double* acc = (double*)malloc(sizeof(double) * D);
  for (int row = j->tid; row < j->M * j->QH; row += j->nthreads) {
    const int t = row / j->QH, qh = row % j->QH;
    const int G = j->QH / j->KVH;
    const uint16_t* qrow = j->q + (size_t)row * D;
    /* orc_attn_partial's arithmetic for this one row over all keys, then orc_attn_merge of the single partial */
    const double scale = 1.0 / sqrt((double)D), log2e = 1.4426950408889634;
    const int h = qh / G, T = j->a + j->M;
    double mx = -INFINITY;
    double* s = (double*)malloc(sizeof(double) * (size_t)T);
    for (int kp = 0; kp < T; ++kp) {
      double dot = -INFINITY;
      if (key_valid(kp, t, j->M, j->a, j->start, j->window, j->causal)) {
        const uint16_t* kr = j->k + ((size_t)kp * j->KVH + h) * D;
        dot = 0.0;
        for (int d = 0; d < D; ++d) dot += h2d(qrow[d]) * h2d(kr[d]);
        dot *= scale * log2e;
        if (dot > mx) mx = dot;
      }
      s[kp] = dot;
    }
    double sum = 0.0;
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    if (mx != -INFINITY)
      for (int kp = 0; kp < T; ++kp) {
        if (s[kp] == -INFINITY) continue;
        const double p = exp2(s[kp] - mx);
        sum += p;
        const uint16_t* vr = j->v + ((size_t)kp * j->KVH + h) * D;
        for (int d = 0; d < D; ++d) acc[d] += p * h2d(vr[d]);
      }
    free(s);
    m = mx;
    l = sum;
    orc_attn_merge(1, 1, D, &m, &l, acc, j->out + (size_t)row * D);
  }
  free(acc);
  return NULL;
}

void orc_verify_attention_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                             int a, int start, int window, int causal, double* out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  attn64_job jobs[256];
  for (int i = 0; i < threads; ++i) {
    attn64_job j = {q, k, v, M, QH, KVH, D, a, start, window, causal, threads, i, out};
    jobs[i] = j;
    pthread_create(&th[i], NULL, attn64_worker, &jobs[i]);
  }
  for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
}

/* fp32 multi-threaded restatement (same masks) used as the timed CPU baseline. */
typedef struct {
  const uint16_t *q, *k, *v;
  int M, QH, KVH, D, a, start, window, causal, nthreads, tid;
  float* out;
} attn_job;

static void* attn_worker(void* arg) {
  const attn_job* j = (const attn_job*)arg;
  const int G = j->QH / j->KVH, T = j->a + j->M, D = j->D;
  const float c = (float)(1.4426950408889634 / sqrt((double)D));
  float* s = (float*)malloc(sizeof(float) * (size_t)T * G);
  float* kf = (float*)malloc(sizeof(float) * D);
  float* acc = (float*)malloc(sizeof(float) * (size_t)G * D);
  float* qf = (float*)malloc(sizeof(float) * (size_t)G * D);
  for (int task = j->tid; task < j->KVH * j->M; task += j->nthreads) {
    const int h = task / j->M, t = task % j->M;
    for (int g = 0; g < G; ++g)
      for (int d = 0; d < D; ++d) qf[g * D + d] = orc_f16_to_f32(j->q[((size_t)t * j->QH + h * G + g) * D + d]);
    float mx[64];
    for (int g = 0; g < G; ++g) mx[g] = -INFINITY;
    for (int kp = 0; kp < T; ++kp) {
      const int ok = key_valid(kp, t, j->M, j->a, j->start, j->window, j->causal);
      if (ok)
        for (int d = 0; d < D; ++d) kf[d] = orc_f16_to_f32(j->k[((size_t)kp * j->KVH + h) * D + d]);
      for (int g = 0; g < G; ++g) {
        float dot = -INFINITY;
        if (ok) {
          dot = 0.f;
          for (int d = 0; d < D; ++d) dot += qf[g * D + d] * kf[d];
          dot *= c;
          if (dot > mx[g]) mx[g] = dot;
        }
        s[(size_t)kp * G + g] = dot;
      }
    }
    float l[64];
    for (int g = 0; g < G; ++g) l[g] = 0.f;
    memset(acc, 0, sizeof(float) * (size_t)G * D);
    for (int kp = 0; kp < T; ++kp) {
      if (s[(size_t)kp * G] == -INFINITY) continue;
      for (int d = 0; d < D; ++d) kf[d] = orc_f16_to_f32(j->v[((size_t)kp * j->KVH + h) * D + d]);
      for (int g = 0; g < G; ++g) {
        const float p = exp2f(s[(size_t)kp * G + g] - mx[g]);
        l[g] += p;
        for (int d = 0; d < D; ++d) acc[g * D + d] += p * kf[d];
      }
    }
    for (int g = 0; g < G; ++g)
      for (int d = 0; d < D; ++d)
        j->out[((size_t)t * j->QH + h * G + g) * D + d] = l[g] > 0 ? acc[g * D + d] / l[g] : 0.f;
  }
  free(s);
  free(kf);
  free(acc);
  free(qf);
  return NULL;
}

void orc_verify_attention_f32_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, int M, int QH, int KVH, int D,
                                 int a, int start, int window, int causal, float* out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  attn_job jobs[256];
  for (int i = 0; i < threads; ++i) {
    attn_job j = {q, k, v, M, QH, KVH, D, a, start, window, causal, threads, i, out};
    jobs[i] = j;
    pthread_create(&th[i], NULL, attn_worker, &jobs[i]);
  }
  for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------ argmax key, penalty */

/* dspark.hip:967-971: ordered float bits in the high word, 0xFFFFFFFF - index in the low word; the max key is the
 * largest value and, among equal values, the smallest index (torch.argmax, internal/sample/sample.go:108-117). */
uint64_t orc_argmax_key(float v, uint32_t idx) {
  uint32_t u;
  memcpy(&u, &v, 4);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - idx);
}

uint32_t orc_key_index(uint64_t key) { return 0xffffffffu - (uint32_t)key; }

/* head_run<false, M>, dspark.hip:2222-2232 (isnew) and 2284-2294 (fp16 rounding, penalty, key). */
void orc_verify_argmax(const float* logits, int M, int V, const uint32_t* seen_bits, const int32_t* tokens, float rep,
                       float inv_rep, uint64_t* best_keys) {
  int isnew[ORC_MT_MAX] = {0};
  for (int t = 1; t < M; ++t) {
    const int32_t dt = tokens[t];
    isnew[t] = ((seen_bits[dt >> 5] >> (dt & 31)) & 1u) == 0;
  }
  for (int t = 0; t < M; ++t) {
    uint64_t best = 0;
    for (int r = 0; r < V; ++r) {
      const float v = logits[(size_t)t * V + r];
      const float vr = orc_f16_to_f32(orc_f32_to_f16(v));
      int hit = ((seen_bits[r >> 5] >> (r & 31)) & 1u) != 0;
      for (int j = 1; j <= t && j < M; ++j)
        if (isnew[j] && r == tokens[j]) hit = 1;
      const float pv = hit ? (vr > 0.f ? vr * inv_rep : vr * rep) : vr;
      const uint64_t key = orc_argmax_key(pv, (uint32_t)r);
      if (key > best) best = key;
    }
    best_keys[t] = best;
  }
}

/* Host sampler's repetition penalty, internal/sample/sample.go:75-90. */
void orc_penalize_rep(float* lg, int n, const int32_t* seen, int nseen, float rep) {
  if (rep == 1.f || rep == 0.f) return;
  char* mark = (char*)calloc((size_t)n, 1);
  for (int i = 0; i < nseen; ++i)
    if (seen[i] >= 0 && seen[i] < n) mark[seen[i]] = 1;
  for (int i = 0; i < n; ++i)
    if (mark[i]) lg[i] = lg[i] > 0 ? lg[i] / rep : lg[i] * rep;
  free(mark);
}

/* internal/sample/sample.go:108-117: first maximum. */
int32_t orc_argmax_first(const float* lg, int n) {
  int best = 0;
  float bv = -INFINITY;
  for (int i = 0; i < n; ++i)
    if (lg[i] > bv) {
      best = i;
      bv = lg[i];
    }
  return best;
}

/* ------------------------------------------------------------------ accept / commit */

/* dspark.hip:2852-2859 (acceptance) and 2880-2913 (books). */
int orc_accept_commit(orc_state* st, const int32_t* best_tok, int m, int skip_now, int32_t* out_tokens, uint32_t* seen) {
  int acc = 0;
  for (int t = 0; t < m - 1; ++t) {
    if (best_tok[t] != st->tokens[t + 1]) break;
    ++acc;
  }
  const int commit = acc + 1;
  const int32_t bonus = best_tok[acc];
  int count = st->count;
  for (int i = 1; i <= acc; ++i) out_tokens[count++] = st->tokens[i];
  out_tokens[count++] = bonus;
  for (int i = 1; i <= acc; ++i) {
    const int32_t tk = st->tokens[i];
    seen[tk >> 5] |= 1u << (tk & 31);
  }
  seen[bonus >> 5] |= 1u << (bonus & 31);
  int stop = 0;
  if (st->eos >= 0)
    for (int i = count - commit; i < count; ++i) stop = stop || out_tokens[i] == st->eos;
  const int aa = st->a;
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
  return acc;
}

/* dspark.hip:2860-2877: positions a..a+acc receive the verified tokens' K/V. */
void orc_kv_commit(uint16_t* cache, const uint16_t* fresh, int a, int acc, int row) {
  for (int c = 0; c <= acc; ++c) memcpy(cache + (size_t)(a + c) * row, fresh + (size_t)c * row, sizeof(uint16_t) * row);
}

/* ------------------------------------------------------------------ int8 K/V records (reference KV format) */

/* quantize_pair, kernels/ops.hip:212-224 (= dspark.hip:933-944): amax over the D values, scale = max(amax / 127, 1e-6),
 * inv = 1 / scale, a = x * inv, a + 0.5 (a >= 0) or a - 0.5, clamped to [-128, 127], truncated. Each step is one IEEE
 * binary32 operation; `volatile` keeps the compiler from fusing the multiply and the add. Returns the scale. */
float orc_rec_quantize(const float* x, int D, int8_t* q) {
  float amax = 0.f;
  for (int i = 0; i < D; ++i) amax = fmaxf(amax, fabsf(x[i]));
  volatile float scale = fmaxf(amax / 127.f, 1e-6f);
  volatile float inv = 1.f / scale;
  for (int i = 0; i < D; ++i) {
    volatile float a = x[i] * inv;
    volatile float r = a >= 0.f ? a + 0.5f : a - 0.5f;
    q[i] = (int8_t)truncf(fminf(fmaxf(r, -128.f), 127.f));
  }
  return scale;
}

/* kv_write, kernels/ops.hip:235-251, with the engine's layout (internal/model/engine.go:30-32: KVBlock = 32 KVH Rec,
 * kv_head = Rec, kv_slot = KVH Rec): record of (pos, h) at page bt[pos / 32] (identity without a table), offset
 * ((pos % 32) KVH + h) Rec; K int8[128] | f32 k scale | V int8[128] | f32 v scale. k, v: fp32 [n][KVH][128]. */
void orc_kv_write_rec(const float* k, const float* v, int n, int KVH, int pos0, const int32_t* bt, uint8_t* pages) {
  const int D = 128, rec = 2 * D + 8;
  for (int t = 0; t < n; ++t) {
    const int pos = pos0 + t;
    const int phys = bt ? bt[pos / 32] : pos / 32;
    for (int h = 0; h < KVH; ++h) {
      uint8_t* r = pages + (size_t)phys * 32 * KVH * rec + ((size_t)(pos % 32) * KVH + h) * rec;
      const float ks = orc_rec_quantize(k + ((size_t)t * KVH + h) * D, D, (int8_t*)r);
      const float vs = orc_rec_quantize(v + ((size_t)t * KVH + h) * D, D, (int8_t*)(r + D + 4));
      memcpy(r + D, &ks, 4);
      memcpy(r + 2 * D + 4, &vs, 4);
    }
  }
}

/* Query quantization of the int8 attention, query_fresh (dspark.hip:1020-1035): per 32-dim group
 * s = max(amax / 127, 1e-20), q8 = rint(q * (1 / s)) (the reference multiplies by the hardware reciprocal of s, within
 * one ulp of 1 / s, so a value that lands within an ulp of a rounding boundary can differ by one unit). q fp16
 * [rows][D]; q8 [rows][D]; qs [rows][D / 32]. */
void orc_rec_quantize_q(const uint16_t* q, int rows, int D, int8_t* q8, float* qs) {
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < D / 32; ++g) {
      const uint16_t* src = q + (size_t)r * D + 32 * g;
      float amax = 0.f;
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(orc_f16_to_f32(src[i])));
      volatile float s = fmaxf(amax / 127.f, 1e-20f);
      volatile float inv = 1.f / s;
      for (int i = 0; i < 32; ++i) {
        volatile float a = orc_f16_to_f32(src[i]) * inv;
        q8[(size_t)r * D + 32 * g + i] = (int8_t)nearbyintf(a);
      }
      qs[(size_t)r * (D / 32) + g] = s;
    }
}

/* fp64 attention over dequantized values: q [M][QH][D], k, v [T][KVH][D] as doubles; the masks and merge of
 * orc_verify_attention (dspark.hip:1308-1312, 2006-2012). */
void orc_verify_attention_d(const double* q, const double* k, const double* v, int M, int QH, int KVH, int D, int a,
                            int start, int window, int causal, double* out) {
  const int G = QH / KVH, T = a + M;
  const double scale = 1.0 / sqrt((double)D), log2e = 1.4426950408889634;
  double* s = (double*)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
  for (int t = 0; t < M; ++t)
    for (int qh = 0; qh < QH; ++qh) {
      const int h = qh / G, row = t * QH + qh;
      const double* qr = q + (size_t)row * D;
      double mx = -INFINITY;
      for (int kp = 0; kp < T; ++kp) {
        double dot = -INFINITY;
        if (key_valid(kp, t, M, a, start, window, causal)) {
          const double* kr = k + ((size_t)kp * KVH + h) * D;
          dot = 0.0;
          for (int d = 0; d < D; ++d) dot += qr[d] * kr[d];
          dot *= scale * log2e;
          if (dot > mx) mx = dot;
        }
        s[kp] = dot;
      }
      double sum = 0.0;
      double* o = out + (size_t)row * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      if (mx != -INFINITY) {
        for (int kp = 0; kp < T; ++kp) {
          if (s[kp] == -INFINITY) continue;
          const double p = exp2(s[kp] - mx);
          sum += p;
          const double* vr = v + ((size_t)kp * KVH + h) * D;
          for (int d = 0; d < D; ++d) o[d] += p * vr[d];
        }
      }
      for (int d = 0; d < D; ++d) o[d] = sum > 0 ? o[d] / sum : 0.0;
    }
  free(s);
}

/* The reference's int8 verify attention as the fp64 softmax attention of its int8 operands (the reference's own
 * accuracy claim is against exactly this, benchmarks/verify_attention.txt): Q quantized per 32-dim group
 * (orc_rec_quantize_q), K and V of position kpos and head h read from the record pages (through bt) and dequantized
 * (q x scale) as they are used, so memory stays at the pages whatever the context. Masks and softmax as
 * orc_verify_attention_d, term for term. */
static const uint8_t* rec_at(const uint8_t* pages, const int32_t* bt, int KVH, int pos, int h) {
  const int phys = bt ? bt[pos / 32] : pos / 32;
  return pages + (size_t)phys * 32 * KVH * 264 + ((size_t)(pos % 32) * KVH + h) * 264;
}

void orc_verify_attention_rec(const uint16_t* q, const uint8_t* pages, const int32_t* bt, int M, int QH, int KVH,
                              int a, int start, int window, int causal, double* out) {
  const int D = 128, T = a + M, rows = M * QH, G = QH / KVH;
  const double scale = 1.0 / sqrt((double)D), log2e = 1.4426950408889634;
  int8_t* q8 = (int8_t*)malloc((size_t)rows * D);
  float* qs = (float*)malloc(sizeof(float) * (size_t)rows * (D / 32));
  double* s = (double*)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
  double qd[128];
  orc_rec_quantize_q(q, rows, D, q8, qs);
  for (int t = 0; t < M; ++t)
    for (int qh = 0; qh < QH; ++qh) {
      const int h = qh / G, row = t * QH + qh;
      for (int d = 0; d < D; ++d) qd[d] = (double)q8[(size_t)row * D + d] * (double)qs[(size_t)row * (D / 32) + d / 32];
      double mx = -INFINITY;
      for (int kp = 0; kp < T; ++kp) {
        double dot = -INFINITY;
        if (key_valid(kp, t, M, a, start, window, causal)) {
          const uint8_t* r = rec_at(pages, bt, KVH, kp, h);
          float ks;
          memcpy(&ks, r + D, 4);
          dot = 0.0;
          for (int d = 0; d < D; ++d) dot += qd[d] * ((double)(int8_t)r[d] * (double)ks);
          dot *= scale * log2e;
          if (dot > mx) mx = dot;
        }
        s[kp] = dot;
      }
      double sum = 0.0;
      double* o = out + (size_t)row * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      if (mx != -INFINITY) {
        for (int kp = 0; kp < T; ++kp) {
          if (s[kp] == -INFINITY) continue;
          const double p = exp2(s[kp] - mx);
          sum += p;
          const uint8_t* r = rec_at(pages, bt, KVH, kp, h);
          float vs;
          memcpy(&vs, r + 2 * D + 4, 4);
          for (int d = 0; d < D; ++d) o[d] += p * ((double)(int8_t)r[D + 4 + d] * (double)vs);
        }
      }
      for (int d = 0; d < D; ++d) o[d] = sum > 0 ? o[d] / sum : 0.0;
    }
  free(q8);
  free(qs);
  free(s);
}

/* ------------------------------------------------------------------ weight formats */

static float round_even(float f) { return (float)nearbyint((double)f); }

/* internal/weights/quant.go:115-144. */
void orc_quantize_rows_int8(const uint16_t* w, int rows, int k, int8_t* q, float* scales) {
  for (int r = 0; r < rows; ++r) {
    float m = 0.f;
    for (int j = 0; j < k; ++j) {
      const float v = fabsf(orc_f16_to_f32(w[(size_t)r * k + j]));
      if (v > m) m = v;
    }
    if (m < 1e-8f) m = 1e-8f;
    const float s = m / 127.f;
    scales[r] = s;
    for (int j = 0; j < k; ++j) {
      float v = round_even(orc_f16_to_f32(w[(size_t)r * k + j]) / s);
      if (v > 127.f) v = 127.f;
      if (v < -127.f) v = -127.f;
      q[(size_t)r * k + j] = (int8_t)v;
    }
  }
}

/* internal/weights/quant.go:24-29. */
int orc_pack_srow(int k) { return (k / 512 == 4) ? 16 : 64; }

/* internal/weights/quant.go:66-104: q = RNE(w / s) clamped to +-127, s = fp16(max|w| / 127) per 128 inputs,
 * stored biased (q + 128); scales [row][quarter][i] with SQ = SRow / 4 entries per quarter. */
void orc_pack_g128(const uint16_t* w, int rows, int k, uint8_t* biased, uint16_t* scales) {
  const int groups = k / 128, ni = groups / 4, sq = orc_pack_srow(k) / 4;
  memset(scales, 0, sizeof(uint16_t) * (size_t)rows * 4 * sq);
  for (int r = 0; r < rows; ++r) {
    const uint16_t* src = w + (size_t)r * k;
    uint8_t* dst = biased + (size_t)r * k;
    uint16_t* sc = scales + (size_t)r * 4 * sq;
    for (int g = 0; g < groups; ++g) {
      float m = 0.f;
      for (int j = 0; j < 128; ++j) {
        const float v = fabsf(orc_f16_to_f32(src[g * 128 + j]));
        if (v > m) m = v;
      }
      if (m < 1e-8f) m = 1e-8f;
      const uint16_t h = orc_f32_to_f16(m / 127.f);
      const float s = orc_f16_to_f32(h);
      for (int j = 0; j < 128; ++j) {
        float q = round_even(orc_f16_to_f32(src[g * 128 + j]) / s);
        if (q > 127.f) q = 127.f;
        if (q < -127.f) q = -127.f;
        dst[g * 128 + j] = (uint8_t)((int)q + 128);
      }
      const int quarter = g % 4, i = g / 4;
      if (i < ni) sc[quarter * sq + i] = h;
    }
  }
}

/* cmd/pack/main.go:281-293: [groups][64 rows][16 pieces][16 B] -> [groups][16 pieces][64 rows][16 B]. */
void orc_transpose_lanes(const uint8_t* src, uint8_t* dst, int64_t n) {
  const int64_t row = 256, piece = 16, group = 64 * 256;
  memcpy(dst, src, (size_t)n);
  for (int64_t g = 0; g + group <= n; g += group)
    for (int r = 0; r < 64; ++r)
      for (int p = 0; p < 16; ++p) memcpy(dst + g + p * 64 * piece + r * piece, src + g + r * row + p * piece, piece);
}

/* ------------------------------------------------------------------ GEMMs */

void orc_gemm_i8(const uint16_t* x, const uint8_t* w, int biased, const uint16_t* scale, int M, int N, int K, double* y) {
  double* xf = (double*)malloc(sizeof(double) * (size_t)M * K);
  for (int64_t i = 0; i < (int64_t)M * K; ++i) xf[i] = h2d(x[i]);
  for (int r = 0; r < N; ++r) {
    const uint8_t* wr = w + (size_t)r * K;
    const double s = h2d(scale[r]);
    for (int t = 0; t < M; ++t) {
      double acc = 0.0;
      const double* xr = xf + (size_t)t * K;
      for (int k = 0; k < K; ++k) {
        const int q = biased ? (int)wr[k] - 128 : (int)(int8_t)wr[k];
        acc += (double)q * xr[k];
      }
      y[(size_t)t * N + r] = acc * s;
    }
  }
  free(xf);
}

/* Per-128-column group scales (weights.Pack, internal/weights/quant.go:66-104; applied per group as gemv_phase does,
 * dspark.hip:553-580): y[t][r] = sum_g gs[g][r] * sum_{k in g} q[r][k] x[t][k], gs fp16 [K/128][N], fp64. */
void orc_gemm_g128(const uint16_t* x, const uint8_t* w, const uint16_t* gs, int M, int N, int K, double* y) {
  const int G = K / 128;
  for (int r = 0; r < N; ++r) {
    const uint8_t* wr = w + (size_t)r * K;
    for (int t = 0; t < M; ++t) {
      double acc = 0.0;
      for (int g = 0; g < G; ++g) {
        double part = 0.0;
        for (int k = 128 * g; k < 128 * g + 128; ++k) part += (double)((int)wr[k] - 128) * h2d(x[(size_t)t * K + k]);
        acc += part * h2d(gs[(size_t)g * N + r]);
      }
      y[(size_t)t * N + r] = acc;
    }
  }
}

/* LFM3_X8's activation format: per 16 values one fp32 scale, int8 codes (norm_compute, kernels/dspark.hip:802-823;
 * x_fill, 883-904). */
void orc_quantize_x16(const float* x, int64_t n, int8_t* q, float* s) {
  for (int64_t p = 0; p < n / 16; ++p) {
    float m = 0.f;
    for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(x[16 * p + j]));
    const float sc = fmaxf(m / 127.f, 1e-20f);
    const float inv = 1.f / sc;
    s[p] = sc;
    for (int j = 0; j < 16; ++j) q[16 * p + j] = (int8_t)(int)rintf(x[16 * p + j] * inv);
  }
}

/* unit_dot_r under LFM3_X8 (kernels/dspark.hip:541-566): per 16-column piece the exact integer dot of the biased
 * weights (q + 128, XOR 0x80 = q) with the int8 codes, times fp32(group scale * piece scale). */
void orc_gemm_x8(const int8_t* q, const float* s, const uint8_t* w, const uint16_t* gs, int M, int N, int K, double* y) {
  const int P = K / 16;
  for (int r = 0; r < N; ++r) {
    const uint8_t* wr = w + (size_t)r * K;
    for (int t = 0; t < M; ++t) {
      double acc = 0.0;
      for (int p = 0; p < P; ++p) {
        int32_t d = 0;
        for (int k = 16 * p; k < 16 * p + 16; ++k) d += ((int)wr[k] - 128) * (int)q[(size_t)t * K + k];
        const float f = orc_f16_to_f32(gs[(size_t)(p / 8) * N + r]) * s[(size_t)t * P + p];
        acc += (double)f * (double)d;
      }
      y[(size_t)t * N + r] = acc;
    }
  }
}

void orc_gemm_f16(const uint16_t* x, const uint16_t* w, int M, int N, int K, double* y) {
  double* xf = (double*)malloc(sizeof(double) * (size_t)M * K);
  double* wf = (double*)malloc(sizeof(double) * (size_t)K);
  for (int64_t i = 0; i < (int64_t)M * K; ++i) xf[i] = h2d(x[i]);
  for (int r = 0; r < N; ++r) {
    for (int k = 0; k < K; ++k) wf[k] = h2d(w[(size_t)r * K + k]);
    for (int t = 0; t < M; ++t) {
      double acc = 0.0;
      const double* xr = xf + (size_t)t * K;
      for (int k = 0; k < K; ++k) acc += wf[k] * xr[k];
      y[(size_t)t * N + r] = acc;
    }
  }
  free(xf);
  free(wf);
}

void orc_row_argmax(const float* y, int M, int N, int32_t* idx) {
  for (int t = 0; t < M; ++t) {
    uint64_t best = 0;
    for (int r = 0; r < N; ++r) {
      const uint64_t key = orc_argmax_key(y[(size_t)t * N + r], (uint32_t)r);
      if (key > best) best = key;
    }
    idx[t] = (int32_t)orc_key_index(best);
  }
}

/* ------------------------------------------------------------------ layer pieces */

/* norm_compute's RMS (dspark.hip:722-843; eps 1e-5 in the target): y = x * rsqrt(mean(x^2) + eps) * w. */
void orc_rms_norm(const float* x, const uint16_t* w, int n, float eps, float* y) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
  const double inv = 1.0 / sqrt(ss / n + eps);
  for (int i = 0; i < n; ++i) y[i] = (float)(x[i] * inv * h2d(w[i]));
}

/* Pairs (i, i + D/2) rotate by pos * base^(-2i/D) for i < rot; the rest pass through (engine.go:428-461,
 * the zero-tail table; norm_rope dspark.hip:946-951). */
void orc_rope(float* x, int D, int rot, double base, int pos) {
  for (int i = 0; i < D / 2; ++i) {
    if (i >= rot) continue;
    const double inv = 1.0 / pow(base, (2.0 * i) / D);
    const double f = (double)pos * inv;
    const double c = cos(f), s = sin(f);
    const double a = x[i], b = x[i + D / 2];
    x[i] = (float)(a * c - b * s);
    x[i + D / 2] = (float)(b * c + a * s);
  }
}

/* conv_wave, dspark.hip:2191-2214, one channel and one token. hist holds the K-1 previous bx (oldest first). */
float orc_conv_step(float B, float C, float X, const float* w, int K, float* hist) {
  const float bx = orc_f16_to_f32(orc_f32_to_f16(B * X));
  double conv = (double)w[K - 1] * bx;
  for (int k = 0; k < K - 1; ++k) conv += (double)w[k] * hist[k];
  for (int k = 0; k + 1 < K - 1; ++k) hist[k] = hist[k + 1];
  if (K > 1) hist[K - 2] = bx;
  return orc_f16_to_f32(orc_f32_to_f16((float)(C * conv)));
}

float orc_silu(float x) { return (float)((double)x / (1.0 + exp(-(double)x))); }
