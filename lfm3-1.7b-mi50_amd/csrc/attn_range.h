// Verify attention's key range evaluated on the device (kernels that take a from the State at run time).
#pragma once
#include "common.h"
#include "dspark.h"
#include "dspark_internal.h"

namespace dspark {

// The same plan evaluated on the device from the State's a (and, for the drafter, ctx_lo): page range, pages per
// split, unmasked range.
__device__ inline void attn_range(AttnParams& p, int a, int ctx_lo) {
  p.a = a;
  if (p.drafter) {
    // drafter ring: context [max(ctx_lo, a - window), a) for every block token, block keys in both directions
    p.start = max(ctx_lo, a - p.window);
    p.window = 0;
    p.causal = 0;
  } else if (p.window > 0) {
    p.start = max(0, a - p.window + 1);
  }
  const int lo0 = min(a, max(p.start, p.window > 0 ? a - p.window + 1 : 0));  // the block's keys from a
  const int lo_last = max(p.start, p.window > 0 ? a + p.M - p.window : 0);
  const int hi_last = a + p.M - 1;
  p.full_lo = lo_last;
  p.full_hi = p.causal ? a : hi_last;
  p.page0 = lo0 / PAGE;
  p.npages = hi_last / PAGE - p.page0 + 1;
  p.pps = (p.npages + p.S - 1) / p.S;
}

// A key-split kernel's prologue with a State: run, a and ctx_lo read in one round trip (scalar loads of one line; the
// empty asm takes all three before the run test, which would otherwise put the other two behind it). Returns false
// when the round is stopped.
__device__ inline bool attn_state_range(AttnParams& p) {
  const int run = p.st->run, a = p.st->a, lo = p.st->ctx_lo;
  asm volatile("" ::"s"(run), "s"(a), "s"(lo));
  if (run == 0) return false;
  attn_range(p, a, lo);
  return true;
}

}  // namespace dspark
