#!/usr/bin/env python3
"""Writes tests/golden/vectors.npz: small seeded input/output vectors of the DSpark step's pieces, computed by the
CPU oracle (oracle/), so GPU tests can check the HIP path against committed outputs and CPU tests can check that the
oracle still reproduces them.

Cases (all seeds fixed here):
  attn{i}_*      verify attention: q/k/v fp16 bits, the geometry, and the fp64 oracle output (float64)
  argmax_*       C1-style verify argmax + acceptance/commit: fp16 logits, seen bitmap, draft tokens, u64 keys, the
                 State words and emitted tokens after the commit
  gemm_*         int8 GEMM with per-row fp16 scales: x fp16 bits, biased weight bytes, scales, fp64 output
  head_*         fp16 crop head + row argmax: x, w fp16 bits, fp64 output, argmax rows (N = 320)

Run from the repository root: python3 tests/golden/make_vectors.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vectors.npz")

# (M, QH, KVH, D, a, start, window, causal, seed)
ATTN = [
    (9, 8, 2, 64, 150, 0, 0, 1, 11),     # causal verify block, ragged context (not a page multiple)
    (16, 8, 2, 64, 70, 10, 0, 0, 12),    # drafter: bidirectional block over a ring range starting at 10
    (5, 8, 2, 128, 120, 61, 64, 1, 13),  # reference head_dim, sliding window 64 (start = a - window + 1)
    (4, 4, 1, 64, 0, 0, 0, 1, 14),       # empty cache: the causal block alone
]
STATE_KW = dict(rounds_left=32, budget=512, eos=-1, stop_at=1056, run=1, skip_rounds=1)


def seen_bitmap(V, toks):
    bits = np.zeros((V + 31) // 32, np.uint32)
    for t in toks:
        bits[t >> 5] |= np.uint32(1 << (int(t) & 31))
    return bits


def main():
    orc.lib()
    out = {}
    out["attn_cases"] = np.array(ATTN, np.int64)
    for i, (M, QH, KVH, D, a, start, window, causal, seed) in enumerate(ATTN):
        q = orc.normal_f16(seed, (M, QH, D))
        k = orc.normal_f16(seed + 1, (a + M, KVH, D))
        v = orc.normal_f16(seed + 2, (a + M, KVH, D))
        out[f"attn{i}_q"], out[f"attn{i}_k"], out[f"attn{i}_v"] = q, k, v
        out[f"attn{i}_out"] = orc.verify_attention(q, k, v, a, start, window, bool(causal))

    # verify argmax + acceptance/commit: M = 9, V = 4096, rep 1.3, the first 5 drafts planted as the argmax
    M, V, a, rep, seed = 9, 4096, 1024, 1.3, 21
    rng = np.random.default_rng(seed)
    logits16 = orc.normal_f16(seed, (M, V))
    logits = orc.f16_to_f32(logits16)
    bits = seen_bitmap(V, rng.integers(0, V, 100))
    tokens = np.zeros(M, np.int32)
    tokens[0] = int(rng.integers(0, V))
    for t in range(1, M):
        am = int(orc.keys_to_tokens(orc.verify_argmax(logits[:t], bits, tokens[:t], rep=rep))[t - 1])
        tokens[t] = am if t <= 5 else (am + 1 + int(rng.integers(0, V - 1))) % V
    keys = orc.verify_argmax(logits, bits, tokens, rep=rep)
    st = orc.new_state(a=a, anchor=int(tokens[0]), tokens=tokens, **STATE_KW)
    emitted = np.zeros(64, np.int32)
    bits_after = bits.copy()
    acc = orc.accept_commit(st, orc.keys_to_tokens(keys), M, emitted, bits_after)
    out.update(argmax_meta=np.array([M, V, a, seed], np.int64), argmax_rep=np.float64(rep),
               argmax_logits=logits16, argmax_seen=bits, argmax_tokens=tokens, argmax_keys=keys,
               argmax_acc=np.int64(acc), argmax_state=np.array([getattr(st, f) for f in STATE_FIELDS], np.int64),
               argmax_state_tokens=np.array(list(st.tokens)[:M], np.int32), argmax_emitted=emitted,
               argmax_seen_after=bits_after)

    # int8 GEMM: M = 5, N = 96, K = 256
    M, N, K = 5, 96, 256
    x = orc.normal_f16(31, (M, K))
    w = orc.int8_uniform(32, (N, K))
    s = orc.f32_to_f16(np.random.default_rng(33).uniform(0.5, 1.5, N).astype(np.float32) / np.float32(127 * 16))
    out.update(gemm_x=x, gemm_wb=(w.astype(np.int16) + 128).astype(np.uint8), gemm_s=s, gemm_out=orc.gemm_i8(x, w, s))

    # fp16 crop head + row argmax: M = 3, N = 320, K = 128 (N a multiple of the 16-row strip)
    M, N, K = 3, 320, 128
    x = orc.normal_f16(41, (M, K))
    w = orc.normal_f16(42, (N, K), scale=float(1 / np.sqrt(K)))
    y = orc.gemm_f16(x, w)
    out.update(head_x=x, head_w=w, head_out=y, head_argmax=orc.row_argmax(y.astype(np.float32)))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(out)} arrays")


STATE_FIELDS = ["a", "anchor", "count", "rounds_left", "limit", "budget", "eos", "M", "ctx_new", "ctx_pos", "ctx_lo",
                "run", "force_m", "rounds_done", "accepted", "verified", "miss", "skip", "skip_after", "skip_rounds",
                "stop_at", "ckpt_slot"]

if __name__ == "__main__":
    main()
