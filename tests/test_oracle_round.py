"""Pins of the round restatement's composition (oracle/round.py) against closed forms, on the CPU.

The GPU engine round is checked against oracle/round.py (tests/test_gpu_engine.py); these tests check that restatement
itself where the reference holds no vectors for it:
  * the Markov/confidence draft loop (dspark.hip:2633-2664, markov_phase 2322-2366): the cap on drafts, the
    confidence gate (including a stop in mid-chain and a NaN confidence), the argmax -> crop_ids mapping, and the
    transition term -- a chain with zero transition weights follows argmax(base[j]) alone, and one-hot weights make
    the chain a permutation cycle worked out by hand;
  * the sandwich norm (norm_compute, dspark.hip:722-843): a hand-computed 4-wide case, the plain norm when there is
    no branch output, and the scale invariance of the branch's own RMS;
  * the per-head q/k norm and RoPE (query_fresh, dspark.hip:999-1061): rotations compose over positions.
"""
import types

import numpy as np
import pytest

from oracle import round as rnd

THR = -0.4  # the reference's confidence threshold (dspark.go:79-93)


def markov_weights(N=32, R=16, V=200, block=9, max_drafts=8, conf_bias=0.0, seed=0, w2q=None, w1q=None, c2=None,
                   crop_ids=None):
    rng = np.random.default_rng(seed)
    d = types.SimpleNamespace(crop_rows=N, markov_rank=R, vocab=V, block=block, max_drafts=max_drafts,
                              conf_bias=conf_bias, conf_thr=THR)
    w2q = rng.integers(-127, 128, (N, R)) if w2q is None else w2q
    w1q = rng.integers(-127, 128, (V, R)) if w1q is None else w1q
    t = {
        "markov.w2q": np.asarray(w2q, np.int8).reshape(-1).view(np.uint8),
        "markov.w1q": np.asarray(w1q, np.int8).reshape(-1).view(np.uint8),
        "markov.w2s": np.full(N, 1 / 512, np.float32),
        "markov.w1s": np.full(V, 1 / 64, np.float32),
        "conf_c2": np.zeros(V, np.float32) if c2 is None else np.asarray(c2, np.float32),
        "crop_ids": (rng.permutation(V)[:N] if crop_ids is None else np.asarray(crop_ids)).astype(np.int32),
    }
    return rnd.Weights(d, t)


def state(a=100, anchor=5, limit=10 ** 6, budget=512, count=0):
    return {"a": a, "anchor": anchor, "limit": limit, "budget": budget, "count": count}


def base_rows(N, B, seed=1, conf=1.0):
    """base [B][N + 1]: crop-head scores, then the confidence row (column N)."""
    b = np.random.default_rng(seed).standard_normal((B, N + 1))
    b[:, N] = conf
    return b


def test_markov_without_transition_follows_base_argmax():
    N, B = 32, 9
    W = markov_weights(N=N, block=B, w2q=np.zeros((N, 16), int))
    base = base_rows(N, B)
    toks, M, _ = rnd.markov(W, state(anchor=7), base)
    crop = W.t["crop_ids"]
    want = [7] + [int(crop[int(np.argmax(base[j, :N]))]) for j in range(B - 1)]
    assert toks == want and M == B


def test_markov_one_hot_transition_is_a_cycle():
    # w1q[v] = 64 e_{v % R}; w2q[r] = 127 e_{(r + 1) % R} for r < R, 0 otherwise: from token v the only nonzero
    # score is row r = (v - 1) % R, so the next token is crop_ids[(v - 1) % R] (base is zero).
    N, R, V, B = 32, 16, 200, 9
    w1q = np.zeros((V, R), int)
    w1q[np.arange(V), np.arange(V) % R] = 64
    w2q = np.zeros((N, R), int)
    w2q[np.arange(R), (np.arange(R) + 1) % R] = 127
    crop = np.arange(100, 100 + N)
    W = markov_weights(N=N, R=R, V=V, block=B, w1q=w1q, w2q=w2q, crop_ids=crop)
    base = np.zeros((B, N + 1))
    base[:, N] = 1.0
    toks, M, _ = rnd.markov(W, state(anchor=37), base)
    want = [37]
    for _ in range(B - 1):
        want.append(int(crop[(want[-1] - 1) % R]))
    assert toks == want and M == B


def test_markov_draft_cap():
    N, B = 32, 9
    W = markov_weights(N=N, block=B, max_drafts=5)
    base = base_rows(N, B)
    assert rnd.markov(W, state(), base)[1] == 6                      # max_drafts
    assert rnd.markov(W, state(a=100, limit=104), base)[1] == 4      # limit - a - 1 drafts
    assert rnd.markov(W, state(budget=10, count=7), base)[1] == 3    # budget - count - 1 drafts
    assert rnd.markov(W, state(a=100, limit=101), base)[1] == 1      # no room: the anchor alone
    W8 = markov_weights(N=N, block=4, max_drafts=8)
    assert rnd.markov(W8, state(), base_rows(N, 4))[1] == 4          # block - 1 drafts


def test_markov_confidence_gate():
    N, B, V = 32, 9, 200
    # conf = base[j][N] + c2[prev] + conf_bias against THR = -0.4, strictly: >= passes
    W = markov_weights(N=N, block=B, V=V)
    assert rnd.markov(W, state(), base_rows(N, B, conf=-0.5))[1] == 1
    assert rnd.markov(W, state(), base_rows(N, B, conf=np.float32(-0.4)))[1] == B
    assert rnd.markov(markov_weights(N=N, block=B, conf_bias=-1.0), state(), base_rows(N, B, conf=0.5))[1] == 1
    nan = base_rows(N, B)
    nan[0, N] = np.nan
    assert rnd.markov(W, state(), nan)[1] == 1
    # a stop in mid-chain: c2 of the third draft's token is -100, so the fourth step's confidence fails
    base = base_rows(N, B)
    toks, _, _ = rnd.markov(W, state(anchor=3), base)
    c2 = np.zeros(V, np.float32)
    c2[toks[3]] = -100.0
    W2 = markov_weights(N=N, block=B, V=V, c2=c2)
    toks2, M2, _ = rnd.markov(W2, state(anchor=3), base)
    assert toks2 == toks[:4] and M2 == 4


def test_sandwich_norm_hand_case():
    eps = 1e-5
    h = np.array([[1.0, -2.0, 3.0, 0.5]])
    v = np.array([[2.0, 0.0, -2.0, 4.0]])
    pw = np.array([1.0, 0.5, 2.0, 1.0])
    nw = np.array([0.5, 1.0, 1.0, 2.0])
    h_new, x = rnd.resnorm(h, v, pw, nw, 1, eps)
    rms_v = np.sqrt((4 + 0 + 4 + 16) / 4 + eps)                       # sqrt(6 + eps)
    want_h = h + v / rms_v * pw
    assert np.allclose(h_new, want_h, rtol=0, atol=1e-12)
    rms_h = np.sqrt((want_h ** 2).sum() / 4 + eps)
    assert np.allclose(x, (want_h / rms_h * nw).astype(np.float16), rtol=0, atol=0)
    # no branch output: the plain RMS norm of h; no sandwich: v is added unscaled
    _, x0 = rnd.resnorm(h, None, None, nw, 1, eps)
    assert np.array_equal(x0, (h / np.sqrt((h ** 2).sum() / 4 + eps) * nw).astype(np.float16).astype(np.float64))
    h1, _ = rnd.resnorm(h, v, None, nw, 0, eps)
    assert np.array_equal(h1, h + v)


def test_sandwich_branch_scale_invariance():
    rng = np.random.default_rng(3)
    h = rng.standard_normal((3, 64))
    v = rng.standard_normal((3, 64))
    pw = rng.uniform(0.5, 1.5, 64)
    nw = rng.uniform(0.5, 1.5, 64)
    a, _ = rnd.resnorm(h, v, pw, nw, 1, 0.0)
    b, _ = rnd.resnorm(h, 1000.0 * v, pw, nw, 1, 0.0)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("rot", [32, 16])
def test_rope_rows_compose_over_positions(rot):
    D, P = 64, 40
    theta = 1e4 ** (-np.arange(D // 2) * 2.0 / D)
    ang = np.arange(P)[:, None] * theta[None, :]
    table = np.concatenate([np.cos(ang), np.sin(ang)], 1)
    x = np.random.default_rng(4).standard_normal(D)
    # rotating by p then by q is rotating by p + q (exact table, fp64)
    p, q = 7, 11
    shift = np.concatenate([np.cos(q * theta), np.sin(q * theta)])[None, :]
    shifted = np.zeros((P, D))
    shifted[p] = shift
    twice = rnd.rope_rows(rnd.rope_rows(x, p, table, rot), p, shifted, rot)
    assert np.allclose(twice, rnd.rope_rows(x, p + q, table, rot), atol=1e-12)
    # pairs past `rot` pass through; position 0 is the identity
    y = rnd.rope_rows(x, 5, table, rot)
    assert np.array_equal(y[rot:D // 2], x[rot:D // 2]) and np.array_equal(y[D // 2 + rot:], x[D // 2 + rot:])
    assert np.allclose(rnd.rope_rows(x, 0, table, rot), x)


def test_norm_head_unit_rms():
    x = np.random.default_rng(5).standard_normal(64) * 7.0
    y = rnd.norm_head(x, np.ones(64), 0.0)
    assert abs(np.sqrt((y ** 2).mean()) - 1.0) < 1e-12
    assert np.allclose(rnd.norm_head(x, np.full(64, 2.0), 0.0), 2.0 * y)
