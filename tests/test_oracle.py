"""Pins the CPU oracle against the reference's own KATs, independent library routines and closed forms.

Nothing here retypes an oracle formula: each check compares against numpy / torch, a reference test vector, or a
mathematical identity chosen so a dropped term, a wrong sign or a transposed operand fails it.
"""
import math

import numpy as np
import pytest


# ---------------------------------------------------------------- fp16 (internal/fp16/fp16.go)
def test_f16_widen_all_halves(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_round_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                  3 * 2.0 ** -25, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -12), np.inf, -np.inf], dtype=np.float32),
        # exact ties at every exponent: 1 + (2k+1) * 2^-11 rounds to even
        (np.float32(1.0) + (2 * np.arange(0, 1024, dtype=np.float32) + 1) * np.float32(2.0 ** -11)),
    ]).astype(np.float32)
    got = orc.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert orc.f32_to_f16(np.array([np.nan], np.float32))[0] & 0x7C00 == 0x7C00


# ---------------------------------------------------------------- generators
def test_generators_deterministic_and_normal(orc):
    a = orc.normal_f16(7, (100000,))
    b = orc.normal_f16(7, (100000,))
    assert np.array_equal(a, b)
    # counter-based: an offset window reproduces the same values
    c = orc.normal_f16(7, (1000,), offset=5000)
    assert np.array_equal(c, a[5000:6000])
    f = orc.f16_to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 0.02 and abs(f.std() - 1.0) < 0.02
    assert abs(np.mean(f ** 4) - 3.0) < 0.1  # Gaussian kurtosis
    q = orc.int8_uniform(3, (200000,))
    assert q.min() == -127 and q.max() == 127
    assert abs(q.astype(np.float64).mean()) < 0.5


# ---------------------------------------------------------------- argmax / penalty (internal/sample/sample_test.go)
def test_argmax_keeps_first_maximum(orc, kats):
    kat = kats["argmax_first_max"]  # sample_test.go:9-13
    assert orc.argmax_first(np.array(kat["logits"], np.float32)) == kat["want"]
    keys = [orc.argmax_key(float(v), i) for i, v in enumerate(kat["logits"])]
    assert orc.key_index(max(keys)) == kat["want"]


def test_repetition_penalty_signs(orc, kats):
    kat = kats["repetition_penalty_signs"]  # sample_test.go:15-25
    lg = orc.penalize_rep(np.array(kat["logits"], np.float32), np.array(kat["seen"], np.int32),
                          float(kat["repetition_penalty"]))
    assert lg.tolist() == kat["want"]
    # the kernel form (multiply by the host's fp32 1/rep, dspark.go:575-578) gives the same on these values
    seen = np.zeros(1, np.uint32)
    for t in kat["seen"]:
        seen[0] |= np.uint32(1 << t)
    keys = orc.verify_argmax(np.array([kat["logits"]], np.float32), seen, [0], rep=float(kat["repetition_penalty"]))
    assert orc.key_index(int(keys[0])) == int(np.argmax(kat["want"]))


def test_greedy_draw(orc, kats):
    kat = kats["greedy_draw"]  # sample_test.go:53-57 (greedy Draw is Argmax)
    assert orc.argmax_first(np.array(kat["logits"], np.float32)) == kat["want"]


def test_argmax_key_orders_like_value_then_index(orc):
    rng = np.random.default_rng(2)
    v = rng.standard_normal(500).astype(np.float32)
    v[::7] = v[3]  # plant exact ties
    v[10] = -np.inf
    keys = np.array([orc.argmax_key(float(x), i) for i, x in enumerate(v)], dtype=np.uint64)
    order_keys = np.argsort(keys, kind="stable")
    order_ref = sorted(range(len(v)), key=lambda i: (float(v[i]), -i))
    assert order_keys.tolist() == order_ref


def _numpy_verify_argmax(logits, seen_bits, tokens, rep):
    """Independent vectorised statement of the penalised fp16 argmax (dspark.hip:2222-2294)."""
    M, V = logits.shape
    seen = ((seen_bits[np.arange(V) >> 5] >> (np.arange(V) & 31)) & 1).astype(bool)
    inv = np.float32(1.0) / np.float32(rep)
    out = []
    for t in range(M):
        vr = logits[t].astype(np.float16).astype(np.float32)
        hit = seen.copy()
        for j in range(1, t + 1):
            dj = tokens[j]
            if not ((seen_bits[dj >> 5] >> (dj & 31)) & 1):
                hit[dj] = True
        pv = np.where(hit, np.where(vr > 0, vr * inv, vr * np.float32(rep)), vr).astype(np.float32)
        out.append(int(np.argmax(pv)))  # numpy argmax: first maximum
    return np.array(out)


@pytest.mark.parametrize("rep", [1.0, 1.3])
def test_verify_argmax_matches_numpy(orc, rep):
    rng = np.random.default_rng(5)
    M, V = 9, 4096
    logits = rng.standard_normal((M, V)).astype(np.float32)
    logits[:, 100] = logits[:, 50]  # exact ties after fp16 rounding
    seen_bits = np.zeros(V // 32, np.uint32)
    for t in rng.integers(0, V, 300):
        seen_bits[t >> 5] |= np.uint32(1 << (t & 31))
    tokens = rng.integers(0, V, M).astype(np.int32)
    # drafts equal to the row argmax of an earlier position, some of them unseen, to exercise the in-block rule
    for t in range(1, M):
        tokens[t] = int(np.argmax(logits[t - 1]))
    keys = orc.verify_argmax(logits, seen_bits, tokens, rep=rep)
    got = orc.keys_to_tokens(keys)
    want = _numpy_verify_argmax(logits, seen_bits, tokens, rep)
    assert got.tolist() == want.tolist()


# ---------------------------------------------------------------- weights (internal/weights/quant_test.go)
def test_quantize_rows_int8_kat(orc, kats):
    kat = kats["quantize_rows_int8"]  # quant_test.go:9-34
    w = orc.f32_to_f16(np.array(kat["w"], np.float32))
    q, s = orc.quantize_rows_int8(w, kat["rows"], kat["k"])
    assert s[0] == np.float32(1.0 / 127)
    assert q[0].tolist() == kat["want_q_row0"]
    assert s[1] == np.float32(1e-8) / np.float32(127)
    assert q[1].tolist() == kat["want_q_row1"]


def test_pack_rows_are_independent(orc):
    rows, k = 3, 2048
    w = orc.f32_to_f16(((np.arange(rows * k) % 251) - 125).astype(np.float32) * np.float32(1e-3))
    b_all, s_all = orc.pack_g128(w, rows, k)
    b_one, s_one = orc.pack_g128(w[k:2 * k], 1, k)
    assert np.array_equal(b_all[1], b_one[0])
    assert np.array_equal(s_all[1], s_one[0])
    # dequantised values reproduce the input within half a step
    s = orc.f16_to_f32(s_all[1][:4 * 4].reshape(4, 4))  # [quarter][i], group g = 4 i + quarter
    deq = np.array([(int(b_all[1][j]) - 128) * s[(j // 128) % 4][(j // 128) // 4] for j in range(k)])
    assert np.max(np.abs(deq - orc.f16_to_f32(w[k:2 * k]))) <= np.max(s) / 2 + 1e-6


def test_transpose_lanes_kat(orc):
    # cmd/pack/main_test.go:8-28
    rows, rank = 128, 256
    src = (np.arange(rows * rank) * 31 % 256).astype(np.uint8)
    dst = orc.transpose_lanes(src)
    for g in range(2):
        for r in range(0, 64, 7):
            for p in range(16):
                for b in (0, 5, 15):
                    frm = (g * 64 + r) * rank + p * 16 + b
                    to = g * 64 * rank + p * 64 * 16 + r * 16 + b
                    assert dst[to] == src[frm]


# ---------------------------------------------------------------- verify attention
def _np_attention(q, k, v, a, start, window, causal):
    """Independent numpy fp64 statement: full softmax with an explicit mask matrix. Context keys (kpos < a) need
    kpos >= start and the window, block keys j = kpos - a only j <= t (causal) or j < M: start and window bound the
    context keys alone (dspark.hip:1311-1312, 2006-2012)."""
    qf = q.view(np.float16).astype(np.float64)
    kf = k.view(np.float16).astype(np.float64)
    vf = v.view(np.float16).astype(np.float64)
    M, QH, D = qf.shape
    KVH = kf.shape[1]
    G = QH // KVH
    T = a + M
    out = np.zeros((M, QH, D))
    kpos = np.arange(T)
    for t in range(M):
        ctx = kpos < a
        valid = ~ctx | (kpos >= start)
        if window:
            valid &= ~ctx | (kpos > a + t - window)
        j = kpos - a
        valid &= ctx | ((j <= t) if causal else (j < M))
        for qh in range(QH):
            h = qh // G
            s = (kf[:T, h, :] @ qf[t, qh]) / math.sqrt(D)
            s = np.where(valid, s, -np.inf)
            if not np.isfinite(s).any():
                continue
            p = np.exp(s - s.max())
            out[t, qh] = (p / p.sum()) @ vf[:T, h, :]
    return out


@pytest.mark.parametrize("M,QH,KVH,D,a,start,window,causal", [
    (9, 32, 8, 64, 100, 0, 0, True),
    (4, 16, 4, 128, 77, 0, 0, True),
    (5, 16, 4, 128, 300, 45, 256, True),   # sliding layer: start = a - window + 1
    (9, 16, 4, 128, 50, 10, 0, False),     # drafter: ring range, bidirectional block
    (1, 8, 8, 64, 0, 0, 0, True),          # empty cache: the token attends only to itself
    (16, 32, 8, 64, 33, 0, 0, True),
    (9, 16, 4, 128, 50, 53, 0, True),      # start inside the block: no context keys, the block's keys all kept
    (9, 16, 4, 128, 50, 56, 0, False),     # the same, bidirectional
    (16, 16, 4, 64, 100, 90, 8, True),     # window shorter than the block: later rows see block keys only
])
def test_attention_matches_numpy(orc, M, QH, KVH, D, a, start, window, causal):
    q = orc.normal_f16(11, (M, QH, D))
    k = orc.normal_f16(12, (a + M, KVH, D))
    v = orc.normal_f16(13, (a + M, KVH, D))
    got = orc.verify_attention(q, k, v, a, start, window, causal)
    want = _np_attention(q, k, v, a, start, window, causal)
    assert np.max(np.abs(got - want)) < 1e-12


def test_attention_matches_torch_sdpa(orc):
    torch = pytest.importorskip("torch")
    M, QH, KVH, D, a = 8, 32, 8, 64, 200
    q = orc.normal_f16(21, (M, QH, D))
    k = orc.normal_f16(22, (a + M, KVH, D))
    v = orc.normal_f16(23, (a + M, KVH, D))
    got = orc.verify_attention(q, k, v, a)
    G = QH // KVH
    qt = torch.from_numpy(q.view(np.float16).astype(np.float64)).permute(1, 0, 2)          # [QH][M][D]
    kt = torch.from_numpy(k.view(np.float16).astype(np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
    vt = torch.from_numpy(v.view(np.float16).astype(np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
    mask = torch.ones(M, a + M, dtype=torch.bool)
    mask[:, a:] = torch.tril(torch.ones(M, M, dtype=torch.bool))
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask).permute(1, 0, 2).numpy()
    assert np.max(np.abs(got - ref)) < 1e-10


def test_attention_closed_forms(orc):
    M, QH, KVH, D = 3, 4, 1, 64
    # zero query: every valid key has equal weight -> output is the mean of the visible V rows
    a = 10
    q = np.zeros((M, QH, D), np.uint16)
    k = orc.normal_f16(31, (a + M, KVH, D))
    v = orc.normal_f16(32, (a + M, KVH, D))
    got = orc.verify_attention(q, k, v, a)
    vf = v.view(np.float16).astype(np.float64)
    for t in range(M):
        assert np.allclose(got[t, 0], vf[:a + t + 1, 0].mean(0), atol=1e-12)
    # one visible key (empty cache, first token): output is that key's V exactly
    got = orc.verify_attention(orc.normal_f16(33, (M, QH, D)), k[:M], v[:M], 0)
    assert np.array_equal(got[0, 2], vf[0, 0])
    # window 1: each context key is outside; only the token's own fresh prefix counts
    got = orc.verify_attention(orc.normal_f16(34, (1, QH, D)), k[:a + 1], v[:a + 1], a, window=1)
    assert np.array_equal(got[0, 1], vf[a, 0])


def test_split_merge_identity(orc):
    M, QH, KVH, D, a = 4, 8, 2, 64, 500
    q = orc.normal_f16(41, (M, QH, D))
    k = orc.normal_f16(42, (a + M, KVH, D))
    v = orc.normal_f16(43, (a + M, KVH, D))
    direct = orc.verify_attention(q, k, v, a).reshape(M * QH, D)
    cuts = [0, 37, 38, 200, 499, 501, a + M]
    parts = [orc.attn_partial(q, k, v, a, k0, k1) for k0, k1 in zip(cuts[:-1], cuts[1:])]
    # an all-masked split (keys beyond the last token) must contribute nothing
    parts.append(orc.attn_partial(q, k, v, a, a + M, a + M))
    merged = orc.attn_merge(*zip(*parts))
    assert np.max(np.abs(merged - direct)) < 1e-12


def test_attention_f32_mt_close_to_fp64(orc):
    M, QH, KVH, D, a = 9, 32, 8, 64, 1024
    q = orc.normal_f16(51, (M, QH, D))
    k = orc.normal_f16(52, (a + M, KVH, D))
    v = orc.normal_f16(53, (a + M, KVH, D))
    want = orc.verify_attention(q, k, v, a)
    got = orc.verify_attention_f32_mt(q, k, v, a, threads=4)
    assert np.max(np.abs(got - want)) < 2e-4


@pytest.mark.parametrize("window,causal,start", [(0, True, 0), (40, True, 470), (0, False, 100)])
def test_attention_mt_is_the_fp64_oracle(orc, window, causal, start):
    """The threaded fp64 form gives the single-threaded oracle's bits (same arithmetic per row)."""
    M, QH, KVH, D, a = 9, 16, 4, 128, 500
    q = orc.normal_f16(61, (M, QH, D))
    k = orc.normal_f16(62, (a + M, KVH, D))
    v = orc.normal_f16(63, (a + M, KVH, D))
    want = orc.verify_attention(q, k, v, a, start, window, causal)
    got = orc.verify_attention_mt(q, k, v, a, start, window, causal, threads=5)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- acceptance / commit (dspark.hip:2848-2913)
def _round(orc, tokens, best, a=1024, count=0, budget=512, stop_at=1056, eos=-1, rounds_left=32):
    st = orc.new_state(a=a, anchor=tokens[0], count=count, rounds_left=rounds_left, budget=budget, eos=eos,
                       stop_at=stop_at, tokens=tokens, run=1, skip_rounds=1)
    out = np.zeros(600, np.int32)
    seen = np.zeros(4096, np.uint32)
    acc = orc.accept_commit(st, np.asarray(best, np.int32), len(tokens), out, seen)
    return acc, st, out, seen


def test_accept_all_none_partial(orc):
    toks = [5, 10, 11, 12, 13]
    acc, st, out, seen = _round(orc, toks, [10, 11, 12, 13, 99])       # 100% planted
    assert acc == 4 and st.a == 1024 + 5 and out[:5].tolist() == [10, 11, 12, 13, 99] and st.anchor == 99
    acc, st, out, _ = _round(orc, toks, [7, 11, 12, 13, 99])            # 0%
    assert acc == 0 and st.a == 1025 and out[:1].tolist() == [7] and st.ctx_new == 1 and st.miss == 1
    acc, st, out, seen = _round(orc, toks, [10, 11, 4, 13, 99])         # stops at the first mismatch
    assert acc == 2 and st.a == 1027 and out[:3].tolist() == [10, 11, 4] and st.accepted == 2 and st.verified == 5
    assert (seen[0] >> 10) & 1 and (seen[0] >> 4) & 1 and not (seen[0] >> 12) & 1
    assert st.tokens[0] == 4 and st.ctx_pos == 1024 and st.rounds_done == 1 and st.run == 1


def test_commit_stop_rules(orc):
    toks = [5, 10, 11, 12]
    _, st, _, _ = _round(orc, toks, [10, 11, 12, 13], eos=11)           # EOS inside the accepted prefix
    assert st.run == 0 and st.count == 4
    _, st, _, _ = _round(orc, toks, [10, 11, 12, 13], stop_at=1027)     # passes stop_at
    assert st.run == 0 and st.a == 1028
    _, st, _, _ = _round(orc, toks, [10, 11, 12, 13], budget=3)         # budget
    assert st.run == 0
    _, st, _, _ = _round(orc, toks, [10, 11, 12, 13], rounds_left=1)    # last round
    assert st.run == 0 and st.rounds_left == 0


def test_kv_commit_positions(orc):
    cache = orc.normal_f16(61, (40, 2, 4))
    before = cache.copy()
    fresh = orc.normal_f16(62, (5, 2, 4))
    orc.kv_commit(cache, fresh, 30, 2)
    assert np.array_equal(cache[30:33], fresh[:3])
    assert np.array_equal(cache[:30], before[:30]) and np.array_equal(cache[33:], before[33:])


# ---------------------------------------------------------------- GEMMs
def test_gemm_i8_matches_numpy(orc):
    M, N, K = 16, 96, 256
    x = orc.normal_f16(71, (M, K))
    w = orc.int8_uniform(72, (N, K))
    s = orc.f32_to_f16(np.random.default_rng(3).uniform(0.001, 0.01, N).astype(np.float32))
    y = orc.gemm_i8(x, w, s)
    ref = (x.view(np.float16).astype(np.float64) @ w.astype(np.float64).T) * s.view(np.float16).astype(np.float64)
    assert np.max(np.abs(y - ref)) < 1e-9
    yb = orc.gemm_i8(x, (w.astype(np.int16) + 128).astype(np.uint8), s, biased=True)
    assert np.array_equal(y, yb)


def test_gemm_f16_and_row_argmax(orc):
    M, N, K = 4, 300, 128
    x = orc.normal_f16(81, (M, K))
    w = orc.normal_f16(82, (N, K), scale=1 / 16)
    y = orc.gemm_f16(x, w)
    ref = x.view(np.float16).astype(np.float64) @ w.view(np.float16).astype(np.float64).T
    assert np.max(np.abs(y - ref)) < 1e-9
    y32 = y.astype(np.float32)
    y32[1, 7] = y32[1, 200] = y32[1].max() + 1  # tie: the smaller index wins
    assert orc.row_argmax(y32).tolist() == [int(np.argmax(r)) for r in y32]
    assert orc.row_argmax(y32)[1] == 7


# ---------------------------------------------------------------- layer pieces
def test_rms_norm_rope_conv(orc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(2048).astype(np.float32)
    w = orc.f32_to_f16(rng.uniform(0.5, 1.5, 2048).astype(np.float32))
    y = orc.rms_norm(x, w)
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w.view(np.float16).astype(np.float64)
    assert np.max(np.abs(y - ref)) < 1e-5
    # RoPE is a rotation: norms of the pairs are preserved, position 0 is the identity, the zero tail passes through
    v = rng.standard_normal(64).astype(np.float32)
    r = orc.rope(v, 16, 1e6, 12345)
    assert np.allclose(np.hypot(r[:32], r[32:]), np.hypot(v[:32], v[32:]), atol=1e-5)
    assert np.array_equal(r[16:32], v[16:32]) and np.array_equal(r[48:], v[48:])
    assert np.allclose(orc.rope(v, 32, 1e4, 0), v)
    # pair 0 turns by exactly pos radians
    e = np.zeros(64, np.float32)
    e[0] = 1
    r = orc.rope(e, 32, 1e4, 3)
    assert abs(r[0] - math.cos(3)) < 1e-6 and abs(r[32] - math.sin(3)) < 1e-6
    # short conv k=3 against np.convolve over the bx sequence
    B, C, X = (rng.standard_normal(6).astype(np.float32) for _ in range(3))
    wk = rng.standard_normal(3).astype(np.float32)
    hist = np.zeros(2, np.float32)
    ys = [orc.conv_step(float(B[i]), float(C[i]), float(X[i]), wk, hist) for i in range(6)]
    bx = (B * X).astype(np.float16).astype(np.float64)
    full = np.convolve(bx, wk[::-1].astype(np.float64))[:6]
    ref = (C * full).astype(np.float32).astype(np.float16).astype(np.float32)
    assert np.allclose(ys, ref, atol=1e-3)
