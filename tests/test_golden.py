"""The committed golden fixtures: the oracle reproduces tests/golden/vectors.npz from its stored inputs, and the
fixtures themselves satisfy the reference's own invariants (so a regenerated file with a planted mistake fails here
before any GPU test compares against it)."""
import numpy as np

from golden.make_vectors import STATE_FIELDS


def test_attention_vectors(orc, golden):
    for i, (M, QH, KVH, D, a, start, window, causal, seed) in enumerate(golden["attn_cases"].tolist()):
        q, k, v = golden[f"attn{i}_q"], golden[f"attn{i}_k"], golden[f"attn{i}_v"]
        assert q.shape == (M, QH, D) and k.shape == (a + M, KVH, D) and v.shape == k.shape
        got = orc.verify_attention(q, k, v, a, start, window, bool(causal))
        np.testing.assert_allclose(got, golden[f"attn{i}_out"], rtol=0, atol=1e-12)
        # inputs are the seeded generator's: the fixture and the oracle's generator agree
        assert np.array_equal(q, orc.normal_f16(seed, (M, QH, D)))


def test_argmax_commit_vectors(orc, golden):
    M, V, a, _ = golden["argmax_meta"].tolist()
    rep = float(golden["argmax_rep"])
    logits = orc.f16_to_f32(golden["argmax_logits"])
    keys = orc.verify_argmax(logits, golden["argmax_seen"], golden["argmax_tokens"], rep=rep)
    assert np.array_equal(keys, golden["argmax_keys"])
    tokens = golden["argmax_tokens"]
    st = orc.new_state(a=a, anchor=int(tokens[0]), tokens=tokens, rounds_left=32, budget=512, eos=-1, stop_at=1056,
                       run=1, skip_rounds=1)
    emitted = np.zeros(64, np.int32)
    bits = golden["argmax_seen"].copy()
    acc = orc.accept_commit(st, orc.keys_to_tokens(keys), M, emitted, bits)
    assert acc == int(golden["argmax_acc"])
    assert [getattr(st, f) for f in STATE_FIELDS] == golden["argmax_state"].tolist()
    assert np.array_equal(emitted, golden["argmax_emitted"])
    assert np.array_equal(bits, golden["argmax_seen_after"])
    # the fixture planted five argmax drafts, then a miss: greedy acceptance stops at 5
    assert acc == 5 and golden["argmax_state"][STATE_FIELDS.index("a")] == a + acc + 1
    best = orc.keys_to_tokens(keys)
    assert golden["argmax_emitted"][:acc + 1].tolist() == best[:acc + 1].tolist()


def test_gemm_and_head_vectors(orc, golden):
    w = (golden["gemm_wb"].astype(np.int16) - 128).astype(np.int8)
    np.testing.assert_allclose(orc.gemm_i8(golden["gemm_x"], w, golden["gemm_s"]), golden["gemm_out"], rtol=0,
                               atol=1e-12)
    # independent form: fp64 numpy of the same int8 x scale product
    x = orc.f16_to_f32(golden["gemm_x"]).astype(np.float64)
    s = orc.f16_to_f32(golden["gemm_s"]).astype(np.float64)
    np.testing.assert_allclose(golden["gemm_out"], (x @ w.astype(np.float64).T) * s[None, :], rtol=1e-12, atol=1e-12)
    y = orc.gemm_f16(golden["head_x"], golden["head_w"])
    np.testing.assert_allclose(y, golden["head_out"], rtol=0, atol=1e-12)
    assert np.array_equal(golden["head_argmax"], np.argmax(golden["head_out"].astype(np.float32), axis=1))
