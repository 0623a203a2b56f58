"""Pins the oracle's int8 K/V record functions (quantize_pair, the record layout, the query's group quantization and
the fp64 attention of dequantized operands) against closed forms, bounds and independent numpy restatements.
CPU only. Reference: kernels/ops.hip:212-251, internal/model/engine.go:30-32, kernels/dspark.hip:1020-1046.
"""
import numpy as np
import pytest

from oracle import oracle as orc


def np_quantize_pair(x):
    """quantize_pair in numpy float32 arithmetic (each operation one IEEE binary32 rounding)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x))
    scale = np.maximum(np.float32(amax) / np.float32(127), np.float32(1e-6)).astype(np.float32)
    inv = (np.float32(1) / scale).astype(np.float32)
    a = (x * inv).astype(np.float32)
    a = np.where(a >= 0, a + np.float32(0.5), a - np.float32(0.5)).astype(np.float32)
    return np.trunc(np.clip(a, -128, 127)).astype(np.int8), np.float32(scale)


def test_quantize_closed_forms():
    # amax 127 -> scale exactly 1: q is x rounded half away from zero
    x = np.zeros(128, np.float32)
    x[:9] = [127, -127, 63.5, -63.5, 0.5, -0.5, 1.49, -2.5, 2.5]
    q, s = orc.rec_quantize(x)
    assert s == np.float32(1.0)
    assert q[:9].tolist() == [127, -127, 64, -64, 1, -1, 1, -3, 3] and not q[9:].any()
    # all zeros: the 1e-6 floor, all codes 0
    q, s = orc.rec_quantize(np.zeros(128, np.float32))
    assert s == np.float32(1e-6) and not q.any()
    # below the floor: scale stays 1e-6, codes are x / 1e-6 rounded
    x = np.zeros(128, np.float32)
    x[0], x[1] = 1e-7, -6e-7
    q, s = orc.rec_quantize(x)
    assert s == np.float32(1e-6) and q[0] == 0 and q[1] == -1
    # exact multiples of the scale come back exactly
    s0 = np.float32(0.25)
    codes = np.arange(-127, 128, 2, dtype=np.int32)[:128]
    x = (codes.astype(np.float32) * s0).astype(np.float32)
    x[0] = -127 * s0
    q, s = orc.rec_quantize(x)
    assert s == s0
    assert np.array_equal(q.astype(np.int32), np.round(x / s0).astype(np.int32))


@pytest.mark.parametrize("seed", range(6))
def test_quantize_bounds_and_numpy(seed):
    rng = np.random.default_rng(seed)
    scale_in = [1.0, 1e-3, 30.0, 1e-7, 5.0, 0.01][seed]
    x = (rng.standard_normal(128) * scale_in).astype(np.float32)
    q, s = orc.rec_quantize(x)
    qn, sn = np_quantize_pair(x)
    assert s == sn and np.array_equal(q, qn)
    assert np.abs(q.astype(np.int32)).max() <= 127
    amax = np.abs(x).max()
    if amax / 127 >= 1e-6:
        assert np.abs(q.astype(np.int32)).max() == 127
    err = np.abs(x.astype(np.float64) - q.astype(np.float64) * float(s))
    assert err.max() <= 0.5 * float(s) * (1 + 1e-5)


def test_record_layout():
    rng = np.random.default_rng(7)
    n, KVH, pos0 = 70, 4, 5
    k = rng.standard_normal((n, KVH, 128)).astype(np.float32)
    v = (rng.standard_normal((n, KVH, 128)) * 3).astype(np.float32)
    bt = np.array([4, 0, 2, 1, 3], dtype=np.int32)
    pages = orc.kv_write_rec(k, v, orc.rec_pages(6, KVH), pos0=pos0, bt=bt)
    for t in (0, 1, 26, 27, 31, 69):
        pos = pos0 + t
        for h in range(KVH):
            kq, ks, vq, vs = orc.rec_read(pages, pos, h, bt)
            kq2, ks2 = np_quantize_pair(k[t, h])
            vq2, vs2 = np_quantize_pair(v[t, h])
            assert np.array_equal(kq, kq2) and ks == ks2 and np.array_equal(vq, vq2) and vs == vs2
            # byte offsets of engine.go:30-32: page * 32 KVH 264 + (slot KVH + h) 264
            flat = pages.reshape(-1)
            off = int(bt[pos // 32]) * 32 * KVH * 264 + ((pos % 32) * KVH + h) * 264
            assert np.array_equal(flat[off:off + 128].view(np.int8), kq2)
            assert flat[off + 128:off + 132].view(np.float32)[0] == ks2
    assert not pages[5].any()                   # a page the table never names stays zero
    assert not pages[int(bt[0]), :pos0].any()  # slots before pos0


def test_query_group_quantization():
    rng = np.random.default_rng(3)
    q = orc.f32_to_f16(rng.standard_normal((12, 128)).astype(np.float32) * 2)
    q8, qs = orc.rec_quantize_q(q)
    qf = orc.f16_to_f32(q).reshape(12, 4, 32)
    s = np.maximum(np.abs(qf).max(axis=2) / np.float32(127), np.float32(1e-20)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    want = np.rint((qf * inv[:, :, None]).astype(np.float32)).astype(np.int8).reshape(12, 128)
    assert np.array_equal(qs, s) and np.array_equal(q8, want)
    assert np.abs(q8.astype(np.int32)).max() == 127


def test_fp64_attention_of_doubles_matches_fp16_oracle():
    q = orc.normal_f16(41, (5, 16, 128))
    k = orc.normal_f16(42, (300, 4, 128))
    v = orc.normal_f16(43, (300, 4, 128))
    for a, start, window, causal in ((295, 0, 0, True), (295, 100, 0, False), (295, 0, 64, True)):
        want = orc.verify_attention(q, k, v, a, start, window, causal)
        got = orc.verify_attention_d(orc.f16_to_f32(q), orc.f16_to_f32(k), orc.f16_to_f32(v), a, start, window,
                                     causal)
        assert np.max(np.abs(got - want)) <= 1e-12


def test_record_attention_is_attention_of_dequantized_operands():
    M, QH, KVH, a = 9, 16, 4, 200
    T = a + M
    rng = np.random.default_rng(11)
    k = rng.standard_normal((T, KVH, 128)).astype(np.float32)
    v = rng.standard_normal((T, KVH, 128)).astype(np.float32)
    bt = np.random.default_rng(1).permutation(9)[:7].astype(np.int32)
    pages = orc.kv_write_rec(k, v, orc.rec_pages(9, KVH), bt=bt)
    q = orc.normal_f16(12, (M, QH, 128))
    got = orc.verify_attention_rec(q, pages, a, bt=bt)
    # the same in numpy: dequantize, then the fp64 oracle
    q8, qs = orc.rec_quantize_q(q.reshape(-1, 128))
    qd = (q8.astype(np.float64).reshape(-1, 4, 32) * qs[:, :, None].astype(np.float64)).reshape(M, QH, 128)
    kd = np.empty((T, KVH, 128))
    vd = np.empty((T, KVH, 128))
    for pos in range(T):
        for h in range(KVH):
            kq, ks, vq, vs = orc.rec_read(pages, pos, h, bt)
            kd[pos, h] = kq.astype(np.float64) * float(ks)
            vd[pos, h] = vq.astype(np.float64) * float(vs)
    want = orc.verify_attention_d(qd, kd, vd, a)
    assert np.max(np.abs(got - want)) <= 1e-12
    # quantization moves the result little from the fp32 attention of the unquantized operands
    ref = orc.verify_attention_d(orc.f16_to_f32(q), k, v, a)
    assert np.max(np.abs(got - ref)) < 0.05
    # a single visible key returns its dequantized V
    one = orc.verify_attention_rec(q[:1], pages, 0, causal=True, bt=bt)
    kq, ks, vq, vs = orc.rec_read(pages, 0, 1, bt)
    assert np.allclose(one[0, 4:8], vq.astype(np.float64) * float(vs), atol=1e-12)
