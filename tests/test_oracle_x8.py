"""Pins the oracle's LFM3_X8 arithmetic: the per-16-column int8 quantization of GEMM inputs and the GEMM over int8
codes with per-piece activation scales and per-128-column weight scales. CPU only. Reference: kernels/dspark.hip:24-26
(LFM3_X8 is the default build), 541-566 (unit_dot_r), 802-823 (norm_compute), 883-904 (x_fill)."""
import numpy as np
import pytest

from oracle import oracle as orc


def test_integer_pieces_with_max_127_are_their_own_codes():
    """A piece of integers whose largest magnitude is 127 has scale exactly 1 and codes equal to the values."""
    rng = np.random.default_rng(1)
    x = rng.integers(-126, 127, (5, 64)).astype(np.float32)
    x[:, ::16] = 127 * np.where(rng.random((5, 4)) < 0.5, -1, 1)
    q, s = orc.quantize_x16(x)
    assert np.all(s == 1.0)
    assert np.array_equal(q.astype(np.float32), x)


def test_round_trip_bound_max_code_and_floor():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((7, 256)) * rng.uniform(1e-3, 30, (7, 1))).astype(np.float32)
    x[3, 32:48] = 0.0  # an all-zero piece: the 1e-20 floor, every code 0
    q, s = orc.quantize_x16(x)
    pieces = x.reshape(7, 16, 16)
    amax = np.abs(pieces).max(axis=2)
    assert np.array_equal(s, np.maximum(amax / np.float32(127), np.float32(1e-20)))
    assert s[3, 2] == np.float32(1e-20) and not q[3, 32:48].any()
    deq = q.reshape(7, 16, 16).astype(np.float64) * s[:, :, None].astype(np.float64)
    assert np.all(np.abs(deq - pieces) <= 0.5 * s[:, :, None] * (1 + 1e-6))
    # the piece's largest magnitude takes the code +-127
    arg = np.abs(pieces).argmax(axis=2)
    top = np.take_along_axis(q.reshape(7, 16, 16), arg[:, :, None], axis=2)[:, :, 0]
    live = amax > 0
    assert np.all(np.abs(top[live]) == 127)


@pytest.mark.parametrize("K", [256, 2048])
def test_x8_gemm_is_the_group_gemm_of_codes_times_piece_scales(K):
    """fp64 numpy: y = sum_p fp32(gs[p / 8] * s_p) * (w_p . q_p); with unit piece scales it is the per-128-column
    GEMM of the codes (orc_gemm_g128 on integer-valued fp16 x)."""
    rng = np.random.default_rng(K)
    M, N = 4, 48
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    q, s = orc.quantize_x16(x)
    w = rng.integers(1, 256, (N, K), dtype=np.uint8)
    gs = orc.f32_to_f16(rng.uniform(0.001, 0.02, (K // 128, N)).astype(np.float32))
    got = orc.gemm_x8(q, s, w, gs)
    gsf = orc.f16_to_f32(gs)
    wq = w.astype(np.float64) - 128
    want = np.zeros((M, N))
    for p in range(K // 16):
        d = q[:, 16 * p:16 * p + 16].astype(np.float64) @ wq[:, 16 * p:16 * p + 16].T
        f = (gsf[p // 8][None, :] * s[:, p][:, None]).astype(np.float32).astype(np.float64)
        want += f * d
    assert np.allclose(got, want, rtol=1e-13, atol=1e-13)
    ones = np.ones_like(s)
    codes16 = orc.f32_to_f16(q.astype(np.float32))
    assert np.allclose(orc.gemm_x8(q, ones, w, gs), orc.gemm_g128(codes16, w, gs), rtol=1e-13, atol=1e-13)
    # and the x8 result stays within the quantization error of the unquantized fp64 product
    exact = sum((x[:, 128 * g:128 * g + 128].astype(np.float64) @ wq[:, 128 * g:128 * g + 128].T) * gsf[g][None, :]
                for g in range(K // 128))
    step = np.repeat(s, 16, axis=1).astype(np.float64)  # [M][K] code step of each input
    bound = (0.5 * step) @ np.abs(wq * np.repeat(gsf, 128, axis=0).T).T + 1e-9
    assert np.all(np.abs(got - exact) <= bound * (1 + 1e-6))


def test_round_weights_mm_x8_matches_the_c_oracle():
    """oracle/round.py's vectorized LFM3_X8 GEMM (Weights.mm) against orc_gemm_x8 on the same codes and scales."""
    from types import SimpleNamespace
    from oracle import round as rnd
    rng = np.random.default_rng(7)
    M, N, K = 9, 64, 512
    w = rng.integers(1, 256, (N, K), dtype=np.uint8)
    gs = orc.f32_to_f16(rng.uniform(0.001, 0.02, (K // 128, N)).astype(np.float32))
    W = rnd.Weights(SimpleNamespace(weight_format=1, x_format=1), {"t.w": w.ravel(), "t.s": gs.ravel()})
    wq, s = W.gemm_w("t", N, K)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32).astype(np.float64)
    q, sc = orc.quantize_x16(x.astype(np.float32))
    assert np.allclose(W.mm(x, wq, s), orc.gemm_x8(q, sc, w, gs), rtol=1e-12, atol=1e-12)
