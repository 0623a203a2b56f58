"""Pins the oracle's GEMM over per-128-column weight scales (the reference's weights.Pack format) and the library's
host converter of the packer's scale layout. CPU only. Reference: internal/weights/quant.go:13-29, 66-104."""
import numpy as np
import pytest

from conftest import load_host
from oracle import oracle as orc


def test_uniform_group_scales_reduce_to_row_scales():
    """All groups of a row sharing one scale: the group GEMM equals the per-row-scale GEMM (the same integer sums)."""
    rng = np.random.default_rng(1)
    M, N, K = 5, 48, 512
    x = orc.f32_to_f16(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(1, 256, (N, K), dtype=np.uint8)
    s = orc.f32_to_f16((rng.uniform(0.5, 1.5, N) / 100).astype(np.float32))
    gs = np.tile(s, (K // 128, 1))
    got = orc.gemm_g128(x, w, gs)
    want = orc.gemm_i8(x, w, s, biased=True)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))


def test_numpy_restatement_and_group_isolation():
    rng = np.random.default_rng(2)
    M, N, K = 3, 32, 384
    x = orc.f32_to_f16(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(1, 256, (N, K), dtype=np.uint8)
    gs = orc.f32_to_f16(rng.uniform(0.001, 0.02, (K // 128, N)).astype(np.float32))
    q = w.astype(np.float64) - 128
    xf = orc.f16_to_f32(x).astype(np.float64)
    gsf = orc.f16_to_f32(gs).astype(np.float64)
    want = sum((xf[:, 128 * g:128 * g + 128] @ q[:, 128 * g:128 * g + 128].T) * gsf[g][None, :] for g in range(K // 128))
    assert np.allclose(orc.gemm_g128(x, w, gs), want, rtol=1e-12, atol=1e-12)
    # a scale of group 1 only moves the columns of group 1
    gs2 = gs.copy()
    gs2[1] = orc.f32_to_f16(np.zeros(N, np.float32))
    d = orc.gemm_g128(x, w, gs) - orc.gemm_g128(x, w, gs2)
    assert np.allclose(d, (xf[:, 128:256] @ q[:, 128:256].T) * gsf[1][None, :], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("K", [2048, 7680])
def test_packed_weights_reproduce_the_matrix(K):
    """weights.Pack (orc_pack_g128) then the layout converter then the group GEMM: within the quantization bound of the
    fp16 matrix product (half a code step per weight), and the converter matches the packer's index rule."""
    host = load_host()
    rng = np.random.default_rng(K)
    M, N = 4, 32
    wf = orc.f32_to_f16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    biased, packed = orc.pack_g128(wf, N, K)
    srow = 16 if K // 512 == 4 else 64
    sq = srow // 4
    gs = host.g128_scales(packed.reshape(N, srow), N, K)
    for g in range(K // 128):
        assert np.array_equal(gs[g], packed.reshape(N, srow)[:, (g % 4) * sq + g // 4])
    x = orc.f32_to_f16(rng.standard_normal((M, K)).astype(np.float32))
    got = orc.gemm_g128(x, biased, gs)
    xf = orc.f16_to_f32(x).astype(np.float64)
    want = xf @ orc.f16_to_f32(wf).astype(np.float64).T
    step = np.repeat(orc.f16_to_f32(gs).astype(np.float64), 128, axis=0)  # [K][N] code step of each weight
    bound = np.abs(xf) @ (0.5 * step) + 1e-9
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("K", [128, 384, 640, 7552])
def test_converter_refuses_unpacked_groups(K):
    """weights.Pack stores group g's scale only while g / 4 < groups / 4 (quant.go:96-99): a K that is not a multiple
    of 512 leaves trailing groups without a stored scale, so the converter refuses it instead of reading padding."""
    host = load_host()
    srow = 16 if K // 512 == 4 else 64
    packed = np.ones((4, srow), dtype=np.uint16)
    with pytest.raises(host.DsparkError):
        host.g128_scales(packed, 4, K)


def test_converter_against_the_packers_layout_at_1024():
    """K = 1024 (8 groups, SRow 64): every group's scale comes from the slot the packer wrote, none from padding."""
    host = load_host()
    rng = np.random.default_rng(1024)
    N, K = 16, 1024
    wf = orc.f32_to_f16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    _, packed = orc.pack_g128(wf, N, K)
    packed = packed.reshape(N, 64)
    gs = host.g128_scales(packed, N, K)
    amax = np.abs(orc.f16_to_f32(wf).astype(np.float32)).reshape(N, K // 128, 128).max(axis=2)
    assert np.array_equal(gs.T, orc.f32_to_f16(np.maximum(amax, 1e-8) / 127))
