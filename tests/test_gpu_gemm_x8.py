"""GPU parity of the int8 GEMM with the reference's default activation format (LFM3_X8, kernels/dspark.hip:24-26:
the input as int8 with one fp32 scale per 16 columns, int8 x int8 products; unit_dot_r 541-566) through the C ABI,
against the fp64 oracle (orc_gemm_x8). Two input forms:

* codes given (the norm kernel's output): x holds the int8 codes as integer-valued fp16 and xscale their scales. The
  integer dots are exact on both sides, so GPU and oracle differ only in the fp32 summation order of the scaled
  pieces: bar 1e-4 x the largest output.
* fp16 x quantized as it is loaded (x_fill, 883-904): the GPU takes 1 / s with the hardware reciprocal, as the
  reference does, the oracle with IEEE fp32; a product x * (1 / s) within an ulp of a rounding midpoint can then take
  the neighbouring code on one side, one code step on one input: bar 1e-3 x the largest output.

Shapes: the reference geometry's GEMMs at 1, 9 and 16 tokens, both kernels (X per wave, X^T through LDS)."""
import numpy as np
import pytest

from conftest import load_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def case(torch, orc, M, N, K, epilogue, seed, given):
    host = load_host()
    print(f"case gemm_x8 M={M} N={N} K={K} epi={epilogue} codes_given={given}", flush=True)
    rng = np.random.default_rng(seed)
    xf = (rng.standard_normal((M, K)) * rng.uniform(0.2, 4.0, (M, 1))).astype(np.float32)
    x16 = orc.f32_to_f16(xf)
    wb = rng.integers(1, 256, (N, K), dtype=np.uint8)
    gs = orc.f32_to_f16((rng.uniform(0.5, 1.5, (K // 128, N)) / (73.3 * np.sqrt(K))).astype(np.float32))
    if given:
        q, s = orc.quantize_x16(xf)
        xin = orc.f32_to_f16(q.astype(np.float32))
        xsd = torch.from_numpy(s).cuda()
    else:
        q, s = orc.quantize_x16(orc.f16_to_f32(x16))
        xin = x16
        xsd = None
    want = orc.gemm_x8(q, s, wb, gs)
    xd = torch.from_numpy(xin.view(np.float16)).cuda()
    wd = torch.from_numpy(wb).cuda()
    gd = torch.from_numpy(gs.view(np.float16)).cuda()
    bar = 1e-4 if given else 1e-3
    if epilogue == 0:
        y, _ = host.gemm_i8_g128_x8(xd, wd, gd, xscale=xsd)
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
        ref = want
    else:
        y16 = torch.empty((M, N // 2), dtype=torch.float16, device="cuda")
        host.gemm_i8_g128_x8(xd, wd, gd, xscale=xsd, epilogue=1, y_f16=y16)
        torch.cuda.synchronize()
        got = y16.cpu().numpy().astype(np.float64)
        g, u = want[:, 0::2], want[:, 1::2]
        ref = (g / (1 + np.exp(-g))) * u
        bar = max(bar, 2e-3)  # the fp16 store of the activation
    scale = np.max(np.abs(ref))
    err = np.max(np.abs(got - ref))
    print(f"max-abs {err:.3e} = {err / scale:.2e} x scale {scale:.2f}", flush=True)
    assert err <= bar * scale, f"max-abs {err} (scale {scale})"
    # the int8 input is not the fp16 one: the result must move by about the quantization error, not by nothing
    if epilogue == 0 and not given:
        plain = orc.gemm_g128(x16, wb, gs)
        assert np.max(np.abs(plain - want)) > 1e-6 * scale
    # run-to-run identical
    if epilogue == 0:
        y2, _ = host.gemm_i8_g128_x8(xd, wd, gd, xscale=xsd)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


@pytest.mark.parametrize("given", [True, False])
@pytest.mark.parametrize("M,N,K,epilogue", [
    (9, 2048, 2048, 0),      # out projection
    (9, 3088, 2048, 0),      # attention mix
    (9, 15360, 2048, 1),     # w13, gated SiLU (X^T through LDS)
    (9, 2048, 7680, 0),      # w2 (60 groups)
    (9, 2048, 10240, 0),     # fc over 5 taps
    (1, 2048, 2048, 0),      # one token
    (16, 3072, 2048, 0),     # drafter mix at 16 tokens
    (9, 128000, 2048, 0),    # LM head (X^T through LDS)
])
def test_gemm_x8_matches_oracle(dev, orc, M, N, K, epilogue, given):
    case(dev, orc, M, N, K, epilogue, 90 + M + N // 16 + K // 128, given)


def test_gemm_x8_refuses_row_scales(dev):
    """int8 x goes with per-128-column weight scales only: K not a multiple of 128 is refused before any launch."""
    torch = dev
    host = load_host()
    x = torch.zeros((4, 192), dtype=torch.float16, device="cuda")
    w = torch.zeros((16, 192), dtype=torch.uint8, device="cuda")
    gs = torch.zeros((1, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(host.DsparkError, match="EINVAL"):
        host.gemm_i8_g128_x8(x, w, gs)
