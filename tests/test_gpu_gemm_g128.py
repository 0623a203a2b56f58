"""GPU parity of the int8 GEMM over per-128-column weight scales (the reference's weights.Pack format) through the C
ABI, against the fp64 oracle (orc_gemm_g128). Bar: max-abs <= 2e-3 x the largest output (fp32 accumulation of fp16
products against fp64), and for the gated epilogues the same bar on the activation. Shapes: the reference geometry's
GEMMs (hidden 2048, FFN 7680, 16/4/128 attention mix, 5-tap fc, 128000-row head) at 1, 9 and 16 tokens."""
import numpy as np
import pytest

from conftest import load_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def case(torch, orc, M, N, K, epilogue, seed):
    host = load_host()
    print(f"case gemm_g128 M={M} N={N} K={K} epi={epilogue}", flush=True)
    rng = np.random.default_rng(seed)
    x = orc.normal_f16(seed, (M, K))
    wb = rng.integers(1, 256, (N, K), dtype=np.uint8)
    gs = orc.f32_to_f16((rng.uniform(0.5, 1.5, (K // 128, N)) / (73.3 * np.sqrt(K))).astype(np.float32))
    want = orc.gemm_g128(x, wb, gs)
    xd = torch.from_numpy(x.view(np.float16)).cuda()
    wd = torch.from_numpy(wb).cuda()
    gd = torch.from_numpy(gs.view(np.float16)).cuda()
    if epilogue == 0:
        y, _ = host.gemm_i8_g128(xd, wd, gd)
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
        ref = want
    else:
        y16 = torch.empty((M, N // 2 if epilogue == 1 else N), dtype=torch.float16, device="cuda")
        host.gemm_i8_g128(xd, wd, gd, epilogue=epilogue, y_f16=y16)
        torch.cuda.synchronize()
        got = y16.cpu().numpy().astype(np.float64)
        if epilogue == 1:
            g, u = want[:, 0::2], want[:, 1::2]
            ref = (g / (1 + np.exp(-g))) * u
        else:
            ref = want / (1 + np.exp(-want))
    err = np.max(np.abs(got - ref))
    scale = max(1.0, np.max(np.abs(ref))) if epilogue else np.max(np.abs(ref))
    assert err <= 2e-3 * scale, f"max-abs {err} (scale {scale})"
    # run-to-run identical
    if epilogue == 0:
        y2, _ = host.gemm_i8_g128(xd, wd, gd)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


@pytest.mark.parametrize("M,N,K,epilogue", [
    (9, 2048, 2048, 0),      # out projection
    (9, 3088, 2048, 0),      # attention mix (16 q + 4 k + 4 v heads of 128, 16 gates, 16-row aligned)
    (9, 15360, 2048, 1),     # w13, gated SiLU
    (9, 2048, 7680, 0),      # w2 (60 groups)
    (9, 2048, 10240, 0),     # fc over 5 taps
    (1, 2048, 2048, 2),      # one token, SiLU
    (16, 3072, 2048, 0),     # drafter mix at 16 tokens
    (9, 128000, 2048, 0),    # LM head
])
def test_gemm_g128_matches_oracle(dev, orc, M, N, K, epilogue):
    case(dev, orc, M, N, K, epilogue, 40 + M + N // 16 + K // 128)
