"""dspark_verify_attention_noalloc (the entry point that allocates nothing) against dspark_verify_attention, through
the C ABI: two calls in a row on one GPU, the second with a smaller input, each bit-identical to the workspace entry
point's output on the same arguments and within the fp64 oracle's 2e-3 max-abs; a shape whose partials exceed the
static scratch array is refused before any launch."""
import ctypes

import numpy as np
import pytest

from conftest import load_host

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def test_noalloc_matches_the_workspace_entry_point(dev, orc):
    torch = dev
    host = load_host()
    lib = host.lib()
    sh = host.stream_handle()
    f16 = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.float16)).cuda()
    cases = [(33, 32, 8, 64, 6000, True), (9, 16, 4, 128, 1500, False)]  # the second call is smaller
    for i, (M, QH, KVH, D, a, gated) in enumerate(cases):
        print(f"case noalloc call {i}: M={M} QH={QH} KVH={KVH} D={D} a={a}", flush=True)
        q = orc.normal_f16(1200 + i, (M, QH, D))
        k = orc.normal_f16(1300 + i, (a + M, KVH, D))
        v = orc.normal_f16(1400 + i, (a + M, KVH, D))
        kp, vp = host.kv_to_pages(f16(k), f16(v))
        qd = f16(q)
        gate = torch.from_numpy(np.random.default_rng(i).standard_normal((M, QH)).astype(np.float32)).cuda() if gated \
            else None
        ref = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
        host.verify_attention(qd, kp, vp, a, out_f32=ref, gate=gate)
        out = torch.full((M, QH, D), float("nan"), dtype=torch.float32, device="cuda")
        out16 = torch.full((M, QH, D), float("nan"), dtype=torch.float16, device="cuda")
        args = host.attn_args(qd, kp, vp, a, out=out16, out_f32=out, gate=gate)
        args.workspace, args.workspace_bytes = None, 0  # ignored by the entry point
        host.check(lib.dspark_verify_attention_noalloc(ctypes.byref(args), sh), "dspark_verify_attention_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: max diff {(out - ref).abs().max().item()}"
        assert torch.equal(out16, ref.to(torch.float16))
        want = orc.verify_attention(q, k, v, a)
        if gated:
            want = want * (1.0 / (1.0 + np.exp(-gate.cpu().numpy().astype(np.float64))))[:, :, None]
        assert np.max(np.abs(out.cpu().numpy() - want)) <= TOL


def test_noalloc_refuses_partials_beyond_its_scratch(dev):
    host = load_host()
    lib = host.lib()
    torch = dev
    M, QH, KVH, D, a = 64, 64, 16, 128, 20000  # 256 rows per KV head, 64 splits: > 16 MiB of partials
    q = torch.zeros((M, QH, D), dtype=torch.float16, device="cuda")
    kp, vp = host.kv_pages_alloc((a + M + 31) // 32, KVH, D)
    out = torch.zeros((M, QH, D), dtype=torch.float32, device="cuda")
    args = host.attn_args(q, kp, vp, a, out_f32=out, splits=64)
    assert lib.dspark_verify_attention_workspace(ctypes.byref(args)) > 16 << 20
    assert lib.dspark_verify_attention_noalloc(ctypes.byref(args), host.stream_handle()) == 1002
