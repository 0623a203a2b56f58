"""The HIP path through the C ABI against the committed golden vectors (tests/golden/vectors.npz): verify attention
within 2e-3 max-abs, argmax keys / acceptance / State / emitted tokens / seen bitmap bit-exact, int8 GEMM within 2e-3
of the output scale, crop-head argmax exact (the fixture's rows have no near ties)."""
import numpy as np
import pytest

from conftest import load_host
from golden.make_vectors import STATE_FIELDS

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def f16(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).cuda()


def test_golden_attention(dev, golden):
    torch = dev
    host = load_host()
    for i, (M, QH, KVH, D, a, start, window, causal, _) in enumerate(golden["attn_cases"].tolist()):
        print(f"case golden attn{i} M={M} QH={QH} KVH={KVH} D={D} a={a} start={start} window={window} "
              f"causal={causal}", flush=True)
        kp, vp = host.kv_to_pages(f16(torch, golden[f"attn{i}_k"]), f16(torch, golden[f"attn{i}_v"]))
        qd = f16(torch, golden[f"attn{i}_q"])
        out = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
        host.verify_attention(qd, kp, vp, a, start, window, bool(causal), out_f32=out)
        torch.cuda.synchronize()
        err = np.max(np.abs(out.cpu().numpy() - golden[f"attn{i}_out"]))
        assert err <= TOL, f"attn{i}: max-abs {err}"


def test_golden_argmax_commit(dev, golden):
    torch = dev
    host = load_host()
    M, V, a, _ = golden["argmax_meta"].tolist()
    rep = float(golden["argmax_rep"])
    tokens = golden["argmax_tokens"]
    print(f"case golden argmax M={M} V={V} rep={rep}", flush=True)
    st = host.state_tensor(a=a, anchor=int(tokens[0]), tokens=tokens, rounds_left=32, budget=512, eos=-1,
                           stop_at=1056, run=1, skip_rounds=1)
    seen = torch.from_numpy(golden["argmax_seen"].view(np.int32).copy()).cuda()
    best = host.verify_argmax(f16(torch, golden["argmax_logits"]), seen, st, rep=rep)
    torch.cuda.synchronize()
    assert np.array_equal(best.cpu().numpy().view(np.uint64), golden["argmax_keys"])
    out = torch.zeros(64, dtype=torch.int32, device="cuda")
    host.accept_commit(st, best, M, out, seen)
    torch.cuda.synchronize()
    gst = host.state_from_tensor(st)
    assert [getattr(gst, f) for f in STATE_FIELDS] == golden["argmax_state"].tolist()
    assert list(gst.tokens)[:M] == golden["argmax_state_tokens"].tolist()
    assert np.array_equal(out.cpu().numpy(), golden["argmax_emitted"])
    assert np.array_equal(seen.cpu().numpy().view(np.uint32), golden["argmax_seen_after"])


def test_golden_gemm_and_head(dev, golden):
    torch = dev
    host = load_host()
    print("case golden gemm_i8 + head", flush=True)
    y = host.gemm_i8(f16(torch, golden["gemm_x"]), torch.from_numpy(golden["gemm_wb"]).cuda(),
                     f16(torch, golden["gemm_s"]))
    torch.cuda.synchronize()
    want = golden["gemm_out"]
    assert np.max(np.abs(y.cpu().numpy().astype(np.float64) - want)) <= TOL * np.max(np.abs(want))
    yh = torch.empty(golden["head_out"].shape, dtype=torch.float32, device="cuda")
    best = host.head_argmax(f16(torch, golden["head_x"]), f16(torch, golden["head_w"]), y_f32=yh)
    torch.cuda.synchronize()
    assert np.max(np.abs(yh.cpu().numpy() - golden["head_out"])) <= TOL
    top2 = np.sort(golden["head_out"], axis=1)[:, -2:]
    assert np.all(top2[:, 1] - top2[:, 0] > 1e-3)  # no near ties in the fixture: the argmax is exact
    assert host.keys_to_tokens(best).cpu().numpy().tolist() == golden["head_argmax"].tolist()
