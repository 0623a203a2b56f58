"""GPU parity of verify attention (through the C ABI) against the fp64 CPU oracle.

Bar: max-abs error <= 2e-3 against the oracle on the same seeded fp16 inputs, plus
run-to-run bit identity. Shapes cover the configs' geometry (32/8/64), the reference geometry (16/4/128), causal and
bidirectional blocks, sliding windows, a paged block table, empty and ragged contexts.
"""
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


def f16(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).cuda()


def run_case(torch, orc, host, M, QH, KVH, D, a, start=0, window=0, causal=True, seed=100, paged=False, splits=0):
    print(f"case M={M} QH={QH} KVH={KVH} D={D} a={a} start={start} window={window} causal={causal} paged={paged}",
          flush=True)
    T = a + M
    q = orc.normal_f16(seed, (M, QH, D))
    k = orc.normal_f16(seed + 1, (T, KVH, D))
    v = orc.normal_f16(seed + 2, (T, KVH, D))
    want = orc.verify_attention(q, k, v, a, start, window, causal)
    npages = (T + 31) // 32
    bt = None
    if paged:
        perm = np.random.default_rng(seed).permutation(npages + 3)[:npages].astype(np.int32)
        bt = torch.from_numpy(perm).cuda()
        kp, vp = host.kv_pages_alloc(npages + 3, KVH, D)
        # cache rows 0..a-1 then the verified tokens' rows a..a+M-1 (the append a verify round does)
        host.kv_write(f16(torch, k[:a]), f16(torch, v[:a]), kp, vp, 0, bt)
        host.kv_write(f16(torch, k[a:]), f16(torch, v[a:]), kp, vp, a, bt)
    else:
        kp, vp = host.kv_to_pages(f16(torch, k), f16(torch, v))
    qd = f16(torch, q)
    out32 = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
    out16 = torch.empty((M, QH, D), dtype=torch.float16, device="cuda")
    host.verify_attention(qd, kp, vp, a, start, window, causal, out=out16, out_f32=out32, block_table=bt,
                          splits=splits)
    torch.cuda.synchronize()
    got = out32.cpu().numpy().astype(np.float64)
    err = np.max(np.abs(got - want))
    assert err <= TOL, f"max-abs {err}"
    err16 = np.max(np.abs(out16.cpu().numpy().astype(np.float64) - want))
    assert err16 <= TOL, f"fp16 output max-abs {err16}"
    # bit-identical on a second run
    out32b = torch.empty_like(out32)
    host.verify_attention(qd, kp, vp, a, start, window, causal, out_f32=out32b, block_table=bt, splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out32, out32b)
    return err


@pytest.mark.parametrize("M,QH,KVH,D,a,start,window,causal,paged", [
    (9, 32, 8, 64, 1024, 0, 0, True, False),      # C1 geometry
    (16, 32, 8, 64, 4096, 0, 0, True, False),     # C2 shape at a short context
    (1, 32, 8, 64, 777, 0, 0, True, False),       # single token, ragged context
    (16, 32, 8, 64, 0, 0, 0, True, False),        # empty cache: causal block only
    (5, 32, 8, 64, 3000, 2745, 256, True, False), # sliding window (start = a - window + 1)
    (16, 32, 8, 64, 2000, 300, 0, False, False),  # drafter: ring range, bidirectional block
    (9, 16, 4, 128, 1500, 0, 0, True, False),     # reference geometry
    (9, 16, 4, 128, 1000, 745, 256, True, True),  # reference sliding layer, paged
    (16, 32, 8, 64, 5000, 0, 0, True, True),      # permuted block table
    (33, 32, 8, 64, 2048, 0, 0, True, False),     # C5 block (M = 33): one page lane, 4 pages per lane per step
    (33, 32, 8, 64, 3100, 0, 0, True, True),      # same, permuted block table, ragged last step
    (24, 32, 8, 64, 2500, 0, 0, True, True),      # 6 row blocks: two page lanes, 2 pages per lane per step
    (64, 32, 8, 64, 1500, 200, 0, False, False),  # 16 row blocks, bidirectional block
    (64, 32, 8, 64, 1500, 0, 0, True, False),     # 16 row blocks, causal block over three pages
    (64, 16, 4, 64, 300, 0, 0, True, True),       # the same with 4 KV heads, permuted block table
    (64, 16, 4, 64, 300, 261, 40, True, False),   # sliding window shorter than the block (later rows see block keys only)
    (33, 32, 8, 64, 2048, 2017, 32, True, False), # the same at 33 tokens, window of one page
    (16, 32, 8, 64, 300, 305, 0, True, False),    # start inside the block: it bounds context keys only
    (9, 16, 4, 128, 300, 304, 0, False, True),    # the same, bidirectional, permuted block table
    (16, 32, 8, 64, 300, 900, 0, True, False),    # start past the block's last position: no context key, block keys kept
    (9, 16, 4, 128, 300, 5000, 0, False, True),   # the same, bidirectional, permuted block table
    (33, 16, 4, 128, 1700, 0, 0, True, True),     # reference geometry, 9 row blocks: one page per step, Q apart
    (24, 16, 4, 128, 900, 0, 0, True, False),     # reference geometry, 6 row blocks
])
def test_verify_attention_matches_oracle(dev, orc, M, QH, KVH, D, a, start, window, causal, paged):
    host = load_host()
    run_case(dev, orc, host, M, QH, KVH, D, a, start, window, causal, paged=paged)


@pytest.mark.parametrize("splits", [1, 3, 64])
def test_verify_attention_split_counts(dev, orc, splits):
    host = load_host()
    run_case(dev, orc, host, 16, 32, 8, 64, 3000, splits=splits, seed=300)


@pytest.mark.parametrize("M,D,a,splits", [(16, 64, 5000, 0), (33, 64, 2048, 0), (9, 128, 1500, 0), (16, 64, 3000, 64)])
def test_one_call_matches_two_phases(dev, orc, M, D, a, splits):
    """dspark_verify_attention gives the same bits as its two phases called apart (split pass, then merge), call after
    call on one workspace that starts out filled with NaN bytes, with the sigmoid gate."""
    torch = dev
    host = load_host()
    lib = host.lib()
    QH, KVH = (32, 8) if D == 64 else (16, 4)
    print(f"case one-call M={M} D={D} a={a} splits={splits}", flush=True)
    T = a + M
    q = orc.normal_f16(700 + M, (M, QH, D))
    k = orc.normal_f16(701 + M, (T, KVH, D))
    v = orc.normal_f16(702 + M, (T, KVH, D))
    kp, vp = host.kv_to_pages(f16(torch, k), f16(torch, v))
    ws = host.Workspace()
    gate = torch.from_numpy(np.random.default_rng(M).standard_normal((M, QH)).astype(np.float32)).cuda()
    ref = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
    qd = f16(torch, q)  # attn_args keeps raw pointers: the tensors must stay alive while args is used
    args = host.attn_args(qd, kp, vp, a, out_f32=ref, gate=gate, splits=splits)
    need = lib.dspark_verify_attention_workspace(ctypes.byref(args))
    buf = ws.get(need)
    buf.fill_(0xFF)  # all-NaN partials: the split pass must write every partial the merge reads
    args.workspace, args.workspace_bytes = buf.data_ptr(), buf.numel()
    sh = host.stream_handle()
    host.check(lib.dspark_verify_attention_splits(ctypes.byref(args), sh), "splits")
    host.check(lib.dspark_verify_attention_combine(ctypes.byref(args), sh), "combine")
    torch.cuda.synchronize()
    want = orc.verify_attention(q, k, v, a) * (1.0 / (1.0 + np.exp(-gate.cpu().numpy().astype(np.float64))))[:, :, None]
    assert np.max(np.abs(ref.cpu().numpy() - want)) <= TOL
    for rep in range(3):
        out = torch.full((M, QH, D), float("nan"), dtype=torch.float32, device="cuda")
        args.out_f32 = out.data_ptr()
        host.check(lib.dspark_verify_attention(ctypes.byref(args), sh), "verify_attention")
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.max(np.abs(got - want)) <= TOL, f"call {rep}: max-abs {np.max(np.abs(got - want))} vs the oracle"
        diff = np.abs(got - ref.cpu().numpy())
        assert torch.equal(out, ref), f"call {rep}: max diff {diff.max()} at {np.unravel_index(diff.argmax(), diff.shape)}, " \
                                      f"{int((diff > 0).sum())} of {diff.size} differ"


def test_verify_attention_c2_full_context(dev, orc):
    """C2 at its real shape: ctx 32768, M = 16, 32/8/64, one layer."""
    host = load_host()
    run_case(dev, orc, host, 16, 32, 8, 64, 32768, seed=400)


def test_verify_attention_gate(dev, orc):
    torch = dev
    host = load_host()
    M, QH, KVH, D, a = 9, 32, 8, 64, 600
    q = orc.normal_f16(500, (M, QH, D))
    k = orc.normal_f16(501, (a + M, KVH, D))
    v = orc.normal_f16(502, (a + M, KVH, D))
    gate = np.random.default_rng(5).standard_normal((M, QH)).astype(np.float32)
    want = orc.verify_attention(q, k, v, a) * (1.0 / (1.0 + np.exp(-gate.astype(np.float64))))[:, :, None]
    kp, vp = host.kv_to_pages(f16(torch, k), f16(torch, v))
    out32 = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
    host.verify_attention(f16(torch, q), kp, vp, a, out_f32=out32, gate=torch.from_numpy(gate).cuda())
    torch.cuda.synchronize()
    assert np.max(np.abs(out32.cpu().numpy() - want)) <= TOL


def test_kv_write_layout(dev, orc):
    """K pages hold the operand order of include/dspark.h, V pages are transposed; pages past the write stay zero."""
    torch = dev
    host = load_host()
    for D in (64, 128):
        T, KVH = 70, 4
        k = orc.normal_f16(600 + D, (T, KVH, D))
        v = orc.normal_f16(601 + D, (T, KVH, D))
        kp, vp = host.kv_to_pages(f16(torch, k), f16(torch, v), n_pages=4)
        torch.cuda.synchronize()
        kpn = kp.cpu().numpy().view(np.uint16).reshape(4, KVH, 32 * D)
        vpn = vp.cpu().numpy().view(np.uint16).reshape(4, KVH, D, 32)
        idx = host.k_page_index(D)
        assert sorted(idx.ravel().tolist()) == list(range(32 * D))  # a permutation of the block
        for pos in (0, 5, 31, 32, 45, 69):
            pg, sl = divmod(pos, 32)
            assert np.array_equal(kpn[pg][:, idx[sl]], k[pos])
            assert np.array_equal(vpn[pg][:, :, sl], v[pos])
        kb, vb = host.kv_from_pages(kp, vp, range(T))
        assert np.array_equal(kb.view(np.uint16), k) and np.array_equal(vb.view(np.uint16), v)
        assert not kpn[3].any()
