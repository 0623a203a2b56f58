"""GPU tests at the configs' full sizes:

* verify attention at context 131072 (C5: 32 query / 8 KV heads, head_dim 64), for the 33-token block and for 16
  tokens, against the fp64 C oracle at 2e-3 max-abs (the oracle's threaded form, which gives its single-threaded bits);
* full DSpark rounds on random-init models of the C4 geometry (16 layers: 10 gated short-conv k=3 + 6 GQA 32/8/64,
  hidden 2048, FFN 8192, vocab 65536, 4-layer drafter): block 33 at context 131072 (C5) with drafts planted at 0 %,
  50 % and 100 % acceptance -- a rollback in every round of the first two -- and block 16 at context 32768 (C4); and the
  reference model's geometry on the reference's storage formats (int8 K/V records, per-128-column weight scales) at
  context 131072 with its 9-token block and 3 drafts. The
  property checked at these sizes is the one a speculative round must keep whatever is drafted: the committed tokens
  are exactly the target's greedy chain (one-token verify rounds), each round commits its accepted prefix plus the
  target's token, and the State's position and counters follow.
"""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, load_host

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def bench_module():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench
    return bench


@pytest.mark.parametrize("M,paged", [(33, False), (16, True)])
def test_verify_attention_c5_context(dev, orc, M, paged):
    torch = dev
    host = load_host()
    QH, KVH, D, a = 32, 8, 64, 131072
    print(f"case C5 attention M={M} a={a} paged={paged}", flush=True)
    T = a + M
    q = orc.normal_f16(900 + M, (M, QH, D))
    k = orc.normal_f16(901 + M, (T, KVH, D))
    v = orc.normal_f16(902 + M, (T, KVH, D))
    npages = (T + 31) // 32
    f16 = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.float16)).cuda()
    bt = None
    if paged:
        bt = torch.from_numpy(np.random.default_rng(M).permutation(npages + 5)[:npages].astype(np.int32)).cuda()
        kp, vp = host.kv_pages_alloc(npages + 5, KVH, D)
        host.kv_write(f16(k[:a]), f16(v[:a]), kp, vp, 0, bt)
        host.kv_write(f16(k[a:]), f16(v[a:]), kp, vp, a, bt)
    else:
        kp, vp = host.kv_to_pages(f16(k), f16(v))
    qd = f16(q)
    out32 = torch.empty((M, QH, D), dtype=torch.float32, device="cuda")
    out16 = torch.empty((M, QH, D), dtype=torch.float16, device="cuda")
    host.verify_attention(qd, kp, vp, a, out=out16, out_f32=out32, block_table=bt)
    torch.cuda.synchronize()
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    want = orc.verify_attention_mt(q, k, v, a, threads=threads)
    err = float(np.max(np.abs(out32.cpu().numpy().astype(np.float64) - want)))
    err16 = float(np.max(np.abs(out16.cpu().numpy().astype(np.float64) - want)))
    print(f"max-abs fp32 {err:.3e}, fp16 {err16:.3e}", flush=True)
    assert err <= TOL and err16 <= TOL
    again = torch.empty_like(out32)
    host.verify_attention(qd, kp, vp, a, out_f32=again, block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(again, out32)


def planted_rounds(torch, host, eng, a0, anchor, rounds, p, seed):
    """Greedy chain from a0, drafts planted from it with probability p; runs `rounds` rounds with planted drafts and
    checks the commits. Returns the commits per round."""
    bench = bench_module()
    B, nd, V = eng.desc.block, eng.desc.max_drafts, eng.desc.vocab
    chain = bench.greedy_chain(eng, host, torch, a0, anchor, (rounds + 1) * B)
    rng = np.random.default_rng(seed)
    ok = rng.random(len(chain)) < p
    planted = np.where(ok, chain, (chain + 1 + rng.integers(0, V - 1, len(chain))) % V).astype(np.int32)
    planted = np.where(ok, chain, np.where(planted == chain, (chain + 1) % V, planted)).astype(np.int32)
    buf = eng.download("plant", np.int32)
    buf[a0 + 1:a0 + 1 + len(chain)] = planted
    eng.upload("plant", buf)
    bench.engine_state(eng, a0, anchor)
    commits = []
    for _ in range(rounds):
        before = eng.state().count
        eng.round(-1, a0)
        torch.cuda.synchronize()
        commits.append(eng.state().count - before)
    st = eng.state()
    got = eng.download("out_tokens", np.int32)[:st.count]
    assert got.tolist() == chain[:st.count].tolist(), "committed tokens differ from the greedy chain"
    assert st.a == a0 + st.count and st.rounds_done == rounds
    c = 0
    for k in commits:  # round at chain index c drafts chain indices c .. c + nd - 1; the first wrong one ends it
        bad = [i for i in range(c, c + nd) if planted[i] != chain[i]]
        assert k == ((bad[0] - c + 1) if bad else nd + 1), (c, k, commits)
        c += k
    assert st.accepted == st.count - rounds and st.verified == rounds * (nd + 1)
    return commits


@pytest.mark.parametrize("case", ["c5", "c4", "ref"])
def test_planted_rounds_full_geometry(dev, case):
    """c5 / c4: the C4-geometry model; ref: the reference model's geometry (24 layers, 16/4/128, FFN 7680, vocab
    128000, 3-layer drafter, 3 drafts from position 57344) on the reference's storage formats (int8 K/V records,
    per-128-column weight scales) at context 131072, which runs the record attention at 4096 pages and the group-scale
    GEMMs at their widest plans (the 128000-row head through LDS, w2 in bands)."""
    torch = dev
    host = load_host()
    bench = bench_module()
    desc_ = None
    if case == "c5":
        ctx, block, rates = 131072, 33, (1.0, 0.5, 0.0)
    elif case == "ref":
        ctx, block, rates = 131072, 9, (1.0, 0.5, 0.0)
        desc_ = host.ref_desc(block=9, max_drafts=3)
    else:
        ctx, block, rates = 32768, 16, (0.7,)
    print(f"case planted rounds {case}: ctx {ctx} block {block}", flush=True)
    desc, eng = bench.engine_setup(host, torch, ctx, block, 20261201 + ctx + block, desc_)
    assert eng.max_context > 131072 or case == "c4"
    nd = eng.desc.max_drafts
    for i, p in enumerate(rates):
        commits = planted_rounds(torch, host, eng, ctx, 17, 4, p, 7 + i)
        print(f"p={p}: commits per round {commits}", flush=True)
        if p == 0.0:
            assert commits == [1] * 4
        if p == 1.0:
            assert commits == [nd + 1] * 4
        if 0 < p < 1:
            assert any(k < nd + 1 for k in commits)  # rollback happened
    eng.close()
