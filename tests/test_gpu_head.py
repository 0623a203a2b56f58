"""GPU parity of the greedy verify argmax, acceptance/commit, the int8 verify GEMM and the cropped head argmax,
through the C ABI, against the CPU oracle. Integer/index results (keys, acceptance, commit offsets, emitted tokens)
must be bit-exact; GEMM values within 2e-3 relative of the fp64 oracle; head argmax exact except where the oracle's
top two values are within the GEMM's rounding (a near tie, the only exception north_star allows)."""
import numpy as np
import pytest

from conftest import load_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def f16(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).cuda()


def seen_bitmap(V, toks):
    bits = np.zeros((V + 31) // 32, np.uint32)
    for t in toks:
        bits[t >> 5] |= np.uint32(1 << (t & 31))
    return bits


def c1_round(orc, seed, M=9, V=65536, plant=0.5, rep=1.0, nseen=200):
    """BASELINE config C1's acceptance half: seeded fp16 logits, drafts planted as the previous position's argmax."""
    rng = np.random.default_rng(seed)
    logits = orc.f16_to_f32(orc.normal_f16(seed, (M, V)))
    seen_toks = rng.integers(0, V, nseen)
    bits = seen_bitmap(V, seen_toks)
    tokens = np.zeros(M, np.int32)
    tokens[0] = int(rng.integers(0, V))
    for t in range(1, M):
        keys = orc.verify_argmax(logits[:t], bits, tokens[:max(t, 1)], rep=rep)
        am = int(orc.keys_to_tokens(keys)[t - 1])
        if rng.random() < plant:
            tokens[t] = am
        else:
            d = int(rng.integers(0, V))
            tokens[t] = d if d != am else (d + 1) % V
    return logits, bits, tokens


@pytest.mark.parametrize("seed,plant,rep", [(1, 0.5, 1.0), (2, 1.0, 1.0), (3, 0.0, 1.0), (4, 0.5, 1.3), (5, 1.0, 1.3)])
def test_verify_argmax_and_commit_c1(dev, orc, seed, plant, rep):
    torch = dev
    host = load_host()
    M, V, a = 9, 65536, 1024
    print(f"case C1 seed={seed} plant={plant} rep={rep}", flush=True)
    logits, bits, tokens = c1_round(orc, seed, M, V, plant, rep)
    want_keys = orc.verify_argmax(logits, bits, tokens, rep=rep)
    for dt in (torch.float32, torch.float16):
        lg = torch.from_numpy(logits).cuda().to(dt)
        st = host.state_tensor(a=a, anchor=int(tokens[0]), tokens=tokens, rounds_left=32, budget=512, eos=-1,
                               stop_at=1056, run=1, skip_rounds=1)
        seen = torch.from_numpy(bits.view(np.int32)).cuda()
        best = host.verify_argmax(lg, seen, st, rep=rep)
        torch.cuda.synchronize()
        got = best.cpu().numpy().view(np.uint64)
        assert np.array_equal(got, want_keys), (got, want_keys)
    # acceptance + commit on the device State, against the oracle's books
    out = torch.zeros(600, dtype=torch.int32, device="cuda")
    host.accept_commit(st, best, M, out, seen)
    torch.cuda.synchronize()
    gst = host.state_from_tensor(st)
    ost = orc.new_state(a=a, anchor=int(tokens[0]), tokens=tokens, rounds_left=32, budget=512, eos=-1, stop_at=1056,
                        run=1, skip_rounds=1)
    oout = np.zeros(600, np.int32)
    obits = bits.copy()
    acc = orc.accept_commit(ost, orc.keys_to_tokens(want_keys), M, oout, obits)
    for f in host.STATE_FIELDS:
        assert getattr(gst, f) == getattr(ost, f), f
    assert list(gst.tokens)[:M] == list(ost.tokens)[:M]
    assert np.array_equal(out.cpu().numpy(), oout)
    assert np.array_equal(seen.cpu().numpy().view(np.uint32), obits)
    assert gst.a == a + acc + 1  # KV commit offset
    if plant == 1.0 and rep == 1.0:
        assert acc == M - 1
    if plant == 0.0:
        assert acc == 0


def test_commit_stop_rules_on_device(dev, orc):
    torch = dev
    host = load_host()
    V = 4096
    for kw in (dict(eos=11), dict(stop_at=1027), dict(budget=3), dict(rounds_left=1), dict(skip=2)):
        base = dict(a=1024, anchor=5, tokens=[5, 10, 11, 12], rounds_left=32, budget=512, eos=-1, stop_at=1056,
                    run=1, skip_rounds=1, skip_after=2, miss=1)
        base.update(kw)
        skip_now = 1 if kw.get("skip") else 0
        keys = np.array([orc.argmax_key(1.0, t) for t in (10, 11, 12, 13)], np.uint64)
        st = host.state_tensor(**base)
        best = torch.from_numpy(keys.view(np.int64)).cuda()
        out = torch.zeros(64, dtype=torch.int32, device="cuda")
        seen = torch.zeros(V // 32, dtype=torch.int32, device="cuda")
        host.accept_commit(st, best, 4, out, seen, skip_now=skip_now)
        torch.cuda.synchronize()
        gst = host.state_from_tensor(st)
        ost = orc.new_state(**base)
        oout = np.zeros(64, np.int32)
        acc = orc.accept_commit(ost, np.array([10, 11, 12, 13], np.int32), 4, oout, np.zeros(V // 32, np.uint32),
                                skip_now=skip_now)
        for f in host.STATE_FIELDS:
            assert getattr(gst, f) == getattr(ost, f), (kw, f)


COMMIT_EDGE = {
    # name: (State tokens[0..m-1], the verify argmax tokens best[0..m-1], State fields, skip_now)
    "mid_miss": ([5, 10, 11, 12], [10, 99, 12, 13], {}, 0),                      # acc 1: the second draft misses
    "miss_to_skip": ([5, 10, 11, 12], [7, 8, 9, 13], dict(miss=1, skip_after=2, skip_rounds=3), 0),  # acc 0
    "eos_bonus": ([5, 10, 11, 12], [10, 11, 77, 13], dict(eos=77), 0),           # the bonus token is eos
    "eos_first_draft": ([5, 77, 11, 12], [77, 11, 12, 13], dict(eos=77), 0),     # an accepted draft is eos
    "one_row": ([5], [42], {}, 0),                                               # m = 1: the bonus alone
    "all_64": ([5] + [100 + j for j in range(1, 64)], [100 + j for j in range(1, 64)] + [999], {}, 0),
    "same_word": ([5, 40, 40, 41], [40, 40, 41, 63], {}, 0),                     # one seen word, a token twice
    "skip_round": ([5, 10, 11, 12], [7, 8, 9, 13], dict(skip=2, miss=1, skip_after=2), 1),
    "count_carried": ([5, 10, 11, 12], [10, 11, 12, 13], dict(count=17, accepted=40, verified=90), 0),
}


@pytest.mark.parametrize("case", sorted(COMMIT_EDGE))
def test_commit_edge_cases_on_device(dev, orc, case):
    """Acceptance + commit on the device against the oracle's books: misses at every position, the skip/miss
    counters, eos among the drafts and as the bonus, one row, all 64 rows accepted, several committed tokens in one
    seen word (the same token twice), a skip round, counters carried in. Every State field, the State's tokens, the
    emitted tokens and the seen bitmap are compared."""
    torch = dev
    host = load_host()
    V = 4096
    tokens, best_tok, fields, skip_now = COMMIT_EDGE[case]
    m = len(tokens)
    base = dict(a=1024, anchor=tokens[0], tokens=tokens, rounds_left=32, budget=4096, eos=-1, stop_at=4096, run=1,
                skip_rounds=1, skip_after=0, miss=0)
    base.update(fields)
    keys = np.array([orc.argmax_key(1.0, t) for t in best_tok], np.uint64)
    st = host.state_tensor(**base)
    best = torch.from_numpy(keys.view(np.int64)).cuda()
    out = torch.full((128,), -7, dtype=torch.int32, device="cuda")
    seen0 = np.zeros(V // 32, np.uint32)
    seen0[3] = 0x80000001  # bits already set stay set
    seen = torch.from_numpy(seen0.view(np.int32).copy()).cuda()
    host.accept_commit(st, best, m, out, seen, skip_now=skip_now)
    torch.cuda.synchronize()
    gst = host.state_from_tensor(st)
    ost = orc.new_state(**base)
    oout = np.full(128, -7, np.int32)
    oseen = seen0.copy()
    acc = orc.accept_commit(ost, np.array(best_tok, np.int32), m, oout, oseen, skip_now=skip_now)
    for f in host.STATE_FIELDS:
        assert getattr(gst, f) == getattr(ost, f), (case, f, getattr(gst, f), getattr(ost, f))
    assert [gst.tokens[i] for i in range(64)] == [ost.tokens[i] for i in range(64)], case
    np.testing.assert_array_equal(out.cpu().numpy(), oout, err_msg=case)
    np.testing.assert_array_equal(seen.cpu().numpy().view(np.uint32), oseen, err_msg=case)
    expect_acc = {"mid_miss": 1, "miss_to_skip": 0, "eos_bonus": 2, "eos_first_draft": 3, "one_row": 0, "all_64": 63,
                  "same_word": 3, "skip_round": 0, "count_carried": 3}[case]
    assert acc == expect_acc, (case, acc)


def test_commit_refuses_a_full_output_buffer(dev, orc):
    """A commit that would write past out_cap writes nothing and stops the run: State.run = 0, every other State
    word, the emitted tokens and the seen bitmap unchanged."""
    torch = dev
    host = load_host()
    V = 4096
    base = dict(a=1024, anchor=5, tokens=[5, 10, 11, 12], rounds_left=32, budget=4096, eos=-1, stop_at=4096, run=1,
                count=2)
    keys = np.array([orc.argmax_key(1.0, t) for t in (10, 11, 99, 13)], np.uint64)  # acc 2: 3 tokens to commit
    st = host.state_tensor(**base)
    before = host.state_from_tensor(st)
    best = torch.from_numpy(keys.view(np.int64)).cuda()
    out = torch.full((4,), -7, dtype=torch.int32, device="cuda")  # out_cap 4 < count 2 + 3
    seen = torch.zeros(V // 32, dtype=torch.int32, device="cuda")
    host.accept_commit(st, best, 4, out, seen)
    torch.cuda.synchronize()
    after = host.state_from_tensor(st)
    assert after.run == 0
    for f in host.STATE_FIELDS:
        if f != "run":
            assert getattr(after, f) == getattr(before, f), f
    assert [after.tokens[i] for i in range(4)] == [5, 10, 11, 12]
    assert out.cpu().tolist() == [-7, -7, -7, -7]
    assert int(seen.abs().sum()) == 0


@pytest.mark.parametrize("M,N,K,epilogue", [
    (16, 12288, 2048, 0),   # K-sliced, 4 strips x 4 ranges, X^T in LDS
    (16, 2048, 8192, 0),    # long K: split across workgroups
    (9, 1024, 2048, 1),     # K-sliced, 1 strip x 4 ranges, each wave loads its own X, gated epilogue
    (16, 512, 1024, 2),     # same, SiLU epilogue
    (1, 64, 128, 0),        # two ranges of one chunk (fewer chunks than ranges)
    (16, 1024, 192, 0),     # three chunks over four ranges: an empty range
    (16, 2048, 4096, 0),    # own-X ranges of 16 chunks (two batches)
    (24, 4096, 1024, 0),    # K-sliced, two token blocks
    (16, 32768, 2048, 0),   # K-sliced, 8 strips x 2 ranges of 16 chunks
    (16, 16400, 2048, 0),   # 1025 strips: 5 strips x 3 ranges (205 groups), the last group part-empty
    (16, 65536, 1024, 0),   # 16 strips x 1 range of 16 chunks
    (16, 16384, 1344, 0),   # ragged ranges: 21 chunks over 4 (X^T in LDS)
    (16, 8192, 1344, 0),    # ragged own-X ranges
    (33, 256, 2048, 0),     # three token blocks: K-sliced, X^T one token block per pass (weights kept in registers)
    (24, 2048, 2048, 0),    # two token blocks in two passes
    (40, 6144, 2048, 1),    # three token blocks, gated epilogue
    (48, 16384, 2048, 2),   # three token blocks, 4 strips x 4 ranges, SiLU epilogue
    (64, 2048, 2048, 0),    # four token blocks
    (36, 1024, 1344, 0),    # passes over ragged ranges (21 chunks over 4)
    (33, 1024, 4096, 0),    # one token block's X^T per pass (128 KB)
    (33, 1024, 8192, 0),    # X^T of one token block over 128 KB: K split across workgroups
    (64, 128, 256, 0),
])
def test_gemm_i8_matches_oracle(dev, orc, M, N, K, epilogue):
    torch = dev
    host = load_host()
    print(f"case gemm M={M} N={N} K={K} epi={epilogue}", flush=True)
    x = orc.normal_f16(700 + M, (M, K))
    w = orc.int8_uniform(701 + N, (N, K))
    s = orc.f32_to_f16(np.random.default_rng(N).uniform(0.5, 1.5, N).astype(np.float32) / np.float32(127 * np.sqrt(K)))
    want = orc.gemm_i8(x, w, s)
    wb = torch.from_numpy((w.astype(np.int16) + 128).astype(np.uint8)).cuda()
    y = host.gemm_i8(f16(torch, x), wb, f16(torch, s), epilogue=epilogue)
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    scale = np.max(np.abs(want))
    if epilogue == 0:
        assert np.max(np.abs(got - want)) <= 2e-3 * scale
    elif epilogue == 1:
        g, u = want[:, 0::2], want[:, 1::2]
        ref = (g / (1 + np.exp(-g))) * u
        assert np.max(np.abs(got - ref)) <= 2e-3 * max(1.0, np.max(np.abs(ref)))
    else:
        ref = want / (1 + np.exp(-want))
        assert np.max(np.abs(got - ref)) <= 2e-3 * max(1.0, np.max(np.abs(ref)))


@pytest.mark.parametrize("M,N,K", [(33, 2048, 8192), (40, 1024, 8192), (33, 512, 8192)])
def test_gemm_split_calls_share_one_workspace(dev, orc, M, N, K):
    """Split-K GEMMs in a row on one workspace (the last split of each row group sums the partials and resets its
    counter): every call matches the oracle on its own inputs and repeats are bit-identical."""
    torch = dev
    host = load_host()
    lib = host.lib()
    print(f"case gemm split calls M={M} N={N} K={K}", flush=True)
    need = lib.dspark_gemm_i8_workspace(M, N, K)
    assert need > M * N * 4  # split: partials + counters
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    w = orc.int8_uniform(901 + N, (N, K))
    s = orc.f32_to_f16(np.random.default_rng(N + 1).uniform(0.5, 1.5, N).astype(np.float32) / np.float32(127 * np.sqrt(K)))
    wb = torch.from_numpy((w.astype(np.int16) + 128).astype(np.uint8)).cuda()
    sd = f16(torch, s)
    wso = host.Workspace()
    wso.buf = ws
    first = None
    for call in range(4):
        x = orc.normal_f16(910 + call % 3, (M, K))
        want = orc.gemm_i8(x, w, s)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        host.gemm_i8(f16(torch, x), wb, sd, y_f32=y, workspace=wso)
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
        assert np.max(np.abs(got - want)) <= 2e-3 * np.max(np.abs(want)), f"call {call}"
        if call == 0:
            first = y.clone()
        if call == 3:
            assert torch.equal(y, first)  # same inputs as call 0: same bits
    # a counter left non-zero would have kept every later call's groups from finishing (NaN outputs above)


def test_gemm_split_shapes_share_one_workspace(dev, orc):
    """Split-K GEMMs of different shapes and split counts in a row on one workspace (the engine's pattern: a wide
    split writes partials where a narrower split's arrival counters would sit if counters followed the partials):
    every call matches the oracle, and a second pass over the same calls gives the same bits."""
    torch = dev
    host = load_host()
    lib = host.lib()
    shapes = [(33, 2048, 8192), (33, 2048, 10240), (40, 6144, 8192), (48, 3104, 8192), (33, 1024, 6144), (64, 2048, 10240)]
    need = max(lib.dspark_gemm_i8_workspace(M, N, K) for M, N, K in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    wso = host.Workspace()
    wso.buf = ws
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        assert lib.dspark_gemm_i8_workspace(M, N, K) > 0  # every shape splits K
        w = orc.int8_uniform(950 + i, (N, K))
        s = orc.f32_to_f16(np.random.default_rng(i).uniform(0.5, 1.5, N).astype(np.float32) / np.float32(127 * np.sqrt(K)))
        x = orc.normal_f16(960 + i, (M, K))
        cases.append((M, N, K, w, s, x, orc.gemm_i8(x, w, s)))
    outs = []
    for rep in range(2):
        for i, (M, N, K, w, s, x, want) in enumerate(cases):
            print(f"case gemm mixed shapes pass={rep} M={M} N={N} K={K}", flush=True)
            wb = torch.from_numpy((w.astype(np.int16) + 128).astype(np.uint8)).cuda()
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            host.gemm_i8(f16(torch, x), wb, f16(torch, s), y_f32=y, workspace=wso)
            torch.cuda.synchronize()
            got = y.cpu().numpy().astype(np.float64)
            assert np.max(np.abs(got - want)) <= 2e-3 * np.max(np.abs(want)), (rep, M, N, K)
            if rep == 0:
                outs.append(y)
            else:
                assert torch.equal(y, outs[i]), (M, N, K)


@pytest.mark.parametrize("M,N,K", [(16, 16384, 2048), (9, 4096, 2048), (33, 1024, 512)])
def test_head_argmax_matches_oracle(dev, orc, M, N, K):
    torch = dev
    host = load_host()
    print(f"case head M={M} N={N} K={K}", flush=True)
    x = orc.normal_f16(800 + M, (M, K))
    w = orc.normal_f16(801 + N, (N, K), scale=float(1 / np.sqrt(K)))
    want = orc.gemm_f16(x, w)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    best = host.head_argmax(f16(torch, x), f16(torch, w), y_f32=y)
    torch.cuda.synchronize()
    got_y = y.cpu().numpy().astype(np.float64)
    assert np.max(np.abs(got_y - want)) <= 2e-3
    idx = host.keys_to_tokens(best).cpu().numpy()
    # the key must be the argmax of the GPU's own fp32 values (bit-exact fold) ...
    assert idx.tolist() == orc.row_argmax(y.cpu().numpy()).tolist()
    # ... and match the oracle's argmax unless the oracle's top two are a near tie
    for t in range(M):
        o = int(np.argmax(want[t]))
        if idx[t] != o:
            top = np.sort(want[t])[-2:]
            assert top[1] - top[0] < 1e-4, (t, idx[t], o, top)
    # bit-identical rerun
    best2 = host.head_argmax(f16(torch, x), f16(torch, w))
    torch.cuda.synchronize()
    assert torch.equal(best, best2)
