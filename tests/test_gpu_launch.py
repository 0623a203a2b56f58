"""GPU checks of the draftLaunch boundary (dspark_engine_launch) and the request-level entry points around it, through
the C ABI on small seeded geometries:

* a launch against the same rounds enqueued one by one (dspark_engine_round) and against the oracle's books
  (orc.accept_commit driven round by round with the draft cap of dspark.hip:2633-2640 and the launch's State setup of
  internal/model/dspark.go:543-566): emitted tokens, count, boundary, every State word, the stop at the block
  boundary, eos, budget, the per-launch draft cap, the rounds limit, miss carried in, a repetition penalty;
* the conv state at launch boundaries (dspark.hip:2415-2431, 2921-2947): the running slot loaded before the first
  round, written back at the end, and the checkpoint at stop_at, against the oracle's conv history;
* drafter context seeding (captureTap + projectPrompt, dspark.go:439-492) against the oracle's projection;
* InitSeen (engine.go:617-629).

Drafts are planted from the target's own greedy chain (one-token verify rounds), so every round's acceptance is known
in advance: tokens, counts and State words are compared bit for bit."""
import ctypes

import numpy as np
import pytest

from conftest import load_host, rope_numpy
from test_gpu_engine import GEOMETRIES, make_weights, setup_caches

pytestmark = pytest.mark.gpu

A0, CTX_LO, ANCHOR = 300, 150, 17


def ulp16(x):
    """The fp16 spacing at magnitude x (>= 1): values the GPU and the oracle both round to fp16 at the same points
    differ by a last-bit flip when their fp32 sums differ in order (measured: <= 1 ulp)."""
    return 2.0 ** (np.floor(np.log2(max(1.0, float(x)))) - 10)


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def conv_rings(eng):
    return {nm: eng.download(nm, np.uint16) for nm in eng.names() if nm.startswith("conv.L")}


def greedy_chain(eng, torch, n, rep=1.0, prompt=()):
    """The target's greedy continuation of position A0 (one-token verify rounds), with the conv rings restored after."""
    rings = conv_rings(eng)
    eng.init_seen(prompt, rep)
    eng.set_state(a=A0, anchor=ANCHOR, count=0, rounds_left=1 << 20, limit=eng.max_context, budget=1 << 20, eos=-1,
                  ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, run=1, skip_rounds=1, stop_at=eng.max_context, ckpt_slot=-1,
                  tokens=[ANCHOR])
    for _ in range(n):
        eng.round(1, A0)
    torch.cuda.synchronize()
    st = eng.state()
    assert st.count == n, (st.count, n)
    chain = eng.download("out_tokens", np.int32)[:n].copy()
    for nm, buf in rings.items():
        eng.upload(nm, buf)
    return chain


def plant(eng, chain, wrong, vocab):
    """plant[A0 + 1 + i] = chain[i], except chain indices in `wrong` (a different token)."""
    planted = chain.copy()
    for i in wrong:
        planted[i] = (chain[i] + 1) % vocab
    buf = eng.download("plant", np.int32)
    buf[A0 + 1:A0 + 1 + len(planted)] = planted
    eng.upload("plant", buf)
    return planted


def oracle_books(orc, host, eng, chain, planted, args):
    """The launch replayed on the CPU: the State as dspark.go:543-566 sets it, then per round the draft cap
    (dspark.hip:2633-2640), the planted drafts and the target's tokens (the chain) through orc.accept_commit."""
    B, md_model = eng.desc.block, eng.desc.max_drafts
    stop = min((args["a"] // 32 + 1) * 32, eng.max_context)
    limit = min(stop + B, eng.max_context)
    md = min(args.get("max_drafts", 0), md_model) if args.get("max_drafts", 0) > 0 else md_model
    st = orc.new_state(a=args["a"], anchor=args["anchor"], count=0, rounds_left=args["rounds"], limit=limit,
                       budget=min(args["budget"], 512), eos=args["eos"], ctx_new=args["ctx_new"],
                       ctx_pos=args["ctx_pos"], ctx_lo=args["ctx_lo"], run=1, force_m=args["force_m"],
                       miss=args.get("miss", 0), skip=args.get("skip", 0),
                       skip_rounds=1, stop_at=stop, ckpt_slot=args.get("ckpt_slot", -1), tokens=[args["anchor"]])
    out = np.zeros(4096, np.int32)
    seen = np.zeros((eng.desc.vocab + 31) // 32, np.uint32)
    while st.run:
        a = st.a
        skip_now = st.skip
        # a skip round verifies the anchor alone (dspark.hip:2441-2444); otherwise the draft cap of dspark.hip:2640
        cap = 0 if skip_now > 0 else max(min(min(md, B - 1), min(st.limit - a, st.budget - st.count) - 1), 0)
        tokens = [st.anchor] + [int(planted[a + j - A0 - 1]) for j in range(1, cap + 1)]
        for j, t in enumerate(tokens):
            st.tokens[j] = t
        best = np.array([chain[a + t - A0] for t in range(cap + 1)], np.int32)
        orc.accept_commit(st, best, cap + 1, out, seen, skip_now=1 if skip_now > 0 else 0)
    return st, out[:st.count].copy(), stop


LAUNCH_CASES = {
    # name: (launch arguments beyond a / anchor, chain indices planted wrong)
    "all_right": (dict(), ()),
    "rollbacks": (dict(), (2, 9, 10, 17)),
    "budget": (dict(budget=10), ()),
    "eos": (dict(eos="chain5"), ()),
    "draft_cap": (dict(max_drafts=3), (6,)),
    "rounds": (dict(rounds=2), (4,)),
    "miss_carried": (dict(miss=2), (0, 1, 8)),
    "skip": (dict(skip=2), (5,)),  # two skip rounds (the anchor alone), then drafted rounds
    "skip_cap": (dict(skip=1, max_drafts=3), (7,)),
}


@pytest.mark.parametrize("name", sorted(LAUNCH_CASES))
def test_launch_matches_rounds_and_oracle_books(dev, orc, name):
    torch = dev
    host = load_host()
    desc = host.model_desc(**GEOMETRIES["small"])
    eng = host.Engine(desc, 512)
    make_weights(eng, desc, 41)
    setup_caches(eng, host, desc, A0, CTX_LO, 141)
    print(f"case launch {name}", flush=True)
    chain = greedy_chain(eng, torch, 48)
    extra, wrong = LAUNCH_CASES[name]
    planted = plant(eng, chain, wrong, desc.vocab)
    args = dict(a=A0, anchor=ANCHOR, budget=512, eos=-1, rep=1.0, rounds=32, ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO,
                force_m=-1)
    args.update(extra)
    if args["eos"] == "chain5":
        args["eos"] = int(chain[5])
    want_st, want_out, stop = oracle_books(orc, host, eng, chain, planted, args)
    rings = conv_rings(eng)

    # the launch
    eng.init_seen([])
    toks, res = eng.launch(**args)
    torch.cuda.synchronize()
    assert toks == want_out.tolist(), (toks, want_out.tolist())
    assert toks == chain[:len(toks)].tolist()  # speculative rounds commit exactly the greedy chain
    assert res.count == want_st.count and res.boundary == stop
    assert (res.rounds, res.accepted, res.verified) == (want_st.rounds_done, want_st.accepted, want_st.verified)
    for f in host.STATE_FIELDS:
        if f != "M":
            assert getattr(res.state, f) == getattr(want_st, f), (f, getattr(res.state, f), getattr(want_st, f))
    # no round was put on the stream that found the State stopped (an eos stop may leave rounds in flight idle)
    if args["eos"] < 0:
        assert res.rounds_enqueued == res.rounds, (res.rounds_enqueued, res.rounds)
    else:
        assert res.rounds <= res.rounds_enqueued <= args["rounds"]
    if "max_drafts" in extra or "skip" in extra:
        # bare rounds verify 1 + the model's max_drafts and skip nothing: the launch's own cap and skip rounds have
        # no one-by-one counterpart (test_launch_cap_and_penalty_do_not_stick covers rounds after such a launch)
        eng.close()
        return

    # the same rounds enqueued one by one from the State the launch sets
    for nm, buf in rings.items():
        eng.upload(nm, buf)
    eng.init_seen([])
    st0 = dict(a=A0, anchor=ANCHOR, count=0, rounds_left=args["rounds"], limit=want_st.limit,
               budget=min(args["budget"], 512), eos=args["eos"], ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, run=1,
               force_m=-1, miss=args.get("miss", 0), skip_rounds=1, stop_at=stop, ckpt_slot=-1, tokens=[ANCHOR])
    eng.set_state(**st0)
    for _ in range(args["rounds"]):
        eng.round(-1, A0)
    torch.cuda.synchronize()
    st = eng.state()
    for f in host.STATE_FIELDS:
        assert getattr(st, f) == getattr(res.state, f), f
    assert eng.download("out_tokens", np.int32)[:st.count].tolist() == toks
    eng.close()


def test_launch_cap_and_penalty_do_not_stick(dev, orc):
    """A launch's draft cap and penalty are its own: after a 3-draft launch with rep 1.3, a bare planted round drafts
    up to the model's max_drafts again (verifies 1 + 7 tokens) and commits the unpenalised greedy chain."""
    torch = dev
    host = load_host()
    desc = host.model_desc(**GEOMETRIES["small"])
    eng = host.Engine(desc, 512)
    make_weights(eng, desc, 43)
    setup_caches(eng, host, desc, A0, CTX_LO, 143)
    print("case launch cap/rep reset", flush=True)
    chain = greedy_chain(eng, torch, 24)
    plant(eng, chain, (), desc.vocab)
    rings = conv_rings(eng)
    eng.init_seen([])
    _, res = eng.launch(A0, ANCHOR, rep=1.3, max_drafts=3, ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, force_m=-1)
    torch.cuda.synchronize()
    assert res.verified <= 4 * res.rounds  # the launch verified at most 1 + 3 tokens a round
    for nm, buf in rings.items():
        eng.upload(nm, buf)
    eng.init_seen([])
    eng.set_state(a=A0, anchor=ANCHOR, count=0, rounds_left=1, limit=eng.max_context, budget=1 << 20, eos=-1,
                  ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, run=1, skip_rounds=1, stop_at=eng.max_context,
                  ckpt_slot=-1, tokens=[ANCHOR])
    eng.round(-1, A0)
    torch.cuda.synchronize()
    st = eng.state()
    assert st.verified == 1 + desc.max_drafts, st.verified
    assert st.count == 1 + desc.max_drafts  # every planted draft of the unpenalised chain accepted
    assert eng.download("out_tokens", np.int32)[:st.count].tolist() == chain[:st.count].tolist()
    eng.close()


def test_launch_with_repetition_penalty(dev, orc):
    """rep != 1 with a seeded prompt mask: the launch commits the greedy chain of the penalised target, and InitSeen
    resets the mask between requests (a second launch from the same start gives the same tokens)."""
    torch = dev
    host = load_host()
    desc = host.model_desc(**GEOMETRIES["small"])
    eng = host.Engine(desc, 512)
    make_weights(eng, desc, 42)
    setup_caches(eng, host, desc, A0, CTX_LO, 142)
    prompt = list(range(100, 160)) + [ANCHOR]
    print("case launch rep=1.3", flush=True)
    chain = greedy_chain(eng, torch, 40, rep=1.3, prompt=prompt)
    plain = greedy_chain(eng, torch, 40)
    assert not np.array_equal(chain, plain), "the penalty changes nothing on this model: pick a larger rep"
    plant(eng, chain, (3,), desc.vocab)
    rings = conv_rings(eng)
    outs = []
    for _ in range(2):
        for nm, buf in rings.items():
            eng.upload(nm, buf)
        eng.init_seen(prompt, 1.3)
        toks, res = eng.launch(A0, ANCHOR, rep=1.3, ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, force_m=-1)
        torch.cuda.synchronize()
        outs.append(toks)
    assert outs[0] == outs[1] == chain[:len(outs[0])].tolist()
    seen = eng.download("seen", np.uint32)
    bits = {int(w) * 32 + b for w in range(seen.size) for b in range(32) if (seen[w] >> b) & 1}
    assert bits == set(prompt) | set(outs[1])
    eng.close()


def test_launch_refuses_bad_arguments(dev):
    host = load_host()
    desc = host.model_desc(**dict(GEOMETRIES["small"], conv_slots=4))
    eng = host.Engine(desc, 512)
    for bad in (dict(a=512), dict(a=-1), dict(anchor=desc.vocab), dict(budget=0), dict(rounds=0),
                dict(conv_slot=4), dict(ckpt_slot=2), dict(conv_slot=0, ckpt_slot=4), dict(ctx_new=9)):
        kw = dict(a=A0, anchor=ANCHOR)
        kw.update(bad)
        with pytest.raises(host.DsparkError, match="EINVAL"):
            eng.launch(**kw)
    eng.close()


def test_conv_state_load_store_and_checkpoint(dev, orc):
    """A launch with conv_slot 0 loads the history before A0 from slot 0 (the ring rows there are scrambled first: the
    rounds then commit the same greedy chain only if the load restored them), and at its end slot 0 holds the history
    before the final a and the checkpoint slot the history before stop_at -- equal to the oracle's conv history of
    the committed tokens. A launch that stops short of the boundary writes no checkpoint."""
    torch = dev
    host = load_host()
    from oracle import round as rnd
    desc = host.model_desc(**dict(GEOMETRIES["small"], conv_slots=4))
    H, km1, B = desc.hidden, desc.conv_kernel - 1, desc.block
    eng = host.Engine(desc, 512)
    weights = make_weights(eng, desc, 43)
    C = setup_caches(eng, host, desc, A0, CTX_LO, 143)
    print("case conv state", flush=True)
    chain = greedy_chain(eng, torch, 48)
    plant(eng, chain, (), desc.vocab)
    conv_layers = [i for i in range(desc.n_layers) if desc.layer_kind[i] == 0]
    # slot 0 = the history before A0 (the rings' rows A0 - km1 .. A0 - 1), then those ring rows scrambled
    slot0 = {}
    for i in conv_layers:
        ring = eng.download(f"conv.L{i}", np.uint16).reshape(128, H)
        state = np.zeros((4, H, km1), np.uint16)
        for k in range(km1):
            state[0, :, k] = ring[(A0 - km1 + k) % 128]
        slot0[i] = state[0].copy()
        eng.upload(f"conv_state.L{i}", state)
        ring[[(A0 - km1 + k) % 128 for k in range(km1)]] = np.float16(7.0).view(np.uint16)
        eng.upload(f"conv.L{i}", ring)
    eng.init_seen([])
    toks, res = eng.launch(A0, ANCHOR, ctx_new=1, ctx_pos=A0 - 1, ctx_lo=CTX_LO, force_m=-1, conv_slot=0, ckpt_slot=2)
    torch.cuda.synchronize()
    assert toks == chain[:len(toks)].tolist()
    stop, a1 = res.boundary, res.state.a
    assert a1 >= stop == 320 and res.ckpt_written == 1

    # the oracle's conv history of the committed positions: the verify pass over each round's block (all drafts were
    # accepted, so the rounds verified [anchor, chain...] in blocks of B from A0)
    W = rnd.Weights(desc, weights)
    rope = rnd.h2f(rope_numpy(desc.rope_base, desc.rope_pairs, desc.head_dim, eng.max_context + B + 1))
    seq = [ANCHOR] + chain.tolist()
    for a in range(A0, a1, B):
        rnd.verify(W, C, dict(a=a), seq[a - A0:a - A0 + B], rope)
    for i in conv_layers:
        got = eng.download(f"conv_state.L{i}", np.uint16).reshape(4, H, km1).view(np.float16).astype(np.float64)
        for slot, pos in ((0, a1), (2, stop)):
            want = rnd.conv_state(C, i, pos, km1, H)
            err = np.max(np.abs(got[slot] - want))
            print(f"layer {i} slot {slot} (history before {pos}): max-abs {err:.3e}", flush=True)
            assert err <= 2 * ulp16(np.max(np.abs(want)))
        ring = eng.download(f"conv.L{i}", np.uint16).reshape(128, H)
        for k in range(km1):  # the loaded rows (positions before A0, which no round writes) hold slot 0's state
            assert np.array_equal(ring[(A0 - km1 + k) % 128], slot0[i][:, k])
    # conv_copy: slot 2 -> 3, bit for bit
    eng.conv_copy(2, 3)
    torch.cuda.synchronize()
    for i in conv_layers:
        s = eng.download(f"conv_state.L{i}", np.uint16).reshape(4, H, km1)
        assert np.array_equal(s[3], s[2])
    # a one-token launch from a1 does not reach its boundary: no checkpoint written, slot 1 untouched
    before = {i: eng.download(f"conv_state.L{i}", np.uint16).reshape(4, H, km1)[1].copy() for i in conv_layers}
    _, res2 = eng.launch(a1, int(res.state.anchor), budget=1, ctx_new=res.state.ctx_new, ctx_pos=res.state.ctx_pos,
                         ctx_lo=CTX_LO, conv_slot=0, ckpt_slot=1)
    torch.cuda.synchronize()
    assert res2.count == 1 and res2.ckpt_written == 0
    for i in conv_layers:
        assert np.array_equal(eng.download(f"conv_state.L{i}", np.uint16).reshape(4, H, km1)[1], before[i])
    eng.close()


@pytest.mark.parametrize("geom,first,n,context", [("small", 150, 100, 140), ("ref_small", 40, 61, 40)])
def test_prompt_projection_matches_oracle(dev, orc, geom, first, n, context):
    """captureTap + projectPrompt: prompt hidden states of the tapped layers -> drafter ring K/V rows of every drafter
    layer, against the oracle's projection. Rows of positions before tap_from are skipped by the capture; the
    projection runs in chunks of the block size, the last one partial."""
    torch = dev
    host = load_host()
    from oracle import round as rnd
    desc = host.model_desc(**GEOMETRIES[geom])
    H, KVH, D = desc.hidden, desc.kv_heads, desc.head_dim
    eng = host.Engine(desc, 512)
    weights = make_weights(eng, desc, 44)
    print(f"case prompt projection {geom} first={first} n={n}", flush=True)
    rng = np.random.default_rng(144)
    rows = first + n - context
    h = rng.standard_normal((desc.n_taps, rows, H)).astype(np.float16)
    for slot in range(desc.n_taps):
        eng.capture_tap(slot, torch.from_numpy(h[slot]).cuda(), context, first)
    eng.project_prompt(first, first + n)
    torch.cuda.synchronize()
    W = rnd.Weights(desc, weights)
    C = rnd.Caches()
    T = eng.max_context + desc.block
    for j in range(desc.draft_layers):
        C.ring[j] = (np.zeros((T, KVH, D)), np.zeros((T, KVH, D)))
    rope = rnd.h2f(rope_numpy(desc.rope_base, desc.rope_pairs, D, T + 1))
    rnd.project_prompt(W, C, h[:, first - context:].astype(np.float64), first, rope)
    bt = torch.from_numpy(eng.download("ring_table", np.int32))
    for j in range(desc.draft_layers):
        kp = torch.from_numpy(eng.download(f"ring.D{j}.k", np.uint16)).view(torch.float16).reshape(-1, KVH, 32, D)
        vp = torch.from_numpy(eng.download(f"ring.D{j}.v", np.uint16)).view(torch.float16).reshape(-1, KVH, D, 32)
        kr, vr = host.kv_from_pages(kp, vp, range(first, first + n), bt)
        wk, wv = C.ring[j][0][first:first + n], C.ring[j][1][first:first + n]
        kerr = np.max(np.abs(kr.astype(np.float64) - wk))
        verr = np.max(np.abs(vr.astype(np.float64) - wv))
        print(f"drafter layer {j}: ring K max-abs {kerr:.3e} (scale {np.max(np.abs(wk)):.2f}), V max-abs {verr:.3e} "
              f"(scale {np.max(np.abs(wv)):.2f})", flush=True)
        assert kerr <= 2 * ulp16(np.max(np.abs(wk))) and verr <= 2 * ulp16(np.max(np.abs(wv)))
        # positions outside [first, first + n) were not written
        ko, _ = host.kv_from_pages(kp, vp, [first - 1, first + n], bt)
        assert not np.any(ko)
    for bad in ((first + 1, first + n), (first, first + desc.draft_window + 1)):
        with pytest.raises(host.DsparkError, match="EINVAL"):
            eng.project_prompt(*bad)
    with pytest.raises(host.DsparkError, match="EINVAL"):
        eng.capture_tap(desc.n_taps, torch.from_numpy(h[0]).cuda(), context, first)
    eng.close()


def test_init_seen(dev):
    torch = dev
    host = load_host()
    desc = host.model_desc(**GEOMETRIES["small"])
    eng = host.Engine(desc, 512)
    eng.init_seen([5, 7, 2047, 5, desc.vocab, -3], 1.25)
    torch.cuda.synchronize()
    seen = eng.download("seen", np.uint32)
    bits = {int(w) * 32 + b for w in range(seen.size) for b in range(32) if (seen[w] >> b) & 1}
    assert bits == {5, 7, 2047}
    rep = eng.download("rep", np.float32)[:2]
    assert rep[0] == np.float32(1.25) and rep[1] == np.float32(1.0) / np.float32(1.25)
    eng.init_seen([], 0.0)  # rep 0 means none
    torch.cuda.synchronize()
    assert not eng.download("seen", np.uint32).any() and eng.download("rep", np.float32)[0] == 1.0
    eng.close()


def test_phase_trace(dev):
    """Traced rounds record every phase in order (begin, context, drafter, crop head, Markov, each verify layer, LM head,
    commit) with a non-decreasing clock, number the rounds that run, record nothing for a stopped round, and commit
    the same tokens as untraced rounds from the same start."""
    torch = dev
    host = load_host()
    desc = host.model_desc(**GEOMETRIES["small"])
    eng = host.Engine(desc, 512)
    make_weights(eng, desc, 45)
    setup_caches(eng, host, desc, A0, CTX_LO, 145)
    print("case phase trace", flush=True)
    rings = conv_rings(eng)
    st0 = dict(a=A0, anchor=ANCHOR, count=0, rounds_left=3, limit=eng.max_context, budget=512, eos=-1, ctx_new=1,
               ctx_pos=A0 - 1, ctx_lo=CTX_LO, run=1, skip_rounds=1, stop_at=eng.max_context, ckpt_slot=-1,
               tokens=[ANCHOR])
    outs = []
    for traced in (False, True):
        for nm, buf in rings.items():
            eng.upload(nm, buf)
        eng.init_seen([])
        eng.set_state(**st0)
        eng.trace(traced)
        for _ in range(4):  # the fourth round finds run == 0 (rounds_left was 3)
            eng.round(0, A0)
        torch.cuda.synchronize()
        st = eng.state()
        outs.append((st.count, eng.download("out_tokens", np.int32)[:st.count].tolist(),
                     [getattr(st, f) for f in host.STATE_FIELDS]))
    assert outs[0] == outs[1]
    marks = eng.trace_read()
    eng.trace(False)
    per_round = [host.TRACE_PHASES[p] for p in (0, 1, 2, 3, 4)] + \
        [f"verify_L{i}" for i in range(desc.n_layers)] + ["lm_head", "commit"]
    assert len(marks) == 3 * len(per_round), len(marks)
    for r in range(3):
        got = [host.trace_phase_name(p) for (rr, p, _) in marks[r * len(per_round):(r + 1) * len(per_round)]]
        assert got == per_round and all(rr == r for (rr, _, _) in marks[r * len(per_round):(r + 1) * len(per_round)])
    clocks = [c for (_, _, c) in marks]
    assert all(b >= a for a, b in zip(clocks, clocks[1:])) and clocks[-1] > clocks[0]
    eng.close()


@pytest.mark.parametrize("geom", ["small", "mid", "ref_rec", "ref_rec_fresh", "ref_x8"])
def test_stopped_round_writes_nothing(dev, geom, monkeypatch):
    """A round enqueued on a stopped State (run == 0) leaves every engine buffer as it was: pools, rings, conv state,
    State, outputs and every scratch buffer (each kernel issues its first loads before it tests run, and must write
    nothing when run == 0; dspark.hip:2438-2440 leaves the persistent loop at run == 0)."""
    torch = dev
    host = load_host()
    if geom.endswith("_fresh"):
        monkeypatch.setenv("DSPARK_FRESH_REC_PPS", "1")
    desc = host.model_desc(**GEOMETRIES[geom])
    eng = host.Engine(desc, 512)
    make_weights(eng, desc, 47)
    setup_caches(eng, host, desc, A0, CTX_LO, 147)
    print(f"case stopped round {geom}", flush=True)
    eng.set_state(a=A0, anchor=ANCHOR, count=0, rounds_left=3, limit=eng.max_context, budget=512, eos=-1, ctx_new=1,
                  ctx_pos=A0 - 1, ctx_lo=CTX_LO, run=0, skip_rounds=1, stop_at=eng.max_context, ckpt_slot=-1,
                  tokens=[ANCHOR])
    torch.cuda.synchronize()
    before = {n: eng.download(n, np.uint8) for n in eng.names()}
    for m in (0, 1):  # a drafting round, and a verify-only round of one token
        eng.round(m, A0)
    torch.cuda.synchronize()
    changed = [n for n in eng.names() if not np.array_equal(eng.download(n, np.uint8), before[n])]
    assert not changed, changed
    eng.close()
