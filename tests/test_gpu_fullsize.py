"""Full-size DSpark rounds against the oracle, teacher-forced layer by layer (through the engine's C ABI).

The round parity test (test_gpu_engine.py) compares whole rounds with the oracle at small geometries. The GEMM plans
that carry the real rounds (w13 16384 x 2048 in strips and K ranges, the 65536- and 128000-row LM heads with X^T in
LDS, w2 over K = 8192 or 7680 in two bands, tile-major weights and operand-order activations) only run at the full
geometries, so here one round runs at:

* the C4 geometry (16 layers, 10 conv k=3 + 6 GQA 32/8/64, hidden 2048, FFN 8192, vocab 65536,
  4-layer drafter, 16-token blocks) at context 32768, fp16 K/V pages and per-row weight scales;
* the reference geometry (24 layers, 16/4/128, conv k=7, sliding 256, FFN 7680, vocab 128000, 3-layer drafter,
  9-token blocks) at context 4096 on the reference's formats: int8 K/V records and per-128-column weight scales.

With the engine's layer-boundary dumps on (dspark_engine_debug_layers), every drafter and target layer is recomputed
by oracle/round.py from the GPU's own input to that layer (the residual and the added FFN output), and its output is
compared with the GPU's next dump; the cropped head from the GPU's last drafter dump; the LM head from the GPU's own
final activations. So a defect in one kernel shows at its layer instead of being lost among the fp16 last-bit
differences that a multi-layer pass carries forward. Bars: every layer output (residual and FFN output) within
LAYER_REL of its largest magnitude (int8 records: LAYER_REL_REC, where a K/V element at a code boundary moves one
code step, 1/127 of its row's range; int8 x: LAYER_REL_X8, where a GEMM input that GPU and oracle round to
neighbouring fp16 values, or to the same value within an fp32 ulp of a code midpoint, takes codes one step apart,
1/127 of its 16-column piece's range -- measured 4.9e-3 for drafter and 7.6e-3 for target FFN outputs, against
5.1e-4 with fp16 x); cropped-head outputs and LM-head logits within 2e-3 max-abs; argmax
keys and the commit books bit-exact.
"""
import ctypes

import numpy as np
import pytest

from conftest import load_host, rope_numpy

pytestmark = pytest.mark.gpu

LAYER_REL = 1e-3
LAYER_REL_REC = 5e-3
LAYER_REL_X8 = 2e-2
LOGIT_TOL = 2e-3
RUNTIME = ("kv.", "ring.", "conv.", "state", "seen", "out_tokens", "rep", "h0", "h1", "x16", "mix", "q16", "gate",
           "y16", "vout", "a16", "w2out", "ctx", "ckv_out", "taps", "logits", "base", "keys", "ws_", "rope",
           "ring_table", "tap_x", "plant", "conv_state", "trace", "debug_layers", "x_scales", "y_scales", "xc16", "xc_scales")


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


def weights_of(eng):
    """Host copies of every weight tensor, in the dtypes oracle/round.py reads."""
    out = {}
    for n in eng.names():
        if n.startswith(RUNTIME):
            continue
        if (n.endswith(".w") and not n.endswith("conv.w")) or n in ("markov.w2q", "markov.w1q"):
            dt = np.uint8
        elif n in ("markov.w2s", "markov.w1s", "conf_c2"):
            dt = np.float32
        elif n == "crop_ids":
            dt = np.int32
        else:
            dt = np.uint16
        out[n] = eng.download(n, dt)
    return out


def xop_rows(buf, rows, K, tbs):
    """Rows [rows][K] of an activation buffer in the matrix cores' operand order (xop_elem of csrc/common.h)."""
    t = np.arange(rows)[:, None]
    k = np.arange(K)[None, :]
    idx = ((((k >> 6) * tbs + (t >> 4)) * 2 + ((k >> 3) & 1)) * 64 + ((k >> 4) & 3) * 16 + (t & 15)) * 8 + (k & 7)
    return buf[idx]


def rec_values(pages_u8, KVH, positions, table=None):
    """Dequantized K and V ([n][KVH][128] fp64) of record pages at the given positions."""
    recs = pages_u8.reshape(-1, 32, KVH, 264)
    pos = np.asarray(positions)
    phys = table[pos // 32] if table is not None else pos // 32
    r = recs[phys, pos % 32]  # [n][KVH][264]
    kq = r[:, :, :128].copy().view(np.int8).astype(np.float64)
    ks = r[:, :, 128:132].copy().view(np.float32).astype(np.float64)
    vq = r[:, :, 132:260].copy().view(np.int8).astype(np.float64)
    vs = r[:, :, 260:264].copy().view(np.float32).astype(np.float64)
    return kq * ks, vq * vs


def setup_full(eng, host, desc, a, ctx_lo, seed):
    """Seeded caches (target K/V for positions < a, drafter rings for [ctx_lo, a), conv histories, taps) written
    through the library's own writers; the oracle's caches hold what the pages hold (the fp16 values, or the
    dequantized records)."""
    import torch
    from oracle import round as rnd
    rng = np.random.default_rng(seed)
    lib = host.lib()
    B, H, KVH, D = desc.block, desc.hidden, desc.kv_heads, desc.head_dim
    T = eng.max_context + B
    rec = desc.kv_format == 1
    C = rnd.Caches()

    def write(kname, vname, pos0, n, bt_name=None):
        k = rng.standard_normal((n, KVH, D)).astype(np.float32)
        v = rng.standard_normal((n, KVH, D)).astype(np.float32)
        bt = ctypes.c_void_p(eng.tensor(bt_name)[0]) if bt_name else None
        K = np.zeros((T, KVH, D))
        V = np.zeros((T, KVH, D))
        if rec:
            kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
            ptr_, nbytes = eng.tensor(kname)
            host.check(lib.dspark_kv_write_rec(ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()), KVH * D,
                                               ctypes.c_void_p(ptr_), bt, nbytes // (32 * KVH * 264), KVH, pos0, n,
                                               None), "kv_write_rec")
            torch.cuda.synchronize()
            table = eng.download(bt_name, np.int32) if bt_name else None
            K[pos0:pos0 + n], V[pos0:pos0 + n] = rec_values(eng.download(kname, np.uint8), KVH,
                                                             range(pos0, pos0 + n), table)
        else:
            k16, v16 = k.astype(np.float16), v.astype(np.float16)
            kd, vd = torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda()
            kptr, kbytes = eng.tensor(kname)
            host.check(lib.dspark_kv_write(ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()), KVH * D,
                                           ctypes.c_void_p(kptr), ctypes.c_void_p(eng.tensor(vname)[0]), bt,
                                           kbytes // (KVH * 32 * D * 2), KVH, D, pos0, n, None), "kv_write")
            torch.cuda.synchronize()
            K[pos0:pos0 + n], V[pos0:pos0 + n] = k16, v16
        return K, V

    for i in range(desc.n_layers):
        if desc.layer_kind[i] == 0:
            ring = rng.standard_normal((128, H)).astype(np.float16)
            eng.upload(f"conv.L{i}", ring.view(np.uint16))
            C.conv[i] = {pos: ring[pos % 128].astype(np.float64) for pos in range(a - desc.conv_kernel + 1, a)}
        else:
            C.kv[i] = write(f"kv.L{i}.rec" if rec else f"kv.L{i}.k", f"kv.L{i}.v", 0, a)
    for j in range(desc.draft_layers):
        C.ring[j] = write(f"ring.D{j}.rec" if rec else f"ring.D{j}.k", f"ring.D{j}.v", ctx_lo, a - ctx_lo,
                          "ring_table")
    taps = rng.standard_normal((desc.n_taps, B, H)).astype(np.float32)
    eng.upload("taps", taps)
    C.taps = taps.astype(np.float64)
    return C


def ring_rows(eng, desc, j, positions):
    """The GPU's drafter ring j at the given positions (fp64 values of its fp16 pages or dequantized records)."""
    import torch
    host = load_host()
    table = eng.download("ring_table", np.int32)
    if desc.kv_format == 1:
        return rec_values(eng.download(f"ring.D{j}.rec", np.uint8), desc.kv_heads, positions, table)
    KVH, D = desc.kv_heads, desc.head_dim
    kr, vr = host.kv_from_pages(
        torch.from_numpy(eng.download(f"ring.D{j}.k", np.uint16)).view(torch.float16).reshape(-1, KVH, 32, D),
        torch.from_numpy(eng.download(f"ring.D{j}.v", np.uint16)).view(torch.float16).reshape(-1, KVH, D, 32),
        positions, torch.from_numpy(table))
    return kr.astype(np.float64), vr.astype(np.float64)


def rel_err(got, want):
    return float(np.max(np.abs(got - want)) / max(1e-30, np.max(np.abs(want))))


@pytest.mark.parametrize("geom", ["c4", "ref", "ref_x8"])
def test_full_size_round_teacher_forced(dev, orc, geom):
    """ref_x8: the reference geometry on its formats with its default activation format, int8 x per 16 columns
    (LFM3_X8, kernels/dspark.hip:24-26)."""
    torch = dev
    host = load_host()
    from oracle import round as rnd
    if geom == "c4":
        desc, a = host.c4_desc(block=16), 32768
    else:
        desc, a = host.ref_desc(x_format=1 if geom == "ref_x8" else 0), 4096
    print(f"case full-size round {geom} ctx={a}", flush=True)
    B, H, V, N = desc.block, desc.hidden, desc.vocab, desc.crop_rows
    DL, NL = desc.draft_layers, desc.n_layers
    MV = min(B, 1 + desc.max_drafts)
    eng = host.Engine(desc, a + 64)
    eng.init_random(20261203 + a)
    torch.cuda.synchronize()
    ctx_lo, ctx_new = a - desc.draft_window, 3
    C = setup_full(eng, host, desc, a, ctx_lo, 77 + a)
    st0 = dict(a=a, anchor=17, count=0, rounds_left=1, limit=a + 40, budget=512, eos=-1, ctx_new=ctx_new,
               ctx_pos=a - ctx_new, ctx_lo=ctx_lo, run=1, skip_rounds=1, stop_at=a + 64, ckpt_slot=-1, tokens=[17])
    eng.set_state(**st0)
    eng.init_seen([])
    eng.debug_layers(True)
    eng.round(0, a)
    torch.cuda.synchronize()
    eng.debug_layers(False)
    st = eng.state()
    dumps = eng.download("debug_layers", np.float32).reshape(DL + NL + 2, 2, B, H).astype(np.float64)
    crop_n = (N + 1 + 15) // 16 * 16
    base_gpu = eng.download("base", np.float32)[:B * crop_n].reshape(B, crop_n)[:, :N + 1].astype(np.float64)
    logits_gpu = eng.download("logits", np.float32)[:MV * V].reshape(MV, V)
    keys_gpu = eng.download("keys", np.uint64)[:MV]
    x_fin = xop_rows(eng.download("x16", np.uint16), MV, H, (B + 15) // 16).view(np.float16).astype(np.float64)
    x8 = desc.x_format == 1
    if x8:  # x16 holds the final norm's int8 codes, x_scales their scales
        x_sc = eng.download("x_scales", np.float32).reshape((B + 15) // 16 * 16, -1)[:MV, :H // 16]
    W = rnd.Weights(desc, weights_of(eng))
    rope = rnd.h2f(rope_numpy(desc.rope_base, desc.rope_pairs, desc.head_dim, eng.max_context + B + 1))
    rope_swa = None
    if desc.rope_base_swa > 0:
        rope_swa = rnd.h2f(rope_numpy(desc.rope_base_swa, desc.rope_pairs_swa, desc.head_dim, eng.max_context + B + 1))
    bar = LAYER_REL_X8 if desc.x_format == 1 else (LAYER_REL_REC if desc.kv_format == 1 else LAYER_REL)
    worst = {}

    # context projection from the seeded taps into the drafter rings (fp16 pages: one ulp; records: one code step)
    rnd.context_projection(W, C, st0, rope)
    pos = list(range(a - ctx_new, a))
    for j in range(DL):
        gk, gv = ring_rows(eng, desc, j, pos)
        wk, wv = C.ring[j][0][a - ctx_new:a], C.ring[j][1][a - ctx_new:a]
        e = max(rel_err(gk, wk), rel_err(gv, wv))
        worst["context"] = max(worst.get("context", 0.0), e)
        assert e <= (1.5 / 127 if desc.kv_format == 1 else LAYER_REL), ("context projection", j, e)
        # the drafter layers below read the ring as the GPU wrote it
        C.ring[j][0][a - ctx_new:a], C.ring[j][1][a - ctx_new:a] = gk, gv

    # drafter layers, each from the GPU's own input
    for j in range(DL):
        h, v = dumps[j, 0], (dumps[j, 1] if j else None)
        h2, v2 = rnd.drafter_layer(W, C, j, h, v, a, ctx_lo, rope)
        eh, ev = rel_err(dumps[j + 1, 0], h2), rel_err(dumps[j + 1, 1], v2)
        print(f"drafter layer {j}: residual {eh:.2e}, FFN output {ev:.2e} (relative to the largest magnitude)",
              flush=True)
        worst["drafter"] = max(worst.get("drafter", 0.0), eh, ev)
        assert eh <= bar and ev <= bar, ("drafter layer", j, eh, ev)
    base = rnd.crop_head(W, dumps[DL, 0], dumps[DL, 1])
    berr = float(np.max(np.abs(base_gpu - base)))
    print(f"cropped head: max-abs {berr:.2e} (scale {np.max(np.abs(base)):.2f})", flush=True)
    assert berr <= LOGIT_TOL

    # target layers over the verify rows, each from the GPU's own input
    for i in range(NL):
        s_ = DL + 1 + i
        h, v = dumps[s_, 0, :MV], (dumps[s_, 1, :MV] if i else None)
        _, h2, v2 = rnd.verify_layer(W, C, i, h, v, a, rope, rope_swa, threads=16)
        eh, ev = rel_err(dumps[s_ + 1, 0, :MV], h2), rel_err(dumps[s_ + 1, 1, :MV], v2)
        print(f"target layer {i} (kind {desc.layer_kind[i]}): residual {eh:.2e}, FFN output {ev:.2e}", flush=True)
        worst["target"] = max(worst.get("target", 0.0), eh, ev)
        assert eh <= bar and ev <= bar, ("target layer", i, eh, ev)

    # the final norm (fp16 values: at most one rounding step apart; int8 x: the same scales within fp32 rounding and
    # codes at most one step apart) and the LM head from the GPU's own activations
    _, x_orc = rnd.final_x(W, dumps[DL + 1 + NL, 0, :MV], dumps[DL + 1 + NL, 1, :MV])
    if x8:
        q_orc, s_orc = orc.quantize_x16(x_orc.astype(np.float32))
        assert np.all(np.abs(x_sc - s_orc) <= 1e-5 * s_orc), "final norm scales"
        dq = np.abs(x_fin - q_orc.astype(np.float64))
        print(f"final norm codes: {int(np.count_nonzero(dq))} of {dq.size} one step apart", flush=True)
        assert dq.max() <= 1 and np.count_nonzero(dq) <= dq.size // 100, "final norm codes"
        logits = rnd.lm_head(W, x_fin, xs=x_sc)
    else:
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x_orc), 2.0 ** -14))) - 10)
        assert np.all(np.abs(x_fin - x_orc) <= ulp), "final norm"
        logits = rnd.lm_head(W, x_fin)
    lerr = float(np.max(np.abs(logits_gpu - logits)))
    print(f"LM head: max-abs {lerr:.2e} (scale {np.max(np.abs(logits)):.2f}); worst layer errors {worst}", flush=True)
    assert lerr <= LOGIT_TOL

    # argmax keys of the GPU's logits bit-exact with the oracle's key rule; the commit books from those keys
    verified = [17] + list(st.tokens)[1:st.M] + list(st.tokens)[st.M:MV]
    seen = eng.download("seen", np.uint32)
    want_keys = orc.verify_argmax(logits_gpu, seen, np.array(verified[:MV], np.int32))
    assert np.array_equal(keys_gpu, want_keys)
    ost = orc.new_state(**dict(st0, tokens=verified[:st.M]))
    out = np.zeros(1024, np.int32)
    acc = orc.accept_commit(ost, orc.keys_to_tokens(keys_gpu), st.M, out, np.zeros_like(seen))
    for f in host.STATE_FIELDS:
        if f != "M":
            assert getattr(st, f) == getattr(ost, f), f
    assert st.a == a + acc + 1
    eng.close()
