"""CPU restatement of one DSpark round -- TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg).

Composes the pinned pieces of liborc.so (fp16 RNE, fp64 verify attention, penalised argmax keys, acceptance/commit)
with numpy statements of the layer arithmetic, following the reference's dspark_kernel section by section:
  context projection   dspark.hip:2487-2518, 2682-2705 (tap norms -> fc -> hidden norm -> ckv -> k norm + RoPE)
  drafter block        dspark.hip:2463-2486, 2706-2780 (kind 3: no sandwich norms, no gate, bidirectional block)
  cropped head         dspark.hip:2564-2587
  Markov/confidence    dspark.hip:2322-2366, 2633-2664
  verify               dspark.hip:2519-2846 (sandwich norms 722-843, conv_wave 2191-2214, query_fresh 999-1061,
                       gated combine 2132-2185, LM head + argmax 2219-2318)
  commit               dspark.hip:2848-2913
Rounding points are the ones the GPU path uses: GEMM inputs, attention Q/K/V and conv/attention/FFN outputs are
fp16; residuals, GEMM outputs and scores are wider (fp64 here).
"""
import numpy as np

from . import oracle as orc


def f16(x):
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def h2f(u16):
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float64)


class Weights:
    """Host copies of an engine's tensors (names as include/dspark.h's engine documents)."""

    def __init__(self, desc, tensors):
        self.d = desc
        self.t = tensors
        # LFM3_X8 (kernels/dspark.hip:24-26): every int8 GEMM's input quantized per 16 columns (x_format 1)
        self.x8 = getattr(desc, "x_format", 0) == 1

    def mm(self, x, w, s):
        """The int8 GEMM of the model's activation format: fp16-valued x (gemm), or under LFM3_X8 x (fp32-valued from
        a norm, fp16-valued otherwise) quantized per 16 columns and multiplied as unit_dot_r does (dspark.hip:541-566):
        per piece the exact integer dot times fp32(group scale * piece scale), summed in fp64."""
        if not self.x8:
            return gemm(x, w, s)
        assert s.ndim == 2, "LFM3_X8 goes with per-128-column weight scales"
        q, sc = orc.quantize_x16(np.asarray(x, np.float64).astype(np.float32))
        M, K = q.shape
        P = K // 16
        qp = q.astype(np.float64).reshape(M, P, 16).transpose(1, 0, 2)        # [P][M][16]
        wp = w.reshape(w.shape[0], P, 16).transpose(1, 2, 0)                  # [P][16][N]
        d = np.matmul(qp, wp)                                                 # [P][M][N] exact integers
        f = (np.repeat(s, 8, axis=0)[:, None, :].astype(np.float32) *
             sc.T[:, :, None]).astype(np.float32).astype(np.float64)          # [P][M][N] fp32(gs * s_p)
        return (f * d).sum(axis=0)

    def f16(self, name, shape=None):
        a = h2f(self.t[name])
        return a.reshape(shape) if shape else a

    def gemm_w(self, name, rows, cols):
        """(q [rows][cols], scales): per-row scales [rows], or (weight_format 1) per-128-column group scales
        [cols / 128][rows] from the tensor's [cols / 128][N] layout (N its allocated rows)."""
        w = (self.t[name + ".w"][:rows * cols].astype(np.int16) - 128).reshape(rows, cols).astype(np.float64)
        if getattr(self.d, "weight_format", 0):
            raw = self.t[name + ".s"]
            n_alloc = raw.size // (cols // 128)
            s = h2f(raw).reshape(cols // 128, n_alloc)[:, :rows]
        else:
            s = h2f(self.t[name + ".s"][:rows])
        return w, s


def gemm(x16, w, s):
    """y = (x @ q^T) * scale (per output row), or with per-128-column group scales s [K/128][N] the sum over groups of
    each group's products times its scale (gemv_phase, dspark.hip:553-580); fp64; x already fp16-valued."""
    if s.ndim == 2:
        return sum((x16[:, 128 * g:128 * g + 128] @ w[:, 128 * g:128 * g + 128].T) * s[g][None, :]
                   for g in range(s.shape[0]))
    return (x16 @ w.T) * s[None, :]


def resnorm(h_old, v, post_w, norm_w, sandwich, eps, x8=False):
    """norm_compute (dspark.hip:722-843) for a block of rows: returns (h_new, x fp16-valued), or with x8 (LFM3_X8,
    dspark.hip:802-823: the norm quantizes its fp32 value) x fp32-valued."""
    H = norm_w.shape[0]
    h = np.zeros_like(v if v is not None else h_old) if h_old is None else h_old.copy()
    if v is not None:
        a = 1.0 / np.sqrt((v * v).sum(1, keepdims=True) / H + eps) if sandwich else 1.0
        pw = post_w if post_w is not None else 1.0
        h = h + (v * a) * pw
    inv = 1.0 / np.sqrt((h * h).sum(1, keepdims=True) / H + eps)
    x = h * inv * norm_w[None, :]
    return h, (x.astype(np.float32).astype(np.float64) if x8 else f16(x))


def rope_rows(x, pos, table, rot):
    """x [D] (one head), rotated by the table row of `pos` (cos | sin, fp16 values), pairs (i, i + D/2), i < rot."""
    D = x.shape[0]
    half = D // 2
    c = table[pos, :half]
    s = table[pos, half:]
    y = x.copy()
    i = np.arange(rot)
    y[i] = x[i] * c[i] - x[i + half] * s[i]
    y[i + half] = x[i + half] * c[i] + x[i] * s[i]
    return y


def norm_head(x, w, eps):
    D = x.shape[0]
    return x / np.sqrt((x * x).sum() / D + eps) * w


class Caches:
    """Logical K/V per attention layer ([positions][KVH][D] fp16 values), conv rings, drafter rings, taps."""

    def __init__(self):
        self.kv = {}      # target layer -> (K, V) arrays [T][KVH][D] (fp64 holding fp16 values)
        self.ring = {}    # drafter layer -> (K, V) arrays indexed by absolute position
        self.conv = {}    # target layer -> {position: bx [H]}
        self.taps = None  # [n_taps][B][H]


def attn_fp16(q16, K, V, a, M, start, window, causal, threads=1):
    """fp64 verify attention via liborc (q [M][QH][D], K/V [T][KVH][D], all fp16-valued); threads > 1: the threaded
    form of the same arithmetic."""
    to16 = lambda x: np.ascontiguousarray(np.asarray(x, np.float64).astype(np.float16).view(np.uint16))
    T = a + M
    if threads > 1:
        return orc.verify_attention_mt(to16(q16), to16(K[:T]), to16(V[:T]), a, start, window, causal, threads)
    return orc.verify_attention(to16(q16), to16(K[:T]), to16(V[:T]), a, start, window, causal)


def attn_rec(q16, K, V, a, M, start, window, causal, threads=1):
    """The int8-record attention (dspark.hip:1020-1035, 1215-1412): q (fp16-valued) quantized per 32-dim group, K/V
    [T][KVH][D] already the dequantized record values (kv_store), fp64 softmax of those operands."""
    QH, D = q16.shape[1], q16.shape[2]
    q8, qs = orc.rec_quantize_q(np.asarray(q16, np.float64).astype(np.float16).view(np.uint16).reshape(-1, D))
    qd = (q8.astype(np.float64).reshape(-1, D // 32, 32) * qs.astype(np.float64)[:, :, None]).reshape(M, QH, D)
    T = a + M
    return orc.verify_attention_d(qd, K[:T], V[:T], a, start, window, causal)


def kv_store(d, K, V, pos, h, k, v):
    """K/V of (pos, KV head h) into the logical cache: fp16 values, or (kv_format 1) the dequantized quantize_pair
    record of the fp32 values (kernels/ops.hip:212-224)."""
    if getattr(d, "kv_format", 0):
        kq, ks = orc.rec_quantize(np.asarray(k, np.float64).astype(np.float32))
        vq, vs = orc.rec_quantize(np.asarray(v, np.float64).astype(np.float32))
        K[pos, h] = kq.astype(np.float64) * float(ks)
        V[pos, h] = vq.astype(np.float64) * float(vs)
    else:
        K[pos, h] = f16(k)
        V[pos, h] = f16(v)


def attention(d, q16, K, V, a, M, start, window, causal, threads=1):
    return (attn_rec if getattr(d, "kv_format", 0) else attn_fp16)(q16, K, V, a, M, start, window, causal, threads)


def context_projection(W, C, st, rope):
    """The round's context projection (sec 0): the taps of the last round's committed positions ctx_pos ..
    ctx_pos + ctx_new - 1 (C.taps, the residual stream after each tapped layer) into the drafter rings."""
    d = W.d
    H, B = d.hidden, d.block
    n_new, pos0 = st["ctx_new"], st["ctx_pos"]
    if n_new <= 0:
        return
    tn = W.f16("tap_norms", (d.n_taps, H))
    xs = [resnorm(C.taps[b][:B], None, None, tn[b], 0, d.eps, W.x8)[1] for b in range(d.n_taps)]
    project_rows(W, C, np.concatenate(xs, axis=1)[:n_new], pos0, rope)


def tap_rows(W, h16, slot):
    """captureTap (dspark.go:439-459 -> ops.hip:89-101 rms_norm): fp16(h / rms(h) * tap_norms[slot]) per row."""
    d = W.d
    w = W.f16("tap_norms", (d.n_taps, d.hidden))[slot]
    return resnorm(np.asarray(h16, np.float64), None, None, w, 0, d.eps)[1]


def project_prompt(W, C, h16_taps, first, rope):
    """captureTap + projectPrompt (dspark.go:439-492): h16_taps [n_taps][n][H] (fp16-valued hidden states after each
    tapped layer for positions first .. first + n - 1) -> drafter ring rows of those positions."""
    x = np.concatenate([tap_rows(W, h16_taps[b], b) for b in range(W.d.n_taps)], axis=1)
    project_rows(W, C, x, first, rope)


def project_rows(W, C, x, pos0, rope):
    """x [n][n_taps * H] (normed taps, fp16-valued) -> fc -> hidden norm -> ckv -> per drafter layer k norm + RoPE
    (the drafter's table) and v -> ring rows pos0 .. pos0 + n - 1 (dspark.hip:2682-2705, 2487-2518)."""
    d = W.d
    H = d.hidden
    n_new = x.shape[0]
    fw, fs = W.gemm_w("fc", H, d.n_taps * H)
    c = W.mm(x, fw, fs)
    _, x2 = resnorm(None, c, None, W.f16("hidden_norm"), 0, d.eps, W.x8)
    KVH, D = d.kv_heads, d.head_dim
    rows = d.draft_layers * 2 * KVH * D
    cw, cs = W.gemm_w("ckv", rows, H)
    kv = W.mm(x2, cw, cs)
    for j in range(d.draft_layers):
        kn = W.f16(f"D{j}.k_norm")
        K, V = C.ring[j]
        for t in range(n_new):
            pos = pos0 + t
            row = kv[t, j * 2 * KVH * D:(j + 1) * 2 * KVH * D]
            for h in range(KVH):
                k = norm_head(row[h * D:(h + 1) * D], kn, d.eps)
                kv_store(d, K, V, pos, h, rope_rows(k, pos, rope, d.rope_pairs),
                         row[KVH * D + h * D:KVH * D + (h + 1) * D])


def drafter_layer(W, C, j, h, v_prev, a, ctx_lo, rope):
    """Drafter layer j over the block rows of the residual h (v_prev: the previous layer's FFN output, None for the
    first): kind 3, no sandwich post-norms, no gate, attention to the ring context [max(ctx_lo, a - window), a) and the
    whole block (dspark.hip:2706-2780, 2531). Stores the block's K/V in ring j. Returns (h, v) for the next layer."""
    d = W.d
    H, QH, KVH, D = d.hidden, d.q_heads, d.kv_heads, d.head_dim
    B = h.shape[0]
    pre = f"D{j}."
    h, x = resnorm(h, v_prev, None, W.f16(pre + "op_norm"), 0, d.eps, W.x8)
    rows = QH * D + 2 * KVH * D
    mw, ms = W.gemm_w(pre + "mix", rows, H)
    mix = W.mm(x, mw, ms)
    qn, kn = W.f16(pre + "q_norm"), W.f16(pre + "k_norm")
    K, V = C.ring[j]
    q16 = np.zeros((B, QH, D))
    for t in range(B):
        pos = a + t
        for qh in range(QH):
            q16[t, qh] = f16(rope_rows(norm_head(mix[t, qh * D:(qh + 1) * D], qn, d.eps), pos, rope, d.rope_pairs))
        for hh in range(KVH):
            o = QH * D + hh * D
            ov = QH * D + KVH * D + hh * D
            kv_store(d, K, V, pos, hh, rope_rows(norm_head(mix[t, o:o + D], kn, d.eps), pos, rope, d.rope_pairs),
                     mix[t, ov:ov + D])
    start = max(ctx_lo, a - d.draft_window)
    o = attention(d, q16, K, V, a, B, start, 0, False)
    y = f16(o.reshape(B, QH * D))
    ow, os_ = W.gemm_w(pre + "out", H, H)
    vout = W.mm(y, ow, os_)
    h, x = resnorm(h, vout, None, W.f16(pre + "ffn_norm"), 0, d.eps, W.x8)
    ww, ws = W.gemm_w(pre + "w13", 2 * d.draft_ffn, H)
    gu = W.mm(x, ww, ws)
    g, u = gu[:, 0::2], gu[:, 1::2]
    act = f16(g / (1.0 + np.exp(-g)) * u)
    w2, s2 = W.gemm_w(pre + "w2", H, d.draft_ffn)
    return h, W.mm(act, w2, s2)


def crop_head(W, h, v_prev):
    """Draft norm + cropped head (dspark.hip:2564-2587): base [B][crop_rows + 1] (fp64)."""
    d = W.d
    _, x = resnorm(h, v_prev, None, W.f16("draft_norm"), 0, d.eps, W.x8)
    cw, cs = W.gemm_w("crop", d.crop_rows + 1, d.hidden)
    return W.mm(x, cw, cs)


def drafter_block(W, C, st, rope):
    """Returns base [B][crop_rows + 1] (fp64): the cropped head over the drafter block."""
    d = W.d
    H, B = d.hidden, d.block
    emb = W.f16("embed", (d.vocab, H))
    toks = [st["anchor"]] + [d.mask_token] * (B - 1)
    h = emb[toks]
    v_prev = None
    for j in range(d.draft_layers):
        h, v_prev = drafter_layer(W, C, j, h, v_prev, st["a"], st["ctx_lo"], rope)
    return crop_head(W, h, v_prev)


def markov(W, st, base):
    """Draft tokens and the verified count M (dspark.hip:2633-2664); returns (tokens list, M, per-step z rows)."""
    d = W.d
    N, R = d.crop_rows, d.markov_rank
    w2q = W.t["markov.w2q"][:N * R].view(np.int8).reshape(N, R).astype(np.int64)
    w2s = W.t["markov.w2s"][:N].astype(np.float32)
    w1q = W.t["markov.w1q"].view(np.int8).reshape(d.vocab, R).astype(np.int64)
    w1s = W.t["markov.w1s"].astype(np.float32)
    c2 = W.t["conf_c2"].astype(np.float32)
    crop_ids = W.t["crop_ids"][:N].astype(np.int64)
    a = st["a"]
    cap = min(min(d.max_drafts, d.block - 1), min(st["limit"] - a, st["budget"] - st["count"]) - 1)
    prev = st["anchor"]
    toks = [prev]
    zs = []
    for j in range(max(cap, 0)):
        conf = np.float32(base[j, N]) + c2[prev] + np.float32(d.conf_bias)
        if not conf >= np.float32(d.conf_thr):
            break
        dots = (w2q @ w1q[prev]).astype(np.float64)   # exact integers
        # fmaf(dot, w2s * w1s, base): one rounding of the exact product plus base
        z = (dots * (w2s * w1s[prev]).astype(np.float64) + base[j, :N].astype(np.float32).astype(np.float64)).astype(np.float32)
        zs.append(z)
        r = int(orc.row_argmax(z[None, :].astype(np.float32))[0])
        prev = int(crop_ids[r])
        toks.append(prev)
    return toks, len(toks), zs


def verify_layer(W, C, i, h, v_prev, a, rope, rope_swa=None, threads=1):
    """Target layer i over the verify rows of the residual h (v_prev: the previous layer's FFN output, None for layer
    0): sandwich norm, conv (conv_wave) or attention (query_fresh, verify attention, gated combine), out GEMM, sandwich
    norm, gated FFN (dspark.hip:2519-2846). Updates layer i's K/V cache or conv ring at positions a .. a + rows - 1.
    Returns (h after the first norm's add -- the tap of layer i - 1 --, h, v) with (h, v) the next layer's input."""
    d = W.d
    H, QH, KVH, D, I = d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.ffn
    B = h.shape[0]
    pre = f"L{i}."
    post = W.f16(f"L{i - 1}.post_ffn_norm") if i else None
    h, x = resnorm(h, v_prev, post, W.f16(pre + "op_norm"), 1, d.eps, W.x8)
    h_in = h
    kind = d.layer_kind[i]
    if kind == 0:
        mw, ms = W.gemm_w(pre + "mix", 3 * H, H)
        mix = W.mm(x, mw, ms)
        cw = W.f16(pre + "conv.w", (H, d.conv_kernel))
        ring = C.conv[i]
        Kc = d.conv_kernel
        y = np.zeros((B, H))
        for t in range(B):
            Bv, Cv, Xv = mix[t, 0::3], mix[t, 1::3], mix[t, 2::3]
            bx = f16(Bv * Xv)
            conv = cw[:, Kc - 1] * bx
            for k in range(Kc - 1):
                conv = conv + cw[:, k] * ring[a + t - (Kc - 1) + k]
            ring[a + t] = bx
            y[t] = f16(Cv * conv)
    else:
        rows = QH * D + 2 * KVH * D + QH
        rows16 = (rows + 15) // 16 * 16
        mw, ms = W.gemm_w(pre + "mix", rows16, H)
        mix = W.mm(x, mw, ms)
        qn, kn = W.f16(pre + "q_norm"), W.f16(pre + "k_norm")
        K, V = C.kv[i]
        own = kind == 2 and getattr(d, "rope_base_swa", 0) > 0
        table = rope_swa if own else rope
        rot = d.rope_pairs_swa if own else d.rope_pairs
        q16 = np.zeros((B, QH, D))
        for t in range(B):
            pos = a + t
            for qh in range(QH):
                q16[t, qh] = f16(rope_rows(norm_head(mix[t, qh * D:(qh + 1) * D], qn, d.eps), pos, table, rot))
            for hh in range(KVH):
                o = QH * D + hh * D
                ov = QH * D + KVH * D + hh * D
                kv_store(d, K, V, pos, hh, rope_rows(norm_head(mix[t, o:o + D], kn, d.eps), pos, table, rot),
                         mix[t, ov:ov + D])
        window = d.window if kind == 2 else 0
        start = max(0, a - window + 1) if window else 0
        o = attention(d, q16, K, V, a, B, start, window, True, threads)
        gate = mix[:, (QH + 2 * KVH) * D:(QH + 2 * KVH) * D + QH].astype(np.float32).astype(np.float64)
        y = f16((o * (1.0 / (1.0 + np.exp(-gate)))[:, :, None]).reshape(B, QH * D))
    ow, os_ = W.gemm_w(pre + "out", H, H)
    vout = W.mm(y, ow, os_)
    h, x = resnorm(h, vout, W.f16(pre + "post_op_norm"), W.f16(pre + "ffn_norm"), 1, d.eps, W.x8)
    ww, ws = W.gemm_w(pre + "w13", 2 * I, H)
    gu = W.mm(x, ww, ws)
    g, u = gu[:, 0::2], gu[:, 1::2]
    act = f16(g / (1.0 + np.exp(-g)) * u)
    w2, s2 = W.gemm_w(pre + "w2", H, I)
    return h_in, h, W.mm(act, w2, s2)


def final_x(W, h, v_prev):
    """The final norm of the verify pass: (h, x), x the LM head's input (fp16-valued, or fp32-valued under
    LFM3_X8)."""
    d = W.d
    return resnorm(h, v_prev, W.f16(f"L{d.n_layers - 1}.post_ffn_norm"), W.f16("final_norm"), 1, d.eps, W.x8)


def lm_head(W, x, row_chunk=16384, xs=None):
    """Logits [rows][V] (fp64) of the int8 LM head (head_run, dspark.hip:2219-2318) for x (as W.mm takes it), or for
    int8 codes x with their piece scales xs (LFM3_X8 input already quantized), by row chunks of the head (its fp64
    copy would be 8 bytes per weight)."""
    d = W.d
    H, V = d.hidden, d.vocab
    out = np.zeros((x.shape[0], V))
    for r0 in range(0, V, row_chunk):
        r1 = min(V, r0 + row_chunk)
        if getattr(d, "weight_format", 0):
            raw = W.t["head.s"]
            sraw = raw.reshape(H // 128, raw.size // (H // 128))[:, r0:r1]
            s = h2f(sraw)
        else:
            s = h2f(W.t["head.s"][r0:r1])
        if xs is not None:
            wb = W.t["head.w"][r0 * H:r1 * H].reshape(r1 - r0, H)
            out[:, r0:r1] = orc.gemm_x8(np.asarray(x).astype(np.int8), xs, wb, np.ascontiguousarray(sraw))
            continue
        w = (W.t["head.w"][r0 * H:r1 * H].astype(np.int16) - 128).reshape(r1 - r0, H).astype(np.float64)
        out[:, r0:r1] = W.mm(x, w, s)
    return out


def verify(W, C, st, tokens, rope, rope_swa=None):
    """Logits [m][V] (fp64) of the verify pass over the first m = min(len(tokens), block) tokens (the reference
    verifies m = 1 + drafts, dspark.hip:2657); updates K/V caches, conv rings and taps. Sliding layers (kind 2)
    rotate with rope_swa and d.rope_pairs_swa when the description gives them their own table (rope_base_swa > 0;
    internal/model/engine.go:333-338), else with `rope` and d.rope_pairs."""
    d = W.d
    H, B = d.hidden, d.block
    emb = W.f16("embed", (d.vocab, H))
    toks = [t if 0 <= t < d.vocab else 0 for t in tokens[:B]]
    B = len(toks)
    h = emb[toks]
    a = st["a"]
    v_prev = None
    taps = np.zeros((d.n_taps, B, H))
    tap_of = {l: i for i, l in enumerate(d.tap_layer[:d.n_taps])}
    for i in range(d.n_layers):
        h_in, h, v_prev = verify_layer(W, C, i, h, v_prev, a, rope, rope_swa)
        if i and (i - 1) in tap_of:
            taps[tap_of[i - 1]] = h_in
    last = d.n_layers - 1
    h, x = final_x(W, h, v_prev)
    if last in tap_of:
        taps[tap_of[last]] = h
    C.taps = taps
    hw, hs = W.gemm_w("head", d.vocab, H)
    return W.mm(x, hw, hs)


def conv_state(C, layer, pos, km1, H):
    """The conv state slot before position `pos` (dspark.hip:2921-2947): element [c][k] = history of position
    pos - km1 + k, channel c (the reference's [H][conv_k - 1] layout, engine.go:546-547)."""
    out = np.zeros((H, km1))
    for k in range(km1):
        out[:, k] = C.conv[layer][pos - km1 + k]
    return out
