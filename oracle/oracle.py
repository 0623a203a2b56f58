"""ctypes view of the CPU oracle (liborc.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the
checker. The C sources (dspark_oracle.c) cite the reference file:line each function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")

_lib = None

c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)
c_i32p = ctypes.POINTER(ctypes.c_int32)
c_u32p = ctypes.POINTER(ctypes.c_uint32)
c_u64p = ctypes.POINTER(ctypes.c_uint64)
c_u8p = ctypes.POINTER(ctypes.c_uint8)
c_i8p = ctypes.POINTER(ctypes.c_int8)

MT_MAX = 64

STATE_FIELDS = ["a", "anchor", "count", "rounds_left", "limit", "budget", "eos", "M", "ctx_new", "ctx_pos",
                "ctx_lo", "run", "force_m", "rounds_done", "accepted", "verified", "miss", "skip", "skip_after",
                "skip_rounds", "stop_at", "ckpt_slot"]


class OrcState(ctypes.Structure):
    """struct State of dspark.hip:134-158 with tokens[] widened to MT_MAX."""
    _fields_ = [(n, ctypes.c_int32) for n in STATE_FIELDS] + [("tokens", ctypes.c_int32 * MT_MAX)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16_n": (None, [c_f32p, c_u16p, ctypes.c_int64]),
            "orc_f16_to_f32_n": (None, [c_u16p, c_f32p, ctypes.c_int64]),
            "orc_mix64": (ctypes.c_uint64, [ctypes.c_uint64]),
            "orc_gen_normal_f16": (None, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64, ctypes.c_float, c_u16p]),
            "orc_gen_int8_uniform": (None, [ctypes.c_uint64, ctypes.c_int64, c_i8p]),
            "orc_gen_uniform_u32": (None, [ctypes.c_uint64, ctypes.c_int64, ctypes.c_uint32, c_u32p]),
            "orc_verify_attention": (None, [c_u16p, c_u16p, c_u16p] + [ctypes.c_int] * 8 + [c_f64p]),
            "orc_attn_partial": (None, [c_u16p, c_u16p, c_u16p] + [ctypes.c_int] * 10 + [c_f64p, c_f64p, c_f64p]),
            "orc_attn_merge": (None, [ctypes.c_int] * 3 + [c_f64p, c_f64p, c_f64p, c_f64p]),
            "orc_verify_attention_f32_mt": (None, [c_u16p, c_u16p, c_u16p] + [ctypes.c_int] * 8 + [c_f32p, ctypes.c_int]),
            "orc_verify_attention_mt": (None, [c_u16p, c_u16p, c_u16p] + [ctypes.c_int] * 8 + [c_f64p, ctypes.c_int]),
            "orc_argmax_key": (ctypes.c_uint64, [ctypes.c_float, ctypes.c_uint32]),
            "orc_key_index": (ctypes.c_uint32, [ctypes.c_uint64]),
            "orc_verify_argmax": (None, [c_f32p, ctypes.c_int, ctypes.c_int, c_u32p, c_i32p, ctypes.c_float,
                                         ctypes.c_float, c_u64p]),
            "orc_penalize_rep": (None, [c_f32p, ctypes.c_int, c_i32p, ctypes.c_int, ctypes.c_float]),
            "orc_argmax_first": (ctypes.c_int32, [c_f32p, ctypes.c_int]),
            "orc_accept_commit": (ctypes.c_int, [ctypes.POINTER(OrcState), c_i32p, ctypes.c_int, ctypes.c_int, c_i32p,
                                                 c_u32p]),
            "orc_kv_commit": (None, [c_u16p, c_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "orc_quantize_rows_int8": (None, [c_u16p, ctypes.c_int, ctypes.c_int, c_i8p, c_f32p]),
            "orc_pack_srow": (ctypes.c_int, [ctypes.c_int]),
            "orc_pack_g128": (None, [c_u16p, ctypes.c_int, ctypes.c_int, c_u8p, c_u16p]),
            "orc_transpose_lanes": (None, [c_u8p, c_u8p, ctypes.c_int64]),
            "orc_gemm_i8": (None, [c_u16p, c_u8p, ctypes.c_int, c_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   c_f64p]),
            "orc_gemm_g128": (None, [c_u16p, c_u8p, c_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_f64p]),
            "orc_quantize_x16": (None, [c_f32p, ctypes.c_int64, c_i8p, c_f32p]),
            "orc_gemm_x8": (None, [c_i8p, c_f32p, c_u8p, c_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_f64p]),
            "orc_gemm_f16": (None, [c_u16p, c_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_f64p]),
            "orc_row_argmax": (None, [c_f32p, ctypes.c_int, ctypes.c_int, c_i32p]),
            "orc_rms_norm": (None, [c_f32p, c_u16p, ctypes.c_int, ctypes.c_float, c_f32p]),
            "orc_rope": (None, [c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_int]),
            "orc_conv_step": (ctypes.c_float, [ctypes.c_float, ctypes.c_float, ctypes.c_float, c_f32p, ctypes.c_int,
                                               c_f32p]),
            "orc_silu": (ctypes.c_float, [ctypes.c_float]),
            "orc_rec_quantize": (ctypes.c_float, [c_f32p, ctypes.c_int, c_i8p]),
            "orc_kv_write_rec": (None, [c_f32p, c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_i32p, c_u8p]),
            "orc_rec_quantize_q": (None, [c_u16p, ctypes.c_int, ctypes.c_int, c_i8p, c_f32p]),
            "orc_verify_attention_d": (None, [c_f64p, c_f64p, c_f64p] + [ctypes.c_int] * 8 + [c_f64p]),
            "orc_verify_attention_rec": (None, [c_u16p, c_u8p, c_i32p] + [ctypes.c_int] * 7 + [c_f64p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


# ---------------------------------------------------------------- fp16
def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_p(x, c_f32p), _p(out, c_u16p), x.size)
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(_p(h, c_u16p), _p(out, c_f32p), h.size)
    return out


# ---------------------------------------------------------------- generators
def normal_f16(seed, shape, offset=0, scale=1.0):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib().orc_gen_normal_f16(seed, offset, n, scale, _p(out, c_u16p))
    return out.reshape(shape)


def int8_uniform(seed, shape):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.int8)
    lib().orc_gen_int8_uniform(seed, n, _p(out, c_i8p))
    return out.reshape(shape)


def uniform_u32(seed, n, bound):
    out = np.empty(n, dtype=np.uint32)
    lib().orc_gen_uniform_u32(seed, n, bound, _p(out, c_u32p))
    return out


# ---------------------------------------------------------------- int8 K/V records
REC_BYTES = 264


def rec_quantize(x):
    """quantize_pair of one 128-value row (fp32): (int8 [128], scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = lib().orc_rec_quantize(_p(x, c_f32p), x.size, _p(q, c_i8p))
    return q, np.float32(s)


def kv_write_rec(k, v, pages, pos0=0, bt=None):
    """k, v fp32 [n][KVH][128] -> records in `pages` (uint8 [n_pages][32][KVH][264]), in place."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n, KVH, D = k.shape
    assert D == 128 and v.shape == k.shape and pages.dtype == np.uint8 and pages.flags.c_contiguous
    btp = None
    if bt is not None:
        bt = np.ascontiguousarray(bt, dtype=np.int32)
        btp = _p(bt, c_i32p)
    lib().orc_kv_write_rec(_p(k, c_f32p), _p(v, c_f32p), n, KVH, pos0, btp, _p(pages, c_u8p))
    return pages


def rec_pages(n_pages, KVH):
    return np.zeros((n_pages, 32, KVH, REC_BYTES), dtype=np.uint8)


def rec_read(pages, pos, h, bt=None):
    """(k int8 [128], k scale, v int8 [128], v scale) of position pos, KV head h."""
    phys = int(bt[pos // 32]) if bt is not None else pos // 32
    r = pages[phys, pos % 32, h]
    return (r[:128].view(np.int8).copy(), r[128:132].view(np.float32)[0], r[132:260].view(np.int8).copy(),
            r[260:264].view(np.float32)[0])


def rec_quantize_q(q):
    """q fp16 bits [rows][D] -> (int8 [rows][D], group scales fp32 [rows][D / 32])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    rows, D = q.shape
    q8 = np.empty((rows, D), dtype=np.int8)
    qs = np.empty((rows, D // 32), dtype=np.float32)
    lib().orc_rec_quantize_q(_p(q, c_u16p), rows, D, _p(q8, c_i8p), _p(qs, c_f32p))
    return q8, qs


def verify_attention_d(q, k, v, a, start=0, window=0, causal=True):
    """fp64 attention of fp64 operands: q [M][QH][D], k, v [T][KVH][D]."""
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    M, QH, D = q.shape
    KVH = k.shape[1]
    assert k.shape[0] >= a + M and k.shape == v.shape
    out = np.empty((M, QH, D), dtype=np.float64)
    lib().orc_verify_attention_d(_p(q, c_f64p), _p(k, c_f64p), _p(v, c_f64p), M, QH, KVH, D, a, start, window,
                                 int(causal), _p(out, c_f64p))
    return out


def verify_attention_rec(q, pages, a, start=0, window=0, causal=True, bt=None):
    """q fp16 bits [M][QH][128]; pages uint8 [n][32][KVH][264]. fp64 [M][QH][128]."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    pages = np.ascontiguousarray(pages, dtype=np.uint8)
    M, QH, D = q.shape
    KVH = pages.shape[2]
    btp = None
    if bt is not None:
        bt = np.ascontiguousarray(bt, dtype=np.int32)
        btp = _p(bt, c_i32p)
    out = np.empty((M, QH, D), dtype=np.float64)
    lib().orc_verify_attention_rec(_p(q, c_u16p), _p(pages, c_u8p), btp, M, QH, KVH, a, start, window, int(causal),
                                   _p(out, c_f64p))
    return out


# ---------------------------------------------------------------- attention
def verify_attention(q, k, v, a, start=0, window=0, causal=True):
    """q [M][QH][D] u16 (fp16 bits); k, v [T][KVH][D] u16. Returns fp64 [M][QH][D]."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    M, QH, D = q.shape
    KVH = k.shape[1]
    assert k.shape[0] >= a + M and k.shape == v.shape
    out = np.empty((M, QH, D), dtype=np.float64)
    lib().orc_verify_attention(_p(q, c_u16p), _p(k, c_u16p), _p(v, c_u16p), M, QH, KVH, D, a, start, window,
                               int(causal), _p(out, c_f64p))
    return out


def attn_partial(q, k, v, a, k0, k1, start=0, window=0, causal=True):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    M, QH, D = q.shape
    KVH = k.shape[1]
    m = np.empty(M * QH)
    l = np.empty(M * QH)
    acc = np.empty((M * QH, D))
    lib().orc_attn_partial(_p(q, c_u16p), _p(np.ascontiguousarray(k), c_u16p), _p(np.ascontiguousarray(v), c_u16p),
                           M, QH, KVH, D, a, start, window, int(causal), k0, k1, _p(m, c_f64p), _p(l, c_f64p),
                           _p(acc, c_f64p))
    return m, l, acc


def attn_merge(ms, ls, accs):
    S = len(ms)
    rows, D = accs[0].shape
    m = np.ascontiguousarray(np.stack(ms))
    l = np.ascontiguousarray(np.stack(ls))
    acc = np.ascontiguousarray(np.stack(accs))
    out = np.empty((rows, D))
    lib().orc_attn_merge(S, rows, D, _p(m, c_f64p), _p(l, c_f64p), _p(acc, c_f64p), _p(out, c_f64p))
    return out


def verify_attention_mt(q, k, v, a, start=0, window=0, causal=True, threads=8):
    """verify_attention (fp64, the same bits) with its rows spread over threads, for long contexts."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    M, QH, D = q.shape
    KVH = k.shape[1]
    assert k.shape[0] >= a + M and k.shape == v.shape
    out = np.empty((M, QH, D), dtype=np.float64)
    lib().orc_verify_attention_mt(_p(q, c_u16p), _p(np.ascontiguousarray(k, dtype=np.uint16), c_u16p),
                                  _p(np.ascontiguousarray(v, dtype=np.uint16), c_u16p), M, QH, KVH, D, a, start, window,
                                  int(causal), _p(out, c_f64p), threads)
    return out


def verify_attention_f32_mt(q, k, v, a, start=0, window=0, causal=True, threads=1):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    M, QH, D = q.shape
    KVH = k.shape[1]
    out = np.empty((M, QH, D), dtype=np.float32)
    lib().orc_verify_attention_f32_mt(_p(q, c_u16p), _p(np.ascontiguousarray(k), c_u16p),
                                      _p(np.ascontiguousarray(v), c_u16p), M, QH, KVH, D, a, start, window,
                                      int(causal), _p(out, c_f32p), threads)
    return out


# ---------------------------------------------------------------- argmax / accept
def argmax_key(v, idx):
    return lib().orc_argmax_key(v, idx)


def key_index(key):
    return lib().orc_key_index(key)


def verify_argmax(logits, seen_bits, tokens, rep=1.0, inv_rep=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    M, V = logits.shape
    if inv_rep is None:
        inv_rep = float(np.float32(1.0) / np.float32(rep))
    tokens = np.ascontiguousarray(np.resize(np.asarray(tokens, dtype=np.int32), max(M, 1)))
    seen_bits = np.ascontiguousarray(seen_bits, dtype=np.uint32)
    keys = np.empty(M, dtype=np.uint64)
    lib().orc_verify_argmax(_p(logits, c_f32p), M, V, _p(seen_bits, c_u32p), _p(tokens, c_i32p), rep, inv_rep,
                            _p(keys, c_u64p))
    return keys


def keys_to_tokens(keys):
    return (np.uint64(0xFFFFFFFF) - (np.asarray(keys, dtype=np.uint64) & np.uint64(0xFFFFFFFF))).astype(np.int32)


def penalize_rep(lg, seen, rep):
    lg = np.ascontiguousarray(lg, dtype=np.float32).copy()
    seen = np.ascontiguousarray(seen, dtype=np.int32)
    lib().orc_penalize_rep(_p(lg, c_f32p), lg.size, _p(seen, c_i32p), seen.size, rep)
    return lg


def argmax_first(lg):
    lg = np.ascontiguousarray(lg, dtype=np.float32)
    return lib().orc_argmax_first(_p(lg, c_f32p), lg.size)


def new_state(**kw):
    st = OrcState()
    for k, v in kw.items():
        if k == "tokens":
            for i, t in enumerate(v):
                st.tokens[i] = int(t)
        else:
            setattr(st, k, int(v))
    return st


def accept_commit(st, best_tok, m, out_tokens, seen_bits, skip_now=0):
    best_tok = np.ascontiguousarray(best_tok, dtype=np.int32)
    return lib().orc_accept_commit(ctypes.byref(st), _p(best_tok, c_i32p), m, skip_now, _p(out_tokens, c_i32p),
                                   _p(seen_bits, c_u32p))


def kv_commit(cache, fresh, a, acc):
    row = int(np.prod(cache.shape[1:]))
    lib().orc_kv_commit(_p(cache, c_u16p), _p(np.ascontiguousarray(fresh), c_u16p), a, acc, row)


# ---------------------------------------------------------------- weights / GEMM
def quantize_rows_int8(w_f16, rows, k):
    w = np.ascontiguousarray(w_f16, dtype=np.uint16)
    q = np.empty(rows * k, dtype=np.int8)
    s = np.empty(rows, dtype=np.float32)
    lib().orc_quantize_rows_int8(_p(w, c_u16p), rows, k, _p(q, c_i8p), _p(s, c_f32p))
    return q.reshape(rows, k), s


def pack_g128(w_f16, rows, k):
    w = np.ascontiguousarray(w_f16, dtype=np.uint16)
    sr = lib().orc_pack_srow(k)
    b = np.empty(rows * k, dtype=np.uint8)
    s = np.empty(rows * sr, dtype=np.uint16)
    lib().orc_pack_g128(_p(w, c_u16p), rows, k, _p(b, c_u8p), _p(s, c_u16p))
    return b.reshape(rows, k), s.reshape(rows, sr)


def transpose_lanes(src):
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty_like(src)
    lib().orc_transpose_lanes(_p(src, c_u8p), _p(dst, c_u8p), src.size)
    return dst


def gemm_i8(x_f16, w, scale_f16, biased=False):
    x = np.ascontiguousarray(x_f16, dtype=np.uint16)
    w = np.ascontiguousarray(w).view(np.uint8)
    s = np.ascontiguousarray(scale_f16, dtype=np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N))
    lib().orc_gemm_i8(_p(x, c_u16p), _p(w, c_u8p), int(biased), _p(s, c_u16p), M, N, K, _p(y, c_f64p))
    return y


def gemm_g128(x_f16, w_biased, gs_f16):
    """x fp16 bits [M][K]; w biased uint8 [N][K]; gs fp16 bits [K/128][N] -> fp64 [M][N]."""
    x = np.ascontiguousarray(x_f16, dtype=np.uint16)
    w = np.ascontiguousarray(w_biased, dtype=np.uint8)
    gs = np.ascontiguousarray(gs_f16, dtype=np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm_g128(_p(x, c_u16p), _p(w, c_u8p), _p(gs, c_u16p), M, N, K, _p(y, c_f64p))
    return y


def quantize_x16(x):
    """LFM3_X8's per-16-value int8 quantization of fp32 x [..., K] -> (int8 codes, fp32 scales [..., K / 16])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1] + (x.shape[-1] // 16,), dtype=np.float32)
    lib().orc_quantize_x16(_p(x, c_f32p), x.size, _p(q, c_i8p), _p(s, c_f32p))
    return q, s


def gemm_x8(q, s, w_biased, gs_f16):
    """int8 codes [M][K] + piece scales [M][K / 16] times biased int8 weights [N][K] with group scales [K/128][N]."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    w = np.ascontiguousarray(w_biased, dtype=np.uint8)
    gs = np.ascontiguousarray(gs_f16, dtype=np.uint16)
    M, K = q.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm_x8(_p(q, c_i8p), _p(s, c_f32p), _p(w, c_u8p), _p(gs, c_u16p), M, N, K, _p(y, c_f64p))
    return y


def gemm_f16(x_f16, w_f16):
    x = np.ascontiguousarray(x_f16, dtype=np.uint16)
    w = np.ascontiguousarray(w_f16, dtype=np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N))
    lib().orc_gemm_f16(_p(x, c_u16p), _p(w, c_u16p), M, N, K, _p(y, c_f64p))
    return y


def row_argmax(y):
    y = np.ascontiguousarray(y, dtype=np.float32)
    M, N = y.shape
    idx = np.empty(M, dtype=np.int32)
    lib().orc_row_argmax(_p(y, c_f32p), M, N, _p(idx, c_i32p))
    return idx


def rms_norm(x, w_f16, eps=1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_f16, dtype=np.uint16)
    y = np.empty_like(x)
    lib().orc_rms_norm(_p(x, c_f32p), _p(w, c_u16p), x.size, eps, _p(y, c_f32p))
    return y


def rope(x, rot, base, pos):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_rope(_p(x, c_f32p), x.size, rot, base, pos)
    return x


def conv_step(B, C, X, w, hist):
    w = np.ascontiguousarray(w, dtype=np.float32)
    return lib().orc_conv_step(B, C, X, _p(w, c_f32p), w.size, _p(hist, c_f32p))


def silu(x):
    return lib().orc_silu(x)
