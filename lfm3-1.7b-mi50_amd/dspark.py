"""Host-side binding of libdspark_amd.so (the C ABI in include/dspark.h).

ctypes over the C ABI; torch is used only for device memory and the current HIP stream. There is no fallback:
if the library is missing the import fails, and every call raises on a nonzero status.

Mirrors the reference's host path for the DSpark step (internal/model/dspark.go: State words 52-77, draftLaunch
537-621) at the level the C ABI exposes: per-round attention, argmax, acceptance and commit.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdspark_amd.so")

MT_MAX = 64
PAGE = 32

STATE_FIELDS = ["a", "anchor", "count", "rounds_left", "limit", "budget", "eos", "M", "ctx_new", "ctx_pos", "ctx_lo",
                "run", "force_m", "rounds_done", "accepted", "verified", "miss", "skip", "skip_after", "skip_rounds",
                "stop_at", "ckpt_slot"]

ERRORS = {1001: "DSPARK_EINVAL", 1002: "DSPARK_ENOSPACE", 1003: "DSPARK_EUNSUPPORTED"}


class DsparkError(RuntimeError):
    pass


class State(ctypes.Structure):
    """struct dspark_state (include/dspark.h) = struct State of dspark.hip:134-158 with tokens[64]."""
    _fields_ = [(n, ctypes.c_int32) for n in STATE_FIELDS] + [("tokens", ctypes.c_int32 * MT_MAX)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("k_pages", ctypes.c_void_p), ("v_pages", ctypes.c_void_p),
                ("block_table", ctypes.c_void_p), ("kv_pages", ctypes.c_int64), ("out", ctypes.c_void_p), ("out_f32", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("M", ctypes.c_int32), ("QH", ctypes.c_int32), ("KVH", ctypes.c_int32), ("D", ctypes.c_int32),
                ("a", ctypes.c_int32), ("start", ctypes.c_int32), ("window", ctypes.c_int32),
                ("causal", ctypes.c_int32), ("splits", ctypes.c_int32)]


_lib = None

_SIGS = {
    "dspark_abi_version": (ctypes.c_int, []),
    "dspark_page_tokens": (ctypes.c_int, []),
    "dspark_max_tokens": (ctypes.c_int, []),
    "dspark_state_bytes": (ctypes.c_int, []),
    "dspark_verify_attention_workspace": (ctypes.c_size_t, [ctypes.POINTER(AttnArgs)]),
    "dspark_verify_attention": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_verify_attention_splits": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_verify_attention_combine": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_verify_attention_noalloc": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_kv_write": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_kv_write_rec": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_void_p]),
    "dspark_verify_attention_rec_workspace": (ctypes.c_size_t, [ctypes.POINTER(AttnArgs)]),
    "dspark_verify_attention_rec": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_verify_attention_rec_splits": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_verify_attention_rec_combine": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "dspark_rope_table": (ctypes.c_int, [ctypes.c_float, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_void_p]),
    "dspark_verify_argmax_workspace": (ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32]),
    "dspark_verify_argmax": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "dspark_accept_commit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]),
    "dspark_gemm_i8_workspace": (ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    "dspark_gemm_i8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "dspark_gemm_i8_g128": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p]),
    "dspark_gemm_i8_g128_x8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "dspark_g128_scales": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_head_argmax_workspace": (ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32]),
    "dspark_head_argmax_f16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                              ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p]),
}


ABI_VERSION = 5  # dspark_abi_version() of the library these signatures describe


def lib():
    """Load libdspark_amd.so; raises if it has not been built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DsparkError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C {HERE})")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.dspark_abi_version() != ABI_VERSION:
            raise DsparkError(f"{LIB_PATH} has ABI {L.dspark_abi_version()}, this module binds {ABI_VERSION}: "
                              "rebuild it")
        _lib = L
    return _lib


def check(rc, what):
    if rc != 0:
        raise DsparkError(f"{what} failed: {ERRORS.get(rc, 'hipError %d' % rc)}")


# ---------------------------------------------------------------- torch plumbing
def _torch():
    import torch
    return torch


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class Workspace:
    """A growable device byte buffer reused across calls (caller-owned memory, as the reference's engine owns
    every buffer, internal/model/dspark.go:202-223)."""

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None

    def get(self, nbytes):
        torch = _torch()
        nbytes = max(int(nbytes), 256)
        if self.buf is None or self.buf.numel() < nbytes:
            # zero-filled: the split-K GEMM keeps its arrival counters here (left at zero by every call)
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf


# ---------------------------------------------------------------- KV pages
def kv_pages_alloc(n_pages, KVH, D, device="cuda"):
    torch = _torch()
    k = torch.zeros((n_pages, KVH, PAGE, D), dtype=torch.float16, device=device)
    v = torch.zeros((n_pages, KVH, D, PAGE), dtype=torch.float16, device=device)
    return k, v


def kv_write(k, v, k_pages, v_pages, pos0, block_table=None, stream=None):
    """k, v: fp16 [n][KVH][D] (or [n][row] with row >= KVH*D) device tensors."""
    n = k.shape[0]
    KVH, D = k_pages.shape[1], k_pages.shape[3]
    row = k.stride(0)
    assert v.stride(0) == row and k.dtype == v.dtype == _torch().float16
    rc = lib().dspark_kv_write(ptr(k), ptr(v), row, ptr(k_pages), ptr(v_pages), ptr(block_table), k_pages.shape[0], KVH,
                               D, pos0, n, stream_handle(stream))
    check(rc, "dspark_kv_write")


def k_page_index(D):
    """For a (page, head) K block of 32*D halves: flat index of K[key][d], as a [32][D] int64 array (the operand
    order documented in include/dspark.h)."""
    import numpy as np
    key = np.arange(PAGE)[:, None]
    d = np.arange(D)[None, :]
    b = (key >> 2) & 1
    nrow = 4 * (key >> 3) + (key & 3)
    s, g, j = d // 32, (d % 32) // 8, d % 8
    return (((b * (D // 32) + s) * 64 + nrow + 16 * g) * 8 + j).astype(np.int64)


def kv_from_pages(k_pages, v_pages, positions, block_table=None):
    """Read K/V rows of the given positions back from the pages (host copy; for checks and debugging)."""
    import numpy as np
    kp = k_pages.detach().cpu().numpy()
    vp = v_pages.detach().cpu().numpy()
    n_pages, KVH = kp.shape[0], kp.shape[1]
    D = kp.size // (n_pages * KVH * PAGE)
    kflat = kp.reshape(n_pages, KVH, PAGE * D)
    vflat = vp.reshape(n_pages, KVH, D, PAGE)
    idx = k_page_index(D)
    bt = None if block_table is None else block_table.detach().cpu().numpy()
    ks, vs = [], []
    for pos in positions:
        lp, sl = divmod(int(pos), PAGE)
        pg = lp if bt is None else int(bt[lp])
        ks.append(kflat[pg][:, idx[sl]])
        vs.append(vflat[pg][:, :, sl])
    return np.stack(ks), np.stack(vs)


def kv_to_pages(k, v, n_pages=None, block_table=None):
    """Logical fp16 [T][KVH][D] K and V -> freshly allocated page pools (identity table unless given)."""
    T, KVH, D = k.shape
    if n_pages is None:
        n_pages = (T + PAGE - 1) // PAGE
    kp, vp = kv_pages_alloc(n_pages, KVH, D, device=k.device)
    kv_write(k.contiguous(), v.contiguous(), kp, vp, 0, block_table)
    return kp, vp


# ---------------------------------------------------------------- verify attention
def attn_args(q, k_pages, v_pages, a, start=0, window=0, causal=True, out=None, out_f32=None, gate=None,
              block_table=None, splits=0):
    M, QH, D = q.shape
    KVH = k_pages.shape[1]
    args = AttnArgs()
    args.q, args.k_pages, args.v_pages = q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr()
    args.block_table = block_table.data_ptr() if block_table is not None else None
    args.kv_pages = k_pages.shape[0]
    args.out = out.data_ptr() if out is not None else None
    args.out_f32 = out_f32.data_ptr() if out_f32 is not None else None
    args.gate = gate.data_ptr() if gate is not None else None
    args.M, args.QH, args.KVH, args.D = M, QH, KVH, D
    args.a, args.start, args.window, args.causal, args.splits = a, start, window, int(causal), splits
    return args


def verify_attention(q, k_pages, v_pages, a, start=0, window=0, causal=True, out=None, out_f32=None, gate=None,
                     block_table=None, splits=0, workspace=None, stream=None):
    """q fp16 [M][QH][D]; pages hold positions 0..a+M-1. Returns (out fp16, out_f32) tensors as given/created."""
    torch = _torch()
    M, QH, D = q.shape
    if out is None and out_f32 is None:
        out = torch.empty((M, QH, D), dtype=torch.float16, device=q.device)
    args = attn_args(q, k_pages, v_pages, a, start, window, causal, out, out_f32, gate, block_table, splits)
    need = lib().dspark_verify_attention_workspace(ctypes.byref(args))
    if need == 0:
        raise DsparkError("dspark_verify_attention_workspace rejected the arguments")
    ws = (workspace or Workspace(q.device)).get(need)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    check(lib().dspark_verify_attention(ctypes.byref(args), stream_handle(stream)), "dspark_verify_attention")
    return out, out_f32


# ---------------------------------------------------------------- int8 K/V records
REC_BYTES = 264


def rec_pages_alloc(n_pages, KVH, device="cuda"):
    """A record pool: [n_pages][32 slots][KVH][264 bytes] (internal/model/engine.go:30-32)."""
    return _torch().zeros((n_pages, PAGE, KVH, REC_BYTES), dtype=_torch().uint8, device=device)


def kv_write_rec(k, v, pages, pos0, block_table=None, stream=None):
    """k, v: fp32 [n][KVH][128] (or [n][row], row >= KVH*128) device tensors -> quantize_pair records."""
    torch = _torch()
    n = k.shape[0]
    KVH = pages.shape[2]
    row = k.stride(0)
    assert v.stride(0) == row and k.dtype == v.dtype == torch.float32 and pages.dtype == torch.uint8
    rc = lib().dspark_kv_write_rec(ptr(k), ptr(v), row, ptr(pages), ptr(block_table), pages.shape[0], KVH, pos0, n,
                                   stream_handle(stream))
    check(rc, "dspark_kv_write_rec")


def rec_attn_args(q, pages, a, start=0, window=0, causal=True, out=None, out_f32=None, gate=None, block_table=None,
                  splits=0):
    M, QH, D = q.shape
    args = AttnArgs()
    args.q, args.k_pages, args.v_pages = q.data_ptr(), pages.data_ptr(), None
    args.block_table = block_table.data_ptr() if block_table is not None else None
    args.kv_pages = pages.shape[0]
    args.out = out.data_ptr() if out is not None else None
    args.out_f32 = out_f32.data_ptr() if out_f32 is not None else None
    args.gate = gate.data_ptr() if gate is not None else None
    args.M, args.QH, args.KVH, args.D = M, QH, pages.shape[2], D
    args.a, args.start, args.window, args.causal, args.splits = a, start, window, int(causal), splits
    return args


def verify_attention_rec(q, pages, a, start=0, window=0, causal=True, out=None, out_f32=None, gate=None,
                         block_table=None, splits=0, workspace=None, stream=None):
    """q fp16 [M][QH][128]; pages: a record pool holding positions 0..a+M-1."""
    torch = _torch()
    M, QH, D = q.shape
    if out is None and out_f32 is None:
        out = torch.empty((M, QH, D), dtype=torch.float16, device=q.device)
    args = rec_attn_args(q, pages, a, start, window, causal, out, out_f32, gate, block_table, splits)
    need = lib().dspark_verify_attention_rec_workspace(ctypes.byref(args))
    if need == 0:
        raise DsparkError("dspark_verify_attention_rec_workspace rejected the arguments")
    ws = (workspace or Workspace(q.device)).get(need)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    check(lib().dspark_verify_attention_rec(ctypes.byref(args), stream_handle(stream)), "dspark_verify_attention_rec")
    return out, out_f32


# ---------------------------------------------------------------- argmax / accept
def state_tensor(device="cuda", **fields):
    """A device dspark_state initialised from keyword fields (tokens=list)."""
    torch = _torch()
    st = State()
    for k, v in fields.items():
        if k == "tokens":
            for i, t in enumerate(v):
                st.tokens[i] = int(t)
        else:
            setattr(st, k, int(v))
    raw = bytes(st)
    host = torch.frombuffer(bytearray(raw), dtype=torch.int32).clone()
    return host.to(device)


def state_from_tensor(t):
    st = State()
    ctypes.memmove(ctypes.byref(st), bytes(t.cpu().numpy().tobytes()), ctypes.sizeof(State))
    return st


def verify_argmax(logits, seen, st, rep=1.0, inv_rep=None, best=None, workspace=None, stream=None):
    torch = _torch()
    M, V = logits.shape
    f16 = logits.dtype == torch.float16
    if inv_rep is None:
        inv_rep = float(torch.tensor(1.0, dtype=torch.float32) / torch.tensor(rep, dtype=torch.float32))
    if best is None:
        best = torch.empty(M, dtype=torch.int64, device=logits.device)
    need = lib().dspark_verify_argmax_workspace(M, V)
    ws = (workspace or Workspace(logits.device)).get(need)
    rc = lib().dspark_verify_argmax(ptr(logits), int(f16), M, V, ptr(seen), ptr(st), rep, inv_rep, ptr(best), ptr(ws),
                                    ws.numel(), stream_handle(stream))
    check(rc, "dspark_verify_argmax")
    return best


def accept_commit(st, best, M, out_tokens, seen, skip_now=0, stream=None):
    rc = lib().dspark_accept_commit(ptr(st), ptr(best), M, skip_now, ptr(out_tokens), out_tokens.numel(), ptr(seen),
                                    stream_handle(stream))
    check(rc, "dspark_accept_commit")


def keys_to_tokens(keys):
    """u64 keys held in an int64 tensor -> token ids."""
    torch = _torch()
    low = keys & 0xFFFFFFFF
    return (0xFFFFFFFF - low).to(torch.int64)


# ---------------------------------------------------------------- GEMMs
def gemm_i8(x, w_biased, scale, epilogue=0, y_f32=None, y_f16=None, workspace=None, stream=None):
    torch = _torch()
    M, K = x.shape
    N = w_biased.shape[0]
    if epilogue == 0 and y_f32 is None and y_f16 is None:
        y_f32 = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if epilogue != 0 and y_f16 is None:
        y_f16 = torch.empty((M, N // 2 if epilogue == 1 else N), dtype=torch.float16, device=x.device)
    need = lib().dspark_gemm_i8_workspace(M, N, K)
    ws = (workspace or Workspace(x.device)).get(need)
    rc = lib().dspark_gemm_i8(ptr(x), M, K, ptr(w_biased), ptr(scale), N, epilogue, ptr(y_f32), ptr(y_f16), ptr(ws),
                              ws.numel(), stream_handle(stream))
    check(rc, "dspark_gemm_i8")
    return y_f32 if epilogue == 0 and y_f32 is not None else y_f16


def gemm_i8_g128(x, w_biased, gscale, epilogue=0, y_f32=None, y_f16=None, stream=None):
    """x fp16 [M][K] (M <= 16); w uint8 [N][K] biased; gscale fp16 [K/128][N] (per-128-column group scales)."""
    torch = _torch()
    M, K = x.shape
    N = w_biased.shape[0]
    if epilogue == 0 and y_f32 is None and y_f16 is None:
        y_f32 = torch.empty((M, N), dtype=torch.float32, device=x.device)
    rc = lib().dspark_gemm_i8_g128(ptr(x), M, K, ptr(w_biased), ptr(gscale), N, epilogue, ptr(y_f32), ptr(y_f16),
                                   stream_handle(stream))
    check(rc, "dspark_gemm_i8_g128")
    return y_f32, y_f16


def gemm_i8_g128_x8(x, w_biased, gscale, xscale=None, epilogue=0, y_f32=None, y_f16=None, stream=None):
    """The LFM3_X8 form of gemm_i8_g128: x fp16 [M][K] quantized per 16 columns on load (xscale None), or x the int8
    codes as integer-valued fp16 with xscale fp32 [M][K/16]."""
    torch = _torch()
    M, K = x.shape
    N = w_biased.shape[0]
    if epilogue == 0 and y_f32 is None and y_f16 is None:
        y_f32 = torch.empty((M, N), dtype=torch.float32, device=x.device)
    rc = lib().dspark_gemm_i8_g128_x8(ptr(x), ptr(xscale), M, K, ptr(w_biased), ptr(gscale), N, epilogue, ptr(y_f32),
                                      ptr(y_f16), stream_handle(stream))
    check(rc, "dspark_gemm_i8_g128_x8")
    return y_f32, y_f16


def g128_scales(packed, N, K):
    """The packer's scale rows (uint16 [N][SRow]) -> group-major [K/128][N] (host numpy)."""
    import numpy as np
    packed = np.ascontiguousarray(packed, dtype=np.uint16)
    out = np.empty((K // 128, N), dtype=np.uint16)
    check(lib().dspark_g128_scales(packed.ctypes.data_as(ctypes.c_void_p), N, K, out.ctypes.data_as(ctypes.c_void_p)),
          "dspark_g128_scales")
    return out


def head_argmax(x, w, y_f32=None, best=None, workspace=None, stream=None):
    torch = _torch()
    M, K = x.shape
    N = w.shape[0]
    if best is None:
        best = torch.empty(M, dtype=torch.int64, device=x.device)
    need = lib().dspark_head_argmax_workspace(M, N)
    ws = (workspace or Workspace(x.device)).get(need)
    rc = lib().dspark_head_argmax_f16(ptr(x), M, K, ptr(w), N, ptr(y_f32), ptr(best), ptr(ws), ws.numel(),
                                      stream_handle(stream))
    check(rc, "dspark_head_argmax_f16")
    return best


# ---------------------------------------------------------------- the full step (engine)
MAX_LAYERS = 64
MAX_TAPS = 8


class ModelDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("ffn", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("n_layers", ctypes.c_int32), ("layer_kind", ctypes.c_int32 * MAX_LAYERS),
                ("q_heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("conv_kernel", ctypes.c_int32), ("window", ctypes.c_int32), ("rope_base", ctypes.c_float),
                ("rope_pairs", ctypes.c_int32), ("draft_layers", ctypes.c_int32), ("draft_ffn", ctypes.c_int32),
                ("block", ctypes.c_int32), ("max_drafts", ctypes.c_int32), ("crop_rows", ctypes.c_int32),
                ("markov_rank", ctypes.c_int32), ("n_taps", ctypes.c_int32), ("tap_layer", ctypes.c_int32 * MAX_TAPS),
                ("draft_window", ctypes.c_int32), ("ring_positions", ctypes.c_int32), ("mask_token", ctypes.c_int32),
                ("conf_bias", ctypes.c_float), ("conf_thr", ctypes.c_float), ("eps", ctypes.c_float),
                ("rope_base_swa", ctypes.c_float), ("rope_pairs_swa", ctypes.c_int32), ("conv_slots", ctypes.c_int32),
                ("kv_format", ctypes.c_int32), ("weight_format", ctypes.c_int32), ("x_format", ctypes.c_int32)]


class LaunchArgs(ctypes.Structure):
    _fields_ = [("a", ctypes.c_int32), ("anchor", ctypes.c_int32), ("budget", ctypes.c_int32), ("eos", ctypes.c_int32),
                ("rep", ctypes.c_float), ("rounds", ctypes.c_int32), ("ctx_new", ctypes.c_int32),
                ("ctx_pos", ctypes.c_int32), ("ctx_lo", ctypes.c_int32), ("force_m", ctypes.c_int32),
                ("tokens", ctypes.c_int32 * MT_MAX), ("max_drafts", ctypes.c_int32), ("miss", ctypes.c_int32),
                ("skip", ctypes.c_int32), ("conv_slot", ctypes.c_int32), ("ckpt_slot", ctypes.c_int32)]


class LaunchResult(ctypes.Structure):
    _fields_ = [("count", ctypes.c_int32), ("rounds", ctypes.c_int32), ("accepted", ctypes.c_int32),
                ("verified", ctypes.c_int32), ("boundary", ctypes.c_int32), ("ckpt_written", ctypes.c_int32),
                ("state", State), ("rounds_enqueued", ctypes.c_int32)]


_SIGS.update({
    "dspark_engine_create": (ctypes.c_int, [ctypes.POINTER(ModelDesc), ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p)]),
    "dspark_engine_destroy": (None, [ctypes.c_void_p]),
    "dspark_engine_init_random": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]),
    "dspark_engine_tensor": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                            ctypes.POINTER(ctypes.c_size_t)]),
    "dspark_engine_tensor_count": (ctypes.c_int, [ctypes.c_void_p]),
    "dspark_engine_tensor_name": (ctypes.c_char_p, [ctypes.c_void_p, ctypes.c_int32]),
    "dspark_engine_debug_layers": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    "dspark_engine_prepare": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "dspark_engine_round": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_engine_launch": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(LaunchArgs), ctypes.c_void_p, ctypes.c_int32,
                                            ctypes.POINTER(LaunchResult), ctypes.c_void_p]),
    "dspark_engine_init_seen": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_float,
                                               ctypes.c_void_p]),
    "dspark_engine_capture_tap": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                                                 ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_engine_project_prompt": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_engine_conv_copy": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_engine_trace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]),
    "dspark_engine_trace_read": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                                ctypes.POINTER(ctypes.c_int32)]),
})

TRACE_PHASES = {0: "begin", 1: "context", 2: "drafter", 3: "crop_head", 4: "markov", 5: "lm_head", 6: "commit"}
TRACE_VERIFY_LAYER = 16


def trace_phase_name(phase):
    return TRACE_PHASES.get(phase, f"verify_L{phase - TRACE_VERIFY_LAYER}")


def rope_table(base, pairs, head_dim, positions):
    """The RoPE table the engine builds (uint16 fp16 bits [positions][head_dim]: cos | sin), host code of the library."""
    import numpy as np
    out = np.empty((positions, head_dim), np.uint16)
    check(lib().dspark_rope_table(base, pairs, head_dim, positions, out.ctypes.data_as(ctypes.c_void_p)),
          "dspark_rope_table")
    return out


def model_desc(**kw):
    d = ModelDesc()
    d.conv_slots = 1
    for k, v in kw.items():
        if k in ("layer_kind", "tap_layer"):
            arr = getattr(d, k)
            for i, x in enumerate(v):
                arr[i] = int(x)
        else:
            setattr(d, k, v)
    return d


def c4_desc(block=16, vocab=65536):
    """16-layer LFM-style target (10 gated short-conv k=3 + 6 GQA 32/8/64), hidden 2048, FFN 8192,
    vocab 65536, int8 weights; 4-layer drafter proposing 16-token blocks."""
    kinds = [0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 1, 0, 1, 0, 1, 0]
    return model_desc(hidden=2048, ffn=8192, vocab=vocab, n_layers=16, layer_kind=kinds, q_heads=32, kv_heads=8,
                      head_dim=64, conv_kernel=3, window=0, rope_base=1e6, rope_pairs=32, draft_layers=4,
                      draft_ffn=8192, block=block, max_drafts=block - 1, crop_rows=16384, markov_rank=256, n_taps=5,
                      tap_layer=[1, 4, 8, 11, 15], draft_window=2048, ring_positions=4096, mask_token=vocab - 1,
                      conf_bias=3.0, conf_thr=-0.4, eps=1e-5)


def ref_desc(block=9, max_drafts=7, vocab=128000, kv_format=1, weight_format=1, x_format=0):
    """The reference model's geometry (internal/model/engine.go:23-40; internal/model/dspark.go:22-41;
    cmd/pack/main.go:193, 329): 24 target layers in the reference order (13 gated short-conv k=7, 6 full and 5
    sliding-window-256 GQA attention layers, 16/4/128), hidden 2048, gated FFN 7680, vocab 128000; 3 attention-only
    drafter layers (FFN 7680) over 9-token blocks, 16384-row cropped head, Markov rank 256, taps {2, 6, 12, 18, 23},
    drafter window 2048, ring 4096. max_drafts follows the reference policy (7, or 3 from position 57344,
    generate.go:136). RoPE per layer kind as the reference builds it (engine.go:333-338): full attention and the
    drafter at base 1e6 with 32 rotating pairs, sliding layers at base 1e4 with 64. K/V in the reference's int8
    records (264 bytes per position and KV head, quantize_pair; engine.go:30-32, ops.hip:212-251) unless
    kv_format=0 (fp16 pages); int8 weights with the reference's per-128-column fp16 scales (weights.Pack,
    quant.go:66-104) unless weight_format=0 (one scale per row). x_format=1: the GEMM inputs as int8 per 16 columns, the
    reference's default build (LFM3_X8, kernels/dspark.hip:24-26); needs weight_format=1."""
    kinds = [0, 0, 1, 0, 2, 0, 1, 0, 2, 0, 1, 0, 2, 0, 1, 0, 2, 0, 1, 0, 2, 0, 1, 0]
    return model_desc(hidden=2048, ffn=7680, vocab=vocab, n_layers=24, layer_kind=kinds, q_heads=16, kv_heads=4,
                      head_dim=128, conv_kernel=7, window=256, rope_base=1e6, rope_pairs=32, rope_base_swa=1e4,
                      rope_pairs_swa=64, draft_layers=3,
                      draft_ffn=7680, block=block, max_drafts=max_drafts, crop_rows=16384, markov_rank=256, n_taps=5,
                      tap_layer=[2, 6, 12, 18, 23], draft_window=2048, ring_positions=4096, mask_token=vocab - 1,
                      conf_bias=3.0, conf_thr=-0.4, eps=1e-5, kv_format=kv_format, weight_format=weight_format,
                      x_format=x_format)


class Engine:
    """One model + one request's device buffers (dspark_engine_* in include/dspark.h)."""

    def __init__(self, desc, max_context):
        self.desc = desc
        self.max_context = max_context
        h = ctypes.c_void_p()
        check(lib().dspark_engine_create(ctypes.byref(desc), max_context, ctypes.byref(h)), "dspark_engine_create")
        self.h = h

    def close(self):
        if self.h:
            lib().dspark_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name):
        p = ctypes.c_void_p()
        n = ctypes.c_size_t()
        check(lib().dspark_engine_tensor(self.h, name.encode(), ctypes.byref(p), ctypes.byref(n)), f"tensor {name}")
        return p.value, n.value

    def names(self):
        n = lib().dspark_engine_tensor_count(self.h)
        return [lib().dspark_engine_tensor_name(self.h, i).decode() for i in range(n)]

    def init_random(self, seed, stream=None):
        check(lib().dspark_engine_init_random(self.h, seed, stream_handle(stream)), "dspark_engine_init_random")

    def prepare(self, stream=None):
        check(lib().dspark_engine_prepare(self.h, stream_handle(stream)), "dspark_engine_prepare")

    def round(self, force_m=0, plan_a=0, stream=None):
        check(lib().dspark_engine_round(self.h, force_m, plan_a, stream_handle(stream)), "dspark_engine_round")

    def launch(self, a, anchor, budget=512, eos=-1, rep=1.0, rounds=32, ctx_new=0, ctx_pos=0, ctx_lo=0, force_m=0,
               tokens=(), max_out=1024, max_drafts=0, miss=0, skip=0, conv_slot=-1, ckpt_slot=-1, stream=None):
        """draftLaunch (dspark_engine_launch): returns (emitted tokens, LaunchResult)."""
        args = LaunchArgs()
        args.a, args.anchor, args.budget, args.eos, args.rep, args.rounds = a, anchor, budget, eos, rep, rounds
        args.ctx_new, args.ctx_pos, args.ctx_lo, args.force_m = ctx_new, ctx_pos, ctx_lo, force_m
        args.max_drafts, args.miss, args.skip, args.conv_slot, args.ckpt_slot = max_drafts, miss, skip, conv_slot, ckpt_slot
        for i, t in enumerate(tokens):
            args.tokens[i] = int(t)
        out = (ctypes.c_int32 * max_out)()
        res = LaunchResult()
        check(lib().dspark_engine_launch(self.h, ctypes.byref(args), out, max_out, ctypes.byref(res),
                                         stream_handle(stream)), "dspark_engine_launch")
        return list(out[:res.count]), res

    def init_seen(self, tokens, rep=1.0, stream=None):
        """InitSeen (dspark_engine_init_seen): the penalty mask = exactly `tokens`."""
        arr = (ctypes.c_int32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        check(lib().dspark_engine_init_seen(self.h, arr, len(tokens), rep, stream_handle(stream)),
              "dspark_engine_init_seen")

    def capture_tap(self, slot, h, context, tap_from, stream=None):
        """captureTap (dspark_engine_capture_tap): h = fp16 device tensor [tokens][>= hidden] of positions
        context .. context + tokens - 1."""
        check(lib().dspark_engine_capture_tap(self.h, slot, ptr(h), h.stride(0), context, h.shape[0], tap_from,
                                              stream_handle(stream)), "dspark_engine_capture_tap")

    def project_prompt(self, first, end, stream=None):
        check(lib().dspark_engine_project_prompt(self.h, first, end, stream_handle(stream)),
              "dspark_engine_project_prompt")

    def debug_layers(self, enable=True):
        """Layer-boundary dumps into the tensor "debug_layers" (dspark_engine_debug_layers)."""
        check(lib().dspark_engine_debug_layers(self.h, int(enable)), "dspark_engine_debug_layers")

    def trace(self, enable=True, stream=None):
        """Phase tracing on (a fresh trace) or off for the rounds enqueued after this call."""
        check(lib().dspark_engine_trace(self.h, int(enable), stream_handle(stream)), "dspark_engine_trace")

    def trace_read(self, cap=65536):
        """The marks since tracing was turned on: list of (round, phase, clock ns)."""
        import numpy as np
        out = np.zeros(2 * cap, np.uint64)
        n = ctypes.c_int32()
        check(lib().dspark_engine_trace_read(self.h, out.ctypes.data_as(ctypes.c_void_p), cap, ctypes.byref(n)),
              "dspark_engine_trace_read")
        k = min(n.value, cap)
        return [(int(out[2 * i]) >> 32, int(out[2 * i]) & 0xFFFFFFFF, int(out[2 * i + 1])) for i in range(k)]

    def conv_copy(self, src, dst, stream=None):
        check(lib().dspark_engine_conv_copy(self.h, src, dst, stream_handle(stream)), "dspark_engine_conv_copy")

    # host <-> device copies of named tensors (plumbing for tests, loaders and benchmarks)
    def upload(self, name, array):
        import numpy as np
        ptr_, nbytes = self.tensor(name)
        a = np.ascontiguousarray(array)
        assert a.nbytes <= nbytes, (name, a.nbytes, nbytes)
        _hip().hipMemcpy(ctypes.c_void_p(ptr_), a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1)

    def download(self, name, dtype, shape=None):
        import numpy as np
        ptr_, nbytes = self.tensor(name)
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        _hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr_), ctypes.c_size_t(out.nbytes), 2)
        if shape is not None:
            out = out[:int(np.prod(shape))].reshape(shape)
        return out

    def state(self):
        import numpy as np
        raw = self.download("state", np.int32)
        st = State()
        ctypes.memmove(ctypes.byref(st), raw.tobytes(), ctypes.sizeof(State))
        return st

    def set_state(self, **fields):
        import numpy as np
        st = State()
        for k, v in fields.items():
            if k == "tokens":
                for i, t in enumerate(v):
                    st.tokens[i] = int(t)
            else:
                setattr(st, k, int(v))
        self.upload("state", np.frombuffer(bytes(st), dtype=np.int32))


_hip_lib = None


def _hip():
    global _hip_lib
    if _hip_lib is None:
        _hip_lib = ctypes.CDLL("libamdhip64.so")
        _hip_lib.hipMemcpy.restype = ctypes.c_int
        _hip_lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _hip_lib
