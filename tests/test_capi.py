"""CPU checks of the C ABI: the library loads, exports exactly what include/dspark.h declares, and the State struct
keeps the reference's 22 scalar words in order (internal/model/dspark_test.go:8-22 pins the same layout)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, load_host, rope_numpy

HEADER = os.path.join(ROOT, "include", "dspark.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(dspark_[a-z0-9_]+)\s*\(", text))
    inline = set(re.findall(r"static inline [^(]*\b(dspark_[a-z0-9_]+)\s*\(", text))
    return sorted(names - inline)


def test_library_exports_every_declared_symbol():
    host = load_host()
    lib = host.lib()
    names = declared_functions()
    assert len(names) >= 14
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the binding declares a signature for each of them
    assert sorted(host._SIGS) == names


def test_size_queries_and_state_layout():
    host = load_host()
    lib = host.lib()
    assert lib.dspark_abi_version() == 5
    assert lib.dspark_page_tokens() == 32
    assert lib.dspark_max_tokens() == 64
    # 22 scalars (dspark.hip:134-157, dspark.go:52-77 sTokens == 22) then tokens[64]
    assert lib.dspark_state_bytes() == (22 + 64) * 4 == ctypes.sizeof(host.State)
    assert [f[0] for f in host.State._fields_][:22] == host.STATE_FIELDS
    assert host.State.tokens.offset == 22 * 4


def test_workspace_queries_reject_bad_shapes():
    host = load_host()
    lib = host.lib()
    args = host.AttnArgs()
    args.M, args.QH, args.KVH, args.D, args.a = 16, 32, 8, 64, 32768
    args.causal = 1
    ws = lib.dspark_verify_attention_workspace(ctypes.byref(args))
    assert ws > 0
    args.D = 96
    assert lib.dspark_verify_attention_workspace(ctypes.byref(args)) == 0
    args.D, args.M = 64, 65
    assert lib.dspark_verify_attention_workspace(ctypes.byref(args)) == 0
    assert lib.dspark_gemm_i8_workspace(16, 65536, 2048) == 0         # enough 16-row strips: no split, no partials
    # K ranges summed inside one workgroup (2 to 4 token blocks: X^T in passes of one or two token blocks)
    for M, N, K in ((16, 2048, 2048), (9, 6144, 2048), (24, 4096, 1024), (1, 64, 128), (40, 6144, 2048),
                    (33, 512, 1024), (64, 16384, 2048), (40, 1024, 4096)):
        assert lib.dspark_gemm_i8_workspace(M, N, K) == 0, (M, N, K)
    for M, N, K in ((33, 2048, 8192), (40, 1024, 8192), (48, 4096, 8192)):
        # split K: a fixed region of 8192 u32 arrival counters (the same offset for every shape), then the
        # [splits][M][N] fp32 partials, 256-byte rounded
        ws = lib.dspark_gemm_i8_workspace(M, N, K)
        part = ws - 8192 * 4
        splits = part // (M * N * 4)
        assert part % 256 == 0 and part - splits * M * N * 4 < 256, (M, N, K, ws)
        assert splits >= 2 and splits & (splits - 1) == 0, (M, N, K, ws)
    assert lib.dspark_gemm_i8_workspace(16, 2050, 8192) == 0          # N % 16
    assert lib.dspark_head_argmax_workspace(16, 16384) == 16 * 1024 * 8


def test_entry_points_refuse_invalid_arguments_without_launching():
    """Argument errors are reported before any device work (no GPU is needed to reach them)."""
    host = load_host()
    lib = host.lib()
    args = host.AttnArgs()
    args.M, args.QH, args.KVH, args.D, args.a = 16, 30, 8, 64, 10   # QH % KVH != 0
    assert lib.dspark_verify_attention(ctypes.byref(args), None) == 1001
    assert lib.dspark_kv_write(None, None, 512, None, None, None, 100, 8, 64, 0, 1, None) == 1001
    assert lib.dspark_gemm_i8(None, 16, 2048, None, None, 8192, 0, None, None, None, 0, None) == 1001
    assert lib.dspark_accept_commit(None, None, 9, 0, None, 64, None, None) == 1001
    assert lib.dspark_verify_argmax(None, 0, 9, 65536, None, None, 1.0, 1.0, None, None, 0, None) == 1001


def test_bounds_are_checked_on_the_host():
    """Refusals that need sizes, not just pointers: K/V rows past the page pools, an output buffer smaller than a
    verify block, an engine whose K/V pool would reach 2 GiB (the attention kernels' 32-bit offsets). Placeholder
    pointers are never dereferenced: every call below is refused before a launch."""
    host = load_host()
    lib = host.lib()
    fake = ctypes.c_void_p(256)
    # 10 pages hold positions 0..319: rows 300..339 overflow without a block table
    assert lib.dspark_kv_write(fake, fake, 512, fake, fake, None, 10, 8, 64, 300, 40, None) == 1001
    assert lib.dspark_kv_write(fake, fake, 512, fake, fake, None, 0, 8, 64, 0, 1, None) == 1001
    # accept/commit: out_cap below the verify block
    assert lib.dspark_accept_commit(fake, fake, 9, 0, fake, 8, fake, None) == 1001
    # engine pools: C4 geometry pages are 8 heads x 32 keys x 64 dims x 2 B = 32 KiB, so max_context ~2M reaches 2 GiB
    h = ctypes.c_void_p()
    desc = host.c4_desc()
    assert lib.dspark_engine_create(ctypes.byref(desc), 1 << 22, ctypes.byref(h)) == 1001
    assert lib.dspark_engine_create(ctypes.byref(desc), (1 << 16) * 32, ctypes.byref(h)) == 1001
    bad = host.ref_desc()
    bad.rope_pairs_swa = 65  # > head_dim / 2
    assert lib.dspark_engine_create(ctypes.byref(bad), 4096, ctypes.byref(h)) == 1001
    bad = host.ref_desc()
    bad.conv_slots = -1
    assert lib.dspark_engine_create(ctypes.byref(bad), 4096, ctypes.byref(h)) == 1001
    assert not h.value


def test_record_entry_points_check_their_arguments():
    """The int8-record path: workspace sizes of the reference geometry (one key split per workgroup over all four KV
    heads, the fp16 path's partial layout), and refusals before any launch (D, KVH, rows, a V pool, pools of 2 GiB,
    rows past the pool)."""
    host = load_host()
    lib = host.lib()
    fake = ctypes.c_void_p(256)
    args = host.AttnArgs()
    args.M, args.QH, args.KVH, args.D, args.a, args.causal = 9, 16, 4, 128, 131063, 1   # 4096 pages
    ws = lib.dspark_verify_attention_rec_workspace(ctypes.byref(args))
    # 36 rows -> 3 row blocks of 16 per KV head, 4 heads, 256 splits of 16 pages: acc [4][S][48][128] f32 + (m, l)
    S = 256
    acc = 4 * S * 48 * 128 * 4
    assert ws == acc + ((4 * S * 48 * 8 + 255) // 256) * 256, ws
    args.M = 17    # 68 rows per KV head: more than one wave per row block can take
    assert lib.dspark_verify_attention_rec_workspace(ctypes.byref(args)) == 0
    args.M, args.D = 9, 64
    assert lib.dspark_verify_attention_rec_workspace(ctypes.byref(args)) == 0
    args.D, args.KVH, args.QH = 128, 8, 32
    assert lib.dspark_verify_attention_rec_workspace(ctypes.byref(args)) == 0
    args.KVH, args.QH = 4, 16
    args.q, args.k_pages, args.v_pages, args.out = 256, 256, 256, 256   # a V pool: records carry V themselves
    args.kv_pages = 4200
    assert lib.dspark_verify_attention_rec(ctypes.byref(args), None) == 1001
    args.v_pages = None
    args.kv_pages = (1 << 31) // (32 * 4 * 264) + 1                      # pool of 2 GiB or more
    assert lib.dspark_verify_attention_rec(ctypes.byref(args), None) == 1001
    args.kv_pages = 100                                                   # positions past the pool, no block table
    assert lib.dspark_verify_attention_rec(ctypes.byref(args), None) == 1001
    args.kv_pages = 4200
    assert lib.dspark_verify_attention_rec(ctypes.byref(args), None) == 1002   # no workspace
    # writer: 10 pages hold positions 0..319
    assert lib.dspark_kv_write_rec(fake, fake, 512, fake, None, 10, 4, 300, 40, None) == 1001
    assert lib.dspark_kv_write_rec(fake, fake, 256, fake, None, 10, 4, 0, 1, None) == 1001   # row < KVH * 128
    assert lib.dspark_kv_write_rec(None, fake, 512, fake, None, 10, 4, 0, 1, None) == 1001


@pytest.mark.parametrize("base,pairs,D", [(1e6, 32, 128), (1e4, 64, 128), (1e6, 32, 64), (1e4, 16, 64)])
def test_rope_table_matches_the_reference_formula(base, pairs, D):
    """The library's table (what the engine uploads) against a numpy restatement, bit for bit over 70000 positions, plus
    the closed forms: position 0 is cos 1 / sin 0, pairs past `pairs` never rotate, and the first pair's angle is the
    position itself (inv[0] = 1)."""
    import numpy as np
    host = load_host()
    n = 70000
    got = host.rope_table(base, pairs, D, n)
    want = rope_numpy(base, pairs, D, n)
    assert np.array_equal(got, want)
    f = got.view(np.float16).astype(np.float64)
    assert np.all(f[0, :D // 2] == 1.0) and np.all(f[0, D // 2:] == 0.0)
    assert np.all(f[:, pairs:D // 2] == 1.0) and np.all(f[:, D // 2 + pairs:] == 0.0)
    pos = np.arange(n)
    assert np.max(np.abs(f[:, 0] - np.cos(pos))) <= 2 ** -11 and np.max(np.abs(f[:, D // 2] - np.sin(pos))) <= 2 ** -11
    # a wrong base or pair count is caught
    assert not np.array_equal(host.rope_table(base * 10, pairs, D, 64), want[:64])
