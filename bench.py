#!/usr/bin/env python3
"""Benchmark of the DSpark step's hot path on one MI355X.

Default workload ("C2"): verify attention alone, 6 GQA layers (32 query / 8 KV heads,
head_dim 64), fp16 K/V cache at context 32768, 16 verify tokens per step, causal inside the drafted block. A step
runs each layer's verify attention (key-split pass, then the split merge) over pages that already hold the 16 tokens'
own K/V.
Inputs are synthetic N(0,1) fp16 resident in HBM; two full KV sets (2 x 6 x 64 MiB) alternate between steps so the
256 MB Infinity Cache cannot serve a step from the previous one.

Prints one JSON line (the driver's contract) with a `roofline` object for the dominant kernel (the key-split pass,
`verify_attn_lds_kernel`) timed with HIP events on the library's stream, and a `cpu_baseline` object (the C oracle's
fp32 restatement timed on a bounded sample of the same workload, on all CPUs of the job's share and on one). The same
line carries the metric's other half, `headline_tok_s` (greedy decode tok/s of full DSpark rounds at 1k / 32k / 128k
context, beside the reference's published MI50 numbers, on the C4 geometry) and `headline_ref_tok_s` (the same on the
reference model's geometry, draft policy and storage formats), `c5_attention` (verify attention at 131072 keys for 33 and
16 verify tokens) and `ref_int8_record_attention` (verify attention over the reference's int8 K/V records, its
geometry and 9-token block, at 32768 and 131072 keys). `--c2-only` skips those; `--workload` selects the other configs
(c3, c4, c5, tiers, ref with `--ref-formats`), or verify attention alone at any context and block (`attn` over fp16
pages, `rec` over int8 records; `--ctx`, `--tokens`).
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "lfm3-1.7b-mi50_amd")
METRIC = "greedy decode tok/s at 1k/32k/128k ctx; verify-attn HBM GB/s vs roofline"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "verify_attn_c2_traffic.txt")
ROOFLINE_KERNEL = "verify_attn_lds_kernel"


def load_host():
    spec = importlib.util.spec_from_file_location("dspark_amd_host", os.path.join(PKG, "dspark.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def read_traffic():
    """HBM bytes per launch of the key-split pass from the committed rocprofv3 --pmc summary, if present and taken
    from the kernel this build launches (the summary's `kernel:` line)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    vals = {}
    for line in open(TRAFFIC_FILE):
        if ":" in line:
            k, _, v = line.partition(":")
            vals[k.strip()] = v.strip()
    if not vals.get("kernel", "").startswith(ROOFLINE_KERNEL):
        return None
    try:
        return int(float(vals["hbm_bytes_per_launch"]))
    except (KeyError, ValueError):
        return None


def cpu_info():
    """Host CPU: model name, the host's logical CPU count and the CPUs this process may run on (the CPU share a GPU
    job gets on the box; worker pools stay within it)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    return model, os.cpu_count() or 1, max(1, share)


def cpu_baseline_c2(ctx, M, QH, KVH, D, seconds):
    """The CPU oracle (test infrastructure, used here only as the timed baseline) on layers of the same workload: all
    threads of this process's CPU share, then one thread."""
    import numpy as np
    from oracle import oracle as orc
    rng = np.random.default_rng(20261202)
    q = rng.standard_normal((M, QH, D)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((ctx + M, KVH, D)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((ctx + M, KVH, D)).astype(np.float16).view(np.uint16)
    model, nproc, share = cpu_info()
    layer_bytes = ctx * KVH * D * 2 * 2

    def rate(threads, budget):
        layers, t0 = 0, time.perf_counter()
        while True:
            orc.verify_attention_f32_mt(q, k, v, ctx, threads=threads)
            layers += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return layer_bytes * layers / el / 1e9, layers, el

    all_gbs, all_n, all_s = rate(share, seconds)
    one_gbs, one_n, one_s = rate(1, seconds / 2)
    return {"value": round(all_gbs, 3), "unit": "GB/s", "cores": share, "kind": "port",
            "sample": f"{all_n} layers of the C2 workload (ctx {ctx}, {M} verify tokens, {QH}/{KVH} heads, d{D}) through "
                      f"the C oracle's fp32 verify attention on {share} threads in {all_s:.1f} s; single thread: "
                      f"{one_n} layers in {one_s:.1f} s",
            "single_thread": round(one_gbs, 3), "host_nproc": nproc, "cpu_share": share, "cpu_model": model,
            "note": "Go (the reference's host language) is absent on the box, so the reference's CPU path cannot run; "
                    "the all-core figure uses the CPUs this GPU job is given (the box's share per GPU), not every "
                    "core of the host"}


def bench_attention(args, host, torch, L, ctx, M, sets, steps=None, warmup=None, rec=False):
    """Verify attention of L GQA layers at context ctx for M verify tokens, `sets` rotating KV sets (so the Infinity
    Cache cannot serve a step from the previous one). A step = per layer the key-split pass and the merge. fp16 pages:
    32 q / 8 kv heads, head_dim 64 (the configs' geometry); rec: int8 K/V records of the reference geometry (16 q / 4 kv
    heads, head_dim 128, 264 bytes per position and KV head). Returns step time, GB/s, and the split pass's average
    launch time."""
    QH, KVH, D = (16, 4, 128) if rec else (32, 8, 64)
    steps = steps or args.steps
    warmup = args.warmup if warmup is None else warmup
    lib = host.lib()
    dev = "cuda"
    stream = torch.cuda.current_stream()
    sh = host.stream_handle(stream)
    n_pages = (ctx + M + 31) // 32
    g = torch.Generator(device=dev)
    g.manual_seed(20261201 + ctx + M)

    def rnd(*shape):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(torch.float16)

    def rnd32(*shape):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32)

    q = [rnd(M, QH, D) for _ in range(L)]
    out = [torch.empty((M, QH, D), dtype=torch.float16, device=dev) for _ in range(L)]
    if rec:
        # every position's records written by the library's quantize_pair writer from N(0,1) rows
        kv = [[host.rec_pages_alloc(n_pages, KVH) for _ in range(L)] for _ in range(sets)]
        for s_ in range(sets):
            for l in range(L):
                for p0 in range(0, ctx + M, 16384):
                    n = min(16384, ctx + M - p0)
                    host.kv_write_rec(rnd32(n, KVH, D), rnd32(n, KVH, D), kv[s_][l], p0)
        argv = [[host.rec_attn_args(q[l], kv[s_][l], ctx, out=out[l]) for l in range(L)] for s_ in range(sets)]
        need = lib.dspark_verify_attention_rec_workspace(ctypes.byref(argv[0][0]))
        f_all, f_split, f_merge = (lib.dspark_verify_attention_rec, lib.dspark_verify_attention_rec_splits,
                                   lib.dspark_verify_attention_rec_combine)
        layer_bytes = ctx * KVH * host.REC_BYTES
    else:
        kv = [[(rnd(n_pages, KVH, 32, D), rnd(n_pages, KVH, D, 32)) for _ in range(L)] for _ in range(sets)]
        fk = [rnd(M, KVH, D) for _ in range(L)]
        fv = [rnd(M, KVH, D) for _ in range(L)]
        argv = [[host.attn_args(q[l], kv[s_][l][0], kv[s_][l][1], ctx, out=out[l]) for l in range(L)]
                for s_ in range(sets)]
        need = lib.dspark_verify_attention_workspace(ctypes.byref(argv[0][0]))
        f_all, f_split, f_merge = (lib.dspark_verify_attention, lib.dspark_verify_attention_splits,
                                   lib.dspark_verify_attention_combine)
        layer_bytes = ctx * KVH * D * 2 * 2
        # The verified block's K/V rows go into every layer's pages once (in the full step the kernel that produces
        # them writes them); each step then re-verifies the same block.
        for s_ in range(sets):
            for l in range(L):
                host.check(lib.dspark_kv_write(ctypes.c_void_p(fk[l].data_ptr()), ctypes.c_void_p(fv[l].data_ptr()),
                                               KVH * D, ctypes.c_void_p(kv[s_][l][0].data_ptr()),
                                               ctypes.c_void_p(kv[s_][l][1].data_ptr()), None, n_pages, KVH, D, ctx, M,
                                               sh), "kv_write")
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    for s_ in range(sets):
        for l in range(L):
            argv[s_][l].workspace, argv[s_][l].workspace_bytes = ws.data_ptr(), ws.numel()

    def step(i):
        s_ = i % sets
        for l in range(L):
            host.check(f_all(ctypes.byref(argv[s_][l]), sh), "verify_attention")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / steps

    # Dominant kernel: the key-split pass, which streams the K/V pages. Its average launch duration: the same launches
    # back to back with nothing between them, HIP events recorded on the library's stream around all of them,
    # elapsed / launches (launch gaps included, so this errs low). The merge kernel is timed the same way and reported
    # beside it.
    n_launch = steps * L
    t0, t1, t2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    t0.record(stream)
    for i in range(steps):
        for l in range(L):
            host.check(f_split(ctypes.byref(argv[i % sets][l]), sh), "splits")
    t1.record(stream)
    for i in range(steps):
        for l in range(L):
            host.check(f_merge(ctypes.byref(argv[i % sets][l]), sh), "combine")
    t2.record(stream)
    torch.cuda.synchronize()
    kern_avg = t0.elapsed_time(t1) / n_launch
    combine_avg = t1.elapsed_time(t2) / n_launch
    # Per-launch brackets of the split pass (event overhead included, so these err high).
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n_launch)]
    j = 0
    for i in range(steps):
        for l in range(L):
            ev[j][0].record(stream)
            host.check(f_split(ctypes.byref(argv[i % sets][l]), sh), "splits")
            ev[j][1].record(stream)
            j += 1
    torch.cuda.synchronize()
    split_br = sorted(e[0].elapsed_time(e[1]) for e in ev)
    del kv, ws
    torch.cuda.empty_cache()
    return {"layers": L, "ctx": ctx, "M": M, "ms_per_step": ms_per_step, "layer_bytes": layer_bytes,
            "step_gbs": L * layer_bytes / (ms_per_step * 1e-3) / 1e9, "split_avg_ms": kern_avg,
            "split_gbs": layer_bytes / (kern_avg * 1e-3) / 1e9, "merge_avg_ms": combine_avg,
            "split_bracket_median_ms": split_br[len(split_br) // 2]}


def rec_attention_fields(args, host, torch):
    """Verify attention over the reference's int8 K/V records (reference geometry 16/4/128, its 9-token block) at 32k
    and 128k keys: 2 layers; 8 rotating record sets at 32k (16 x 34.6 MB) and 2 at 128k (4 x 138 MB), so a layer's
    records come back after more than the 256 MB Infinity Cache has been read."""
    out = []
    for ctx, sets in ((32768, 8), (131072, 2)):
        r = bench_attention(args, host, torch, 2, ctx, 9, sets, steps=max(8, args.steps // 2), warmup=2, rec=True)
        out.append({"ctx": ctx, "verify_tokens": 9, "record_bytes_per_layer": r["layer_bytes"],
                    "ms_per_layer": round(r["ms_per_step"] / 2, 5), "step_GBs": round(r["step_gbs"], 1),
                    "step_frac": round(r["step_gbs"] / HBM_PEAK_GBS, 4),
                    "split_avg_us": round(r["split_avg_ms"] * 1e3, 2), "split_GBs": round(r["split_gbs"], 1),
                    "split_frac": round(r["split_gbs"] / HBM_PEAK_GBS, 4),
                    "merge_avg_us": round(r["merge_avg_ms"] * 1e3, 2)})
    return out


def bench_c2(args, host, torch):
    r = bench_attention(args, host, torch, 6, 32768, 16, 2)
    L, ctx, M = r["layers"], r["ctx"], r["M"]
    step_bytes = L * r["layer_bytes"]
    achieved = r["split_gbs"]
    traffic = read_traffic()
    res = {
        "metric": METRIC,
        "value": round(r["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1) fp16 K/V/Q resident in HBM, 2 rotating KV sets",
        "config": {"workload": "C2 verify attention (BASELINE configs[1]): 6 GQA layers, 32 q / 8 kv heads, head_dim 64, "
                               "fp16 paged K/V at context 32768, 16 verify tokens causal in block; per layer the key-split "
                               "pass and the split merge (the block's K/V appended once at setup)",
                   "layers": L, "ctx": ctx, "verify_tokens": M, "q_heads": 32, "kv_heads": 8, "head_dim": 64,
                   "algorithmic_bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "verify_attn_lds_kernel (key-split pass)",
                     "algorithmic_bytes_per_launch": r["layer_bytes"],
                     "avg_launch_us": round(r["split_avg_ms"] * 1e3, 2),
                     "bracketed_median_us": round(r["split_bracket_median_ms"] * 1e3, 2),
                     "merge_kernel_avg_us": round(r["merge_avg_ms"] * 1e3, 2),
                     "step_frac": round(r["step_gbs"] / HBM_PEAK_GBS, 4)},
    }
    return res


def c5_attention_fields(args, host, torch):
    """C5's verify attention (context 131072) for the 33-token block and for 16 tokens: 2 layers, 2 rotating KV sets
    (4 x 268 MB)."""
    out = []
    for M in (33, 16):
        r = bench_attention(args, host, torch, 2, 131072, M, 2, steps=max(4, args.steps // 2), warmup=2)
        out.append({"ctx": 131072, "verify_tokens": M, "ms_per_layer": round(r["ms_per_step"] / 2, 5),
                    "step_GBs": round(r["step_gbs"], 1), "step_frac": round(r["step_gbs"] / HBM_PEAK_GBS, 4),
                    "split_avg_us": round(r["split_avg_ms"] * 1e3, 2), "split_GBs": round(r["split_gbs"], 1),
                    "split_frac": round(r["split_gbs"] / HBM_PEAK_GBS, 4),
                    "merge_avg_us": round(r["merge_avg_ms"] * 1e3, 2)})
    return out


MFMA_F16_PEAK_TFLOPS = 2500.0
MI50_TOK_S = {1024: 1174.0, 32768: 687.9, 131072: 423.7}  # README.md:233, 235, 237 (cold, median of 3)
MI50_TAU = {1024: 3.47, 32768: 3.30, 131072: 2.27}         # benchmarks/verify_attention.txt:54-58


def bench_c3(args, host, torch):
    """int8-weight FFN 2048 -> 8192 (SiLU) -> 2048 for M = 16 tokens with one fp16 scale per output
    row, then the 2048 x 16384 fp16 cropped-head projection with its row argmax. Four weight sets rotate (a set returns after 3 x 100.7 MB
    > the 256 MB Infinity Cache)."""
    M, H, I, N = 16, 2048, 8192, 16384
    SETS = 4
    dev = "cuda"
    stream = torch.cuda.current_stream()
    g = torch.Generator(device=dev)
    g.manual_seed(20261201 + 2)

    def u8(*shape):
        return torch.randint(1, 256, shape, generator=g, device=dev, dtype=torch.uint8)  # biased int8 in [-127, 127]

    def scales(rows, K):
        return (torch.rand(rows, generator=g, device=dev) * 0.5 + 0.75).div(73.3 * K ** 0.5).to(torch.float16)

    sets = [dict(up=u8(I, H), up_s=scales(I, H), dn=u8(H, I), dn_s=scales(H, I),
                 crop=(torch.randn((N, H), generator=g, device=dev) / H ** 0.5).to(torch.float16)) for _ in range(SETS)]
    x = torch.randn((M, H), generator=g, device=dev).to(torch.float16)
    hmid = torch.empty((M, I), dtype=torch.float16, device=dev)
    y16 = torch.empty((M, H), dtype=torch.float16, device=dev)
    best = torch.empty(M, dtype=torch.int64, device=dev)
    ws = host.Workspace(dev)

    def up(s):
        host.gemm_i8(x, s["up"], s["up_s"], epilogue=2, y_f16=hmid, workspace=ws)

    def down(s):
        host.gemm_i8(hmid, s["dn"], s["dn_s"], epilogue=0, y_f16=y16, workspace=ws)

    def crop(s):
        host.head_argmax(y16, s["crop"], best=best, workspace=ws)

    def timed(fn, n):
        for i in range(args.warmup):
            fn(sets[i % SETS])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n):
            fn(sets[i % SETS])
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    t_up, t_dn, t_crop = timed(up, args.steps), timed(down, args.steps), timed(crop, args.steps)
    t_step = timed(lambda s: (up(s), down(s), crop(s)), args.steps)
    bytes_up = I * H + 2 * I
    bytes_dn = H * I + 2 * H
    bytes_crop = 2 * N * H
    flops_ffn = 2 * M * H * I * 2
    flops_crop = 2 * M * H * N
    total_bytes = bytes_up + bytes_dn + bytes_crop
    gbs = total_bytes / (t_step * 1e-3) / 1e9

    def k(name, ms, nbytes, flops):
        return {"kernel": name, "us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                "mfma_util": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}

    return {
        "metric": "C3 int8 FFN + crop head: weight GB/s and MFMA utilisation", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t_step, 5),
        "higher_is_better": True, "dtype": "int8 weights, fp16 MFMA, fp32 accumulation",
        "data": "synthetic: int8 uniform [-127, 127] weights, fp16 N(0,1) activations, 4 rotating weight sets",
        "config": {"workload": "C3 (BASELINE configs[2]): M=16, FFN 2048->8192 (SiLU epilogue)->2048 int8 with per-row "
                               "fp16 scales, then 2048x16384 fp16 crop head + row argmax",
                   "algorithmic_bytes_per_step": total_bytes, "flops_per_step": flops_ffn + flops_crop},
        "kernels": [k("up 8192x2048 int8 (gemm_kernel)", t_up, bytes_up, flops_ffn / 2),
                    k("down 2048x8192 int8 (gemm_kernel + split-K reduce)", t_dn, bytes_dn, flops_ffn / 2),
                    k("crop 16384x2048 fp16 + argmax (gemm_kernel<fp16> + fold)", t_crop, bytes_crop, flops_crop)],
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "mfma_util": round((flops_ffn + flops_crop) / (t_step * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)},
    }


def engine_setup(host, torch, ctx, block, seed, desc=None):
    """A random-init model (the C4 geometry with block `block` unless `desc` is given) with every cache filled for
    positions < ctx: target K/V pages, the drafter ring, conv histories and taps hold N(0,1) fp16 / fp32 values."""
    desc = desc if desc is not None else host.c4_desc(block=block)
    eng = host.Engine(desc, ctx + 4096)
    eng.init_random(seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for name in eng.names():
        if name.endswith(".rec"):
            # int8 K/V records: codes uniform in [-127, 127], both scales 1/40 (|K|, |V| up to ~3, as N(0,1) rows give)
            ptr_, nbytes = eng.tensor(name)
            chunk = 264 * (1 << 18)
            for off in range(0, nbytes, chunk):
                n = min(chunk, nbytes - off) // 264
                r = torch.randint(-127, 128, (n, 264), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
                sc = torch.full((n, 1), 1.0 / 40, device="cuda", dtype=torch.float32).view(torch.int8)
                r[:, 128:132] = sc
                r[:, 260:264] = sc
                host._hip().hipMemcpy(ctypes.c_void_p(ptr_ + off), ctypes.c_void_p(r.data_ptr()),
                                      ctypes.c_size_t(264 * n), 3)
        elif name.startswith(("kv.", "ring.D", "conv.")):
            ptr_, nbytes = eng.tensor(name)
            chunk = 64 << 20
            for off in range(0, nbytes, chunk):
                n = min(chunk, nbytes - off) // 2
                t = torch.randn(n, generator=g, device="cuda").to(torch.float16)
                host._hip().hipMemcpy(ctypes.c_void_p(ptr_ + off), ctypes.c_void_p(t.data_ptr()),
                                      ctypes.c_size_t(2 * n), 3)
        elif name == "taps":
            ptr_, nbytes = eng.tensor(name)
            t = torch.randn(nbytes // 4, generator=g, device="cuda")
            host._hip().hipMemcpy(ctypes.c_void_p(ptr_), ctypes.c_void_p(t.data_ptr()), ctypes.c_size_t(nbytes), 3)
    torch.cuda.synchronize()
    return desc, eng


def engine_state(eng, a, anchor, big=1 << 30):
    eng.set_state(a=a, anchor=anchor, count=0, rounds_left=big, limit=eng.max_context, budget=big, eos=-1,
                  ctx_new=1, ctx_pos=a - 1, ctx_lo=max(0, a - 2048), run=1, skip_rounds=1, stop_at=eng.max_context,
                  ckpt_slot=-1, tokens=[anchor])


def greedy_chain(eng, host, torch, a0, anchor, n):
    """The target's greedy continuation of positions a0 + 1 .. a0 + n: one-token verify rounds (force_m = 1).

    The short-conv history is a ring of the last CONV_RING positions, so a chain longer than that overwrites the
    history of positions before a0; the rings are saved before the chain and restored after it, so that rounds
    restarted at a0 see the same history the chain started from (the KV pages are position-indexed and need no
    restore: a round rewrites the rows it verifies before it reads them)."""
    import numpy as np
    torch.cuda.synchronize()
    saved = {nm: eng.download(nm, np.uint16) for nm in eng.names() if nm.startswith("conv.L")}
    engine_state(eng, a0, anchor)
    for _ in range(n):
        eng.round(1, a0)
    torch.cuda.synchronize()
    st = eng.state()
    assert st.count == n, (st.count, n)
    chain = eng.download("out_tokens", np.int32)[:n].copy()
    for nm, buf in saved.items():
        eng.upload(nm, buf)
    return chain


def phase_times(eng, host, torch, mode, a0, anchor, rounds=5):
    """Mean microseconds per round of each phase, from traced rounds (the phase trace, dspark_engine_trace): the time
    from the previous mark to the phase's own mark; traced rounds carry one extra kernel per mark."""
    import collections
    engine_state(eng, a0, anchor)
    eng.trace(True)
    for _ in range(rounds):
        eng.round(mode, a0)
    torch.cuda.synchronize()
    marks = eng.trace_read()
    eng.trace(False)
    acc = collections.OrderedDict()
    for (r0, _, c0), (r1, p1, c1) in zip(marks, marks[1:]):
        if r1 != r0:
            continue
        name = host.trace_phase_name(p1)
        if name.startswith("verify_L"):
            name = "verify_layers"
        acc[name] = acc.get(name, 0.0) + (c1 - c0) / 1e3
    nr = len({r for (r, _, _) in marks}) or 1
    return {k: round(v / nr, 1) for k, v in acc.items()}


def round_bytes(eng, desc, a):
    """Algorithmic HBM bytes of one round at anchor position a: every GEMM weight and scale (int8 target and drafter
    layers, LM head, fp16 cropped head, conv taps) read once; the K/V each attention layer reads (full layers: the a
    cached positions plus the block; sliding layers: the window plus the block; drafter layers: the ring window plus
    the block); one Markov table row and one cropped-head row per draft step. Returns (round bytes, target K/V bytes)."""
    w = sum(eng.tensor(n)[1] for n in eng.names() if n.endswith((".w", ".s")) and not n.startswith("markov."))
    B = desc.block
    # K and V bytes per position: fp16 pages, or int8 records (264 bytes per KV head)
    row = desc.kv_heads * (264 if desc.kv_format else desc.head_dim * 2 * 2)
    kv = 0
    for i in range(desc.n_layers):
        if desc.layer_kind[i] == 1:
            kv += (a + B) * row
        elif desc.layer_kind[i] == 2:
            kv += (min(desc.window, a) + B) * row
    ring = desc.draft_layers * (min(desc.draft_window, a) + B) * row
    chain = desc.max_drafts * 2 * desc.crop_rows * 4
    return w + kv + ring + chain, kv


def run_rounds(eng, torch, mode, a0, anchor, warmup, rounds, hist=False):
    """Timed rounds from position a0; returns (ms per round, committed tokens per round, per-round accepted)."""
    stream = torch.cuda.current_stream()
    engine_state(eng, a0, anchor)
    for _ in range(warmup):
        eng.round(mode, a0)
    torch.cuda.synchronize()
    st0 = eng.state()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(rounds):
        eng.round(mode, a0)
    e1.record(stream)
    torch.cuda.synchronize()
    st1 = eng.state()
    ms = e0.elapsed_time(e1) / rounds
    committed = (st1.count - st0.count) / rounds
    accs = []
    if hist:  # untimed: one round at a time, the State read after each
        for _ in range(rounds):
            before = eng.state().accepted
            eng.round(mode, a0)
            torch.cuda.synchronize()
            accs.append(eng.state().accepted - before)
    return ms, committed, accs, st1


def plant_drafts(eng, chain, a0, p, seed, vocab):
    """plant[a0 + i] = chain token of that position with probability p, else a different token."""
    import numpy as np
    rng = np.random.default_rng(seed)
    ok = rng.random(len(chain)) < p
    planted = np.where(ok, chain, (chain + 1 + rng.integers(0, vocab - 1, len(chain))) % vocab).astype(np.int32)
    planted = np.where(ok, chain, np.where(planted == chain, (chain + 1) % vocab, planted)).astype(np.int32)
    buf = eng.download("plant", np.int32)
    buf[a0 + 1:a0 + 1 + len(chain)] = planted
    eng.upload("plant", buf)


def conv_snapshot(eng):
    import numpy as np
    return {nm: eng.download(nm, np.uint16) for nm in eng.names() if nm.startswith("conv.L")}


def conv_restore(eng, rings):
    for nm, buf in rings.items():
        eng.upload(nm, buf)


def planted_pass(eng, torch, a0, anchor, n_rounds, rings0, cover=0):
    """Untimed: n_rounds planted rounds from a0 (conv rings as at a0), then more until `cover` tokens are out; returns
    the tokens they emitted."""
    import numpy as np
    conv_restore(eng, rings0)
    engine_state(eng, a0, anchor)
    for _ in range(n_rounds):
        eng.round(-1, a0)
    torch.cuda.synchronize()
    while eng.state().count < cover:
        for _ in range(8):
            eng.round(-1, a0)
        torch.cuda.synchronize()
    return eng.download("out_tokens", np.int32)[:eng.state().count].copy()


def settle_chain(eng, host, torch, desc, a0, anchor, need, p, n_rounds, rings0, cover=0, tries=8):
    """The greedy chain the planted drafts replay, checked against what planted rounds actually emit.

    Planted rounds emit the target's own greedy continuation under their own arithmetic (accepted drafts equal the
    target's tokens, the bonus is the target's token). The chain comes from one-token rounds, and where a verify pass
    of M rows resolves a near tie differently (the attention's key splits follow a and M, so the fp32 sums differ in
    order), the emitted tokens leave the chain at some index and every later planted draft is wrong. So: plant, run
    the pass, and where it left the chain take its tokens, extend them by one-token rounds from where the pass
    stopped, plant again; until a pass emits the chain itself. The timed rounds repeat the last pass exactly (every
    reduction has a fixed order), so their acceptance follows the planted draws; the pass runs on until `cover` tokens
    are out, so the launch path's rounds (the same rounds from the same start) are covered too. Returns (chain,
    re-plants)."""
    import numpy as np
    chain = greedy_chain(eng, host, torch, a0, anchor, need)
    fixes = 0
    for _ in range(tries):
        plant_drafts(eng, chain, a0, p, 7, desc.vocab)
        out = planted_pass(eng, torch, a0, anchor, n_rounds, rings0, cover)
        n = len(out)
        if np.array_equal(out, chain[:n]):
            break
        fixes += 1
        ext = greedy_chain(eng, host, torch, a0 + n, int(out[-1]), max(1, need - n))
        chain = np.concatenate([out, ext]).astype(np.int32)
    conv_restore(eng, rings0)
    return chain, fixes


def run_launches(eng, torch, a0, anchor, rings0, n_warm, n_timed):
    """The drop-in path: draftLaunch's loop (internal/model/generate.go:133-162) over dspark_engine_launch, each launch
    from the State the last one left to the next 32-position boundary (32 rounds at most), planted drafts. Host wall
    clock around the timed launches (each launch returns when its State is back on the host)."""
    conv_restore(eng, rings0)
    torch.cuda.synchronize()
    kw = dict(a=a0, anchor=anchor, ctx_new=1, ctx_pos=a0 - 1, miss=0, skip=0)
    lo = max(0, a0 - 2048)
    tok = rounds = enq = 0
    t0 = None
    for i in range(n_warm + n_timed):
        if i == n_warm:
            t0 = time.perf_counter()
        _, res = eng.launch(kw["a"], kw["anchor"], budget=512, rounds=32, ctx_new=kw["ctx_new"],
                            ctx_pos=kw["ctx_pos"], ctx_lo=lo, force_m=-1, miss=kw["miss"], skip=kw["skip"])
        st = res.state
        kw = dict(a=st.a, anchor=st.anchor, ctx_new=st.ctx_new, ctx_pos=st.ctx_pos, miss=st.miss, skip=st.skip)
        if i >= n_warm:
            tok += res.count
            rounds += res.rounds
            enq += res.rounds_enqueued
    wall = time.perf_counter() - t0
    return {"launches": n_timed, "rounds": rounds, "rounds_enqueued": enq, "tokens": tok,
            "ms_per_round": wall * 1e3 / rounds, "tokens_per_round": tok / rounds, "tok_s": tok / wall}


def p_for_tau(tau, drafts):
    """Per-position planting probability whose expected committed tokens per round is tau (truncated geometric)."""
    lo, hi = 0.0, 1.0
    for _ in range(60):
        p = (lo + hi) / 2
        e = sum(p ** k for k in range(1, drafts + 1)) + 1
        lo, hi = (p, hi) if e < tau else (lo, p)
    return (lo + hi) / 2


def bench_engine(args, host, torch, workload):
    """C4 / C5 / tiers / ref: the full DSpark round (context projection, drafter, Markov drafts, verify, greedy argmax,
    acceptance + commit) as HIP-graph replays on a random-init model: the C4 geometry, or for `ref` the reference
    model's geometry and draft policy."""
    out = []
    ref = workload == "ref"
    if workload == "c4":
        cases = [(32768, 16, None)]
    elif workload == "c5":
        cases = [(131072, 33, 0.0), (131072, 33, 0.5), (131072, 33, 1.0)]
    else:  # tiers / ref: the reference's verify block (MT = 9) at the MI50's measured committed tokens per round
        tiers = [int(c) for c in args.tiers.split(",")] if getattr(args, "tiers", "") else (1024, 32768, 131072)
        cases = [(c, 9, ("tau", MI50_TAU[c])) for c in tiers]
    rounds, warm = args.steps, args.warmup
    cache = {}
    for ctx, block, plant in cases:
        # ref: the reference geometry and draft policy (7 drafts, 3 from position 57344, generate.go:136)
        max_drafts = (3 if ctx >= 57344 else 7) if ref else block - 1
        key = (ctx, block, max_drafts)
        if key not in cache:
            for k in list(cache):
                cache.pop(k)[1].close()
            fmt = 0 if args.ref_formats == "fp16" else 1
            x8 = 1 if args.ref_formats == "reference" else 0
            desc_ = (host.ref_desc(block=block, max_drafts=max_drafts, kv_format=fmt, weight_format=fmt, x_format=x8)
                     if ref else None)
            cache[key] = engine_setup(host, torch, ctx, block, 20261201 + ctx + block, desc_)
        desc, eng = cache[key]
        a0, anchor = ctx, 17
        print(f"case {workload} ctx={ctx} block={block} plant={plant}", file=sys.stderr, flush=True)
        rec = {"ctx": ctx, "block": block}
        if plant is None:
            ms, committed, accs, st = run_rounds(eng, torch, 0, a0, anchor, warm, rounds, hist=True)
            import collections
            rec["accepted_histogram"] = dict(sorted(collections.Counter(accs).items()))
        else:
            p = plant if not isinstance(plant, tuple) else p_for_tau(plant[1], desc.max_drafts)
            n_launch = (1, 4) if isinstance(plant, tuple) else (0, 0)  # the tiers also time the drop-in launch path
            cover = (sum(n_launch) + 1) * 32 + block  # positions the launches reach
            need = max((warm + rounds + 1) * block + 2, cover + 8 * block + 2)
            rings0 = conv_snapshot(eng)
            chain, fixes = settle_chain(eng, host, torch, desc, a0, anchor, need, p, warm + rounds, rings0, cover)
            ms, committed, accs, st = run_rounds(eng, torch, -1, a0, anchor, warm, rounds)
            rec["planted_p"] = round(p, 4)
            rec["planted_tau_expected"] = round(1 + sum(p ** k for k in range(1, desc.max_drafts + 1)), 3)
            rec["max_drafts"] = desc.max_drafts
            rec["replants"] = fixes
            if n_launch[1]:
                lr = run_launches(eng, torch, a0, anchor, rings0, *n_launch)
                rec["launch"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in lr.items()}
                rec["launch_tok_s"] = round(lr["tok_s"], 1)
                # the drop-in path against the round rate: time per round (launch boundaries, host round trips and
                # the rounds a launch enqueues included) and tok/s at the same committed tokens per round
                rec["launch_round_time_ratio"] = round(ms / lr["ms_per_round"], 4)
                rec["launch_tok_s_at_mi50_tau"] = round(plant[1] / (lr["ms_per_round"] * 1e-3), 1)
        rec["phase_us"] = phase_times(eng, host, torch, 0 if plant is None else -1, a0, anchor)
        rec.update({"ms_per_round": round(ms, 4), "tokens_per_round": round(committed, 3),
                    "tok_s": round(committed / (ms * 1e-3), 1)})
        rb, kvb = round_bytes(eng, desc, a0)
        rec.update({"round_bytes": rb, "verify_kv_bytes": kvb, "round_GBs": round(rb / (ms * 1e-3) / 1e9, 1),
                    "round_frac": round(rb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        if isinstance(plant, tuple):
            # A round verifies the same tokens whatever is accepted, so its time does not depend on the draws: the
            # rate at exactly the MI50's committed tokens per round is tau / round time (the realised rate above
            # carries the sampling noise of the planted draws).
            rec["tok_s_at_mi50_tau"] = round(plant[1] / (ms * 1e-3), 1)
            rec["mi50_tok_s"] = MI50_TOK_S[ctx]
            rec["vs_mi50"] = round(rec["tok_s_at_mi50_tau"] / MI50_TOK_S[ctx], 3)
        out.append(rec)
        print(json.dumps(rec), file=sys.stderr, flush=True)
    for k in list(cache):
        cache.pop(k)[1].close()
    recf = ref and args.ref_formats != "fp16"
    xf = ("int8 GEMM inputs per 16 columns (LFM3_X8, the reference's default build)" if args.ref_formats == "reference"
          else "fp16 GEMM inputs (the reference's LFM3_F16 build)")
    model = ("reference geometry: 24 layers (13 conv k=7 / 6 full / 5 sliding-256 attention, 16/4/128), FFN 7680, "
             "vocab 128000, 3-layer drafter; " + (f"the reference's int8 K/V records and per-128-column weight scales, {xf}"
                                                  if recf else "fp16 K/V pages and per-row weight scales") if ref
             else "C4 geometry")
    kv = ("int8 K/V records (codes uniform in [-127, 127], scales 1/40)" if recf else "N(0,1) fp16 KV caches")
    scales = "per-128-column fp16 scales" if recf else "per-row fp16 scales"
    return {"metric": f"greedy decode tok/s (DSpark rounds, random-init model, {model})", "workload": workload,
            "rounds": rounds, "warmup": warm, "cases": out,
            "data": f"random-init weights (int8 uniform, {scales}), {kv}; planted drafts "
                    "replay the target's own greedy chain (one-token verify rounds) with per-position probability p"}


def bench_copy(args, torch):
    """Plain device copy of a known size: the calibration point for rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    nbytes = 512 << 20
    src = torch.ones(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    return {"workload": "copy", "bytes_per_copy": nbytes, "GBs_read_plus_write": round(2 * nbytes * args.steps / el / 1e9, 1)}


def trace_summary(path):
    """One round of a rocprofv3 kernel trace (the --kernel-trace --output-format csv file of a round workload): the
    middle round of the longest run of back-to-back rounds with no host copy, trace mark or forced row count among
    them (a round of a timed loop), as kernels by total time and GEMM launch shapes. Reads a CSV; no GPU."""
    import csv
    import collections
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    idx = [i for i, r in enumerate(rows) if "round_begin_kernel" in r["Kernel_Name"]]
    runs, cur = [], []
    for k in range(len(idx) - 1):
        rnd = rows[idx[k]:idx[k + 1]]
        names = [r["Kernel_Name"] for r in rnd]
        if any("trace_mark" in n or "force_m" in n or "rocclr" in n for n in names):
            if cur:
                runs.append(cur)
            cur = []
            continue
        cur.append(rnd)
    if cur:
        runs.append(cur)
    if not runs:
        return "no complete round in the trace"
    best = max(runs, key=len)
    rnd = best[len(best) // 2]

    def name(r):
        n = r["Kernel_Name"].replace("void ", "").replace("dspark::", "")
        return n if n.startswith("_Z") else n.split("(dspark")[0].split("(")[0]
    agg, shapes = collections.OrderedDict(), collections.OrderedDict()
    for r in rnd:
        n, d = name(r), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        a = agg.setdefault(n, [0, 0.0])
        a[0] += 1
        a[1] += d
        if "gemm" in n:
            key = f"{n} {int(r['Grid_Size_X']) // int(r['Workgroup_Size_X'])} x {r['Workgroup_Size_X']}"
            b = shapes.setdefault(key, [0, 0.0])
            b[0] += 1
            b[1] += d
    busy = sum(v[1] for v in agg.values())
    nxt = rows[rows.index(rnd[-1]) + 1]
    span = (int(nxt["Start_Timestamp"]) - int(rnd[0]["Start_Timestamp"])) / 1e3
    out = [f"# round: {len(rnd)} kernels, kernel busy {busy:.1f} us, round_begin to next round_begin under the tracer "
           f"{span:.1f} us (middle of {len(best)} back-to-back rounds)",
           "# kernel, launches per round, total us, average us"]
    for k, v in sorted(agg.items(), key=lambda x: -x[1][1]):
        out.append(f"{k[:64]:64s} {v[0]:4d} {v[1]:8.1f} {v[1] / v[0]:7.2f}")
    out.append("# GEMM launch shapes (workgroups x threads), launches, total us, average us:")
    for k, v in sorted(shapes.items(), key=lambda x: -x[1][1]):
        out.append(f"#   {k[:70]:70s} {v[0]:4d} {v[1]:8.1f} {v[1] / v[0]:7.2f}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", default="c2", choices=["c2", "c3", "c4", "c5", "tiers", "ref", "copy", "attn", "rec"])
    ap.add_argument("--ref-formats", default="reference", choices=["reference", "reference-f16x", "fp16"],
                    help="ref workload: the reference's default build (int8 K/V records, per-128-column weight "
                         "scales, int8 GEMM inputs per 16 columns), the same with fp16 GEMM inputs (its LFM3_F16 "
                         "build), or fp16 K/V pages with per-row scales")
    ap.add_argument("--tiers", default="", help="tiers / ref workloads: comma-separated contexts out of 1024, 32768, "
                                                  "131072 (default all three)")
    ap.add_argument("--ctx", type=int, default=131072, help="attn workload: context (keys before the block)")
    ap.add_argument("--tokens", type=int, default=0, help="attn / rec workload: verify tokens (default 33 / 9)")
    ap.add_argument("--layers", type=int, default=2, help="attn workload: layers per step")
    ap.add_argument("--c2-only", action="store_true",
                    help="default workload without the headline tiers and the C5 and int8-record attention fields")
    ap.add_argument("--trace-summary", default="", metavar="CSV",
                    help="print one round of a rocprofv3 kernel-trace CSV of a round workload and exit (no GPU)")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(args.trace_summary))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.workload == "copy":
        print(json.dumps(bench_copy(args, torch)), flush=True)
        return
    host = load_host()
    if args.workload == "c3":
        print(json.dumps(bench_c3(args, host, torch)), flush=True)
        return
    if args.workload in ("attn", "rec"):
        # verify attention alone at any context and block: the C2 kernels (fp16 pages, 32/8/64), or the int8-record
        # kernels (reference geometry 16/4/128); what the attention profiles run
        rec = args.workload == "rec"
        args.tokens = args.tokens or (9 if rec else 33)
        r = bench_attention(args, host, torch, args.layers, args.ctx, args.tokens, 2, rec=rec)
        print(json.dumps({"metric": "verify attention HBM GB/s", "workload": args.workload, "ctx": args.ctx,
                          "verify_tokens": args.tokens, "layers": args.layers, "steps": args.steps,
                          "ms_per_layer": round(r["ms_per_step"] / args.layers, 5),
                          "step_GBs": round(r["step_gbs"], 1), "split_avg_us": round(r["split_avg_ms"] * 1e3, 2),
                          "split_frac": round(r["split_gbs"] / HBM_PEAK_GBS, 4),
                          "merge_avg_us": round(r["merge_avg_ms"] * 1e3, 2)}), flush=True)
        return
    if args.workload in ("c4", "c5", "tiers", "ref"):
        print(json.dumps(bench_engine(args, host, torch, args.workload)), flush=True)
        return
    res = bench_c2(args, host, torch)
    if not args.c2_only:
        # The metric's other half: greedy decode tok/s at 1k / 32k / 128k (DSpark rounds of the C4-geometry model with
        # the reference's 9-token verify block, drafts planted at the MI50's committed tokens per round), and C5's
        # verify attention at 128k.
        targs = argparse.Namespace(**vars(args))
        targs.steps, targs.warmup = min(args.steps, 20), min(args.warmup, 5)
        tiers = bench_engine(targs, host, torch, "tiers")
        res["headline_tok_s"] = {
            "model": "C4 geometry (16 layers: 10 conv k=3 + 6 GQA 32/8/64, H 2048, FFN 8192, vocab 65536, int8 "
                     "weights; 4-layer drafter), random-init, block 9 (the reference's verify block)",
            "rounds": targs.steps, "warmup": targs.warmup,
            "tiers": [{k: c[k] for k in ("ctx", "ms_per_round", "tokens_per_round", "tok_s", "tok_s_at_mi50_tau",
                                         "mi50_tok_s", "vs_mi50", "planted_tau_expected", "replants", "launch_tok_s",
                                         "launch_tok_s_at_mi50_tau", "launch_round_time_ratio", "launch")}
                      for c in tiers["cases"]],
            "note": "tok_s_at_mi50_tau = the MI50's measured committed tokens per round (benchmarks/"
                    "verify_attention.txt:54-58) / this round time; a round verifies the same tokens whatever is "
                    "accepted, so its time does not depend on the draws; tok_s is the rate of the planted draws; "
                    "launch_* time the drop-in path (dspark_engine_launch, draftLaunch's loop: one launch per "
                    "32-position block, State read back by the host after each) on the same planted chain"}
        # The same tiers on the reference model's geometry, draft policy and default build (int8 K/V records,
        # per-128-column weight scales, int8 GEMM inputs): the configuration the MI50 numbers were measured on.
        rargs = argparse.Namespace(**vars(targs))
        rargs.ref_formats = "reference"
        rtiers = bench_engine(rargs, host, torch, "ref")
        res["headline_ref_tok_s"] = {
            "model": rtiers["metric"], "rounds": targs.steps, "warmup": targs.warmup,
            "tiers": [{k: c[k] for k in ("ctx", "max_drafts", "ms_per_round", "tokens_per_round", "tok_s",
                                         "tok_s_at_mi50_tau", "mi50_tok_s", "vs_mi50", "planted_tau_expected",
                                         "replants", "launch_tok_s", "launch_tok_s_at_mi50_tau",
                                         "launch_round_time_ratio", "launch")}
                      for c in rtiers["cases"]]}
        # The same on the reference's LFM3_F16 build (fp16 GEMM inputs): on MI355X the int8-x products (one masked
        # MFMA pair and a scaled add per 16-column piece) lengthen the latency-bound GEMMs
        fargs = argparse.Namespace(**vars(targs))
        fargs.ref_formats = "reference-f16x"
        ftiers = bench_engine(fargs, host, torch, "ref")
        res["headline_ref_f16x_tok_s"] = {
            "model": ftiers["metric"], "rounds": targs.steps, "warmup": targs.warmup,
            "tiers": [{k: c[k] for k in ("ctx", "max_drafts", "ms_per_round", "tokens_per_round", "tok_s",
                                         "tok_s_at_mi50_tau", "vs_mi50", "launch_tok_s", "launch_round_time_ratio")}
                      for c in ftiers["cases"]]}
        res["c5_attention"] = c5_attention_fields(args, host, torch)
        res["ref_int8_record_attention"] = rec_attention_fields(args, host, torch)
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        res["cpu_baseline"] = cpu_baseline_c2(32768, 16, 32, 8, 64, args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
