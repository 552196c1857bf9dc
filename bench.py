#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one GPU).

Headline metric: qmv HBM GB/s at K=4096 x N=12288, 4-bit gs64,
bf16 (config 2a) -> `value`; qmm TFLOP/s at M=512, N=K=4096 (config 3a) -> the
`qmm` object.  A "step" is one kernel call over one batch of synthetic input
already resident in HBM.  `--copies` independent weight copies are rotated
so the working set (>= 450 MB for qmv) exceeds the 256 MB Infinity Cache;
steps are captured into a HIP graph and replayed, bracketed by HIP events on
the launch stream.  The CPU baseline leg times the oracle's multithreaded
dequantize-and-dot on the host.

    python bench.py [--steps K] [--warmup W] [--only qmv|qmm|all|configs] [--no-cpu] [--no-configs]

The line's "configs" object times the other configurations of the
measurement table (cfg1, cfg2b, cfg3b/3c, cfg4 small-M sweep through the
routed op, cfg5 routed experts) the same way.

HBM traffic (`roofline.traffic`) comes from rocprofv3 counter runs of this
same script, calibrated against a plain device copy of known size:

    rocprofv3 --pmc FETCH_SIZE -d D1 -o run --output-format csv -- python3 bench.py
    rocprofv3 --pmc WRITE_SIZE -d D2 -o run --output-format csv -- python3 bench.py
    rocprofv3 --pmc FETCH_SIZE -d D3 -o run --output-format csv -- python3 bench.py --only copy
    rocprofv3 --pmc WRITE_SIZE -d D4 -o run --output-format csv -- python3 bench.py --only copy
    python bench.py --pmc-summary D1 D2 D3 D4   # -> profiles/traffic.json

`bench.py` reads profiles/traffic.json when it names the kernel being timed.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "qmv HBM GB/s (%peak) K4096×N12288 4b; qmm TFLOPS (%MFMA peak) M=512"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")
COPY_BYTES = 512 << 20         # calibration copy: 512 MiB read + 512 MiB written
QMV_KERNEL = "qmv_lean_kernel<cpq::dev::BF16, 4"
QMM_KERNEL = "qmm_dma_kernel<cpq::dev::BF16"
COPY_KERNEL = "copy"


def algo_bytes(m, n, k, gs, bits, tsize=2):
    """Reference byte formula (qmv_dispatch_bench.rs:37-43) extended to M rows."""
    return n * k * bits // 8 + 2 * n * (k // gs) * tsize + m * k * tsize + m * n * tsize


def make_copies(dev, rng, copies, n, k, gs, bits, dtype):
    from cider_press_amd.synthetic import from_bits, to_bits

    out = []
    host0 = None
    for c in range(copies):
        w = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
        s = to_bits(rng.uniform(0.002, 0.02, size=(n, k // gs)).astype(np.float32), dtype)
        b = to_bits(-float(1 << (bits - 1)) * from_bits(s, dtype), dtype)
        if c == 0:
            host0 = (w, s, b)
        out.append((dev.upload(w.reshape(-1), "u32"), dev.upload(s.reshape(-1), dtype),
                    dev.upload(b.reshape(-1), dtype)))
    return out, host0


class Flusher:
    """Evicts the 256 MB Infinity Cache (and L2) before a timed region with a
    plain read of a 512 MiB buffer nothing else touches.  It reads, so it
    leaves clean lines: a flush that wrote would have its dirty lines written
    back to HBM during the timed region.  Without it the first weight copies
    of the timed replay could still be cache-resident from the untimed one."""

    def __init__(self, dev):
        import ctypes

        self.buf = dev.alloc_buffer(128 << 20, "u32")
        self.sink = dev.alloc_buffer(1, "u32")
        self.ptrs = (ctypes.c_void_p * 1)(self.buf.ptr)
        self.lens = (ctypes.c_size_t * 1)(self.buf.byte_len)

    def flush(self, cmds):
        import ctypes

        from cider_press_amd import _lib

        _lib.check(_lib.lib().cpq_stream_read(cmds.handle, self.ptrs, self.lens, 1, ctypes.c_void_p(self.sink.ptr),
                                              4096))


_FLUSHER = None


def time_graph(dev, steps, warmup, encode_step):
    """Capture `steps` calls in a graph, replay once untimed per warmup batch,
    replay the timed graph once untimed, flush the caches, then time one
    replay between HIP events on the launch stream."""
    global _FLUSHER
    from cider_press_amd.kernels import Event

    if _FLUSHER is None:
        _FLUSHER = Flusher(dev)
    cmds = dev.commands()
    if warmup:
        cmds.begin_capture()
        for i in range(warmup):
            encode_step(cmds, i)
        gw = cmds.end_capture()
        gw.launch(cmds)
        cmds.commit_and_wait()
    cmds.begin_capture()
    for i in range(steps):
        encode_step(cmds, i)
    g = cmds.end_capture()
    g.launch(cmds)          # one untimed replay of the timed graph itself
    _FLUSHER.flush(cmds)    # no weight copy starts the timed replay cache-resident
    cmds.commit_and_wait()
    e0, e1 = Event(), Event()
    cmds.commit_and_wait()  # barrier: nothing in flight before the timed region
    e0.record(cmds)
    g.launch(cmds)
    e1.record(cmds)
    cmds.commit_and_wait()
    return e0.elapsed_ms(e1) / steps


def parity_entry(rep, rows=None):
    """The tolerance report as the line carries it: raw and beyond-rounding
    errors with their bounds (max-abs is judged beyond the output's own
    rounding to T; see oracle.tolerance_report)."""
    out = {"ok": rep["ok"], "rel_l2": rep["rel_l2"], "rel_l2_bound": rep["rel_l2_bound"],
           "max_abs": rep["max_abs"], "max_abs_beyond_rounding": rep["max_abs_beyond_rounding"],
           "max_abs_bound": rep["max_abs_bound"]}
    if rows is not None:
        out["rows_checked"] = rows
    return out


def check_rows(m):
    """Rows the oracle checks for an M-row prefill: all of them up to 512,
    else two whole 128-row tiles plus every 7th row (every position inside a
    tile is covered)."""
    if m <= 512:
        return np.arange(m)
    rows = set(range(0, 128)) | set(range(m - 128, m)) | set(range(0, m, 7))
    return np.array(sorted(rows))


ORACLE_THREADS = min(16, os.cpu_count() or 1)


def bench_qmv(dev, lib, args, rng):
    from cider_press_amd.kernels import qmv as kqmv
    from cider_press_amd.synthetic import make_x

    n, k, gs, bits, dtype = 12288, 4096, 64, 4, "bf16"
    copies, host0 = make_copies(dev, rng, args.copies, n, k, gs, bits, dtype)
    x = make_x(rng, 1, k, dtype)
    X = dev.upload(x.reshape(-1), dtype)
    Y = dev.alloc_buffer(n, dtype)

    def step(cmds, i):
        W, S, B = copies[i % len(copies)]
        kqmv.affine_qmv(cmds, lib, W, S, B, X, Y, k, gs, bits)

    parity = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

        cmds = dev.commands()
        step(cmds, 0)
        cmds.commit_and_wait()
        ref = O.qmm_ref(x, *host0, 1, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
        parity = parity_entry(O.tolerance_report(Y.to_numpy().reshape(1, n), ref, x, k, dtype))
    ms = time_graph(dev, args.steps, args.warmup, step)
    nbytes = algo_bytes(1, n, k, gs, bits)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": ms, "gbs": gbs, "bytes": nbytes, "parity": parity, "host0": host0, "x": x,
            "shape": (n, k, gs, bits), "copies": copies, "X": X}


def bench_qmm(dev, lib, args, rng):
    from cider_press_amd.kernels import qmm as kqmm
    from cider_press_amd.synthetic import make_x

    m, n, k, gs, bits, dtype = 512, 4096, 4096, 64, 4, "bf16"
    copies, host0 = make_copies(dev, rng, args.copies, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    X = dev.upload(x.reshape(-1), dtype)
    Y = dev.alloc_buffer(m * n, dtype)

    def step(cmds, i):
        W, S, B = copies[i % len(copies)]
        kqmm.affine_qmm_t(cmds, lib, W, S, B, X, Y, m, n, k, gs, bits)

    parity = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

        cmds = dev.commands()
        step(cmds, 0)
        cmds.commit_and_wait()
        ref = O.qmm_ref(x, *host0, m, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
        parity = parity_entry(O.tolerance_report(Y.to_numpy().reshape(m, n), ref, x, k, dtype))
    ms = time_graph(dev, args.qmm_steps, args.warmup, step)
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tflops, "flops": flops, "bytes": algo_bytes(m, n, k, gs, bits),
            "parity": parity}


def _weights(dev, rng, copies, n, k, gs, bits, dtype, bias_noise=0.0):
    """Rotated device copies and the host arrays of copy 0 (the parity input)."""
    from cider_press_amd.synthetic import make_weight

    out, host0 = [], None
    for c in range(copies):
        w, s, b = make_weight(rng, n, k, gs, bits, dtype, bias_noise=bias_noise)
        if c == 0:
            host0 = (w, s, b)
        out.append((dev.upload(w.reshape(-1), "u32"), dev.upload(s.reshape(-1), dtype),
                    dev.upload(b.reshape(-1), dtype)))
    return out, host0


def _copies_for(nbytes, min_copies=2, working_set=600 << 20, cap=16):
    """Enough rotated weight copies that the working set exceeds the 256 MB
    Infinity Cache (bounded by `cap`)."""
    return int(max(min_copies, min(cap, -(-working_set // max(nbytes, 1)))))


def bench_configs(dev, lib, args, rng):
    """The remaining configurations of the measurement table: cfg1, cfg2b
    (decode), cfg3b/3c (prefill), cfg4 (small M through the routed op, all
    three quantizations), cfg5 (routed experts).  Same timing method as the
    headline: rotated weight copies, one graph replay between HIP events.
    Every configuration is also checked against the oracle (copy 0, one
    eager call) unless --no-parity."""
    from cider_press_amd.kernels import gather as kg
    from cider_press_amd.kernels import qmm as kqmm
    from cider_press_amd.kernels import qmv as kqmv
    from cider_press_amd.synthetic import make_routing, make_x

    O = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

    steps = args.config_steps
    res = {}

    def eager(fn):
        cmds = dev.commands()
        fn(cmds)
        cmds.commit_and_wait()

    def qmv_case(name, n, k, dtype, bias_noise=0.0):
        gs, bits = 64, 4
        wb = n * k // 2 + 4 * n * (k // gs)
        cps, h0 = _weights(dev, rng, _copies_for(wb), n, k, gs, bits, dtype, bias_noise)
        x = make_x(rng, 1, k, dtype)
        X = dev.upload(x.reshape(-1), dtype)
        Y = dev.alloc_buffer(n, dtype)
        par = None
        if O is not None:
            eager(lambda c: kqmv.affine_qmv(c, lib, *cps[0], X, Y, k, gs, bits))
            ref = O.qmm_ref(x, *h0, 1, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
            par = parity_entry(O.tolerance_report(Y.to_numpy().reshape(1, n), ref, x, k, dtype))
        ms = time_graph(dev, steps, args.warmup,
                        lambda c, i: kqmv.affine_qmv(c, lib, *cps[i % len(cps)], X, Y, k, gs, bits))
        nb = algo_bytes(1, n, k, gs, bits)
        res[name] = {"shape": f"x[1,{k}] . W[{n},{k}]^T 4b gs64 {dtype}", "us": round(ms * 1e3, 2),
                     "GB/s": round(nb / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "copies": len(cps), "parity": par}

    def qmm_case(name, m, n, k):
        gs, bits, dtype = 64, 4, "bf16"
        wb = n * k // 2 + 4 * n * (k // gs)
        cps, h0 = _weights(dev, rng, _copies_for(wb), n, k, gs, bits, dtype)
        x = make_x(rng, m, k, dtype)
        X = dev.upload(x.reshape(-1), dtype)
        Y = dev.alloc_buffer(m * n, dtype)
        par = None
        if O is not None:
            eager(lambda c: kqmm.affine_qmm_t(c, lib, *cps[0], X, Y, m, n, k, gs, bits))
            rows = check_rows(m)
            y = Y.to_numpy().reshape(m, n)
            ref = O.qmm_ref(x[rows], *h0, len(rows), n, k, gs, bits, dtype, threads=ORACLE_THREADS)
            par = parity_entry(O.tolerance_report(y[rows], ref, x[rows], k, dtype), rows=len(rows))
            par["all_finite"] = bool(np.all(np.isfinite(O.bits_to_f32(y, dtype))))
        ms = time_graph(dev, max(10, steps // 4), args.warmup,
                        lambda c, i: kqmm.affine_qmm_t(c, lib, *cps[i % len(cps)], X, Y, m, n, k, gs, bits))
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        res[name] = {"shape": f"X[{m},{k}] . W[{n},{k}]^T 4b gs64 bf16", "us": round(ms * 1e3, 2),
                     "TFLOP/s": round(tf, 1), "mfma_frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "copies": len(cps),
                     "parity": par}

    qmv_case("cfg1", 2048, 2048, "f16", bias_noise=1e-3)
    qmv_case("cfg2b", 4096, 12288, "bf16")
    qmm_case("cfg3b", 512, 12288, 4096)
    qmm_case("cfg3c_n4096", 2048, 4096, 4096)
    qmm_case("cfg3c_n12288", 2048, 12288, 4096)

    # cfg4: small M through the routed op (eval.rs routing), K = N = 4096.
    rows = []
    n = k = 4096
    for bits, gs in ((4, 64), (4, 32), (8, 64)):
        wb = n * k * bits // 8 + 4 * n * (k // gs)
        cps, h0 = _weights(dev, rng, _copies_for(wb), n, k, gs, bits, "bf16")
        for m in (1, 4, 16, 64):
            x = make_x(rng, m, k, "bf16")
            X = dev.upload(x.reshape(-1), "bf16")
            Y = dev.alloc_buffer(m * n, "bf16")
            par = None
            if O is not None:
                eager(lambda c: kqmm.quantized_matmul(c, *cps[0], X, Y, m, n, k, gs, bits))
                ref = O.qmm_ref(x, *h0, m, n, k, gs, bits, "bf16", threads=ORACLE_THREADS)
                par = parity_entry(O.tolerance_report(Y.to_numpy().reshape(m, n), ref, x, k, "bf16"))
            ms = time_graph(dev, steps, args.warmup,
                            lambda c, i: kqmm.quantized_matmul(c, *cps[i % len(cps)], X, Y, m, n, k, gs, bits))
            nb = algo_bytes(m, n, k, gs, bits)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            rows.append({"bits": bits, "gs": gs, "m": m, "us": round(ms * 1e3, 2),
                         "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "TFLOP/s": round(tf, 2), "mfma_frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 5),
                         "kernel": "qmv" if m == 1 else ("small-M" if m <= (64 if n <= 8192 else 32) else "prefill"),
                         "parity": par})
        del cps
    res["cfg4"] = rows

    # cfg5: 128 experts, W_up [768, 2048] and W_down [2048, 768], 4b gs64;
    # 256 tokens routed top-8 (uniform, without replacement) -> 2048 rows.
    e, tokens, topk = 128, 256, 8
    route = make_routing(rng, tokens, topk, e).reshape(-1)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), topk)
    order = np.argsort(route, kind="stable")
    for proj, (n, k) in (("up", (768, 2048)), ("down", (2048, 768))):
        gs, bits = 64, 4
        wb = e * (n * k // 2 + 4 * n * (k // gs))
        cps, h0 = _weights(dev, rng, _copies_for(wb, cap=6), e * n, k, gs, bits, "bf16")
        xin = make_x(rng, tokens if proj == "up" else tokens * topk, k, "bf16")
        X = dev.upload(xin.reshape(-1), "bf16")
        nrows = tokens * topk
        Y = dev.alloc_buffer(nrows * n, "bf16")
        for label, sorted_rows in (("unsorted", False), ("sorted", True)):
            rhs = (route[order] if sorted_rows else route).astype(np.uint32)
            lh = lhs[order] if sorted_rows else lhs
            if proj == "down":
                lh = None  # row r of the down projection reads its own hidden row
            R = dev.upload(rhs, "u32")
            L = dev.upload(lh.astype(np.uint32), "u32") if lh is not None else None

            def call(c, ws, L=L, R=R, sorted_rows=sorted_rows):
                kg.affine_gather_qmm(c, lib, X, *ws, L, R, Y, nrows, n, k, e, gs, bits,
                                     sorted_indices=sorted_rows, x_rows=xin.shape[0])

            par = None
            if O is not None:
                eager(lambda c: call(c, cps[0]))
                ref = O.gather_qmm_ref(xin, lh, rhs, *h0, nrows, n, k, gs, bits, "bf16", threads=ORACLE_THREADS)
                par = parity_entry(O.tolerance_report(Y.to_numpy().reshape(nrows, n), ref, xin, k, "bf16"))
            ms = time_graph(dev, max(10, steps // 2), args.warmup, lambda c, i: call(c, cps[i % len(cps)]))
            touched = len(np.unique(rhs))
            nb = touched * (n * k // 2 + 4 * n * (k // gs)) + nrows * k * 2 + nrows * n * 2
            tf = 2.0 * nrows * n * k / (ms * 1e-3) / 1e12
            res[f"cfg5_{proj}_{label}"] = {
                "shape": f"{nrows} rows x {e} experts W[{n},{k}] 4b gs64 bf16", "us": round(ms * 1e3, 2),
                "GB/s": round(nb / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(tf, 2), "experts_touched": touched, "copies": len(cps), "parity": par}
        del cps
    return res


def bench_ceiling(dev, args, rng, q=None):
    """HBM ceiling of one launch over the qmv config 2a bytes: a plain
    streaming read (cpq_stream_read) of the same kind of rotated copies
    (W, scales, biases, x), timed by the same graph method as the decode
    kernel.  Two grid sizes; the faster one is the ceiling."""
    import ctypes

    from cider_press_amd import _lib

    n, k, gs, bits, dtype = 12288, 4096, 64, 4, "bf16"
    if q is not None and q.get("copies"):
        copies, X = q["copies"], q["X"]
    else:
        copies, _ = make_copies(dev, rng, args.copies, n, k, gs, bits, dtype)
        from cider_press_amd.synthetic import make_x

        X = dev.upload(make_x(rng, 1, k, dtype).reshape(-1), dtype)
    sink = dev.alloc_buffer(1, "u32")
    L = _lib.lib()
    regs = []
    for W, S, B in copies:
        ptrs = (ctypes.c_void_p * 4)(W.ptr, S.ptr, B.ptr, X.ptr)
        lens = (ctypes.c_size_t * 4)(W.byte_len, S.byte_len, B.byte_len, X.byte_len)
        regs.append((ptrs, lens))
    nbytes = sum(int(v) for v in regs[0][1])
    out = {"what": "plain streaming read of the same rotated copies (W, scales, biases, x) in one launch per "
                   "step, same graph method as the decode kernel", "bytes_read": nbytes, "grids": {}}
    best = None
    for nwg in (768, 2048):
        def step(c, i, nwg=nwg):
            ptrs, lens = regs[i % len(regs)]
            _lib.check(L.cpq_stream_read(c.handle, ptrs, lens, 4, ctypes.c_void_p(sink.ptr), nwg))

        ms = time_graph(dev, args.steps, args.warmup, step)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out["grids"][str(nwg)] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1)}
        if best is None or gbs > best:
            best = gbs
    out["GB/s"] = round(best, 1)
    out["frac_of_peak"] = round(best / HBM_PEAK_GBS, 4)
    return out


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, budget_s):
    """Oracle dequantize-and-dot (T-rounded weights, fp32 accumulate) on the
    host: all-core and single-thread qmv GB/s at config 2a, and config 3a
    GFLOP/s on a row sample.  Uses the AVX-512 build where the host has it."""
    from oracle import oracle as O
    from cider_press_amd.synthetic import make_x

    n, k, gs, bits = q["shape"]
    w, s, b = q["host0"]
    threads = min(16, os.cpu_count() or 1)
    isa = O.baseline_isa()

    def timed(fn, seconds):
        fn()  # warm-up
        times, t0 = [], time.perf_counter()
        while time.perf_counter() - t0 < seconds and len(times) < 10000:
            t1 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t1)
        return float(np.median(times)), len(times)

    all_s, all_n = timed(lambda: O.cpu_baseline(q["x"], w, s, b, 1, n, k, gs, bits, "bf16", threads=threads),
                         budget_s * 0.5)
    one_s, one_n = timed(lambda: O.cpu_baseline(q["x"], w, s, b, 1, n, k, gs, bits, "bf16", threads=1),
                         budget_s * 0.25)
    # cfg3a (M=512, N=K=4096) on a sample of 32 activation rows x all 4096
    # output rows of copy 0's first 4096 rows: 2*32*4096*4096 FLOP per call.
    mq, nq = 32, 4096
    xq = make_x(np.random.default_rng(1), mq, k, "bf16")
    wq, sq, bq = w[:nq], s[:nq], b[:nq]
    qmm_s, qmm_n = timed(lambda: O.cpu_baseline(xq, wq, sq, bq, mq, nq, k, gs, bits, "bf16", threads=threads),
                         budget_s * 0.25)
    return {"value": round(q["bytes"] / all_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"qmv config 2a (N=12288, K=4096, 4-bit gs64, bf16), median of {all_n} calls "
                      f"over {budget_s * 0.5:.0f} s, {threads} threads, oracle C dequantize-and-dot ({isa})",
            "nproc": os.cpu_count(), "cpu_model": _cpu_model(), "isa": isa,
            "single_thread_GB/s": round(q["bytes"] / one_s / 1e9, 3), "single_thread_calls": one_n,
            "qmm_cfg3a_GFLOP/s": round(2.0 * mq * nq * k / qmm_s / 1e9, 2),
            "qmm_sample": f"config 3a shape on {mq} of its 512 activation rows (K=N=4096), median of {qmm_n} calls, "
                          f"{threads} threads"}


def bench_copy(args):
    """Calibration leg: torch's device copy of COPY_BYTES, five times."""
    import torch

    src = torch.randint(0, 2**31 - 1, (COPY_BYTES // 4,), dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 5
    return {"calibration": "device copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
            "ms": ms, "gbs": 2 * COPY_BYTES / (ms * 1e-3) / 1e9}


# Launch grids (threads) of the headline dispatches: qmv config 2a runs 768
# workgroups of 256 threads, qmm config 3a 256 workgroups of 512 threads (128
# output tiles of 128 x 128, K split in two).  The same kernels also serve the
# secondary configurations at other grids.
QMV_GRID = 768 * 256
QMM_GRID = 256 * 512


def _pmc_table(d):
    """Mean value per dispatch of every counter in a rocprofv3 --pmc run, by
    (kernel name, grid size): {counter: {(kernel, grid): (mean, dispatches)}}."""
    import csv
    import glob

    acc = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                key = (r["Kernel_Name"], int(r["Grid_Size"]))
                acc.setdefault(r["Counter_Name"], {}).setdefault(key, []).append(float(r["Counter_Value"]))
    return {c: {k: (sum(v) / len(v), len(v)) for k, v in t.items()} for c, t in acc.items()}


def _pmc_per_dispatch(d, counter):
    """Mean counter value (KiB) per dispatch, by (kernel name, grid size),
    from rocprofv3 CSV output."""
    return _pmc_table(d).get(counter, {})


def counter_summary(dirs, min_dispatches=20):
    """Markdown table of every counter of one or more --pmc runs, mean per
    dispatch, one row per (kernel, grid) seen in every run with at least
    `min_dispatches` dispatches (the benchmark's timed kernels, not set-up)."""
    tabs = {}
    for d in dirs:
        tabs.update(_pmc_table(d))
    keys = None
    for t in tabs.values():
        ks = {k for k, (_, n) in t.items() if n >= min_dispatches}
        keys = ks if keys is None else keys & ks
    cols = sorted(tabs)
    print("| kernel | grid | dispatches | " + " | ".join(cols) + " |")
    print("|---|---:|---:|" + "---:|" * len(cols))
    for k in sorted(keys or (), key=lambda kk: (kk[0], kk[1])):
        n = min(tabs[c][k][1] for c in cols)
        vals = " | ".join(f"{tabs[c][k][0]:.6g}" for c in cols)
        print(f"| `{k[0]}` | {k[1]} | {n} | {vals} |")


def trace_summary(d):
    """Per (kernel, grid) durations from a rocprofv3 --kernel-trace run."""
    import csv
    import glob

    acc = {}
    for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                acc.setdefault((r["Kernel_Name"], grid), []).append(dur)
    out = []
    for (name, grid), v in sorted(acc.items(), key=lambda kv: -sum(kv[1])):
        v.sort()
        out.append({"kernel": name, "grid": grid, "calls": len(v), "avg_ns": sum(v) / len(v), "min_ns": v[0],
                    "median_ns": v[len(v) // 2], "max_ns": v[-1]})
    print(json.dumps(out, indent=1))


def pmc_summary(fetch_dir, write_dir, cfetch_dir, cwrite_dir):
    """Scale FETCH_SIZE / WRITE_SIZE per dispatch by the copy calibration and
    write profiles/traffic.json."""

    def pick(tab, needle, grid):
        hits = [(k, v) for k, v in tab.items() if needle in k[0] and k[1] == grid]
        if not hits:
            raise SystemExit(f"no dispatch of a kernel matching {needle!r} at grid {grid}")
        (name, _), val = max(hits, key=lambda kv: kv[1][1])
        return name, val

    fetch, write = _pmc_per_dispatch(fetch_dir, "FETCH_SIZE"), _pmc_per_dispatch(write_dir, "WRITE_SIZE")
    cfetch, cwrite = _pmc_per_dispatch(cfetch_dir, "FETCH_SIZE"), _pmc_per_dispatch(cwrite_dir, "WRITE_SIZE")
    # The calibration copy is the kernel with the largest per-dispatch fetch.
    ckey = max(cfetch, key=lambda k: cfetch[k][0])
    kib = COPY_BYTES / 1024
    f_fac = kib / cfetch[ckey][0]
    w_fac = kib / cwrite[ckey][0]
    out = {"copy_kernel": ckey[0], "copy_fetch_kib": cfetch[ckey][0], "copy_write_kib": cwrite[ckey][0],
           "fetch_factor": f_fac, "write_factor": w_fac, "kernels": {}}
    for tag, needle, grid in (("qmv", QMV_KERNEL, QMV_GRID), ("qmm", QMM_KERNEL, QMM_GRID)):
        name, (fk, nd) = pick(fetch, needle, grid)
        wk = pick(write, needle, grid)[1][0]
        out["kernels"][tag] = {"kernel": name, "grid": grid, "dispatches": nd, "fetch_kib": fk, "write_kib": wk,
                               "traffic_bytes": int(round((fk * f_fac + wk * w_fac) * 1024))}
    os.makedirs(os.path.dirname(TRAFFIC_JSON), exist_ok=True)
    with open(TRAFFIC_JSON, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out, indent=1))


def load_traffic(tag, needle):
    try:
        with open(TRAFFIC_JSON) as fh:
            t = json.load(fh)["kernels"][tag]
    except (OSError, KeyError, ValueError):
        return None
    return t["traffic_bytes"] if needle in t["kernel"] else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--qmm-steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--only", choices=["qmv", "qmm", "all", "copy", "configs", "ceiling"], default="all")
    ap.add_argument("--no-configs", action="store_true", help="skip the cfg1/2b/3b/3c/4/5 table")
    ap.add_argument("--config-steps", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"))
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_DIR")
    ap.add_argument("--counter-summary", nargs="+", metavar="PMC_DIR")
    args = ap.parse_args()

    if args.counter_summary:
        counter_summary(args.counter_summary)
        return

    if args.trace_summary:
        trace_summary(args.trace_summary)
        return

    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return

    if args.gpus != 1:
        print(json.dumps({"error": f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
                                   "(the quantized-matmul path is measured on a single MI355X)"}))
        sys.exit(2)

    from cider_press_amd.kernels import Device, KernelLibrary

    if args.only == "copy":
        print(json.dumps(bench_copy(args)), flush=True)
        return

    dev = Device.system_default()
    lib = KernelLibrary.quantized(dev)
    info = dev.info()
    rng = np.random.default_rng(0)

    line = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded uniform nibbles, U(0.002,0.02) "
            "scales, biases=-8*scale, x~N(0,1))",
            "config": {"workload": "qmv config 2a: x[1,4096] . W[12288,4096]^T, 4-bit gs64, bf16, "
                                   f"{args.copies} rotated weight copies", "device": info["name"],
                       "cu_count": info["cu_count"]}}
    q = None
    if args.only == "ceiling":
        print(json.dumps(bench_ceiling(dev, args, rng)), flush=True)
        return
    if args.only in ("qmv", "all"):
        q = bench_qmv(dev, lib, args, rng)
        line["value"] = round(q["gbs"], 2)
        line["ms_per_step"] = q["ms"]
        line["roofline"] = {"bound": "hbm", "achieved": round(q["gbs"], 2), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(q["gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": load_traffic("qmv", QMV_KERNEL)}
        line["parity"] = {"qmv": q["parity"]}
        c = bench_ceiling(dev, args, rng, q)
        c["qmv_frac_of_ceiling"] = round(q["gbs"] / c["GB/s"], 4)
        line["ceiling"] = c
    if args.only in ("qmm", "all"):
        r = bench_qmm(dev, lib, args, rng)
        line["qmm"] = {"workload": "config 3a: X[512,4096] . W[4096,4096]^T, 4-bit gs64, bf16",
                       "value": round(r["tflops"], 2), "unit": "TFLOP/s", "steps": args.qmm_steps,
                       "ms_per_step": r["ms"],
                       "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                                    "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(r["tflops"] / BF16_MFMA_PEAK_TFLOPS, 4),
                                    "traffic": load_traffic("qmm", QMM_KERNEL)}}
        line.setdefault("parity", {})["qmm"] = r["parity"]
        if args.only == "qmm":
            line["metric"] = METRIC
            line["value"] = round(r["tflops"], 2)
            line["unit"] = "TFLOP/s"
            line["ms_per_step"] = r["ms"]
            line["steps"] = args.qmm_steps
            line["roofline"] = line["qmm"]["roofline"]
    if (args.only == "all" and not args.no_configs) or args.only == "configs":
        line["configs"] = bench_configs(dev, lib, args, rng)
    if q is not None and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(q, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
