#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one GPU).

Headline metric: qmv HBM GB/s at K=4096 x N=12288, 4-bit gs64,
bf16 (config 2a) -> `value`; qmm TFLOP/s at M=512, N=K=4096 (config 3a) -> the
`qmm` object.  A "step" is one kernel call over one batch of synthetic input
already resident in HBM.

Timing method (every row):
  * weight copies are rotated so that the working set of each row is at
    least ROTATE_BYTES (512 MiB = 2 x the 256 MB Infinity Cache); copy c holds
    copy 0's packed words XOR a per-copy random word (uniform nibbles still)
    and copy 0's scales and biases;
  * `--steps` calls (S) are captured into one HIP graph and 2S calls into a
    second; each graph is replayed once untimed, then `reps` times (the two
    interleaved), each replay enqueued right behind a 512 MiB streaming read
    (cache flush) and bracketed by HIP events on the launch stream, with no
    host synchronisation in between: the host submits the replay while the
    GPU reads, so host submission is not in the window;
  * the figure is the marginal time of a step, (median T(2S) - median
    T(S)) / S: a graph replay carries a fixed cost (about 11 us here) that
    this removes, so the figure does not depend on S.  The fixed cost and the
    plain replay mean per step are reported beside it.
One command session serves the whole run.

    python bench.py [--steps K] [--warmup W] [--only qmv|qmm|configs|ceiling|dense|copy] [--no-cpu]
                    [--no-configs] [--no-graph]

`--no-graph` encodes the timed calls directly on the stream (no graph
capture); it is the form used for kernel traces of the whole table.

The line also carries: the single-launch streaming-read ceiling of the
headline bytes (best of several read designs and grids) and of every row's
bytes; the launch floor (a one-workgroup read of 16 bytes per step); a dense
bf16 GEMM anchor (torch.matmul, i.e. hipBLASLt, at the qmm shapes, same timing
method, measurement only); the configs table (cfg1, cfg2b, cfg3b/3c, 8-bit
prefill, cfg4 small-M sweep through the routed op, cfg5 routed experts incl.
decode-shaped routing, the reference's own Qwen2.5-0.5B decode and M=39
prefill shapes), each row checked against the oracle; and the CPU baseline.

HBM traffic (`roofline.traffic`) comes from rocprofv3 counter runs of this
same script, calibrated against a plain device copy of known size:

    rocprofv3 --pmc FETCH_SIZE -d D1 -o run --output-format csv -- python3 bench.py --no-configs --no-cpu
    rocprofv3 --pmc WRITE_SIZE -d D2 -o run --output-format csv -- python3 bench.py --no-configs --no-cpu
    rocprofv3 --pmc FETCH_SIZE -d D3 -o run --output-format csv -- python3 bench.py --only copy
    rocprofv3 --pmc WRITE_SIZE -d D4 -o run --output-format csv -- python3 bench.py --only copy
    python bench.py --pmc-summary D1 D2 D3 D4   # -> profiles/traffic.json
"""
from __future__ import annotations

import argparse
import ctypes
import json
import re
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
ROTATE_BYTES = 512 << 20       # per-row rotated working set: 2 x the 256 MB Infinity Cache
FLUSH_BYTES = 512 << 20        # streaming read before each timed replay
QMV_KERNEL = "qmv_lean_kernel<cpq::dev::BF16, 4"
QMM_KERNEL = "qmm_dma_kernel<cpq::dev::BF16"

# Published reference figures (Apple M4 Max, bf16, 4-bit gs64, effective
# GB/s by the same byte formula): docs/inference/quantized-matmul.md:121-153.
REF_QMV_SHAPES = (  # (K, N, label, x_len, published GB/s)
    (896, 4864, "gate/up_proj", 896, 306.0),
    (4864, 896, "down_proj", 4864, 272.0),
    (896, 151936, "lm_head", 896, 464.0),
    (896, 896, "q/o_proj", 896, 85.0),
    (896, 128, "k/v_proj", 896, 13.0),
    (1024, 896, "q/o_proj K-padded 896->1024", 896, 139.0),
    (1024, 128, "k/v_proj K-padded 896->1024", 896, 22.0),
)
# The reference's prefill benchmark shapes: Qwen2.5-0.5B at M = 39
# (crates/cider-press-kernels/tests/qmm_dispatch_bench.rs:33,150-159); no
# published figure.
REF_QMM_M = 39
REF_QMM_SHAPES = ((896, 896, "q_proj"), (896, 128, "k_proj"), (896, 896, "o_proj"), (896, 4864, "gate/up"),
                  (4864, 896, "down"), (896, 151936, "lm_head"))


def algo_bytes(m, n, k, gs, bits, tsize=2):
    """Reference byte formula (qmv_dispatch_bench.rs:37-43) extended to M rows."""
    return n * k * bits // 8 + 2 * n * (k // gs) * tsize + m * k * tsize + m * n * tsize


def copies_for(copy_bytes, target=ROTATE_BYTES):
    """Rotated copies so the working set is at least `target` bytes."""
    return int(max(2, -(-target // max(int(copy_bytes), 1))))


REPS_OVERRIDE = 0


def reps_for(steps):
    """Timed replays: at least 10, more for short graphs (or --reps)."""
    if REPS_OVERRIDE > 0:
        return REPS_OVERRIDE
    return int(max(10, min(100, 2000 // max(steps, 1))))


ORACLE_THREADS = min(16, os.cpu_count() or 1)


class Harness:
    """One command session for the whole run, the cache-flush buffer, event
    pairs and the graph timing method."""

    def __init__(self, dev, use_graph=True):
        from cider_press_amd import _lib

        self.dev = dev
        self.L = _lib.lib()
        self._check = _lib.check
        self.cmds = dev.commands()
        self.use_graph = use_graph
        self.flush_buf = dev.alloc_buffer(FLUSH_BYTES // 4, "u32")
        self.sink = dev.alloc_buffer(64, "u32")
        self._fp = (ctypes.c_void_p * 1)(self.flush_buf.ptr)
        self._fl = (ctypes.c_size_t * 1)(self.flush_buf.byte_len)
        self.events = []

    def sync(self):
        self.cmds.commit_and_wait()

    def eager(self, fn):
        fn(self.cmds)
        self.sync()

    def flush(self):
        """512 MiB streaming read: evicts the Infinity Cache and L2 and leaves
        only clean lines (nothing is written back inside a timed window)."""
        self._check(self.L.cpq_stream_read_variant(self.cmds.handle, self._fp, self._fl, 1,
                                                   ctypes.c_void_p(self.sink.ptr), 4096, 1))

    def stream_read(self, cmds, ptrs, lens, n, nwg, variant):
        self._check(self.L.cpq_stream_read_variant(cmds.handle, ptrs, lens, n, ctypes.c_void_p(self.sink.ptr),
                                                   nwg, variant))

    def _event_pairs(self, n):
        from cider_press_amd.kernels import Event

        while len(self.events) < n:
            self.events.append((Event(), Event()))
        return self.events[:n]

    def _capture(self, steps, encode_step):
        cmds = self.cmds
        cmds.begin_capture()
        try:
            for i in range(steps):
                encode_step(cmds, i)
        except BaseException:
            try:
                cmds.end_capture().close()
            except Exception:
                pass
            raise
        return cmds.end_capture()

    def time(self, encode_step, steps, warmup, reps=None):
        """Per-step time of `encode_step` as the marginal cost of a step: two
        graphs of S and 2S steps are replayed `reps` times each (interleaved,
        every replay behind the cache flush), and the per-step time is
        (median T(2S) - median T(S)) / S.  A graph replay carries a fixed cost
        of about 11 us on this device whatever it holds (launch of the graph,
        measured with one-step graphs); the difference removes it, so the
        figure does not depend on S.  The fixed cost and the plain replay
        mean per step are reported beside it."""
        reps = reps or reps_for(steps)
        cmds = self.cmds
        graphs = []
        try:
            runs = []
            for s in (steps, 2 * steps):
                if self.use_graph:
                    g = self._capture(s, encode_step)
                    graphs.append(g)
                    runs.append(lambda g=g: g.launch(cmds))
                else:
                    runs.append(lambda s=s: [encode_step(cmds, i) for i in range(s)])
            if warmup:
                if self.use_graph:
                    gw = self._capture(warmup, encode_step)
                    graphs.append(gw)
                    gw.launch(cmds)
                else:
                    for i in range(warmup):
                        encode_step(cmds, i)
            for run in runs:  # one untimed replay of each timed graph
                run()
            self.sync()
            pairs = self._event_pairs(2 * reps)
            for r in range(reps):
                for j, run in enumerate(runs):
                    e0, e1 = pairs[2 * r + j]
                    self.flush()
                    e0.record(cmds)
                    run()
                    e1.record(cmds)
            self.sync()
            t1 = sorted(pairs[2 * r][0].elapsed_ms(pairs[2 * r][1]) * 1e3 for r in range(reps))
            t2 = sorted(pairs[2 * r + 1][0].elapsed_ms(pairs[2 * r + 1][1]) * 1e3 for r in range(reps))
        finally:
            self.sync()
            for gr in graphs:
                gr.close()
        m1, m2 = t1[len(t1) // 2], t2[len(t2) // 2]
        per = (m2 - m1) / steps
        return {"us": per, "us_replay": m1 / steps, "fixed_us": m1 - per * steps,
                "us_min": (t2[0] - t1[0]) / steps, "us_max": (t2[-1] - t1[-1]) / steps, "reps": reps,
                "steps": steps}


class Rotation:
    """Rotated device copies of one quantized weight (or expert table): copy 0
    from the generator, copy c its packed words XOR a per-copy random word."""

    def __init__(self, dev, rng, n, k, gs, bits, dtype, bias_noise=0.0, copies=None):
        from cider_press_amd.synthetic import make_weight

        w, s, b = make_weight(rng, n, k, gs, bits, dtype, bias_noise=bias_noise)
        self.host0 = (w, s, b)
        self.copy_bytes = w.nbytes + s.nbytes + b.nbytes
        self.n_copies = copies or copies_for(self.copy_bytes)
        keys = rng.integers(1, 2**32, size=self.n_copies, dtype=np.uint64).astype(np.uint32)
        Sd = dev.upload(s.reshape(-1), dtype)
        Bd = dev.upload(b.reshape(-1), dtype)
        self.copies = []
        for c in range(self.n_copies):
            wc = w if c == 0 else (w ^ keys[c])
            # Scales and biases differ per copy in address only (same values:
            # the fast-dequantization vote sees the same constants).
            sc = Sd if c == 0 else dev.upload(s.reshape(-1), dtype)
            bc = Bd if c == 0 else dev.upload(b.reshape(-1), dtype)
            self.copies.append((dev.upload(wc.reshape(-1), "u32"), sc, bc))

    def __getitem__(self, i):
        return self.copies[i % self.n_copies]

    @property
    def working_set_mb(self):
        return round(self.n_copies * self.copy_bytes / 2**20, 1)


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


def _timing(t):
    return {"us": round(t["us"], 3), "us_replay": round(t["us_replay"], 3), "fixed_us": round(t["fixed_us"], 2),
            "reps": t["reps"]}


class Ceiling:
    """Single-launch streaming-read ceilings over rotated regions."""

    GRIDS = (768, 1024, 2048, 4096)

    def __init__(self, h):
        self.h = h
        self.best_variant = 1

    def _regs(self, regions_per_copy):
        regs = []
        for rs in regions_per_copy:
            ptrs = (ctypes.c_void_p * len(rs))(*[p for p, _ in rs])
            lens = (ctypes.c_size_t * len(rs))(*[n for _, n in rs])
            regs.append((ptrs, lens, len(rs)))
        return regs

    def measure(self, regions_per_copy, steps, warmup, variants=None, grids=None):
        """Best per-step time over (variant, grid) of a plain read of the same
        rotated regions, one launch per step."""
        regs = self._regs(regions_per_copy)
        variants = variants if variants is not None else (self.best_variant,)
        grids = grids or self.GRIDS
        table, best = {}, None
        for v in variants:
            for nwg in grids:
                def step(c, i, v=v, nwg=nwg):
                    ptrs, lens, n = regs[i % len(regs)]
                    self.h.stream_read(c, ptrs, lens, n, nwg, v)

                t = self.h.time(step, steps, warmup)
                table[f"v{v}_wg{nwg}"] = round(t["us"], 3)
                if best is None or t["us"] < best[0]:
                    best = (t["us"], v, nwg)
        return {"us": round(best[0], 3), "variant": best[1], "grid": best[2], "sweep_us": table}


def _wsb_regions(rot, x_buf=None):
    out = []
    for W, S, B in rot.copies:
        rs = [(W.ptr, W.byte_len), (S.ptr, S.byte_len), (B.ptr, B.byte_len)]
        if x_buf is not None:
            rs.append((x_buf.ptr, x_buf.byte_len))
        out.append(rs)
    return out


def bench_qmv(h, lib, args, rng, ceil):
    from cider_press_amd.kernels import qmv as kqmv
    from cider_press_amd.synthetic import make_x

    n, k, gs, bits, dtype = 12288, 4096, 64, 4, "bf16"
    rot = Rotation(h.dev, rng, n, k, gs, bits, dtype)
    x = make_x(rng, 1, k, dtype)
    X = h.dev.upload(x.reshape(-1), dtype)
    Y = h.dev.alloc_buffer(n, dtype)

    def step(cmds, i):
        kqmv.affine_qmv(cmds, lib, *rot[i], X, Y, k, gs, bits)

    parity = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

        h.eager(lambda c: step(c, 0))
        ref = O.qmm_ref(x, *rot.host0, 1, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
        parity = parity_entry(O.tolerance_report(Y.to_numpy().reshape(1, n), ref, x, k, dtype))
    t = h.time(step, args.steps, args.warmup)
    nbytes = algo_bytes(1, n, k, gs, bits)
    # Ceiling: every read design x grid over the same rotated bytes.
    c = ceil.measure(_wsb_regions(rot, X), args.steps, args.warmup,
                     variants=range(h.L.cpq_stream_read_variant_count()) if not args.no_ceiling else (1,),
                     grids=None if not args.no_ceiling else (1024,))
    ceil.best_variant = c["variant"]
    c["what"] = ("plain streaming read of the same rotated copies (W, scales, biases, x) in one launch per "
                 "step, best over read designs x grids")
    c["bytes_read"] = sum(int(nb) for _, nb in _wsb_regions(rot, X)[0])
    c["GB/s"] = round(c["bytes_read"] / (c["us"] * 1e-6) / 1e9, 1)
    c["frac_of_peak"] = round(c["GB/s"] / HBM_PEAK_GBS, 4)
    gbs = nbytes / (t["us"] * 1e-6) / 1e9
    c["qmv_frac_of_ceiling"] = round(gbs / c["GB/s"], 4)
    return {"t": t, "gbs": gbs, "bytes": nbytes, "parity": parity, "host0": rot.host0, "x": x,
            "shape": (n, k, gs, bits), "copies": rot.n_copies, "working_set_mb": rot.working_set_mb,
            "ceiling": c}


def bench_qmm(h, lib, args, rng):
    from cider_press_amd.kernels import qmm as kqmm
    from cider_press_amd.synthetic import make_x

    m, n, k, gs, bits, dtype = 512, 4096, 4096, 64, 4, "bf16"
    rot = Rotation(h.dev, rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    X = h.dev.upload(x.reshape(-1), dtype)
    Y = h.dev.alloc_buffer(m * n, dtype)

    def step(cmds, i):
        kqmm.affine_qmm_t(cmds, lib, *rot[i], X, Y, m, n, k, gs, bits)

    parity = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

        h.eager(lambda c: step(c, 0))
        ref = O.qmm_ref(x, *rot.host0, m, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
        parity = parity_entry(O.tolerance_report(Y.to_numpy().reshape(m, n), ref, x, k, dtype))
    t = h.time(step, args.qmm_steps, args.warmup)
    flops = 2.0 * m * n * k
    return {"t": t, "tflops": flops / (t["us"] * 1e-6) / 1e12, "flops": flops,
            "bytes": algo_bytes(m, n, k, gs, bits), "parity": parity, "copies": rot.n_copies,
            "working_set_mb": rot.working_set_mb}


def bench_dense(args, shapes=((512, 4096, 4096), (512, 12288, 4096), (2048, 4096, 4096), (2048, 12288, 4096))):
    """Dense anchor: torch.matmul in bf16 (hipBLASLt on ROCm) on X[M,K] . W[N,K]^T,
    rotated bf16 weights (>= 512 MiB), torch graph of `steps` calls, each timed
    replay behind a 512 MiB read, median of the replays.  Measurement only:
    nothing in the package uses it."""
    import torch

    dev = "cuda"
    steps = max(10, min(args.qmm_steps, 50))
    reps = 10
    rows = []
    s = torch.cuda.Stream()
    flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)
    g0 = torch.Generator(device=dev)
    g0.manual_seed(0)
    for m, n, k in shapes:
        wb = n * k * 2
        copies = copies_for(wb)
        X = torch.randn(m, k, device=dev, dtype=torch.bfloat16, generator=g0)
        W0 = (torch.randn(n, k, device=dev, dtype=torch.bfloat16, generator=g0) * 0.02)
        Ws = [W0] + [W0.clone() for _ in range(copies - 1)]
        Y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        with torch.cuda.stream(s):
            for i in range(3):
                torch.matmul(X, Ws[i % copies].t(), out=Y)
        torch.cuda.synchronize()
        gs_ = []
        for n_steps in (steps, 2 * steps):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for i in range(n_steps):
                    torch.matmul(X, Ws[i % copies].t(), out=Y)
            gs_.append(g)
        with torch.cuda.stream(s):
            for g in gs_:
                g.replay()
            ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in gs_]
                  for _ in range(reps)]
            for r in range(reps):
                for g, (e0, e1) in zip(gs_, ev[r]):
                    flush.sum()
                    e0.record(s)
                    g.replay()
                    e1.record(s)
        torch.cuda.synchronize()
        t1 = sorted(ev[r][0][0].elapsed_time(ev[r][0][1]) * 1e3 for r in range(reps))
        t2 = sorted(ev[r][1][0].elapsed_time(ev[r][1][1]) * 1e3 for r in range(reps))
        us = (t2[reps // 2] - t1[reps // 2]) / steps
        tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
        rows.append({"shape": f"X[{m},{k}] . W[{n},{k}]^T bf16", "m": m, "n": n, "k": k, "us": round(us, 3),
                     "us_replay": round(t1[reps // 2] / steps, 3), "TFLOP/s": round(tf, 1),
                     "mfma_frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "copies": copies, "steps": steps,
                     "reps": reps})
        del gs_, g
        del Ws, W0, X, Y
        torch.cuda.empty_cache()
    return {"what": f"torch {torch.__version__} bf16 matmul (hipBLASLt), dense weights, same graph + events method",
            "rows": rows}


def bench_configs(h, lib, args, rng, ceil):
    """The remaining configurations of the measurement table, each checked
    against the oracle (copy 0, one eager call) unless --no-parity, timed by
    the same method, with the single-launch read ceiling of the same bytes."""
    from cider_press_amd.kernels import gather as kg
    from cider_press_amd.kernels import qmm as kqmm
    from cider_press_amd.kernels import qmv as kqmv
    from cider_press_amd.synthetic import make_routing, make_x

    O = None
    if not args.no_parity:
        from oracle import oracle as O  # checker only

    steps, warm = args.config_steps, args.warmup
    res = {}
    pats = [p for p in (args.rows or "").split(",") if p]

    def want(name):
        return not pats or any(p in name for p in pats)

    def hbm(nb, us):
        gbs = nb / (us * 1e-6) / 1e9
        return round(gbs, 1), round(gbs / HBM_PEAK_GBS, 4)

    def with_ceiling(row, rot, x_buf, nb, regions=None):
        if args.no_ceiling:
            return row
        c = ceil.measure(regions or _wsb_regions(rot, x_buf), max(10, steps // 2), warm,
                         grids=(512, 1024, 2048, 4096))
        row["ceiling_us"] = c["us"]
        row["ceiling_GB/s"] = round(nb / (c["us"] * 1e-6) / 1e9, 1)
        row["frac_of_ceiling"] = round(c["us"] / row["us"], 4)
        return row

    def qmv_case(name, n, k, dtype, bias_noise=0.0, x_len=None, routed=False):
        gs, bits = 64, 4
        rot = Rotation(h.dev, rng, n, k, gs, bits, dtype, bias_noise)
        xl = x_len or k
        x = make_x(rng, 1, xl, dtype)
        X = h.dev.upload(x.reshape(-1), dtype)
        Y = h.dev.alloc_buffer(n, dtype)

        def call(c, i):
            kqmv.affine_qmv(c, lib, *rot[i], X, Y, k, gs, bits)

        par = None
        if O is not None:
            h.eager(lambda c: call(c, 0))
            xk = np.zeros((1, k), np.uint16)
            xk[:, :xl] = x
            ref = O.qmm_ref(xk, *rot.host0, 1, n, k, gs, bits, dtype, threads=ORACLE_THREADS)
            par = parity_entry(O.tolerance_report(Y.to_numpy().reshape(1, n), ref, xk, k, dtype))
        t = h.time(call, steps, warm)
        nb = algo_bytes(1, n, k, gs, bits)
        gbs, frac = hbm(nb, t["us"])
        row = {"shape": f"x[1,{xl}] . W[{n},{k}]^T 4b gs64 {dtype}", **_timing(t), "GB/s": gbs, "hbm_frac": frac,
               "copies": rot.n_copies, "working_set_MB": rot.working_set_mb, "parity": par}
        return with_ceiling(row, rot, X, nb)

    def qmm_case(name, m, n, k, bits=4, gs=64, routed=False):
        dtype = "bf16"
        rot = Rotation(h.dev, rng, n, k, gs, bits, dtype)
        x = make_x(rng, m, k, dtype)
        X = h.dev.upload(x.reshape(-1), dtype)
        Y = h.dev.alloc_buffer(m * n, dtype)

        def call(c, i):
            if routed:
                kqmm.quantized_matmul(c, *rot[i], X, Y, m, n, k, gs, bits)
            else:
                kqmm.affine_qmm_t(c, lib, *rot[i], X, Y, m, n, k, gs, bits)

        par = None
        if O is not None:
            h.eager(lambda c: call(c, 0))
            rows = check_rows(m)
            y = Y.to_numpy().reshape(m, n)
            ref = O.qmm_ref(x[rows], *rot.host0, len(rows), n, k, gs, bits, dtype, threads=ORACLE_THREADS)
            par = parity_entry(O.tolerance_report(y[rows], ref, x[rows], k, dtype), rows=len(rows))
            par["all_finite"] = bool(np.all(np.isfinite(O.bits_to_f32(y, dtype))))
        t = h.time(call, steps if m <= 64 else max(10, steps // 4), warm)
        nb = algo_bytes(m, n, k, gs, bits)
        tf = 2.0 * m * n * k / (t["us"] * 1e-6) / 1e12
        gbs, frac = hbm(nb, t["us"])
        row = {"shape": f"X[{m},{k}] . W[{n},{k}]^T {bits}b gs{gs} bf16", **_timing(t), "TFLOP/s": round(tf, 2),
               "mfma_frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "GB/s": gbs, "hbm_frac": frac,
               "copies": rot.n_copies, "working_set_MB": rot.working_set_mb, "parity": par}
        return row, rot, X, nb

    if want("cfg1"):
        res["cfg1"] = qmv_case("cfg1", 2048, 2048, "f16", bias_noise=1e-3)
    if want("cfg2b"):
        res["cfg2b"] = qmv_case("cfg2b", 4096, 12288, "bf16")
    for name, m, n, k, bits in (("cfg3b", 512, 12288, 4096, 4), ("cfg3c_n4096", 2048, 4096, 4096, 4),
                                ("cfg3c_n12288", 2048, 12288, 4096, 4), ("qmm_8bit_m512", 512, 4096, 4096, 8)):
        if want(name):
            row, _, _, _ = qmm_case(name, m, n, k, bits=bits)
            res[name] = row

    # cfg4: small M through the routed op (eval.rs routing), K = N = 4096.
    rows = []
    n = k = 4096
    for bits, gs in ((4, 64), (4, 32), (8, 64)):
        for m in (1, 4, 16, 64):
            if not want(f"cfg4_{bits}b_gs{gs}_m{m}"):
                continue
            row, rot, X, nb = qmm_case(f"cfg4_{bits}b_gs{gs}_m{m}", m, n, k, bits=bits, gs=gs, routed=True)
            row = {"bits": bits, "gs": gs, "m": m, **row}
            rows.append(with_ceiling(row, rot, X, nb))
            del rot
    if rows:
        res["cfg4"] = rows

    # cfg5: 128 experts, W_up [768, 2048] and W_down [2048, 768], 4b gs64;
    # 256 tokens routed top-8 (uniform, without replacement) -> 2048 rows;
    # decode-shaped routing: 1 and 4 tokens x top-8.
    e, topk = 128, 8
    for proj, (n, k) in (("up", (768, 2048)), ("down", (2048, 768))):
        gs, bits = 64, 4
        if not want(f"cfg5_{proj}") and not want(f"cfg5_decode_{proj}") and not any(
                want(f"cfg5_decode_t{t}_{proj}") for t in (1, 4)):
            continue
        rot = Rotation(h.dev, rng, e * n, k, gs, bits, "bf16")
        per_w, per_s = n * k // 8, n * (k // gs)
        for tokens in (256, 4, 1):
            route = make_routing(rng, tokens, topk, e).reshape(-1)
            lhs = np.repeat(np.arange(tokens, dtype=np.uint32), topk)
            order = np.argsort(route, kind="stable")
            xin = make_x(rng, tokens if proj == "up" else tokens * topk, k, "bf16")
            X = h.dev.upload(xin.reshape(-1), "bf16")
            nrows = tokens * topk
            Y = h.dev.alloc_buffer(nrows * n, "bf16")
            labels = (("unsorted", False), ("sorted", True)) if tokens == 256 else (("sorted", True),)
            for label, sorted_rows in labels:
                if not want(f"cfg5_{proj}_{label}" if tokens == 256 else f"cfg5_decode_t{tokens}_{proj}"):
                    continue
                rhs = (route[order] if sorted_rows else route).astype(np.uint32)
                lh = lhs[order] if sorted_rows else lhs
                if proj == "down":
                    lh = None  # row r of the down projection reads its own hidden row
                R = h.dev.upload(rhs, "u32")
                Lb = h.dev.upload(lh.astype(np.uint32), "u32") if lh is not None else None

                def call(c, i, Lb=Lb, R=R, sorted_rows=sorted_rows, X=X, Y=Y, nrows=nrows, xin=xin):
                    kg.affine_gather_qmm(c, lib, X, *rot[i], Lb, R, Y, nrows, n, k, e, gs, bits,
                                         sorted_indices=sorted_rows, x_rows=xin.shape[0])

                par = None
                if O is not None:
                    h.eager(lambda c: call(c, 0))
                    ref = O.gather_qmm_ref(xin, lh, rhs, *rot.host0, nrows, n, k, gs, bits, "bf16",
                                           threads=ORACLE_THREADS)
                    par = parity_entry(O.tolerance_report(Y.to_numpy().reshape(nrows, n), ref, xin, k, "bf16"))
                t = h.time(call, max(10, steps // 2), warm)
                touched = len(np.unique(rhs))
                nb = touched * (n * k // 2 + 4 * n * (k // gs)) + nrows * k * 2 + nrows * n * 2
                tf = 2.0 * nrows * n * k / (t["us"] * 1e-6) / 1e12
                gbs, frac = hbm(nb, t["us"])
                key = f"cfg5_{proj}_{label}" if tokens == 256 else f"cfg5_decode_t{tokens}_{proj}"
                row = {"shape": f"{tokens} tokens x top-{topk} -> {nrows} rows, {e} experts W[{n},{k}] 4b gs64 bf16",
                       **_timing(t), "GB/s": gbs, "hbm_frac": frac, "TFLOP/s": round(tf, 2),
                       "experts_touched": touched, "copies": rot.n_copies, "working_set_MB": rot.working_set_mb,
                       "parity": par}
                # Ceiling: a plain read of the same byte count (touched experts'
                # tables, contiguous) plus the activation rows.
                regs = [[(W.ptr, touched * per_w * 4), (S.ptr, touched * per_s * 2), (B.ptr, touched * per_s * 2),
                         (X.ptr, X.byte_len)] for W, S, B in rot.copies]
                res[key] = with_ceiling(row, rot, X, nb, regions=regs)
        del rot

    # The reference's own benchmark shapes (Qwen2.5-0.5B): decode qmv with its
    # published M4 Max figures beside ours, and M = 39 prefill.
    ref_rows = []
    for k, n, label, xl, pub in REF_QMV_SHAPES:
        if not want("reference_qmv"):
            break
        row = qmv_case(label, n, k, "bf16", x_len=xl)
        ref_rows.append({"label": label, **row, "reference_M4_Max_GB/s": pub,
                         "ratio_to_reference": round(row["GB/s"] / pub, 2)})
    if ref_rows:
        res["reference_qmv_qwen2.5_0.5b"] = ref_rows
    ref_rows = []
    for k, n, label in REF_QMM_SHAPES:
        if not want("reference_qmm"):
            break
        row, rot, X, nb = qmm_case(label, REF_QMM_M, n, k)
        ref_rows.append(with_ceiling({"label": label, **row}, rot, X, nb))
        del rot
    if ref_rows:
        res["reference_qmm_m39_qwen2.5_0.5b"] = ref_rows
    return res


def launch_floor(h, args):
    """Per-step time of a graph of one-workgroup, 16-byte reads: the launch
    cost any kernel here pays."""
    buf = h.dev.alloc_buffer(4, "u32")
    ptrs = (ctypes.c_void_p * 1)(buf.ptr)
    lens = (ctypes.c_size_t * 1)(16)
    t = h.time(lambda c, i: h.stream_read(c, ptrs, lens, 1, 1, 0), args.steps, args.warmup)
    return {"what": "one workgroup reading 16 bytes per step, same graph method", **_timing(t)}


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
    """Host dequantize-and-dot (T-rounded weights, fp32 accumulate), each form
    of oracle/cpu_baseline.c that the host runs (scalar, AVX2, AVX-512): qmv
    config 2a GB/s on all cores and one core, and config 3a GFLOP/s on a row
    sample.  `value` is the fastest all-core form."""
    from oracle import oracle as O
    from cider_press_amd.synthetic import make_x

    n, k, gs, bits = q["shape"]
    w, s, b = q["host0"]
    threads = min(16, os.cpu_count() or 1)
    forms = O.baseline_forms()

    def timed(fn, seconds):
        fn()  # warm-up
        times, t0 = [], time.perf_counter()
        while time.perf_counter() - t0 < seconds and len(times) < 10000:
            t1 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t1)
        return float(np.median(times)), len(times)

    per_form = {}
    share = budget_s / max(1, len(forms))
    mq, nq = 32, 4096
    xq = make_x(np.random.default_rng(1), mq, k, "bf16")
    wq, sq, bq = w[:nq], s[:nq], b[:nq]
    for form in forms:
        all_s, all_n = timed(lambda: O.cpu_baseline(q["x"], w, s, b, 1, n, k, gs, bits, "bf16", threads=threads,
                                                    form=form), share * 0.45)
        one_s, one_n = timed(lambda: O.cpu_baseline(q["x"], w, s, b, 1, n, k, gs, bits, "bf16", threads=1,
                                                    form=form), share * 0.3)
        qmm_s, qmm_n = timed(lambda: O.cpu_baseline(xq, wq, sq, bq, mq, nq, k, gs, bits, "bf16", threads=threads,
                                                    form=form), share * 0.25)
        per_form[form] = {"GB/s": round(q["bytes"] / all_s / 1e9, 3), "calls": all_n,
                          "single_thread_GB/s": round(q["bytes"] / one_s / 1e9, 3), "single_thread_calls": one_n,
                          "qmm_cfg3a_GFLOP/s": round(2.0 * mq * nq * k / qmm_s / 1e9, 2), "qmm_calls": qmm_n}
    best = max(per_form, key=lambda f: per_form[f]["GB/s"])
    return {"value": per_form[best]["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"qmv config 2a (N=12288, K=4096, 4-bit gs64, bf16), median over about "
                      f"{share * 0.45:.0f} s of calls, {threads} threads, {best} form of the C dequantize-and-dot "
                      f"(oracle/cpu_baseline.c); config 3a sampled on {mq} of its 512 activation rows",
            "form": best, "forms": per_form, "nproc": os.cpu_count(), "cpu_model": _cpu_model()}


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


def _short_kernel(name):
    name = re.sub(r"\((unsigned|cpq::).*$", "", name)
    return name.replace("void cpq::(anonymous namespace)::", "").replace("cpq::dev::", "")


def counter_summary(dirs, min_dispatches=20, per_wave=False):
    """Markdown table of every counter of one or more --pmc runs, mean per
    dispatch, one row per (kernel, grid) seen in every run with at least
    `min_dispatches` dispatches (the benchmark's timed kernels, not set-up).
    per_wave: the per-wave figures instead (quad-cycle counters x 4,
    SQ_BUSY_CYCLES / 32 shader engines, MFMA busy and co-issue / 1024 SIMDs)."""
    tabs = {}
    for d in dirs:
        tabs.update(_pmc_table(d))
    keys = None
    for t in tabs.values():
        ks = {k for k, (_, n) in t.items() if n >= min_dispatches}
        keys = ks if keys is None else keys & ks
    keys = sorted(keys or (), key=lambda kk: (kk[0], kk[1]))
    if per_wave:
        print("| kernel | grid | waves | wave life (cyc) | busy (cyc) | VALU instr / wave | MFMA / wave | "
              "s_waitcnt stall / wave (cyc) | VALU active / wave (cyc) | MFMA busy / SIMD (cyc) | "
              "VALU+MFMA co-issue / SIMD (cyc) | FETCH_SIZE (KiB) | LDS bank conflicts |")
        print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
        for k in keys:
            if k[0].startswith("__amd"):
                continue
            v = lambda c: tabs.get(c, {}).get(k, (float("nan"), 0))[0]
            w = v("SQ_WAVES")
            row = [w, v("SQ_WAVE_CYCLES") * 4 / w, v("SQ_BUSY_CYCLES") / 32, v("SQ_INSTS_VALU") / w,
                   v("SQ_INSTS_MFMA") / w, v("SQ_WAIT_INST_ANY") * 4 / w, v("SQ_ACTIVE_INST_VALU") * 4 / w,
                   v("SQ_VALU_MFMA_BUSY_CYCLES") / 1024, v("SQ_VALU_MFMA_COEXEC_CYCLES") / 1024, v("FETCH_SIZE"),
                   v("SQ_LDS_BANK_CONFLICT")]
            print(f"| `{_short_kernel(k[0])}` | {k[1]} | " + " | ".join(f"{x:.0f}" for x in row) + " |")
        return
    cols = sorted(tabs)
    print("| kernel | grid | dispatches | " + " | ".join(cols) + " |")
    print("|---|---:|---:|" + "---:|" * len(cols))
    for k in keys:
        n = min(tabs[c][k][1] for c in cols)
        vals = " | ".join(f"{tabs[c][k][0]:.6g}" for c in cols)
        print(f"| `{k[0]}` | {k[1]} | {n} | {vals} |")


# The bench row each traced (kernel name fragment, launch grid in threads)
# belongs to, for the markdown form of --trace-summary.
TRACE_WORKLOADS = (
    ("qmv_lean_kernel<cpq::dev::BF16, 4, 6, 4, 8, true, false>", 196608, "**cfg2a qmv** (headline)"),
    ("qmv_lean_kernel<cpq::dev::BF16, 4, 6, 12, 8, true, false>", 196608, "cfg2b qmv"),
    ("qmv_lean_kernel<cpq::dev::F16, 4, 6, 4, 4, true, false>", 32768, "cfg1 qmv (f16)"),
    ("qmm_dma_kernel", 131072, "**cfg3a qmm** (headline)"),
    ("qmm_dma_kernel", 196608, "cfg3b"),
    ("qmm_dma_kernel", 262144, "cfg3c N=4096"),
    ("qmm_dma_kernel", 786432, "cfg3c N=12288"),
    ("qmm_staged_kernel<cpq::dev::BF16, 8", 65536, "8-bit prefill M=512"),
    ("qmv_lean_kernel<cpq::dev::BF16, 4, 6, 4, 8, true, false>", 65536, "cfg4 4b gs64 M=1"),
    ("qmv_lean_kernel<cpq::dev::BF16, 4, 5, 4, 8, true, false>", 65536, "cfg4 4b gs32 M=1"),
    ("qmv_lean_kernel<cpq::dev::BF16, 8, 6, 4, 8, true, false>", 65536, "cfg4 8b M=1"),
    ("qmm_lean_rows_kernel<cpq::dev::BF16, 4, 6, 8, 4, false, 16>", 131072, "cfg4 4b gs64 M=4, M=16"),
    ("qmm_lean_rows_kernel<cpq::dev::BF16, 4, 5, 8, 4, false, 16>", 131072, "cfg4 4b gs32 M=4"),
    ("qmm_lean_rows_kernel<cpq::dev::BF16, 4, 5, 8, 4, false, 8>", 131072, "cfg4 4b gs32 M=16"),
    ("qmm_lean_rows_kernel<cpq::dev::BF16, 8, 6, 4, 8, false, 16>", 65536, "cfg4 8b M=4"),
    ("qmm_lean_rows_kernel<cpq::dev::BF16, 8, 6, 8, 4, false, 16>", 131072, "cfg4 8b M=16"),
    ("qmm_small_kernel<cpq::dev::BF16, 4, 4>", 131072, "cfg4 4b M=64 (gs64 and gs32)"),
    ("qmm_small_kernel<cpq::dev::BF16, 8, 4>", 131072, "cfg4 8b M=64"),
    ("gather_expert_kernel", 131072, "cfg5 prefill up / down (sorted + unsorted)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, false, true>", 98304, "cfg5 decode 1 token, up"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 2, false, true>", 131072, "cfg5 decode 1 token, down"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 2, false, true>", 196608, "cfg5 decode 4 tokens, up"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 1, false, true>", 262144, "cfg5 decode 4 tokens, down"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 1, true, true>", 607744, "reference qmv lm_head (K=896; dense form, M=1)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, true, true>", 77824, "reference qmv gate/up (K=896; dense form, M=1)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, true, true>", 14336, "reference qmv q/o, its K-padded twin (dense form, M=1)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, true, true>", 2048, "reference qmv k/v, its K-padded twin (dense form, M=1)"),
    ("qmv_kernel<cpq::dev::BF16, 4, 8, 4, false>", 28672, "reference qmv down (K=4864)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, true, true>", 71680, "reference M=39 q, o (K=896) and down (K=4864) (dense form)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 4, true, true>", 10240, "reference M=39 k_proj (dense form)"),
    ("gather_decode_kernel<cpq::dev::BF16, 4, 2, true, true>", 194560, "reference M=39 gate/up (dense form)"),
    ("qmm_rows_kernel<cpq::dev::BF16, 4, 3, true>", 607744, "reference M=39 lm_head (activations in LDS)"),
    ("stream_read_kernel<256, 8, false, false>", 1048576, "cache flush (512 MiB read) before each timed replay"),
    ("stream_read_kernel<256, 8, false, false>", 262144, "read ceiling leg"),
    ("stream_read_kernel<256, 4, false, false>", 256, "launch floor (one workgroup, 16 B)"),
)


def trace_summary(d, markdown=False):
    """Per (kernel, grid) durations from a rocprofv3 --kernel-trace run: JSON,
    or a markdown table with each row's bench workload (TRACE_WORKLOADS)."""
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
    if not markdown:
        print(json.dumps(out, indent=1))
        return
    print("| workload | kernel | grid (threads) | calls | avg ns | median ns | min ns | max ns |")
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for r in out:
        if r["calls"] < 3:
            continue
        lab = next((l for frag, g, l in TRACE_WORKLOADS if frag in r["kernel"] and r["grid"] == g), "")
        print(f"| {lab} | `{_short_kernel(r['kernel'])}` | {r['grid']} | {r['calls']} | {r['avg_ns']:.0f} | "
              f"{r['median_ns']} | {r['min_ns']} | {r['max_ns']} |")


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
    ap.add_argument("--only", choices=["qmv", "qmm", "all", "copy", "configs", "ceiling", "dense"], default="all")
    ap.add_argument("--no-configs", action="store_true", help="skip the configs table")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense bf16 GEMM anchor")
    ap.add_argument("--no-graph", action="store_true", help="encode timed calls directly (no graph capture)")
    ap.add_argument("--reps", type=int, default=0, help="timed replays per timing (0: by step count)")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the read-ceiling legs (kernel traces)")
    ap.add_argument("--rows", default="", help="configs rows to run: comma-separated name substrings")
    ap.add_argument("--config-steps", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"))
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_DIR")
    ap.add_argument("--markdown", action="store_true", help="with --trace-summary: markdown table by workload")
    ap.add_argument("--counter-summary", nargs="+", metavar="PMC_DIR")
    ap.add_argument("--per-wave", action="store_true", help="with --counter-summary: per-wave figures")
    args = ap.parse_args()

    if args.counter_summary:
        counter_summary(args.counter_summary, per_wave=args.per_wave)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, markdown=args.markdown)
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return

    global REPS_OVERRIDE
    REPS_OVERRIDE = args.reps
    if args.gpus != 1:
        print(json.dumps({"error": f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
                                   "(the quantized-matmul path is measured on a single MI355X)"}))
        sys.exit(2)

    if args.only == "copy":
        print(json.dumps(bench_copy(args)), flush=True)
        return
    if args.only == "dense":
        print(json.dumps(bench_dense(args)), flush=True)
        return

    # The dense anchor runs in a child process started before this process
    # touches the GPU: torch's ROCm build carries its own HIP runtime, which
    # does not see the device once the system runtime libcpq.so links has
    # opened it in the same process.
    dense = None
    if args.only == "all" and not args.no_dense:
        import subprocess

        cmd = [sys.executable, os.path.abspath(__file__), "--only", "dense", "--qmm-steps", str(args.qmm_steps)]
        # Run to completion first: the two processes must not share the GPU
        # while either one times.
        dense = subprocess.run(cmd, capture_output=True, text=True, timeout=600)

    from cider_press_amd.kernels import Device, KernelLibrary

    dev = Device.system_default()
    lib = KernelLibrary.quantized(dev)
    info = dev.info()
    rng = np.random.default_rng(0)
    h = Harness(dev, use_graph=not args.no_graph)
    ceil = Ceiling(h)

    line = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded uniform nibbles, U(0.002,0.02) "
            "scales, biases=-8*scale, x~N(0,1))",
            "config": {"workload": "qmv config 2a: x[1,4096] . W[12288,4096]^T, 4-bit gs64, bf16",
                       "device": info["name"], "cu_count": info["cu_count"],
                       "timing": "median of timed graph replays, each behind a 512 MiB read, no host sync between"
                                 if h.use_graph else "eager launches between events (no graph)"}}
    q = None
    if args.only in ("qmv", "all", "ceiling"):
        q = bench_qmv(h, lib, args, rng, ceil)
        line["value"] = round(q["gbs"], 2)
        line["ms_per_step"] = q["t"]["us"] * 1e-3
        line["config"]["copies"] = q["copies"]
        line["config"]["working_set_MB"] = q["working_set_mb"]
        line["timing"] = _timing(q["t"])
        line["roofline"] = {"bound": "hbm", "achieved": round(q["gbs"], 2), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(q["gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": load_traffic("qmv", QMV_KERNEL)}
        line["parity"] = {"qmv": q["parity"]}
        line["ceiling"] = q["ceiling"]
        line["launch_floor"] = launch_floor(h, args)
        if args.only == "ceiling":
            print(json.dumps(line), flush=True)
            return
    if args.only in ("qmm", "all"):
        r = bench_qmm(h, lib, args, rng)
        line["qmm"] = {"workload": "config 3a: X[512,4096] . W[4096,4096]^T, 4-bit gs64, bf16",
                       "value": round(r["tflops"], 2), "unit": "TFLOP/s", "steps": args.qmm_steps,
                       "ms_per_step": r["t"]["us"] * 1e-3, "timing": _timing(r["t"]), "copies": r["copies"],
                       "working_set_MB": r["working_set_mb"],
                       "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                                    "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(r["tflops"] / BF16_MFMA_PEAK_TFLOPS, 4),
                                    "traffic": load_traffic("qmm", QMM_KERNEL)}}
        line.setdefault("parity", {})["qmm"] = r["parity"]
        if args.only == "qmm":
            line["value"] = round(r["tflops"], 2)
            line["unit"] = "TFLOP/s"
            line["ms_per_step"] = r["t"]["us"] * 1e-3
            line["steps"] = args.qmm_steps
            line["roofline"] = line["qmm"]["roofline"]
    if dense is not None:
        out, err = dense.stdout, dense.stderr
        js = [ln for ln in out.splitlines() if ln.startswith("{")]
        if dense.returncode == 0 and js:
            d = json.loads(js[-1])
            line["dense_anchor"] = d
            if "qmm" in line:
                d0 = d["rows"][0]
                line["qmm"]["dense_anchor_TFLOP/s"] = d0["TFLOP/s"]
                line["qmm"]["vs_dense_anchor"] = round(line["qmm"]["value"] / d0["TFLOP/s"], 3)
        else:  # the anchor is optional measurement
            line["dense_anchor"] = {"error": f"rc={dense.returncode}: {err[-400:]}"}
    if (args.only == "all" and not args.no_configs) or args.only == "configs":
        line["configs"] = bench_configs(h, lib, args, rng, ceil)
    if q is not None and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(q, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
