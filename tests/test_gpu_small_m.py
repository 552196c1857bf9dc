"""GPU parity of the tiled small-M kernel (1 <= M <= 64 rows, 4- and 8-bit
weights, K a multiple of 256) that cpq_quantized_matmul runs below its
prefill threshold, against the CPU oracle (qmm_t_impl semantics,
kernels-mlx/mlx/backend/metal/kernels/quantized.h:1087-1213).

The cases cover each row-block count (M <= 16: one workgroup per 16 columns
over all of K; <= 32 and <= 64: K split over workgroups), K walked in
several chunks, K splits up to 16 parts per tile, a last column tile that is
partly past N, K slices with no unit, both activation types and every group
size; plus bit-identical results across calls and under graph replay."""
import numpy as np
import pytest

from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _routed(device, w_q, s, b, x, m, n, k, gs, bits, dtype, reps=1):
    W = device.upload(w_q.reshape(-1), "u32")
    S = device.upload(s.reshape(-1), dtype)
    B = device.upload(b.reshape(-1), dtype)
    X = device.upload(x.reshape(-1), dtype)
    outs = []
    cmds = device.commands()
    for _ in range(reps):
        Y = device.alloc_buffer(m * n, dtype)
        kqmm.quantized_matmul(cmds, W, S, B, X, Y, m, n, k, gs, bits)
        outs.append(Y)
    cmds.commit_and_wait()
    return [o.to_numpy().reshape(m, n) for o in outs], (W, S, B, X)


@pytest.mark.parametrize("m,n,k,bits,gs,dtype", [
    (2, 4096, 4096, 4, 64, "bf16"),     # one row block, all of K per workgroup
    (4, 4096, 4096, 4, 32, "bf16"),
    (16, 4096, 4096, 8, 64, "bf16"),
    (5, 1024, 8192, 4, 64, "f16"),      # K in two chunks
    (17, 2048, 4096, 4, 128, "bf16"),   # two row blocks, ragged, K split
    (32, 4096, 2048, 8, 32, "f16"),
    (33, 4096, 4096, 4, 64, "f16"),     # four row blocks
    (64, 4096, 4096, 4, 64, "bf16"),
    (64, 4128, 1024, 4, 64, "bf16"),    # last column tile half past N
    (48, 96, 4096, 8, 64, "bf16"),      # two tiles, K split 16
    (7, 160, 256, 4, 64, "bf16"),       # one unit: seven of eight K slices idle
    (9, 8192, 768, 4, 32, "f16"),       # three units
    (64, 12288, 2048, 8, 128, "bf16"),
])
def test_small_m_parity(device, oracle, m, n, k, bits, gs, dtype):
    rng = np.random.default_rng(m * 131 + n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    print(f"small-M m={m} n={n} k={k} bits={bits} gs={gs} {dtype}", flush=True)
    (y,), _ = _routed(device, w_q, s, b, x, m, n, k, gs, bits, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype)
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], rep


def test_small_m_deterministic_and_graph_replay(device, oracle):
    """The K parts are added in part order whatever order their workgroups
    finish in: repeated calls and graph replays give identical bits."""
    m, n, k, gs, bits = 64, 4096, 4096, 64, 4
    rng = np.random.default_rng(4096)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    x = make_x(rng, m, k, "bf16")
    ys, (W, S, B, X) = _routed(device, w_q, s, b, x, m, n, k, gs, bits, "bf16", reps=3)
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    cmds = device.commands()
    Y = device.alloc_buffer(m * n, "bf16")
    cmds.begin_capture()
    kqmm.quantized_matmul(cmds, W, S, B, X, Y, m, n, k, gs, bits)
    graph = cmds.end_capture()
    for _ in range(3):
        Y.write(np.zeros(m * n, np.uint16))
        graph.launch(cmds)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy().reshape(m, n), ys[0])
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16")
    assert oracle.tolerance_report(ys[0], ref, x, k, "bf16")["ok"]


def test_small_m_interleaved_shapes_keep_counters_clean(device, oracle):
    """Launches with different tile counts and splits, back to back on one
    session, share its split-K counters; each must leave them zero for the
    next."""
    rng = np.random.default_rng(77)
    cases = [(64, 4096, 4096, 64), (5, 96, 4096, 64), (40, 4096, 1024, 32), (64, 4096, 4096, 64)]
    cmds = device.commands()
    runs = []
    for m, n, k, gs in cases:
        w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
        x = make_x(rng, m, k, "bf16")
        bufs = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
                device.upload(b.reshape(-1), "bf16"), device.upload(x.reshape(-1), "bf16"))
        Y = device.alloc_buffer(m * n, "bf16")
        kqmm.quantized_matmul(cmds, *bufs, Y, m, n, k, gs, 4)
        runs.append((m, n, k, gs, w_q, s, b, x, bufs, Y))
    cmds.commit_and_wait()
    for m, n, k, gs, w_q, s, b, x, _, Y in runs:
        ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
        y = Y.to_numpy().reshape(m, n)
        assert oracle.tolerance_report(y, ref, x, k, "bf16")["ok"], (m, n, k, gs)


@pytest.mark.parametrize("m,n,k,bits,gs,dtype", [
    (2, 4096, 4096, 4, 64, "bf16"),
    (3, 2048, 8192, 4, 32, "f16"),
    (2, 1056, 16384, 8, 128, "bf16"),   # 16 steps per wave; N not a multiple of 64
    (8, 4096, 8192, 8, 128, "bf16"),
    (13, 4096, 4096, 4, 128, "f16"),
    (16, 12288, 4096, 4, 64, "bf16"),
    (16, 4096, 4096, 8, 64, "bf16"),
    (16, 4096, 4096, 4, 32, "bf16"),    # gs 32, 16 rows: (scale, bias) pairs in LDS, exact path
    (15, 4096, 4096, 4, 32, "bf16"),    # the same layout, single-FMA path
    (15, 2048, 4096, 8, 32, "f16"),
    (8, 4096, 4096, 8, 32, "bf16"),     # 8-bit, K = 4096, up to 8 rows: 4 waves of 8 steps
    (3, 2080, 4096, 8, 64, "f16"),      # the same, N not a multiple of 64
    (5, 4096, 4096, 8, 64, "bf16"),     # 8-bit, steps staged one at a time: a partial 4-row item, exact path
])
def test_decode_layout_rows_parity(device, oracle, m, n, k, bits, gs, dtype):
    """Up to 16 rows on the decode kernel's layout (K of 4096, 8192 or 16384):
    each wave stages M rows of its K range with the rows' slots swizzled.
    At gs 32 with 15 or 16 rows the group constants are kept as (scale,
    bias) pairs (the four-float form does not fit in LDS)."""
    rng = np.random.default_rng(m * 17 + n + k)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    if (bits == 4 and (gs == 64 or m == 16)) or (bits == 8 and m == 5):
        s[:, ::7] = 0  # zero scales: the per-group exact path inside one wave
    x = make_x(rng, m, k, dtype)
    print(f"decode rows m={m} n={n} k={k} bits={bits} gs={gs} {dtype}", flush=True)
    (y,), _ = _routed(device, w_q, s, b, x, m, n, k, gs, bits, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype)
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], rep


@pytest.mark.parametrize("m,n,k,bits,gs", [
    (5, 4096, 1024, 3, 64),     # widths other than 4 and 8
    (20, 2048, 2048, 5, 32),
    (40, 1024, 1024, 6, 128),
    (9, 4096, 896, 4, 64),      # K not a multiple of 256
    (33, 2048, 1152, 8, 128),
    (64, 8192, 512, 2, 32),
])
def test_slab_kernel_parity(device, oracle, m, n, k, bits, gs):
    """Shapes the tiled small-M kernels do not take run the slab kernel (one
    16-column slab of W per workgroup, up to 64 rows per pass)."""
    rng = np.random.default_rng(m * 5 + n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    x = make_x(rng, m, k, "bf16")
    (y,), _ = _routed(device, w_q, s, b, x, m, n, k, gs, bits, "bf16")
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16")
    rep = oracle.tolerance_report(y, ref, x, k, "bf16")
    assert rep["ok"], rep
