"""Full-size parity of every workload bench.py times, through
the C ABI, against the CPU oracle.

Shape of the reference's own parity tests (crates/cider-press-kernels/tests/
qmm_parity.rs:22-87: upload, dispatch, commit_and_wait, compare against the
reference output), at the BASELINE shapes.  Bars: the BASELINE tolerance
(max|y-y_ref| <= 1e-2*||x||_inf*sqrt(K)/64 beyond the output's own rounding,
rel-L2 <= 2e-3) against the oracle's unrounded float64 output.

For the M = 2048 prefill shapes the oracle checks a row subset (two whole
128-row tiles plus every 7th row elsewhere, so every row position inside a
tile is covered) and the whole output is checked by size-independent
properties: finite everywhere, and bit-identical between an eager call and a
replay of the same call captured into a HIP graph (the kernel choice depends
on the shape and the session only).
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.kernels import gather as kg
from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.synthetic import from_bits, make_routing, make_weight, make_x

pytestmark = pytest.mark.gpu

THREADS = 16


def _up(device, w_q, s, b, dtype="bf16"):
    return (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), dtype),
            device.upload(b.reshape(-1), dtype))


def _check(oracle, y, ref, x, k, label, dtype="bf16"):
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], f"{label}: {rep}"


def _rows_subset(m):
    rows = set(range(0, min(m, 128))) | set(range(max(0, m - 128), m)) | set(range(0, m, 7))
    return np.array(sorted(rows))


def _prefill(device, library, oracle, m, n, k, seed, capture):
    rng = np.random.default_rng(seed)
    w_q, s, b = make_weight(rng, n, k, 64, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    W, S, B = _up(device, w_q, s, b)
    X = device.upload(x.reshape(-1), "bf16")
    Y = device.alloc_buffer(m * n, "bf16")
    cmds = device.commands()
    kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, 64, 4)
    cmds.commit_and_wait()
    y = Y.to_numpy().reshape(m, n)
    assert np.all(np.isfinite(from_bits(y, "bf16")))
    if capture:
        Yg = device.alloc_buffer(m * n, "bf16")
        cmds.begin_capture()
        kqmm.affine_qmm_t(cmds, library, W, S, B, X, Yg, m, n, k, 64, 4)
        g = cmds.end_capture()
        for _ in range(2):  # replays with the eager work above in between
            g.launch(cmds)
            cmds.commit_and_wait()
            assert np.array_equal(Yg.to_numpy().reshape(m, n), y), "graph replay differs from the eager call"
    rows = _rows_subset(m) if m > 512 else np.arange(m)
    ref = oracle.qmm_ref(x[rows], w_q, s, b, len(rows), n, k, 64, 4, "bf16", threads=THREADS)
    _check(oracle, y[rows], ref, x[rows], k, f"prefill {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k,capture", [
    (512, 12288, 4096, False),   # config 3b
    (2048, 4096, 4096, True),    # config 3c, N = 4096: eager and captured
    (2048, 12288, 4096, True),   # config 3c, N = 12288: eager and captured
])
def test_prefill_configs(device, library, oracle, m, n, k, capture):
    _prefill(device, library, oracle, m, n, k, m + n, capture)


@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (8, 64)])
@pytest.mark.parametrize("m", [4, 16, 64])
def test_config4_routed(device, library, oracle, m, bits, gs):
    """Config 4 through the runtime's routed op (eval.rs:1293-1394) at K = N = 4096."""
    n = k = 4096
    rng = np.random.default_rng(1000 * m + 10 * bits + gs)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    x = make_x(rng, m, k, "bf16")
    W, S, B = _up(device, w_q, s, b)
    X = device.upload(x.reshape(-1), "bf16")
    Y = device.alloc_buffer(m * n, "bf16")
    cmds = device.commands()
    kqmm.quantized_matmul(cmds, W, S, B, X, Y, m, n, k, gs, bits)
    cmds.commit_and_wait()
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16", threads=THREADS)
    _check(oracle, Y.to_numpy().reshape(m, n), ref, x, k, f"cfg4 m={m} {bits}b gs{gs}")


def _experts(rng, e, n, k):
    ws = [make_weight(rng, n, k, 64, 4, "bf16") for _ in range(e)]
    return tuple(np.concatenate([w[i] for w in ws]) for i in range(3))


@pytest.mark.parametrize("proj,sorted_rows", [("up", True), ("down", False), ("down", True)])
def test_config5_projections(device, library, oracle, proj, sorted_rows):
    """Config 5: 128 experts, 256 tokens routed top-8 without replacement.  The up
    projection reads token rows through lhs_indices; the down projection reads
    its own hidden row (lhs NULL), as in an MoE block."""
    e, tokens, top = 128, 256, 8
    n, k = (768, 2048) if proj == "up" else (2048, 768)
    rng = np.random.default_rng(5 + (proj == "down") + 2 * sorted_rows)
    w_q, s, b = _experts(rng, e, n, k)
    rows = tokens * top
    route = make_routing(rng, tokens, top, e).reshape(-1).astype(np.uint32)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), top)
    if sorted_rows:
        order = np.argsort(route, kind="stable")
        route, lhs = route[order], lhs[order]
    if proj == "down":
        lhs = None
        x = make_x(rng, rows, k, "bf16")
    else:
        x = make_x(rng, tokens, k, "bf16")
    X = device.upload(x.reshape(-1), "bf16")
    W, S, B = _up(device, w_q, s, b)
    L = None if lhs is None else device.upload(lhs, "u32")
    R = device.upload(route, "u32")
    Y = device.alloc_buffer(rows * n, "bf16")
    cmds = device.commands()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L, R, Y, rows, n, k, e, 64, 4, sorted_indices=sorted_rows,
                         x_rows=x.shape[0])
    cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, lhs, route, w_q, s, b, rows, n, k, 64, 4, "bf16", threads=THREADS)
    _check(oracle, Y.to_numpy().reshape(rows, n), ref, x, k, f"cfg5 {proj} sorted={sorted_rows}")


@pytest.mark.parametrize("n,k,gs", [
    (64, 29568, 32),   # a long down projection at decode: 924 groups per row
    (96, 40960, 32),   # 1280 groups per row
    (32, 40960, 64),
])
def test_qmv_long_rows(device, library, oracle, n, k, gs):
    """Rows whose per-row constants fit neither the decode kernel's LDS nor the
    small-M kernel's take a prefill kernel with M = 1 (no LDS constants)."""
    from cider_press_amd.kernels import qmv as kqmv

    rng = np.random.default_rng(k + gs)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, 1, k, "bf16")
    W, S, B = _up(device, w_q, s, b)
    X = device.upload(x.reshape(-1), "bf16")
    Y = device.alloc_buffer(n, "bf16")
    cmds = device.commands()
    kqmv.affine_qmv(cmds, library, W, S, B, X, Y, k, gs, 4)
    cmds.commit_and_wait()
    ref = oracle.qmm_ref(x, w_q, s, b, 1, n, k, gs, 4, "bf16")
    _check(oracle, Y.to_numpy().reshape(1, n), ref, x, k, f"qmv long K={k} gs{gs}")


def test_gather_unsupported_shape_rejected_before_launch(device, library):
    """A routed shape no kernel takes (2-bit, 1280 groups per row) is refused
    with InvalidArgument before anything is enqueued: y is untouched and the
    next wait reports nothing."""
    e, n, k, gs, rows = 2, 32, 40960, 32, 4
    W = device.alloc_buffer(e * n * k * 2 // 32, "u32")
    S = device.alloc_buffer(e * n * k // gs, "bf16")
    X = device.alloc_buffer(rows * k, "bf16")
    R = device.upload(np.array([0, 1, 7, 0], np.uint32), "u32")  # an out-of-range index, too
    Y = device.upload(np.full(rows * n, 0x3F80, np.uint16), "bf16")
    cmds = device.commands()
    with pytest.raises(_lib.InvalidArgument, match="groups per row"):
        kg.affine_gather_qmm(cmds, library, X, W, S, S, None, R, Y, rows, n, k, e, gs, 2)
    cmds.commit_and_wait()  # no stale status from a check kernel
    assert np.all(Y.to_numpy() == 0x3F80)
