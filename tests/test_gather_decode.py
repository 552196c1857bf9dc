"""Routed experts at decode shapes (up to 64 rows): one pass per distinct
expert over its weights (kernels/gather_decode.hip), checked against the
oracle's dense reduction row by row, through the C ABI.  (The per-slab
kernel keeps the shapes this kernel does not take; see test_gpu_parity.)

Covers 1, 2, 4 and 8 tokens x top-8 over 128 experts at config 5's up and
down shapes (sorted and unsorted routing), rows sharing an expert (more than
one pass of rows), 8-bit and f16, every group size, K ranges of several
batches, ragged N, the 64-row limit and the next kernel past it, and index
validation (out-of-range expert or activation row: zeroed, counted, the
other rows exact; a declared-sorted routing with a descent is reported).
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.kernels import gather as kg
from cider_press_amd.synthetic import make_routing, make_weight, make_x

pytestmark = pytest.mark.gpu


def _experts(rng, e, n, k, gs, bits, dtype):
    ws = [make_weight(rng, n, k, gs, bits, dtype) for _ in range(e)]
    return tuple(np.concatenate([w[i] for w in ws]) for i in range(3))


def _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, bits, dtype, sorted_idx=False, fill=None):
    rows = len(rhs)
    X = device.upload(x.reshape(-1), dtype)
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), dtype),
               device.upload(b.reshape(-1), dtype))
    L = None if lhs is None else device.upload(np.asarray(lhs, np.uint32), "u32")
    R = device.upload(np.asarray(rhs, np.uint32), "u32")
    Y = device.upload(np.full(rows * n, fill if fill is not None else 0, np.uint16), dtype)
    cmds = device.commands()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L, R, Y, rows, n, k, e, gs, bits, sorted_indices=sorted_idx,
                         x_rows=x.shape[0])
    return cmds, Y


def _check(oracle, y, ref, x, k, dtype, label):
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], (label, rep)


@pytest.mark.parametrize("tokens", [1, 2, 4, 8])
@pytest.mark.parametrize("proj", ["up", "down"])
@pytest.mark.parametrize("sorted_idx", [False, True])
def test_decode_config5_shapes(device, library, oracle, tokens, proj, sorted_idx):
    e, top, gs = 128, 8, 64
    n, k = (768, 2048) if proj == "up" else (2048, 768)
    rng = np.random.default_rng(100 + tokens + 7 * (proj == "down") + 3 * sorted_idx)
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = make_routing(rng, tokens, top, e).reshape(-1).astype(np.uint32)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), top)
    if sorted_idx:
        order = np.argsort(rhs, kind="stable")
        rhs, lhs = rhs[order], lhs[order]
    if proj == "down":
        lhs = None
        x = make_x(rng, len(rhs), k, "bf16")
    else:
        x = make_x(rng, tokens, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, 4, "bf16", sorted_idx)
    cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, len(rhs), n, k, gs, 4, "bf16", threads=8)
    _check(oracle, Y.to_numpy().reshape(len(rhs), n), ref, x, k, "bf16", f"decode {proj} t={tokens}")


def test_decode_shared_experts_many_passes(device, library, oracle):
    """40 of 64 rows on one expert (ten passes of 4 rows), the rest spread
    over three experts; one expert unused."""
    rng = np.random.default_rng(7)
    e, n, k, gs = 5, 96, 1024, 64
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = np.concatenate([np.full(40, 3), rng.choice([0, 1, 4], size=24)]).astype(np.uint32)
    rng.shuffle(rhs)
    lhs = rng.integers(0, 20, size=64).astype(np.uint32)
    x = make_x(rng, 20, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, 4, "bf16")
    cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, 64, n, k, gs, 4, "bf16")
    _check(oracle, Y.to_numpy().reshape(64, n), ref, x, k, "bf16", "shared experts")


@pytest.mark.parametrize("bits,gs,dtype,k,n,rows", [
    (8, 64, "bf16", 2048, 256, 12),
    (4, 32, "f16", 1024, 128, 12),
    (4, 128, "bf16", 4096, 64, 12),
    (8, 128, "f16", 768, 80, 12),     # ragged N: the last column block half empty
    (4, 64, "bf16", 16384, 32, 4),    # 16 steps per wave: two batches of loads
    (4, 32, "bf16", 128, 48, 12),     # one step: waves without a K range
])
def test_decode_quantizations_and_shapes(device, library, oracle, bits, gs, dtype, k, n, rows):
    rng = np.random.default_rng(bits * 1000 + gs + k + n)
    e = 9
    w_q, s, b = _experts(rng, e, n, k, gs, bits, dtype)
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    lhs = rng.integers(0, 3, size=rows).astype(np.uint32)
    x = make_x(rng, 3, k, dtype)
    cmds, Y = _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, bits, dtype)
    cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, rows, n, k, gs, bits, dtype)
    _check(oracle, Y.to_numpy().reshape(rows, n), ref, x, k, dtype, f"{bits}b gs{gs} {dtype} K={k}")


@pytest.mark.parametrize("rows", [64, 65])
def test_decode_row_limit_and_next_kernel(device, library, oracle, rows):
    """64 rows take the decode kernel, 65 the expert-major kernel: both exact
    to the tolerance on the same routing prefix."""
    rng = np.random.default_rng(64)
    e, n, k, gs = 16, 128, 1024, 64
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    x = make_x(rng, rows, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, None, rhs, n, k, e, gs, 4, "bf16")
    cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, None, rhs, w_q, s, b, rows, n, k, gs, 4, "bf16")
    _check(oracle, Y.to_numpy().reshape(rows, n), ref, x, k, "bf16", f"rows={rows}")


def test_decode_bad_indices_zeroed_and_counted(device, library, oracle):
    rng = np.random.default_rng(9)
    e, n, k, gs, rows, xr = 6, 64, 512, 64, 16, 4
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    lhs = rng.integers(0, xr, size=rows).astype(np.uint32)
    rhs[[2, 11]] = [e, 0xFFFFFFFF]
    lhs[[5, 15]] = [xr, 1000]
    bad = np.array([2, 5, 11, 15])
    x = make_x(rng, xr, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, 4, "bf16", fill=0x3F80)
    with pytest.raises(_lib.InvalidArgument, match="affine_gather_qmm: 4 row"):
        cmds.commit_and_wait()
    y = Y.to_numpy().reshape(rows, n)
    assert not y[bad].any()
    ok = np.setdiff1d(np.arange(rows), bad)
    ref = oracle.gather_qmm_ref(x, lhs[ok], rhs[ok], w_q, s, b, len(ok), n, k, gs, 4, "bf16")
    _check(oracle, y[ok], ref, x, k, "bf16", "valid rows")
    cmds.commit_and_wait()  # the failed wait cleared the status word


def test_decode_sorted_descent_reported(device, library, oracle):
    """A routing declared sorted with one descent is reported once; the
    outputs are still the gather's (this kernel does not rely on the order)."""
    rng = np.random.default_rng(10)
    e, n, k, gs, rows = 8, 32, 256, 64, 8
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = np.array([0, 1, 3, 2, 4, 5, 6, 7], np.uint32)
    x = make_x(rng, rows, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, None, rhs, n, k, e, gs, 4, "bf16", sorted_idx=True)
    with pytest.raises(_lib.InvalidArgument, match="affine_gather_qmm: 1 row"):
        cmds.commit_and_wait()
    ref = oracle.gather_qmm_ref(x, None, rhs, w_q, s, b, rows, n, k, gs, 4, "bf16")
    _check(oracle, Y.to_numpy().reshape(rows, n), ref, x, k, "bf16", "declared sorted")


def test_decode_repeat_calls_and_graph_replay_bit_equal(device, library):
    """Eager calls and replays of a captured call give the same bits."""
    rng = np.random.default_rng(11)
    e, n, k, gs, tokens, top = 32, 256, 1024, 64, 4, 8
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    rhs = make_routing(rng, tokens, top, e).reshape(-1).astype(np.uint32)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), top)
    x = make_x(rng, tokens, k, "bf16")
    cmds, Y = _run(device, library, x, w_q, s, b, lhs, rhs, n, k, e, gs, 4, "bf16")
    cmds.commit_and_wait()
    first = Y.to_numpy()
    X = device.upload(x.reshape(-1), "bf16")
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
               device.upload(b.reshape(-1), "bf16"))
    L, R = device.upload(lhs, "u32"), device.upload(rhs, "u32")
    Y2 = device.alloc_buffer(len(rhs) * n, "bf16")
    cmds.begin_capture()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L, R, Y2, len(rhs), n, k, e, gs, 4, x_rows=tokens)
    g = cmds.end_capture()
    for _ in range(3):
        Y2.write(np.zeros(len(rhs) * n, np.uint16))
        g.launch(cmds)
        cmds.commit_and_wait()
        assert np.array_equal(Y2.to_numpy(), first)
    g.close()
