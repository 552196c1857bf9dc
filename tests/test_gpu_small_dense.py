"""Small-M matmul through the dense form of the routed-decode kernel
(kernels/gather_decode.hip: rows in passes of 8, K in 128-element steps split
over the waves of a workgroup) and through the LDS-resident small-M kernel
(kernels/qmm_rows.hip), checked against the oracle through the C ABI.

affine_qmm_t sends a shape there when the tiled small-M kernel does not take
it (K not a multiple of 256) or would leave most CUs idle (few column tiles
and a K that does not split): the reference's own M = 39 benchmark shapes
(Qwen2.5-0.5B projections, K = 896 and the down projection's K = 4864) are
such shapes.  CPQ_SMALL_DENSE=1 forces the form for every shape it takes, so
the quantizations, group sizes, ragged N, one-step K and the pass boundaries
(M = 8, 9, 64) are covered here too.  affine_qmv sends rows of up to 1024
elements that its lean kernel does not take to the same form (M = 1).
"""
import numpy as np
import pytest

from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.kernels import qmv as kqmv
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _run(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype):
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), dtype),
               device.upload(b.reshape(-1), dtype))
    X = device.upload(x.reshape(-1), dtype)
    Y = device.upload(np.full(m * n, 0x7FC0, np.uint16), dtype)  # NaN fill: every output is written
    cmds = device.commands()
    kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, gs, bits)
    cmds.commit_and_wait()
    return Y.to_numpy().reshape(m, n)


def _check(oracle, y, x, w_q, s, b, m, n, k, gs, bits, dtype, label):
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype, threads=8)
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], (label, rep)


@pytest.mark.parametrize("n,k", [(896, 896), (128, 896), (4864, 896), (896, 4864)])
def test_reference_m39_shapes(device, library, oracle, n, k):
    """The reference's M = 39 prefill shapes on the default routing."""
    m, gs, bits, dtype = 39, 64, 4, "bf16"
    rng = np.random.default_rng(n + k)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    y = _run(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype)
    _check(oracle, y, x, w_q, s, b, m, n, k, gs, bits, dtype, f"M=39 N={n} K={k}")


@pytest.mark.parametrize("m,n,k,gs,bits,dtype", [
    (1, 512, 4096, 64, 4, "bf16"),
    (7, 224, 896, 64, 4, "bf16"),      # N not a multiple of 64: the last column group partly empty
    (8, 256, 2048, 32, 4, "f16"),      # one full pass
    (9, 256, 2048, 128, 8, "bf16"),    # a second pass of one row
    (39, 160, 4864, 64, 4, "bf16"),    # K of 38 steps: uneven wave ranges
    (64, 96, 1024, 64, 8, "f16"),      # the row limit, 8 passes
    (16, 32, 128, 32, 4, "bf16"),      # one step: waves without a K range
    (33, 4096, 4096, 64, 4, "bf16"),   # config 4's shape
    (5, 256, 960, 64, 4, "bf16"),      # K % 128 = 64: a half last step
    (3, 128, 96, 32, 8, "f16"),        # K below one step
    (12, 160, 992, 32, 4, "bf16"),     # K % 128 = 96
])
def test_forced_dense_form(device, library, oracle, monkeypatch, m, n, k, gs, bits, dtype):
    monkeypatch.setenv("CPQ_SMALL_DENSE", "1")
    rng = np.random.default_rng(m * 100 + n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    y = _run(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype)
    _check(oracle, y, x, w_q, s, b, m, n, k, gs, bits, dtype, f"dense {m}x{n}x{k} {bits}b gs{gs} {dtype}")


def test_forced_dense_deterministic_and_near_tiled(device, library, oracle, monkeypatch):
    """Same inputs, dense form vs the tiled small-M kernel: both accumulate in
    fp32 over the same dequantized weights (in different orders), so they
    agree to a couple of output ULPs; and the dense form is deterministic
    (two calls, same bits)."""
    m, n, k, gs = 24, 512, 4096, 64
    rng = np.random.default_rng(5)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    monkeypatch.setenv("CPQ_SMALL_DENSE", "1")
    y1 = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16")
    y2 = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16")
    assert np.array_equal(y1, y2)
    monkeypatch.setenv("CPQ_SMALL_DENSE", "0")
    y3 = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16")
    a, c = oracle.bits_to_f32(y1, "bf16"), oracle.bits_to_f32(y3, "bf16")
    assert np.max(np.abs(a - c)) <= 2 * 2.0 ** -7 * max(1.0, float(np.max(np.abs(c))))


def test_reference_lm_head_m39(device, library, oracle):
    """The reference's M = 39 lm_head shape (N = 151936, K = 896) on the
    default routing (the LDS-resident kernel), rows of every row block
    checked."""
    m, n, k, gs = 39, 151936, 896, 64
    rng = np.random.default_rng(151936)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    y = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16")
    rows = np.array([0, 1, 15, 16, 31, 32, 38])
    ref = oracle.qmm_ref(x[rows], w_q, s, b, len(rows), n, k, gs, 4, "bf16", threads=8)
    rep = oracle.tolerance_report(y[rows], ref, x[rows], k, "bf16")
    assert rep["ok"], rep


# The LDS-resident small-M kernel (kernels/qmm_rows.hip): all M rows of X in
# LDS, one workgroup per 128 columns, every dequantized slice feeding each
# 16-row block.  CPQ_SMALL_ROWS=1 forces it where it applies.
@pytest.mark.parametrize("m,n,k,gs,bits,dtype", [
    (39, 4096, 896, 64, 4, "bf16"),    # the lm_head shape's rows and K
    (1, 256, 128, 64, 4, "bf16"),      # one row, one step
    (16, 160, 896, 32, 4, "f16"),      # N not a multiple of 128: a partly empty workgroup
    (17, 512, 1024, 128, 8, "bf16"),   # a second row block of one row
    (64, 384, 512, 64, 4, "bf16"),     # the row limit, 64 KiB of activations
    (8, 512, 4096, 64, 4, "bf16"),     # 32 steps: four batches
    (33, 256, 1152, 64, 8, "f16"),     # 9 steps: a batch of 8 and a batch of 1
    (48, 128, 768, 32, 4, "bf16"),     # three full row blocks
])
def test_forced_rows_kernel(device, library, oracle, monkeypatch, m, n, k, gs, bits, dtype):
    monkeypatch.setenv("CPQ_SMALL_ROWS", "1")
    rng = np.random.default_rng(m * 1000 + n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    y = _run(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype)
    _check(oracle, y, x, w_q, s, b, m, n, k, gs, bits, dtype, f"rows {m}x{n}x{k} {bits}b gs{gs} {dtype}")


def test_rows_kernel_deterministic_and_graph_replay(device, library, monkeypatch):
    """Eager calls and replays of a captured call give the same bits."""
    monkeypatch.setenv("CPQ_SMALL_ROWS", "1")
    m, n, k, gs = 39, 1024, 896, 64
    rng = np.random.default_rng(12)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    first = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16")
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
               device.upload(b.reshape(-1), "bf16"))
    X = device.upload(x.reshape(-1), "bf16")
    Y = device.alloc_buffer(m * n, "bf16")
    cmds = device.commands()
    cmds.begin_capture()
    kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, gs, 4)
    gr = cmds.end_capture()
    for _ in range(3):
        Y.write(np.zeros(m * n, np.uint16))
        gr.launch(cmds)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy().reshape(m, n), first)
    gr.close()


@pytest.mark.parametrize("n,k,gs,bits,dtype", [
    (4864, 896, 64, 4, "bf16"),     # the reference's gate/up decode shape
    (151936, 896, 64, 4, "bf16"),   # its lm_head
    (1000, 1024, 128, 8, "f16"),    # 8-bit, N not a multiple of 16
    (96, 512, 32, 4, "bf16"),
    (256, 992, 32, 4, "bf16"),      # K % 128 = 96
])
def test_qmv_short_k_dense_route(device, library, oracle, monkeypatch, n, k, gs, bits, dtype):
    """affine_qmv on the dense form (default) and on its own kernels
    (CPQ_QMV_DENSE=0): both within the tolerance of the oracle."""
    rng = np.random.default_rng(n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, 1, k, dtype)
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), dtype),
               device.upload(b.reshape(-1), dtype))
    X = device.upload(x.reshape(-1), dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, 1, n, k, gs, bits, dtype, threads=8)
    for env in ("1", "0"):
        monkeypatch.setenv("CPQ_QMV_DENSE", env)
        Y = device.upload(np.full(n, 0x7FC0, np.uint16), dtype)
        cmds = device.commands()
        kqmv.affine_qmv(cmds, library, W, S, B, X, Y, k, gs, bits)
        cmds.commit_and_wait()
        rep = oracle.tolerance_report(Y.to_numpy().reshape(1, n), ref, x, k, dtype)
        assert rep["ok"], (env, rep)


@pytest.mark.parametrize("k_log,k_pads,gs", [(992, (1024,), 32), (640, (704, 768, 1024), 64)])
def test_qmv_short_k_padding_bit_exact(device, library, k_log, k_pads, gs):
    """K-padding contract on the short-K qmv route at more shapes: zero
    weights, scales and biases past the logical K and a zero activation tail
    give the unpadded output's bits."""
    rng = np.random.default_rng(k_log)
    n = 384
    w_q, s, b = make_weight(rng, n, k_log, gs, 4, "bf16")
    x = make_x(rng, 1, k_log, "bf16")

    def run(wq, ss, bb, k):
        W, S, B = (device.upload(wq.reshape(-1), "u32"), device.upload(ss.reshape(-1), "bf16"),
                   device.upload(bb.reshape(-1), "bf16"))
        xp = np.zeros(k, np.uint16); xp[:k_log] = x.reshape(-1)  # zero activation tail
        X = device.upload(xp, "bf16")
        Y = device.alloc_buffer(n, "bf16")
        cmds = device.commands()
        kqmv.affine_qmv(cmds, library, W, S, B, X, Y, k, gs, 4)
        cmds.commit_and_wait()
        return Y.to_numpy()

    base = run(w_q, s, b, k_log)
    for k in k_pads:
        wp = np.zeros((n, k * 4 // 32), np.uint32); wp[:, :w_q.shape[1]] = w_q
        sp = np.zeros((n, k // gs), np.uint16); sp[:, :s.shape[1]] = s
        bp = np.zeros((n, k // gs), np.uint16); bp[:, :b.shape[1]] = b
        assert np.array_equal(run(wp, sp, bp, k), base), k


# Scale / bias pairs outside the single-FMA dequantization's exactness range
# (a tiny scale under a much larger bias; an f16 subnormal scale), zero
# scales or biases (they fail the packed exponent check and pass the exact
# one) and a -0 bias under a negative scale (fails both).
_SLOW_SB = {"bf16": (0x3000, 0x3C23), "f16": (0x0001, 0x211F)}


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("form", ["rows", "dense"])
def test_small_forms_slow_and_zero_groups(device, library, oracle, monkeypatch, dtype, form):
    monkeypatch.setenv("CPQ_SMALL_ROWS" if form == "rows" else "CPQ_SMALL_DENSE", "1")
    m, n, k, gs = 20, 256, 896, 64
    rng = np.random.default_rng(21)
    w_q, s, b = make_weight(rng, n, k, gs, 4, dtype)
    s[17, 2], b[17, 2] = _SLOW_SB[dtype]
    s[200, k // gs - 1], b[200, k // gs - 1] = _SLOW_SB[dtype]
    s[5, 0] = 0
    b[40, 7] = 0
    s[90, 3], b[90, 3] = 0, 0
    s[131, 13] = s[131, 13] | 0x8000
    b[131, 13] = 0x8000
    x = make_x(rng, m, k, dtype)
    y = _run(device, library, w_q, s, b, x, m, n, k, gs, 4, dtype)
    _check(oracle, y, x, w_q, s, b, m, n, k, gs, 4, dtype, f"{form} slow/zero groups {dtype}")
