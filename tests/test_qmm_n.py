"""affine_qmm_n / affine_qvm (MLX transpose=false, quantized.h:977-1086,
1215-1349): Y = X . dequant(W) with W logically [K, N] (packed along N,
groups along N).  The oracle dequantizes the [K, N] table exactly
(pinned bit-exact elsewhere) and multiplies in float64; the result must meet
the BASELINE tolerance.  Argument checks run on the CPU.
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.synthetic import from_bits, make_weight, make_x


def _check(m=4, n=256, k=512, gs=64, bits=4, dtype="bf16", **over):
    a = dict(w_q_len=k * n * bits // 32, s_len=k * n // gs, b_len=k * n // gs, x_len=m * k, y_len=m * n)
    a.update(over)
    return _lib.lib().cpq_check_qmm_n_args(_lib.DTYPES[dtype], a["w_q_len"], a["s_len"], a["b_len"], a["x_len"],
                                           a["y_len"], m, n, k, gs, bits)


def test_qmm_n_args():
    assert _check() == _lib.OK
    assert _check(m=0, y_len=0, x_len=0) == _lib.OK
    for bad in (dict(w_q_len=1), dict(s_len=3), dict(x_len=7), dict(y_len=9)):
        assert _check(**bad) == _lib.INVALID_ARGUMENT, bad
    assert _check(n=48, w_q_len=512 * 48 // 8, s_len=512 * 48 // 16, b_len=512 * 48 // 16, y_len=4 * 48,
                  gs=16) == _lib.INVALID_ARGUMENT      # N % 32 (and gs 16 unsupported)
    assert _check(k=500, w_q_len=500 * 256 // 8, s_len=500 * 4, b_len=500 * 4, x_len=4 * 500) == _lib.INVALID_ARGUMENT
    assert _check(dtype="f32") == _lib.KERNEL_NOT_FOUND


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,gs,bits,dtype", [
    (1, 4096, 4096, 64, 4, "bf16"),     # qvm at the decode shape (VALU decode kernel, K in parts)
    (1, 1024, 1000, 32, 8, "f16"),      # qvm, K not a multiple of the two-row step
    (1, 12288, 4096, 64, 4, "bf16"),    # qvm, wide N
    (1, 4128, 4096, 32, 4, "f16"),      # qvm, last column block partly past N; 129 groups a row
    (1, 2048, 96, 32, 8, "bf16"),       # qvm, one part
    (1, 96, 8192, 32, 4, "bf16"),       # qvm, one column block, many parts; 3 groups a row
    (1, 1024, 2048, 32, 3, "bf16"),     # qvm at 3 bits: the tiled kernel
    (5, 256, 512, 64, 4, "bf16"),
    (130, 352, 264, 32, 4, "bf16"),     # ragged M, N and K tiles
    (70, 384, 128, 128, 4, "bf16"),
    (64, 128, 256, 32, 2, "bf16"),
    (33, 96, 128, 32, 3, "f16"),
    (17, 160, 192, 32, 5, "bf16"),
    (40, 64, 320, 64, 6, "bf16"),
    (512, 1024, 1024, 64, 8, "bf16"),
])
def test_qmm_n_parity(device, library, oracle, m, n, k, gs, bits, dtype):
    from cider_press_amd.kernels import qmm as kqmm

    rng = np.random.default_rng(m + n + k + bits)
    w_q, s, b = make_weight(rng, k, n, gs, bits, dtype)  # [K, N] table: rows are k
    x = make_x(rng, m, k, dtype)
    W = device.upload(w_q.reshape(-1), "u32")
    S = device.upload(s.reshape(-1), dtype)
    B = device.upload(b.reshape(-1), dtype)
    X = device.upload(x.reshape(-1), dtype)
    Y = device.alloc_buffer(m * n, dtype)
    cmds = device.commands()
    if m == 1:
        kqmm.affine_qvm(cmds, library, W, S, B, X, Y, k, n, gs, bits)
    else:
        kqmm.affine_qmm_n(cmds, library, W, S, B, X, Y, m, n, k, gs, bits)
    cmds.commit_and_wait()
    y = Y.to_numpy()[: m * n].reshape(m, n)
    wd = from_bits(oracle.dequantize(w_q, s, b, k, n, gs, bits, dtype), dtype).astype(np.float64).reshape(k, n)
    ref = from_bits(x, dtype).astype(np.float64).reshape(m, k) @ wd
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], rep


@pytest.mark.gpu
def test_qmm_n_zero_k_writes_zeros(device):
    """K == 0: every output is the empty sum, 0 (zero-length inputs, C ABI)."""
    from cider_press_amd.kernels import _ptr

    Y = device.upload(np.full(3 * 64, 0x3f80, np.uint16), "bf16")
    cmds = device.commands()
    _lib.check(_lib.lib().cpq_affine_qmm_n(cmds.handle, _lib.DTYPES["bf16"], None, 0, None, 0, None, 0, None, 0,
                                           _ptr(Y), 3 * 64, 3, 64, 0, 64, 4))
    cmds.commit_and_wait()
    assert not Y.to_numpy()[: 3 * 64].any()


@pytest.mark.gpu
@pytest.mark.parametrize("rpt,parts", [(2, 1), (4, 3), (4, 16), (2, 64), (4, 5)])
def test_qvm_plans(device, library, oracle, monkeypatch, rpt, parts):
    """Every rows-per-thread step and K split of the decode kernel (forced
    through its tuning hooks) meets the tolerance, and repeated calls give
    identical bits: parts are added in part order whatever order they
    arrive in."""
    from cider_press_amd.kernels import qmm as kqmm

    monkeypatch.setenv("CPQ_QVM_RPT", str(rpt))
    monkeypatch.setenv("CPQ_QVM_PARTS", str(parts))
    n, k, gs, bits = 2080, 4000, 32, 4 if parts != 1 else 8
    rng = np.random.default_rng(rpt * 100 + parts)
    w_q, s, b = make_weight(rng, k, n, gs, bits, "bf16")
    x = make_x(rng, 1, k, "bf16")
    W, S, B, X = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
                  device.upload(b.reshape(-1), "bf16"), device.upload(x.reshape(-1), "bf16"))
    cmds = device.commands()
    ys = []
    for _ in range(3):
        Y = device.alloc_buffer(n, "bf16")
        kqmm.affine_qvm(cmds, library, W, S, B, X, Y, k, n, gs, bits)
        ys.append(Y)
    cmds.commit_and_wait()
    ys = [y.to_numpy()[:n] for y in ys]
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    wd = from_bits(oracle.dequantize(w_q, s, b, k, n, gs, bits, "bf16"), "bf16").astype(np.float64).reshape(k, n)
    ref = from_bits(x, "bf16").astype(np.float64).reshape(1, k) @ wd
    rep = oracle.tolerance_report(ys[0].reshape(1, n), ref, x, k, "bf16")
    assert rep["ok"], rep


@pytest.mark.gpu
def test_qvm_graph_replay_and_shared_counters(device, library, oracle):
    """qvm launches captured in a graph replay bit-equal to eager calls, and
    qvm and split-K small-M launches back to back on one session leave the
    shared arrival words zero for each other."""
    from cider_press_amd.kernels import qmm as kqmm

    rng = np.random.default_rng(5)
    n, k, gs = 4096, 4096, 64
    w_q, s, b = make_weight(rng, k, n, gs, 4, "bf16")
    x = make_x(rng, 1, k, "bf16")
    W, S, B, X = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
                  device.upload(b.reshape(-1), "bf16"), device.upload(x.reshape(-1), "bf16"))
    mw, ms, mb = make_weight(rng, 4096, 4096, 64, 4, "bf16")  # small-M operand, [N, K]
    mx = make_x(rng, 64, 4096, "bf16")
    MW, MS, MB, MX = (device.upload(mw.reshape(-1), "u32"), device.upload(ms.reshape(-1), "bf16"),
                      device.upload(mb.reshape(-1), "bf16"), device.upload(mx.reshape(-1), "bf16"))
    cmds = device.commands()
    Y0 = device.alloc_buffer(n, "bf16")
    kqmm.affine_qvm(cmds, library, W, S, B, X, Y0, k, n, gs, 4)
    cmds.commit_and_wait()
    y0 = Y0.to_numpy()[:n]
    Y, MY = device.alloc_buffer(n, "bf16"), device.alloc_buffer(64 * 4096, "bf16")
    cmds.begin_capture()
    kqmm.affine_qvm(cmds, library, W, S, B, X, Y, k, n, gs, 4)
    kqmm.quantized_matmul(cmds, MW, MS, MB, MX, MY, 64, 4096, 4096, 64, 4)
    kqmm.affine_qvm(cmds, library, W, S, B, X, Y, k, n, gs, 4)
    graph = cmds.end_capture()
    mref = oracle.qmm_ref(mx, mw, ms, mb, 64, 4096, 4096, 64, 4, "bf16")
    for _ in range(3):
        Y.write(np.zeros(n, np.uint16))
        graph.launch(cmds)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy()[:n], y0)
        assert oracle.tolerance_report(MY.to_numpy().reshape(64, 4096), mref, mx, 4096, "bf16")["ok"]
    wd = from_bits(oracle.dequantize(w_q, s, b, k, n, gs, 4, "bf16"), "bf16").astype(np.float64).reshape(k, n)
    ref = from_bits(x, "bf16").astype(np.float64).reshape(1, k) @ wd
    assert oracle.tolerance_report(y0.reshape(1, n), ref, x, k, "bf16")["ok"]
