"""cpq_affine_qmm_t_noalloc: the prefill op on a caller's stream with a static
device scratch array instead of session scratch (no allocation).

Checked against cpq_affine_qmm_t on the same inputs: the no-alloc entry point
runs the kernel a default session runs, so the outputs are bit-identical.
Two calls in a row (the second smaller, so it reuses the array the first one
left behind), a split-K shape whose partial tiles use the array, a replayed
graph capture, and the refusal of a shape whose split needs more scratch than
the array holds.
"""
import ctypes

import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.kernels import _ptr
from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _noalloc(stream, W, S, B, X, Y, m, n, k, gs, bits):
    _lib.check(_lib.lib().cpq_affine_qmm_t_noalloc(
        ctypes.c_void_p(stream), _lib.DTYPES[S.dtype], _ptr(W), len(W), _ptr(S), len(S), _ptr(B), len(B), _ptr(X),
        len(X), _ptr(Y), len(Y), m, n, k, gs, bits))


def _case(device, library, rng, m, n, k, gs):
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
               device.upload(b.reshape(-1), "bf16"))
    X = device.upload(x.reshape(-1), "bf16")
    Y_ref, Y = device.alloc_buffer(m * n, "bf16"), device.alloc_buffer(m * n, "bf16")
    cmds = device.commands()
    kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y_ref, m, n, k, gs, 4)
    cmds.commit_and_wait()
    return W, S, B, X, Y, Y_ref, cmds


def test_noalloc_matches_session_op(device, library, oracle):
    rng = np.random.default_rng(77)
    # config 3a (K split 2: 16 MiB of partial tiles in the static array), then
    # a smaller split-K shape and an unsplit one, each bit-identical to the
    # session op; the smaller calls reuse what the first left in the array.
    for m, n, k, gs in ((512, 4096, 4096, 64), (256, 1024, 2048, 64), (96, 256, 1024, 32)):
        W, S, B, X, Y, Y_ref, cmds = _case(device, library, rng, m, n, k, gs)
        _noalloc(cmds.stream, W, S, B, X, Y, m, n, k, gs, 4)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy(), Y_ref.to_numpy()), (m, n, k)
        if m == 512:
            x = X.to_numpy().reshape(m, k)
            ref = oracle.qmm_ref(x, W.to_numpy().reshape(n, -1), S.to_numpy().reshape(n, -1),
                                 B.to_numpy().reshape(n, -1), m, n, k, gs, 4, "bf16", threads=16)
            rep = oracle.tolerance_report(Y.to_numpy().reshape(m, n), ref, x, k, "bf16")
            assert rep["ok"], rep


def test_noalloc_under_graph_capture(device, library):
    rng = np.random.default_rng(78)
    m, n, k, gs = 512, 2048, 4096, 64
    W, S, B, X, Y, Y_ref, cmds = _case(device, library, rng, m, n, k, gs)
    cmds.begin_capture()
    _noalloc(cmds.stream, W, S, B, X, Y, m, n, k, gs, 4)
    g = cmds.end_capture()
    for _ in range(3):
        Y.write(np.zeros(m * n, np.uint16))
        g.launch(cmds)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy(), Y_ref.to_numpy())


def test_noalloc_refuses_split_beyond_static_scratch(device, library):
    # K = 8192 at gs64 has 128 groups per row, more than one K range of the
    # prefill kernel takes, so a default session splits K over 2: 32 MiB of
    # partial tiles, more than the 16 MiB array.
    m, n, k, gs = 512, 8192, 8192, 64
    W = device.alloc_buffer(n * k // 8, "u32")
    S = device.alloc_buffer(n * k // gs, "bf16")
    X = device.alloc_buffer(m * k, "bf16")
    Y = device.upload(np.full(m * n, 0x3F80, np.uint16), "bf16")
    cmds = device.commands()
    with pytest.raises(_lib.BufferTooLarge, match="static scratch"):
        _noalloc(cmds.stream, W, S, S, X, Y, m, n, k, gs, 4)
    cmds.commit_and_wait()
    assert np.all(Y.to_numpy() == 0x3F80)
