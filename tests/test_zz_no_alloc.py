"""cpq_affine_qmm_t_noalloc: the prefill op on a caller's stream with a static
device scratch array instead of session scratch (no allocation).

Checked against cpq_affine_qmm_t on the same inputs: where the default
session's K split fits the static array the no-alloc entry point runs the
same kernel, so the outputs are bit-identical.  Two calls in a row (the
second smaller, so it reuses the array the first one left behind), a
split-K shape whose partial tiles use the array, a replayed graph capture, a
fresh process whose first call is made under capture, and a shape whose
session split does not fit the array (run with a smaller split, checked
against the oracle).
"""
import ctypes
import os
import subprocess
import sys

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


def test_noalloc_falls_back_when_split_exceeds_static_scratch(device, library, oracle):
    # K = 8192 at gs64 has 128 groups per row, more than one K range of the
    # prefill kernel takes, so a default session splits K over 2: 32 MiB of
    # partial tiles, more than the 16 MiB array.  The entry point then runs
    # the plan made for the array's capacity: within tolerance of the oracle
    # (another summation order than the session op, so not bit-equal to it).
    rng = np.random.default_rng(79)
    m, n, k, gs = 512, 8192, 8192, 64
    W, S, B, X, Y, Y_ref, cmds = _case(device, library, rng, m, n, k, gs)
    for _ in range(2):
        _noalloc(cmds.stream, W, S, B, X, Y, m, n, k, gs, 4)
        cmds.commit_and_wait()
    rows = np.arange(0, m, 8)
    x = X.to_numpy().reshape(m, k)[rows]
    ref = oracle.qmm_ref(x, W.to_numpy().reshape(n, -1), S.to_numpy().reshape(n, -1), B.to_numpy().reshape(n, -1),
                         len(rows), n, k, gs, 4, "bf16", threads=16)
    y = Y.to_numpy().reshape(m, n)[rows]
    rep = oracle.tolerance_report(y, ref, x, k, "bf16")
    assert rep["ok"], rep


_FRESH = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from cider_press_amd import _lib
from cider_press_amd.kernels import Device, KernelLibrary, _ptr
from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.synthetic import make_weight, make_x

dev = Device.system_default()
lib = KernelLibrary.quantized(dev)
rng = np.random.default_rng(80)
m, n, k, gs = 512, 4096, 4096, 64
w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
x = make_x(rng, m, k, "bf16")
W, S, B = dev.upload(w_q.reshape(-1), "u32"), dev.upload(s.reshape(-1), "bf16"), dev.upload(b.reshape(-1), "bf16")
X = dev.upload(x.reshape(-1), "bf16")
Y, Y_ref = dev.alloc_buffer(m * n, "bf16"), dev.alloc_buffer(m * n, "bf16")
cmds = dev.commands()
print("capture: first no-alloc call of the process", flush=True)
cmds.begin_capture()
_lib.check(_lib.lib().cpq_affine_qmm_t_noalloc(
    ctypes.c_void_p(cmds.stream), _lib.DTYPES["bf16"], _ptr(W), len(W), _ptr(S), len(S), _ptr(B), len(B), _ptr(X),
    len(X), _ptr(Y), len(Y), m, n, k, gs, 4))
g = cmds.end_capture()
kqmm.affine_qmm_t(cmds, lib, W, S, B, X, Y_ref, m, n, k, gs, 4)
cmds.commit_and_wait()
ref = Y_ref.to_numpy()
for i in range(3):
    Y.write(np.zeros(m * n, np.uint16))
    g.launch(cmds)
    cmds.commit_and_wait()
    assert np.array_equal(Y.to_numpy(), ref), i
g.close()
print("NOALLOC_FRESH_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_under_capture_in_fresh_process():
    """The per-device set-up runs inside the first call; here that call is
    captured into a graph in a process that never called the entry point."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and "NOALLOC_FRESH_CAPTURE_OK" in r.stdout, (r.returncode, r.stdout[-2000:],
                                                                          r.stderr[-2000:])
