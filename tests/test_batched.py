"""Batched qmv / qmm_t (MLX's `batched` kernels; adjust_matrix_offsets,
quantized.h:1351-1388): every batch element must equal the single-matrix op
on that element's operands bit for bit, for distinct, broadcast and 2-D
batch shapes; and the single-matrix results are pinned to the oracle by the
other parity tests.  Stride checks run through the same entry points.
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _stack(rng, count, n, k, gs, bits, dtype):
    ws = [make_weight(rng, n, k, gs, bits, dtype) for _ in range(count)]
    return [np.stack([w[i] for w in ws]) for i in range(3)]


@pytest.mark.parametrize("shape,wbroad,m,n,k,gs,bits,dtype", [
    ((3,), (False,), 5, 256, 512, 64, 4, "bf16"),          # distinct weights
    ((2, 2), (False, True), 40, 128, 1024, 32, 8, "f16"),  # weights broadcast along dim 1
    ((4,), (True,), 1, 512, 256, 128, 4, "bf16"),          # one weight, four activations
])
def test_qmm_t_batched_matches_single_calls(device, library, oracle, shape, wbroad, m, n, k, gs, bits, dtype):
    from cider_press_amd.kernels import qmm as kqmm

    rng = np.random.default_rng(sum(shape) + m + bits)
    wcount = int(np.prod([1 if b else d for d, b in zip(shape, wbroad)]))
    w_q, s, b = _stack(rng, wcount, n, k, gs, bits, dtype)
    count = int(np.prod(shape))
    x = make_x(rng, count * m, k, dtype).reshape(count, m, k)
    # element strides: weights over the non-broadcast dims (row-major), x dense
    wdims = [d for d, bb in zip(shape, wbroad) if not bb]
    def strides(per):
        out, acc = [], per
        for d, bb in reversed(list(zip(shape, wbroad))):
            out.append(0 if bb else acc)
            acc *= 1 if bb else d
        return tuple(reversed(out))
    wst, sst = strides(n * k * bits // 32), strides(n * k // gs)
    xst = tuple(int(np.prod(shape[i + 1:])) * m * k for i in range(len(shape)))
    W = device.upload(w_q.reshape(-1), "u32"); S = device.upload(s.reshape(-1), dtype)
    B = device.upload(b.reshape(-1), dtype); X = device.upload(x.reshape(-1), dtype)
    Y = device.alloc_buffer(count * m * n, dtype)
    cmds = device.commands()
    kqmm.affine_qmm_t_batched(cmds, library, W, S, B, X, Y, m, n, k, gs, bits, shape, wst, sst, sst, xst)
    cmds.commit_and_wait()
    got = Y.to_numpy()[: count * m * n].reshape(count, m, n)
    for z, idx in enumerate(np.ndindex(*shape)):
        wi = int(np.ravel_multi_index([i for i, bb in zip(idx, wbroad) if not bb], wdims)) if wdims else 0
        W1 = device.upload(w_q[wi].reshape(-1), "u32"); S1 = device.upload(s[wi].reshape(-1), dtype)
        B1 = device.upload(b[wi].reshape(-1), dtype); X1 = device.upload(x[z].reshape(-1), dtype)
        Y1 = device.alloc_buffer(m * n, dtype)
        c1 = device.commands()
        kqmm.affine_qmm_t(c1, library, W1, S1, B1, X1, Y1, m, n, k, gs, bits)
        c1.commit_and_wait()
        assert np.array_equal(got[z], Y1.to_numpy()[: m * n].reshape(m, n)), f"batch element {idx}"
    ref = oracle.qmm_ref(x[0], w_q[0], s[0], b[0], m, n, k, gs, bits, dtype)
    assert oracle.tolerance_report(got[0], ref, x[0], k, dtype)["ok"]


def test_qmv_batched(device, library, oracle):
    from cider_press_amd.kernels import qmv as kqmv

    rng = np.random.default_rng(3)
    count, n, k, gs = 3, 1024, 2048, 64
    w_q, s, b = _stack(rng, count, n, k, gs, 4, "bf16")
    x = make_x(rng, count, k, "bf16")
    W = device.upload(w_q.reshape(-1), "u32"); S = device.upload(s.reshape(-1), "bf16")
    B = device.upload(b.reshape(-1), "bf16"); X = device.upload(x.reshape(-1), "bf16")
    Y = device.alloc_buffer(count * n, "bf16")
    cmds = device.commands()
    kqmv.affine_qmv_batched(cmds, library, W, S, B, X, Y, k, n, gs, 4, (count,), (n * k // 8,), (n * k // gs,),
                            (n * k // gs,), (k,))
    cmds.commit_and_wait()
    got = Y.to_numpy()[: count * n].reshape(count, n)
    for z in range(count):
        ref = oracle.qmm_ref(x[z:z + 1], w_q[z], s[z], b[z], 1, n, k, gs, 4, "bf16")
        rep = oracle.tolerance_report(got[z:z + 1], ref, x[z:z + 1], k, "bf16")
        assert rep["ok"], (z, rep)


def test_batched_stride_checks(device, library):
    from cider_press_amd.kernels import qmm as kqmm

    rng = np.random.default_rng(4)
    m, n, k, gs = 4, 64, 128, 64
    w_q, s, b = _stack(rng, 2, n, k, gs, 4, "bf16")
    W = device.upload(w_q.reshape(-1), "u32"); S = device.upload(s.reshape(-1), "bf16")
    B = device.upload(b.reshape(-1), "bf16"); X = device.upload(make_x(rng, 2 * m, k, "bf16").reshape(-1), "bf16")
    Y = device.alloc_buffer(2 * m * n, "bf16")
    cmds = device.commands()
    wst, sst, xst = n * k // 8, n * k // gs, m * k
    for bad in (((3,), (wst,), (sst,), (xst,)),          # third element past every buffer
                ((2,), (wst + 1,), (sst,), (xst,)),      # weight stride breaks 16-byte rows
                ((2,), (wst,), (sst,), (xst + 4,)),      # activation stride breaks 16-byte rows
                ((2,), (-wst,), (sst,), (xst,))):        # negative stride
        shape, ws, ss, xs = bad
        with pytest.raises(_lib.InvalidArgument):
            kqmm.affine_qmm_t_batched(cmds, library, W, S, B, X, Y, m, n, k, gs, 4, shape, ws, ss, ss, xs)
