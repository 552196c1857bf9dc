"""Batched qmv / qmm_t (MLX's `batched` kernels; adjust_matrix_offsets,
quantized.h:1351-1388): every batch element must meet the tolerance against
the oracle on that element's operands, for distinct, broadcast and 2-D batch
shapes, on each of the three ways a batch runs: one weight shared by every
element with dense activations (a single matmul over all rows), the
decode-layout kernels with the batch in their grid, and one launch per
element.  Repeated calls give identical bits.  Stride checks run through the
same entry points.
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _stack(rng, count, n, k, gs, bits, dtype):
    ws = [make_weight(rng, n, k, gs, bits, dtype) for _ in range(count)]
    return [np.stack([w[i] for w in ws]) for i in range(3)]


def _strides(shape, broad, per):
    """Row-major element strides over the dims that are not broadcast."""
    out, acc = [], per
    for d, bb in reversed(list(zip(shape, broad))):
        out.append(0 if bb else acc)
        acc *= 1 if bb else d
    return tuple(reversed(out))


def _index(idx, shape, broad):
    dims = [d for d, bb in zip(shape, broad) if not bb]
    return int(np.ravel_multi_index([i for i, bb in zip(idx, broad) if not bb], dims)) if dims else 0


def _run_batched(device, library, oracle, shape, wbroad, xbroad, m, n, k, gs, bits, dtype, qmv):
    from cider_press_amd.kernels import qmm as kqmm
    from cider_press_amd.kernels import qmv as kqmv

    rng = np.random.default_rng(sum(shape) + m + n + k + bits)
    wcount = int(np.prod([1 if b else d for d, b in zip(shape, wbroad)]))
    xcount = int(np.prod([1 if b else d for d, b in zip(shape, xbroad)]))
    w_q, s, b = _stack(rng, wcount, n, k, gs, bits, dtype)
    count = int(np.prod(shape))
    x = make_x(rng, xcount * m, k, dtype).reshape(xcount, m, k)
    wst, sst = _strides(shape, wbroad, n * k * bits // 32), _strides(shape, wbroad, n * k // gs)
    xst = _strides(shape, xbroad, m * k)
    W = device.upload(w_q.reshape(-1), "u32"); S = device.upload(s.reshape(-1), dtype)
    B = device.upload(b.reshape(-1), dtype); X = device.upload(x.reshape(-1), dtype)
    outs = []
    cmds = device.commands()
    for _ in range(2):
        Y = device.alloc_buffer(count * m * n, dtype)
        if qmv:
            kqmv.affine_qmv_batched(cmds, library, W, S, B, X, Y, k, n, gs, bits, shape, wst, sst, sst, xst)
        else:
            kqmm.affine_qmm_t_batched(cmds, library, W, S, B, X, Y, m, n, k, gs, bits, shape, wst, sst, sst, xst)
        outs.append(Y)
    cmds.commit_and_wait()
    got = [o.to_numpy()[: count * m * n].reshape(count, m, n) for o in outs]
    assert np.array_equal(got[0], got[1])
    for z, idx in enumerate(np.ndindex(*shape)):
        wi, xi = _index(idx, shape, wbroad), _index(idx, shape, xbroad)
        ref = oracle.qmm_ref(x[xi], w_q[wi], s[wi], b[wi], m, n, k, gs, bits, dtype)
        rep = oracle.tolerance_report(got[0][z], ref, x[xi], k, dtype)
        assert rep["ok"], (idx, rep)


@pytest.mark.parametrize("shape,wbroad,xbroad,m,n,k,gs,bits,dtype", [
    ((3,), (False,), (False,), 5, 256, 512, 64, 4, "bf16"),            # per element (K off the decode layout)
    ((2, 2), (False, True), (False, False), 40, 128, 1024, 32, 8, "f16"),  # per element, weights broadcast on dim 1
    ((4,), (True,), (False,), 1, 512, 256, 128, 4, "bf16"),            # shared weight: one matmul over 4 rows
    ((2, 3), (True, True), (False, False), 8, 4096, 4096, 64, 4, "bf16"),  # shared weight: 48 rows, small-M kernel
    ((3,), (False,), (False,), 4, 1024, 4096, 64, 4, "bf16"),          # decode layout, batch in the grid
    ((5,), (False,), (False,), 16, 512, 8192, 128, 8, "f16"),          # decode layout, 16 rows, 8-bit
    ((3,), (False,), (False,), 6, 1056, 4096, 64, 8, "bf16"),          # decode layout, 8-bit K = 4096: 4 waves
    ((2, 2), (False, True), (True, False), 3, 1024, 4096, 32, 4, "bf16"),  # grid, both operands broadcast on a dim
])
def test_qmm_t_batched_parity(device, library, oracle, shape, wbroad, xbroad, m, n, k, gs, bits, dtype):
    print(f"qmm_t batched {shape} w{wbroad} x{xbroad} m={m} n={n} k={k} b{bits} gs{gs} {dtype}", flush=True)
    _run_batched(device, library, oracle, shape, wbroad, xbroad, m, n, k, gs, bits, dtype, qmv=False)


@pytest.mark.parametrize("shape,wbroad,xbroad,n,k,gs,bits,dtype", [
    ((3,), (False,), (False,), 1024, 2048, 64, 4, "bf16"),             # batch in the decode kernel's grid
    ((2, 3), (False, True), (True, False), 4096, 4096, 32, 8, "f16"),  # grid, 2-D with broadcasts
    ((7,), (False,), (False,), 96, 8192, 128, 4, "bf16"),              # grid, one column block per element
    ((6,), (True,), (False,), 2048, 4096, 64, 4, "bf16"),              # shared weight: one matmul over 6 rows
    ((3,), (False,), (False,), 256, 768, 64, 4, "bf16"),               # per element (K off the decode kernel)
])
def test_qmv_batched_parity(device, library, oracle, shape, wbroad, xbroad, n, k, gs, bits, dtype):
    print(f"qmv batched {shape} w{wbroad} x{xbroad} n={n} k={k} b{bits} gs{gs} {dtype}", flush=True)
    _run_batched(device, library, oracle, shape, wbroad, xbroad, 1, n, k, gs, bits, dtype, qmv=True)


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
