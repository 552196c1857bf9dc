"""Routed-expert plumbing (kernels/moe.hip) against numpy: softmax top-k
(float64 softmax; ranking by (-p, expert)), the stable argsort of the
flattened expert ids for the sort, and a float64 weighted sum for the
combine; then a whole MoE projection (route -> sorted gather_qmm -> combine)
against the oracle's per-row dense reduction.

The reference has no MoE code to pin against (its docs name the feature as
unbuilt), so these are closed forms and a textbook sort: parity for the
route/sort/combine semantics stated in include/cpq.h.
"""
import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.synthetic import from_bits, make_weight, make_x, to_bits

pytestmark = pytest.mark.gpu


def np_route(logits_f32, k, normalize):
    z = logits_f32.astype(np.float64)
    p = np.exp(z - z.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    e = np.arange(p.shape[1])
    order = np.lexsort((np.broadcast_to(e, p.shape), -p), axis=1)[:, :k]
    sc = np.take_along_axis(p, order, axis=1)
    if normalize:
        sc = sc / sc.sum(axis=1, keepdims=True)
    return order.astype(np.uint32), sc


def np_sort(experts_flat, k, n_experts):
    order = np.argsort(experts_flat, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    offsets = np.searchsorted(experts_flat[order], np.arange(n_experts + 1), side="left")
    return (order // k).astype(np.uint32), experts_flat[order].astype(np.uint32), inv.astype(np.uint32), \
        offsets.astype(np.uint32)


def run_route(device, logits_bits, dtype, tokens, E, k, normalize):
    from cider_press_amd.kernels import moe as kmoe

    L = device.upload(logits_bits.reshape(-1), dtype)
    rows = tokens * k
    bufs = {n: device.alloc_buffer(max(1, rows), t) for n, t in
            (("experts", "u32"), ("scores", "f32"), ("lhs", "u32"), ("rhs", "u32"), ("inv", "u32"))}
    off = device.alloc_buffer(E + 1, "u32")
    cmds = device.commands()
    kmoe.moe_route(cmds, L, tokens, E, k, normalize, bufs["experts"], bufs["scores"], bufs["lhs"], bufs["rhs"],
                   bufs["inv"], off)
    cmds.commit_and_wait()
    out = {n: b.to_numpy()[:rows] for n, b in bufs.items()}
    out["offsets"] = off.to_numpy()[:E + 1]
    return out, bufs, off


def _logits(rng, tokens, E, dtype):
    lg = (rng.standard_normal((tokens, E)) * 2.5).astype(np.float32)
    if dtype == "f32":
        return lg, lg
    bits = to_bits(lg, dtype)
    return bits, from_bits(bits, dtype)


@pytest.mark.parametrize("tokens,E,k,normalize,dtype", [
    (256, 128, 8, True, "bf16"),     # config 5 routing
    (100, 64, 2, False, "f32"),
    (33, 1000, 16, True, "f16"),
    (1, 8, 8, False, "bf16"),        # every expert picked
    (700, 60, 4, True, "bf16"),      # several sort blocks, E not a multiple of 64
    (300, 4, 4, False, "bf16"),      # every row of a token on the 4 experts: long equal runs
    (2100, 64, 8, True, "bf16"),     # 66 sort blocks
    (1100, 1000, 2, True, "f16"),    # 9 sort blocks x 1000 experts
])
def test_route_and_sort(device, tokens, E, k, normalize, dtype):
    rng = np.random.default_rng(tokens * 7 + E + k)
    bits, lg = _logits(rng, tokens, E, dtype)
    got, _, _ = run_route(device, bits, dtype, tokens, E, k, normalize)
    ex, sc = np_route(lg, k, normalize)
    assert np.array_equal(got["experts"].reshape(tokens, k), ex)
    np.testing.assert_allclose(got["scores"].reshape(tokens, k), sc, rtol=2e-6, atol=1e-7)
    lhs, rhs, inv, offsets = np_sort(got["experts"], k, E)
    assert np.array_equal(got["lhs"], lhs) and np.array_equal(got["rhs"], rhs)
    assert np.array_equal(got["inv"], inv) and np.array_equal(got["offsets"], offsets)


def test_route_ties_prefer_lower_expert(device):
    tokens, E, k = 3, 70, 5
    lg = np.zeros((tokens, E), np.float32)
    lg[1, [3, 9, 40, 41]] = 1.0          # four equal maxima, then a 66-way tie
    lg[2, ::-1] = np.arange(E) % 2       # alternating 0/1, equal pairs everywhere
    got, _, _ = run_route(device, lg, "f32", tokens, E, k, True)
    ex = got["experts"].reshape(tokens, k)
    assert list(ex[0]) == [0, 1, 2, 3, 4]
    assert list(ex[1]) == [3, 9, 40, 41, 0]
    ones = [e for e in range(E) if lg[2, e] == 1.0]
    assert list(ex[2]) == ones[:5]
    np.testing.assert_allclose(got["scores"].reshape(tokens, k)[0], np.full(5, 0.2), rtol=1e-6)


def test_route_rejects_bad_arguments(device):
    from cider_press_amd.kernels import moe as kmoe

    L = device.alloc_buffer(64, "f32")
    b = {n: device.alloc_buffer(64, t) for n, t in
         (("e", "u32"), ("s", "f32"), ("l", "u32"), ("r", "u32"), ("i", "u32"), ("o", "u32"))}
    cmds = device.commands()
    for E, k in ((4, 5), (2000, 2), (32, 0), (32, 17)):
        with pytest.raises(_lib.InvalidArgument):
            kmoe.moe_route(cmds, L, 1, E, k, True, b["e"], b["s"], b["l"], b["r"], b["i"],
                           device.alloc_buffer(E + 1, "u32"))


@pytest.mark.parametrize("tokens,k,n,dtype", [(256, 8, 2048, "bf16"), (37, 3, 96, "f16"), (1, 1, 8, "bf16")])
def test_combine(device, tokens, k, n, dtype):
    from cider_press_amd.kernels import moe as kmoe

    rng = np.random.default_rng(tokens + k + n)
    rows = tokens * k
    y = make_x(rng, rows, n, dtype)
    sc = rng.uniform(0.0, 1.0, size=rows).astype(np.float32)
    inv = rng.permutation(rows).astype(np.uint32)
    Y = device.upload(y.reshape(-1), dtype)
    S = device.upload(sc, "f32")
    I = device.upload(inv, "u32")
    O = device.alloc_buffer(tokens * n, dtype)
    cmds = device.commands()
    kmoe.moe_combine(cmds, Y, S, I, tokens, k, n, O)
    cmds.commit_and_wait()
    got = from_bits(O.to_numpy()[: tokens * n], dtype).astype(np.float64).reshape(tokens, n)
    yf = from_bits(y, dtype).astype(np.float64).reshape(rows, n)
    ref = np.einsum("tk,tkn->tn", sc.astype(np.float64).reshape(tokens, k), yf[inv].reshape(tokens, k, n))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - (7 if dtype == "bf16" else 10))
    assert np.all(np.abs(got - ref) <= 0.5 * ulp + 1e-5 * (1 + np.abs(ref)))


def test_combine_out_of_range_position(device):
    from cider_press_amd.kernels import moe as kmoe

    tokens, k, n = 4, 2, 16
    y = np.full((tokens * k, n), to_bits(np.float32([1.0]), "bf16")[0], np.uint16)
    inv = np.array([0, 1, 2, 99, 4, 5, 6, 7], np.uint32)
    Y = device.upload(y.reshape(-1), "bf16")
    S = device.upload(np.ones(tokens * k, np.float32), "f32")
    I = device.upload(inv, "u32")
    O = device.alloc_buffer(tokens * n, "bf16")
    cmds = device.commands()
    kmoe.moe_combine(cmds, Y, S, I, tokens, k, n, O)
    with pytest.raises(_lib.InvalidArgument, match="moe_combine: 1"):
        cmds.commit_and_wait()
    got = from_bits(O.to_numpy()[: tokens * n], "bf16").reshape(tokens, n)
    assert np.all(got[[0, 2, 3]] == 2.0) and np.all(got[1] == 1.0)
    cmds.commit_and_wait()


def test_moe_projection_end_to_end(device, library, oracle):
    """route -> sorted gather_qmm -> combine, against per-token float64 sums
    of the oracle's dense rows."""
    from cider_press_amd.kernels import gather as kgather
    from cider_press_amd.kernels import moe as kmoe

    rng = np.random.default_rng(5)
    tokens, E, k, n, kd, gs = 96, 16, 4, 256, 512, 64
    w = [make_weight(rng, n, kd, gs, 4, "bf16") for _ in range(E)]
    w_q = np.concatenate([a[0] for a in w]); s = np.concatenate([a[1] for a in w])
    b = np.concatenate([a[2] for a in w])
    x = make_x(rng, tokens, kd, "bf16")
    bits, lg = _logits(rng, tokens, E, "bf16")
    got, bufs, _ = run_route(device, bits, "bf16", tokens, E, k, True)
    X = device.upload(x.reshape(-1), "bf16")
    W = device.upload(w_q.reshape(-1), "u32"); S = device.upload(s.reshape(-1), "bf16")
    B = device.upload(b.reshape(-1), "bf16")
    rows = tokens * k
    Y = device.alloc_buffer(rows * n, "bf16")
    O = device.alloc_buffer(tokens * n, "bf16")
    cmds = device.commands()
    kgather.affine_gather_qmm(cmds, library, X, W, S, B, bufs["lhs"], bufs["rhs"], Y, rows, n, kd, E, gs, 4,
                              sorted_indices=True, x_rows=tokens)
    kmoe.moe_combine(cmds, Y, bufs["scores"], bufs["inv"], tokens, k, n, O)
    cmds.commit_and_wait()
    ex = got["experts"].reshape(tokens, k)
    sc = got["scores"].astype(np.float64).reshape(tokens, k)
    dense = oracle.gather_qmm_ref(x, np.repeat(np.arange(tokens, dtype=np.uint32), k), ex.reshape(-1), w_q, s, b,
                                  rows, n, kd, gs, 4, "bf16").reshape(tokens, k, n)
    # The expert outputs are stored in T before the combine (as gather_qmm's
    # output is), so the reference rounds them the same way.
    dense_t = from_bits(to_bits(dense.astype(np.float32), "bf16"), "bf16").astype(np.float64)
    ref = np.einsum("tk,tkn->tn", sc, dense_t)
    rep = oracle.tolerance_report(O.to_numpy()[: tokens * n].reshape(tokens, n), ref, x, kd, "bf16")
    assert rep["ok"], rep
