"""Pins the CPU oracle (oracle/cpq_oracle.c) before anything is checked against it.

Each check is independent of the oracle's own formulas: the reference's
committed golden vectors, torch/numpy library conversions, an independent bit
stream implementation, closed forms and brute force.  The planted-mistake
tests at the end compile deliberately wrong oracles and show the pins fail.
"""
import os
import subprocess

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bf16_torch(f32: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(np.ascontiguousarray(f32, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _probe_floats(n=200_000, seed=1):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # ties and near-ties at bf16 / f16 precision
    base = rng.integers(0, 2**32, size=20_000, dtype=np.uint64).astype(np.uint32) & 0xFFFF0000
    ties = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001, (base & 0xFFFE0000) | 0x18000])
    ties = ties.view(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8,
                        3e-38, 1e-45, 3.4e38], np.float32)
    out = np.concatenate([f, ties[np.isfinite(ties)], special]).astype(np.float32)
    return out


def test_bf16_conversion_matches_torch(oracle):
    f = _probe_floats()
    ours = np.array([oracle.c_f32_to_bits(float(v), "bf16") for v in f[:30000]], np.uint16)
    assert np.array_equal(ours, _bf16_torch(f[:30000]))
    # vectorised helper used by the tests
    assert np.array_equal(oracle.f32_to_bits(f, "bf16"), _bf16_torch(f))


def test_f16_conversion_matches_numpy(oracle):
    f = _probe_floats(seed=2)
    f = f[np.abs(f) < 1e5]
    ours = np.array([oracle.c_f32_to_bits(float(v), "f16") for v in f[:30000]], np.uint16)
    assert np.array_equal(ours, f[:30000].astype(np.float16).view(np.uint16))


def test_16bit_to_f32_exhaustive(oracle):
    allb = np.arange(65536, dtype=np.uint16)
    finite_bf = ((allb & 0x7F80) != 0x7F80)
    import torch

    bf = np.array([oracle.c_bits_to_f32(int(b), "bf16") for b in allb[finite_bf]], np.float32)
    ref = torch.from_numpy(allb[finite_bf].view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(bf.view(np.uint32), ref.view(np.uint32))
    finite_h = ((allb & 0x7C00) != 0x7C00)
    h = np.array([oracle.c_bits_to_f32(int(b), "f16") for b in allb[finite_h]], np.float32)
    assert np.array_equal(h.view(np.uint32), allb[finite_h].view(np.float16).astype(np.float32).view(np.uint32))


def test_half_ulp_bounds_t_rounding(oracle):
    """half_ulp (used by the tolerance check) is a tight bound on |RNE_T(v) - v|."""
    rng = np.random.default_rng(8)
    v = (rng.standard_normal(100_000) * np.exp2(rng.integers(-20, 20, 100_000))).astype(np.float32)
    for dtype in ("bf16", "f16"):
        vv = v[np.abs(v) < 6e4] if dtype == "f16" else v
        r = oracle.bits_to_f32(oracle.f32_to_bits(vv, dtype), dtype).astype(np.float64)
        e = np.abs(r - vv.astype(np.float64))
        h = oracle.half_ulp(vv, dtype)
        assert np.all(e <= h * (1 + 1e-12))
        assert np.max(e / h) > 0.99
    assert oracle.half_ulp(np.array([16.0, 15.99, -300.0]), "bf16").tolist() == [0.0625, 0.03125, 1.0]
    assert oracle.half_ulp(np.array([1.0]), "f16")[0] == 2.0 ** -11


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_unpack_is_little_endian_bit_stream(oracle, bits):
    """Element i occupies bits [bits*i, bits*(i+1)) of the row's LE bit stream
    (quantized.h:2565-2600); checked with numpy.unpackbits, not the oracle's shifts."""
    rng = np.random.default_rng(bits)
    k = 256
    words = rng.integers(0, 2**32, size=(3, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    q = oracle.unpack(words, k, bits)
    stream = np.unpackbits(words.view(np.uint8), axis=1, bitorder="little")
    expect = np.zeros((3, k), np.uint32)
    for j in range(bits):
        expect |= stream[:, j::bits][:, :k].astype(np.uint32) << j
    assert np.array_equal(q.astype(np.uint32), expect)
    assert np.array_equal(oracle.pack(q, bits), words)


def test_synthetic_packer_agrees(oracle):
    from cider_press_amd.synthetic import pack_rows

    rng = np.random.default_rng(7)
    for bits in (2, 3, 4, 5, 6, 8):
        q = rng.integers(0, 1 << bits, size=(4, 128), dtype=np.uint32)
        assert np.array_equal(pack_rows(q, bits), oracle.pack(q.astype(np.uint8), bits))


# ---------------------------------------------------------------------------
# The reference's committed goldens
# ---------------------------------------------------------------------------

def test_golden_qmv_bit_exact(oracle):
    """crates/cider-press-kernels/tests/fixtures/qmv.safetensors (K=N=512, MLX qmv_fast)."""
    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmv.safetensors"))
    y = oracle.qmv_mlx(d["x"].reshape(1, -1), d["w_q"], d["scales"], d["biases"], 1, 512, 512, 64, 4, "bf16")
    assert np.array_equal(oracle.f32_to_bits(y, "bf16").reshape(-1), d["y_ref"])


def test_golden_qmm_qwen2(oracle):
    """qmm_qwen2.safetensors (M=8, K=N=896): produced by MLX's generic qmv path.
    Exact on >= 7166/7168 elements; the rest differ by one bf16 ULP (lane
    reduction order)."""
    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmm_qwen2.safetensors"))
    y = oracle.qmv_mlx(d["x"], d["w_q"], d["scales"], d["biases"], 8, 896, 896, 64, 4, "bf16")
    yb = oracle.f32_to_bits(y, "bf16")
    assert (yb == d["y_ref"]).sum() >= 7166
    ulps = np.abs(yb.astype(np.int32) - d["y_ref"].astype(np.int32))
    assert ulps.max() <= 1


def test_golden_against_dequant_reference(oracle):
    """The dequantize-then-matmul reference reproduces the goldens within the
    reference's own tolerance (max_relative=1e-2, epsilon=5e-2, qmv_parity.rs:79-92)."""
    for name, m, k, n in (("qmv.safetensors", 1, 512, 512), ("qmm_qwen2.safetensors", 8, 896, 896)):
        d = oracle.read_safetensors(os.path.join(GOLDEN, name))
        y = oracle.qmm_ref(d["x"].reshape(m, k), d["w_q"], d["scales"], d["biases"], m, n, k, 64, 4, "bf16")
        e = oracle.bits_to_f32(d["y_ref"], "bf16").reshape(m, n).astype(np.float64)
        assert np.all(np.abs(y - e) <= np.maximum(5e-2, 1e-2 * np.maximum(np.abs(y), np.abs(e))))


# ---------------------------------------------------------------------------
# Dequantize: RNE_T(fmaf(s, q, b))
# ---------------------------------------------------------------------------

def _independent_dequant(q, s_bits, b_bits, gs, dtype):
    """float64 s*q+b (exact for these widths) -> float32 (one RNE) -> T via torch/numpy."""
    from cider_press_amd.synthetic import from_bits

    s = np.repeat(from_bits(s_bits, dtype).astype(np.float64), gs, axis=1)
    b = np.repeat(from_bits(b_bits, dtype).astype(np.float64), gs, axis=1)
    v = (s * q.astype(np.float64) + b).astype(np.float32)
    if dtype == "bf16":
        return _bf16_torch(v)
    return v.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (8, 64), (2, 128), (3, 32), (5, 64), (6, 32)])
def test_dequantize_matches_independent(oracle, dtype, bits, gs):
    from cider_press_amd.synthetic import make_weight

    rng = np.random.default_rng(bits * 100 + gs)
    n, k = 16, 256
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype, bias_noise=1e-3)
    q = oracle.unpack(w_q, k, bits)
    got = oracle.dequantize(w_q, s, b, n, k, gs, bits, dtype)
    assert np.array_equal(got, _independent_dequant(q, s, b, gs, dtype))


def test_dequantize_special_cases(oracle):
    from cider_press_amd.synthetic import from_bits, make_weight, to_bits

    rng = np.random.default_rng(3)
    n, k, gs = 8, 128, 64
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    # q = 0 everywhere -> RNE(b), i.e. b itself
    zero = np.zeros_like(w_q)
    got = oracle.dequantize(zero, s, b, n, k, gs, 4, "bf16")
    assert np.array_equal(got, np.repeat(b, gs, axis=1))
    # b = -8s -> RNE(s*(q-8)); q-8 in {+-1,+-2,+-4,+-8,0} is exact
    q = oracle.unpack(w_q, k, 4).astype(np.float64)
    sf = np.repeat(from_bits(s, "bf16").astype(np.float64), gs, axis=1)
    got = from_bits(oracle.dequantize(w_q, s, b, n, k, gs, 4, "bf16"), "bf16").astype(np.float64)
    expect = from_bits(to_bits((sf * (q - 8)).astype(np.float32), "bf16"), "bf16")
    assert np.array_equal(got, expect)
    pow2 = np.isin(q - 8, [0, 1, -1, 2, -2, 4, -4, 8, -8])
    assert np.array_equal(got[pow2], (sf * (q - 8))[pow2])


# ---------------------------------------------------------------------------
# Reference matmul: closed forms and brute force
# ---------------------------------------------------------------------------

def test_qmm_ref_brute_force_tiny(oracle):
    from cider_press_amd.synthetic import from_bits, make_weight, make_x

    rng = np.random.default_rng(11)
    m, n, k, gs = 3, 5, 64, 32
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16", bias_noise=1e-3)
    x = make_x(rng, m, k, "bf16")
    wd = from_bits(_independent_dequant(oracle.unpack(w_q, k, 4), s, b, gs, "bf16"), "bf16")
    xf = from_bits(x, "bf16")
    brute = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                acc += float(xf[i, kk]) * float(wd[j, kk])
            brute[i, j] = acc
    got = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
    np.testing.assert_allclose(got, brute, rtol=1e-12, atol=1e-12)


def test_qmm_ref_matches_numpy_float64(oracle):
    from cider_press_amd.synthetic import from_bits, make_weight, make_x

    rng = np.random.default_rng(12)
    m, n, k, gs = 7, 96, 512, 64
    for bits in (4, 8):
        w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
        x = make_x(rng, m, k, "bf16")
        wd = from_bits(_independent_dequant(oracle.unpack(w_q, k, bits), s, b, gs, "bf16"), "bf16")
        ref = from_bits(x, "bf16").astype(np.float64) @ wd.astype(np.float64).T
        np.testing.assert_allclose(oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16"), ref,
                                   rtol=1e-12, atol=1e-10)


def test_qmm_ref_invariants(oracle):
    from cider_press_amd.synthetic import from_bits, make_weight, make_x, to_bits

    rng = np.random.default_rng(13)
    m, n, k, gs = 4, 32, 256, 64
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    y = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
    # homogeneity: doubling x (exact in bf16) doubles y exactly
    x2 = to_bits(from_bits(x, "bf16") * 2, "bf16")
    assert np.array_equal(oracle.qmm_ref(x2, w_q, s, b, m, n, k, gs, 4, "bf16"), 2 * y)
    # s = 0: every weight is the bias -> y = sum over groups of b_g * sum(x_g)
    zs = np.zeros_like(s)
    y0 = oracle.qmm_ref(x, w_q, zs, b, m, n, k, gs, 4, "bf16")
    xs = from_bits(x, "bf16").astype(np.float64).reshape(m, k // gs, gs).sum(axis=2)
    np.testing.assert_allclose(y0, xs @ from_bits(b, "bf16").astype(np.float64).T, rtol=1e-12, atol=1e-12)
    # transposition of roles: row j of y for x = e_i picks dequant(W)[j, i]
    eye = to_bits(np.eye(4, k, dtype=np.float32), "bf16")
    ye = oracle.qmm_ref(eye, w_q, s, b, 4, n, k, gs, 4, "bf16")
    wd = from_bits(oracle.dequantize(w_q, s, b, n, k, gs, 4, "bf16"), "bf16")
    assert np.array_equal(ye, wd[:, :4].T.astype(np.float64))


def test_gather_ref_reduces_to_dense(oracle):
    from cider_press_amd.synthetic import make_weight, make_x

    rng = np.random.default_rng(14)
    e, n, k, gs, rows = 4, 32, 128, 64, 9
    w = [make_weight(rng, n, k, gs, 4, "bf16") for _ in range(e)]
    w_q = np.concatenate([t[0] for t in w]); s = np.concatenate([t[1] for t in w]); b = np.concatenate([t[2] for t in w])
    x = make_x(rng, 5, k, "bf16")
    lhs = rng.integers(0, 5, size=rows).astype(np.uint32)
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    y = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, rows, n, k, gs, 4, "bf16")
    for r in range(rows):
        ex = rhs[r]
        dense = oracle.qmm_ref(x[lhs[r]:lhs[r] + 1], w[ex][0], w[ex][1], w[ex][2], 1, n, k, gs, 4, "bf16")
        assert np.array_equal(y[r], dense[0])


def test_cpu_baseline_within_tolerance(oracle):
    from cider_press_amd.synthetic import make_weight, make_x

    rng = np.random.default_rng(15)
    m, n, k, gs = 2, 256, 4096, 64
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
    forms = oracle.baseline_forms()
    assert "scalar" in forms
    for form in forms:
        got = oracle.cpu_baseline(x, w_q, s, b, m, n, k, gs, 4, "bf16", threads=4, form=form)
        rep = oracle.tolerance_report(got, ref, x, k, "bf16")
        assert rep["ok"], (form, rep)


@pytest.mark.parametrize("dtype,bits,gs", [("f16", 4, 32), ("bf16", 8, 64), ("f16", 3, 64), ("bf16", 4, 128)])
def test_cpu_baseline_forms_other_quantizations(oracle, dtype, bits, gs):
    """Every baseline form (the SIMD ones fall back to scalar for widths other
    than 4) against the oracle's float64 reference."""
    from cider_press_amd.synthetic import make_weight, make_x

    rng = np.random.default_rng(17)
    m, n, k = 3, 96, 1024
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype)
    for form in oracle.baseline_forms():
        got = oracle.cpu_baseline(x, w_q, s, b, m, n, k, gs, bits, dtype, threads=3, form=form)
        rep = oracle.tolerance_report(got, ref, x, k, dtype)
        assert rep["ok"], (form, rep)


def test_bf16_tolerance_rejects_factored_form(oracle):
    """Why every kernel rounds dequantized weights to T: MLX's factored form
    (unrounded weights, the qmv arithmetic) exceeds the 2e-3 rel-L2 budget
    against the dequantize-then-matmul reference at the decode shape."""
    from cider_press_amd.synthetic import make_weight, make_x

    rng = np.random.default_rng(16)
    n, k, gs = 2048, 4096, 64
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, 1, k, "bf16")
    ref = oracle.qmm_ref(x, w_q, s, b, 1, n, k, gs, 4, "bf16")
    fac = oracle.qmv_mlx(x, w_q, s, b, 1, n, k, gs, 4, "bf16")
    rep = oracle.tolerance_report(oracle.f32_to_bits(fac, "bf16"), ref, x, k, "bf16")
    assert rep["rel_l2"] > 2e-3
    rounded = oracle.f32_to_bits(ref.astype(np.float32), "bf16")
    assert oracle.tolerance_report(rounded, ref, x, k, "bf16")["ok"]


# ---------------------------------------------------------------------------
# Planted mistakes: the pins above must fail on a wrong oracle
# ---------------------------------------------------------------------------

MUTATIONS = {
    # nibble order reversed within each byte
    "nibble": ("q[i] = (uint8_t)(v & mask);", "q[i] = (uint8_t)((bits == 4 ? (v >> (4 * ((i & 1) ? -1 : 1) + 0)) : v) & mask);"),
    # truncation instead of round-to-nearest-even for bf16
    "trunc": ("u += 0x7fffu + ((u >> 16) & 1u);", "u += 0u;"),
    # bias dropped from the dequantized weight
    "nobias": ("out[r * k + i] = from_f32(fmaf(s, (float)q[i], b), dtype);", "out[r * k + i] = from_f32(s * (float)q[i], dtype);"),
    # wrong group index: element i reads the scale/bias of group (i+1)/gs
    "groupidx": ("size_t g = r * groups_per_row + i / (size_t)gs;", "size_t g = r * groups_per_row + (i + 1) / (size_t)gs;"),
    # last k term dropped from the reference matmul
    "dropk": ("a3 += xr[kk + 3] * (double)wr[kk + 3];",
              "a3 += (kk + 4 < j->k) ? xr[kk + 3] * (double)wr[kk + 3] : 0.0;"),
    # gather ignores the activation-row index
    "lhs": ("size_t xr = lhs ? lhs[r] : r;", "size_t xr = r;"),
}


def _build_mutant(tmp_path, name):
    src = open(os.path.join(os.path.dirname(os.path.dirname(__file__)), "oracle", "cpq_oracle.c")).read()
    old, new = MUTATIONS[name]
    assert old in src
    if name == "nibble":
        # swap the two nibbles of every byte for 4-bit rows
        new = ("{ uint32_t vv = v & mask; if (bits == 4) { size_t j = i ^ 1u; size_t bb = j * 4u; "
               "vv = (row[bb >> 5] >> (bb & 31u)) & mask; } q[i] = (uint8_t)vv; }")
    src = src.replace(old, new)
    c = tmp_path / f"mut_{name}.c"
    c.write_text(src)
    so = tmp_path / f"libmut_{name}.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-pthread", "-o", str(so), str(c), "-lm"],
                   check=True)
    return str(so)


def _pin_failures(mod, oracle):
    """Every pin the planted-mistake test applies; True marks a failed pin."""
    from cider_press_amd.synthetic import from_bits, make_weight, make_x

    d = mod.read_safetensors(os.path.join(GOLDEN, "qmv.safetensors"))
    caught = []
    y = mod.qmv_mlx(d["x"].reshape(1, -1), d["w_q"], d["scales"], d["biases"], 1, 512, 512, 64, 4, "bf16")
    caught.append(not np.array_equal(mod.f32_to_bits(y, "bf16").reshape(-1), d["y_ref"]))
    rng = np.random.default_rng(5)
    w_q, s, b = make_weight(rng, 8, 128, 64, 4, "bf16", bias_noise=1e-3)
    dq = mod.dequantize(w_q, s, b, 8, 128, 64, 4, "bf16")
    caught.append(not np.array_equal(dq, _independent_dequant(oracle.unpack(w_q, 128, 4), s, b, 64, "bf16")))
    fb = np.array([mod.c_f32_to_bits(float(v), "bf16") for v in _probe_floats(5000)], np.uint16)
    caught.append(not np.array_equal(fb, _bf16_torch(_probe_floats(5000))))
    # reference matmul and gather against numpy float64 of independently dequantized W
    x = make_x(rng, 5, 128, "bf16")
    wd = from_bits(_independent_dequant(oracle.unpack(w_q, 128, 4), s, b, 64, "bf16"), "bf16").astype(np.float64)
    xf = from_bits(x, "bf16").astype(np.float64)
    caught.append(not np.allclose(mod.qmm_ref(x, w_q, s, b, 5, 8, 128, 64, 4, "bf16"), xf @ wd.T,
                                  rtol=1e-12, atol=1e-10))
    lhs = np.array([4, 0, 3, 1], np.uint32)
    rhs = np.zeros(4, np.uint32)
    yg = mod.gather_qmm_ref(x, lhs, rhs, w_q, s, b, 4, 8, 128, 64, 4, "bf16")
    caught.append(not np.allclose(yg, xf[lhs] @ wd.T, rtol=1e-12, atol=1e-10))
    return caught


def _load_oracle_copy(oracle, so):
    import importlib

    spec = importlib.util.spec_from_file_location("mutant_oracle", oracle.__file__)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if so is not None:
        mod.LIB_PATH = so
        mod._lib = None
    return mod


def test_pins_hold_for_unmutated_oracle(oracle):
    assert not any(_pin_failures(_load_oracle_copy(oracle, None), oracle))


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(oracle, tmp_path, name):
    mod = _load_oracle_copy(oracle, _build_mutant(tmp_path, name))
    assert any(_pin_failures(mod, oracle)), f"mutation {name} slipped through every pin"
