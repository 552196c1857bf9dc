"""GPU parity of the HIP path against the CPU oracle (all calls go through the C ABI).

Bars: dequantized weights bit-exact; matmul outputs within the BASELINE
tolerance against the oracle's unrounded float64 output
(max|y-y_ref| <= 1e-2*||x||_inf*sqrt(K)/64 and rel-L2 <= 2e-3), plus the
reference's own tolerance on its committed goldens
(max_relative=1e-2, epsilon=5e-2; crates/cider-press-kernels/tests/qmv_parity.rs:79-92).
"""
import os

import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.kernels import dequantize as kdq
from cider_press_amd.kernels import gather as kg
from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.kernels import qmv as kqmv
from cider_press_amd.synthetic import from_bits, make_routing, make_weight, make_x

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _ref_tol_ok(got_bits, ref_bits, dtype="bf16"):
    a = from_bits(got_bits, dtype).astype(np.float64)
    e = from_bits(ref_bits, dtype).astype(np.float64)
    return np.all(np.abs(a - e) <= np.maximum(5e-2, 1e-2 * np.maximum(np.abs(a), np.abs(e))))


def _upload_weight(device, w_q, s, b, dtype):
    return (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), dtype),
            device.upload(b.reshape(-1), dtype))


def run_qmv(device, library, w_q, s, b, x, n, k, gs, bits, dtype):
    W, S, B = _upload_weight(device, w_q, s, b, dtype)
    X = device.upload(x.reshape(-1), dtype)
    Y = device.alloc_buffer(n, dtype)
    cmds = device.commands()
    kqmv.affine_qmv(cmds, library, W, S, B, X, Y, k, gs, bits)
    cmds.commit_and_wait()
    return Y.to_numpy().reshape(1, n)


def run_qmm(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype, routed=False):
    W, S, B = _upload_weight(device, w_q, s, b, dtype)
    X = device.upload(x.reshape(-1), dtype)
    Y = device.alloc_buffer(m * n, dtype)
    cmds = device.commands()
    if routed:
        kqmm.quantized_matmul(cmds, W, S, B, X, Y, m, n, k, gs, bits)
    else:
        kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, gs, bits)
    cmds.commit_and_wait()
    return Y.to_numpy().reshape(m, n)


def assert_tol(oracle, got, ref, x, k, dtype, label=""):
    rep = oracle.tolerance_report(got, ref, x, k, dtype)
    assert rep["ok"], f"{label}: {rep}"
    return rep


# ---------------------------------------------------------------------------
# The reference's goldens, through the reference-shaped API
# ---------------------------------------------------------------------------

def test_golden_qmv_fast_bf16_gs64_b4(device, library, oracle):
    """qmv_parity.rs:37-93 on the HIP path."""
    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmv.safetensors"))
    W, S, B = _upload_weight(device, d["w_q"], d["scales"], d["biases"], "bf16")
    X = device.upload(d["x"], "bf16")
    Y = device.alloc_buffer(512, "bf16")
    cmds = device.commands()
    kqmv.affine_qmv_bf16(cmds, library, W, S, B, X, Y, 512, 64, 4)
    cmds.commit_and_wait()
    y = Y.to_numpy()
    assert _ref_tol_ok(y, d["y_ref"])
    ref = oracle.qmm_ref(d["x"].reshape(1, -1), d["w_q"], d["scales"], d["biases"], 1, 512, 512, 64, 4, "bf16")
    assert_tol(oracle, y.reshape(1, -1), ref, d["x"], 512, "bf16", "qmv golden")


def test_golden_qmm_t_bf16_gs64_b4(device, library, oracle):
    """qmm_parity.rs:35-88 (M=8, K=N=896) on the HIP path, both entry points."""
    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmm_qwen2.safetensors"))
    ref = oracle.qmm_ref(d["x"], d["w_q"], d["scales"], d["biases"], 8, 896, 896, 64, 4, "bf16")
    for routed in (False, True):
        y = run_qmm(device, library, d["w_q"], d["scales"], d["biases"], d["x"], 8, 896, 896, 64, 4, "bf16",
                    routed=routed)
        assert _ref_tol_ok(y, d["y_ref"])
        assert_tol(oracle, y, ref, d["x"], 896, "bf16", f"qmm golden routed={routed}")


# ---------------------------------------------------------------------------
# Dequantize: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (4, 128), (8, 64), (8, 32), (2, 64), (3, 32), (5, 64),
                                     (6, 128)])
def test_dequantize_bit_exact(device, library, oracle, dtype, bits, gs):
    rng = np.random.default_rng(bits * 1000 + gs)
    n, k = 96, 512
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype, bias_noise=1e-3)
    W, S, B = _upload_weight(device, w_q, s, b, dtype)
    out = device.alloc_buffer(n * k, dtype)
    cmds = device.commands()
    kdq.affine_dequantize(cmds, library, W, S, B, out, gs, bits)
    cmds.commit_and_wait()
    got = out.to_numpy().reshape(n, k)
    assert np.array_equal(got, oracle.dequantize(w_q, s, b, n, k, gs, bits, dtype))


@pytest.mark.parametrize("n,k,bits,gs", [
    (37, 96, 4, 32),       # 444 eight-element pieces: a partly filled last wave
    (45, 160, 8, 32),
    (4100, 8192, 4, 64),   # more pieces than one pass of the grid covers
])
def test_dequantize_bit_exact_ragged_and_large(device, library, oracle, n, k, bits, gs):
    """Sizes that leave a wave's 256 pieces partly filled, and one larger
    than a single pass of the grid-stride loop."""
    rng = np.random.default_rng(n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16", bias_noise=1e-3)
    W, S, B = _upload_weight(device, w_q, s, b, "bf16")
    out = device.upload(np.full(n * k + 64, 0x7FC0, np.uint16), "bf16")  # sentinel past the end
    cmds = device.commands()
    from cider_press_amd.kernels import _ptr
    _lib.check(_lib.lib().cpq_affine_dequantize(cmds.handle, _lib.DTYPES["bf16"], _ptr(W), len(W), _ptr(S), len(S),
                                                _ptr(B), len(B), _ptr(out), n * k, gs, bits))
    cmds.commit_and_wait()
    got = out.to_numpy()
    assert np.array_equal(got[: n * k].reshape(n, k), oracle.dequantize(w_q, s, b, n, k, gs, bits, "bf16"))
    assert (got[n * k:] == 0x7FC0).all()


def test_dequantize_reference_entry_point_and_special_values(device, library, oracle):
    """affine_dequantize_bf16_gs64_b4 (dequantize.rs:58-137) at the reference
    test's 128x64 shape, with ties, tiny and large scales mixed in."""
    rng = np.random.default_rng(99)
    rows, cols = 128, 64
    w_q, s, b = make_weight(rng, rows, cols, 64, 4, "bf16")
    special_s = np.array([0x0001, 0x0080, 0x3F80, 0x3F81, 0x4780, 0x0000, 0x8080, 0x3C01], np.uint16)
    special_b = np.array([0x0000, 0x8001, 0xBF80, 0x3F7F, 0xC780, 0x7F00, 0x0080, 0xBC01], np.uint16)
    s = s.copy(); b = b.copy()
    s[:8, 0] = special_s
    b[:8, 0] = special_b
    W, S, B = _upload_weight(device, w_q, s, b, "bf16")
    out = device.alloc_buffer(rows * cols, "bf16")
    cmds = device.commands()
    kdq.affine_dequantize_bf16_gs64_b4(cmds, library, W, S, B, out)
    cmds.commit_and_wait()
    assert np.array_equal(out.to_numpy().reshape(rows, cols),
                          oracle.dequantize(w_q, s, b, rows, cols, 64, 4, "bf16"))


def test_dequantize_empty_is_noop(device, library):
    W = device.alloc_buffer(0, "u32")
    S = device.alloc_buffer(0, "bf16")
    out = device.alloc_buffer(0, "bf16")
    cmds = device.commands()
    kdq.affine_dequantize_bf16_gs64_b4(cmds, library, W, S, S, out)
    cmds.commit_and_wait()


# ---------------------------------------------------------------------------
# qmv (decode)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,gs,bits,dtype,noise", [
    (2048, 2048, 64, 4, "f16", 1e-3),      # config 1
    (12288, 4096, 64, 4, "bf16", 0.0),     # config 2a (fused gate+up)
    (4096, 12288, 64, 4, "bf16", 0.0),     # config 2b (down)
    (4096, 4096, 32, 4, "bf16", 0.0),      # config 4, 4-bit gs32
    (4096, 4096, 64, 8, "bf16", 0.0),      # config 4, 8-bit gs64
    (896, 896, 64, 4, "bf16", 0.0),        # Qwen2.5-0.5B q/o (generic-variant shape)
    (131, 960, 64, 4, "bf16", 0.0),        # ragged N, K not a 512 multiple
    (7, 128, 128, 4, "bf16", 0.0),         # tiny
    (512, 512, 64, 2, "bf16", 0.0),
    (256, 512, 32, 3, "bf16", 0.0),
    (256, 512, 64, 5, "f16", 0.0),
    (256, 512, 64, 6, "bf16", 0.0),
])
def test_qmv_parity(device, library, oracle, n, k, gs, bits, dtype, noise):
    rng = np.random.default_rng(n + k + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype, bias_noise=noise)
    x = make_x(rng, 1, k, dtype)
    y = run_qmv(device, library, w_q, s, b, x, n, k, gs, bits, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, 1, n, k, gs, bits, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"qmv {n}x{k} b{bits} gs{gs} {dtype}")


def test_qmv_k_padding_is_bit_exact(device, library, oracle):
    """K-padding contract (qmv_padded_parity.rs:10-72): zero q/s/b pad groups and a
    zeroed activation tail add exactly +0.0, for both pad targets (960 and 1024)."""
    rng = np.random.default_rng(5)
    n, k_log, gs = 896, 896, 64
    w_q, s, b = make_weight(rng, n, k_log, gs, 4, "bf16")
    x = make_x(rng, 1, k_log, "bf16")
    base = run_qmv(device, library, w_q, s, b, x, n, k_log, gs, 4, "bf16")
    for k_pad in (960, 1024):
        wp = np.zeros((n, k_pad * 4 // 32), np.uint32); wp[:, :w_q.shape[1]] = w_q
        sp = np.zeros((n, k_pad // gs), np.uint16); sp[:, :s.shape[1]] = s
        bp = np.zeros((n, k_pad // gs), np.uint16); bp[:, :b.shape[1]] = b
        W, S, B = _upload_weight(device, wp, sp, bp, "bf16")
        X = device.upload(x.reshape(-1), "bf16")  # 896 elements; 512-B rounding covers 1024
        assert X.alloc_len >= k_pad * 2
        Y = device.alloc_buffer(n, "bf16")
        cmds = device.commands()
        kqmv.affine_qmv_bf16(cmds, library, W, S, B, X, Y, k_pad, gs, 4)
        cmds.commit_and_wait()
        assert np.array_equal(Y.to_numpy(), base.reshape(-1)), k_pad
    # negative control: a corrupted logical weight byte changes the output
    w_bad = w_q.copy(); w_bad[0, 0] ^= 0x5
    assert not np.array_equal(run_qmv(device, library, w_bad, s, b, x, n, k_log, gs, 4, "bf16"), base)


def test_qmv_capacity_rejected_before_launch(device, library):
    W = device.alloc_buffer(8 * 1024 // 8, "u32")
    S = device.alloc_buffer(8 * 16, "bf16")
    X = device.alloc_buffer(256, "bf16")      # 512 B allocation, K=1024 needs 2048 B
    Y = device.alloc_buffer(8, "bf16")
    cmds = device.commands()
    with pytest.raises(_lib.InvalidArgument):
        kqmv.affine_qmv_bf16(cmds, library, W, S, S, X, Y, 1024, 64, 4)


# ---------------------------------------------------------------------------
# qmm (prefill) and the routed small-M path
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k,gs,bits,dtype", [
    (512, 4096, 4096, 64, 4, "bf16"),      # config 3a
    (512, 1024, 4096, 64, 8, "bf16"),
    (300, 640, 1024, 32, 4, "bf16"),       # ragged M
    (129, 256, 512, 128, 4, "f16"),
    (64, 4096, 4096, 64, 4, "bf16"),       # config 4 at M=64
    (33, 96, 256, 64, 2, "bf16"),
    (40, 64, 384, 32, 6, "bf16"),
    (2, 32, 128, 64, 4, "bf16"),
    (96, 160, 4096, 32, 4, "f16"),         # staged kernel: 3-slot ring (128 groups), N and M tails
    (136, 224, 2048, 64, 8, "f16"),        # staged kernel, 8-bit, f16
    (256, 128, 12288, 128, 4, "bf16"),     # staged kernel, long K
])
def test_qmm_t_parity(device, library, oracle, m, n, k, gs, bits, dtype):
    rng = np.random.default_rng(m * 7 + n + bits)
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, bits, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"qmm {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 2, 4, 15, 16, 17, 31, 32, 33, 64, 65, 200])
@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 64), (4, 32)])
def test_quantized_matmul_routes_all_m(device, library, oracle, m, bits, gs):
    n, k = 512, 1024
    rng = np.random.default_rng(m * 3 + bits + gs)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    x = make_x(rng, m, k, "bf16")
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, bits, "bf16", routed=True)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", f"routed m={m}")


# Routed small-M shapes (up to 64 rows while N <= 8192) across the three
# small-M kernels: the decode layout with M rows, the tiled small-M kernel and
# the slab kernel.
@pytest.mark.parametrize("m,n,k,bits,gs", [
    (5, 8192, 1024, 4, 64),     # 1 row block, 4 waves (512 slabs)
    (20, 8192, 1024, 8, 64),    # 2 row blocks, 4 waves
    (20, 4096, 2048, 4, 32),    # 2 row blocks, 8 waves
    (48, 4096, 1024, 4, 64),    # 4 row blocks (M <= 64 at N <= 8192)
    (64, 8192, 512, 4, 128),    # 33..64 rows with N >= 32 x CUs: two slabs per workgroup
    (48, 8192, 256, 4, 64),     # two slabs, three row blocks
    (36, 8192, 512, 8, 32),     # two slabs, 8-bit, a ragged row block
])
def test_small_m_wave_counts(device, library, oracle, m, n, k, bits, gs):
    rng = np.random.default_rng(m + n + k)
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    x = make_x(rng, m, k, "bf16")
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, bits, "bf16", routed=True)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", f"small-M m={m} n={n}")


@pytest.mark.parametrize("m,n,k,gs", [
    (4, 256, 12288, 32),    # slab constants 98 KiB: past the default dynamic-LDS limit
    (40, 128, 12288, 32),   # 64-row blocks at the same size
    (3, 64, 40960, 32),     # constants would not fit in LDS: the prefill path takes it
])
def test_small_m_long_k(device, library, oracle, m, n, k, gs):
    rng = np.random.default_rng(m + k)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, 4, "bf16", routed=True)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", f"small-M long K m={m} k={k}")


def test_gather_per_slab_long_k(device, library, oracle):
    """The per-slab routed kernel (K beyond the expert-major kernel's LDS, and
    more rows than the decode kernel takes) with 98 KiB of slab constants."""
    rng = np.random.default_rng(12288)
    e, n, k, gs, rows = 2, 64, 12288, 32, 70
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, rows, k, "bf16")
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    y = run_gather(device, library, x, w_q, s, b, None, rhs, rows, n, k, e, gs, 4, "bf16", False)
    ref = oracle.gather_qmm_ref(x, None, rhs, w_q, s, b, rows, n, k, gs, 4, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", "gather per-slab long K")


# The 4-bit prefill path runs the two-waves-per-SIMD kernel ("dma": 128 x 128
# tiles, both operands streamed into LDS, K split over 1, 2 or 4 workgroups,
# partial tiles summed by the last to finish), else the one-wave wide-tile
# kernel ("wide"), else the staged kernel.  CPQ_QMM_SPLIT forces the split,
# CPQ_QMM_DMA=0 / CPQ_QMM_WIDE=0 turn the first two off.
_KERNEL_ENV = {"dma": ("1", "1"), "wide": ("0", "1"), "staged": ("0", "0")}


def _use_kernel(monkeypatch, kern):
    dma, wide = _KERNEL_ENV[kern]
    monkeypatch.setenv("CPQ_QMM_DMA", dma)
    monkeypatch.setenv("CPQ_QMM_WIDE", wide)
    # affine_qmm_t sends small M to the small-M kernels; these tests force
    # the prefill kernels at every M.
    monkeypatch.setenv("CPQ_SKINNY_MAX_M", "1")


@pytest.mark.parametrize("kern", ["dma", "wide"])
@pytest.mark.parametrize("m,n,k,gs,dtype,split", [
    (256, 512, 2048, 64, "bf16", 1),
    (256, 512, 2048, 64, "bf16", 2),
    (512, 4096, 4096, 64, "bf16", 2),      # config 3a
    (300, 640, 4096, 32, "bf16", 4),       # ragged M
    (200, 352, 4096, 64, "f16", 2),        # ragged M and a partial column tile
    (200, 352, 4096, 64, "f16", 4),
    (129, 256, 2048, 128, "bf16", 1),
    (129, 256, 2048, 128, "bf16", 2),
    (64, 4096, 4096, 64, "bf16", 4),       # config 4 at M = 64
])
def test_qmm_wide_parity(device, library, oracle, monkeypatch, m, n, k, gs, dtype, split, kern):
    _use_kernel(monkeypatch, kern)
    monkeypatch.setenv("CPQ_QMM_SPLIT", str(split))
    rng = np.random.default_rng(m + n + split)
    w_q, s, b = make_weight(rng, n, k, gs, 4, dtype)
    x = make_x(rng, m, k, dtype)
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, 4, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"{kern} split={split} {m}x{n}x{k}")


# Scale / bias pairs outside the single-FMA fast path's exactness range: a
# tiny scale under a much larger bias (bf16 exponent gap 24), or an f16
# subnormal scale.  Their column tile takes the generic dequantization; the
# other tiles stay fast.
_SLOW_SB = {"bf16": (0x3000, 0x3C23), "f16": (0x0001, 0x211F)}


_KERNEL_SPLITS = [("dma", 2), ("dma", 1), ("wide", 2), ("wide", 1), ("staged", 1)]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("kern,split", _KERNEL_SPLITS)
def test_qmm_mixed_fast_and_slow_tiles(device, library, oracle, monkeypatch, dtype, kern, split):
    _use_kernel(monkeypatch, kern)
    monkeypatch.setenv("CPQ_QMM_SPLIT", str(split))
    m, n, k, gs = 160, 384, 2048, 64
    rng = np.random.default_rng(5)
    w_q, s, b = make_weight(rng, n, k, gs, 4, dtype)
    s[130, 3], b[130, 3] = _SLOW_SB[dtype]
    s[300, k // gs - 1], b[300, k // gs - 1] = _SLOW_SB[dtype]
    x = make_x(rng, m, k, dtype)
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, 4, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"mixed {kern} split={split}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("kern,split", _KERNEL_SPLITS)
def test_qmm_zero_scales_and_biases(device, library, oracle, monkeypatch, dtype, kern, split):
    """Zero scales or biases fail the packed exponent check but pass the
    exact predicate, so their tiles stay on the fast dequantization; a -0
    bias under a negative scale does not (the fast path would give +0)."""
    _use_kernel(monkeypatch, kern)
    monkeypatch.setenv("CPQ_QMM_SPLIT", str(split))
    m, n, k, gs = 130, 384, 2048, 64
    rng = np.random.default_rng(9)
    w_q, s, b = make_weight(rng, n, k, gs, 4, dtype)
    s[5, 0] = 0                      # zero scale: w = b
    b[40, 7] = 0                     # zero bias
    s[200, 3], b[200, 3] = 0, 0      # both zero
    s[301, 31] = s[301, 31] | 0x8000  # negative scale over a -0 bias: generic path
    b[301, 31] = 0x8000
    x = make_x(rng, m, k, dtype)
    y = run_qmm(device, library, w_q, s, b, x, m, n, k, gs, 4, dtype)
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"zeros {kern} split={split}")


@pytest.mark.parametrize("kern", ["dma", "wide"])
def test_qmm_wide_split_is_deterministic(device, library, oracle, monkeypatch, kern):
    """The split-K sum adds the parts in k order whatever order the
    workgroups finish in: repeated calls give identical bits."""
    _use_kernel(monkeypatch, kern)
    monkeypatch.setenv("CPQ_QMM_SPLIT", "4")
    m, n, k, gs = 512, 1024, 4096, 64
    rng = np.random.default_rng(9)
    w_q, s, b = make_weight(rng, n, k, gs, 4, "bf16")
    x = make_x(rng, m, k, "bf16")
    W, S, B = _upload_weight(device, w_q, s, b, "bf16")
    X = device.upload(x.reshape(-1), "bf16")
    outs = []
    cmds = device.commands()
    for _ in range(3):
        Y = device.alloc_buffer(m * n, "bf16")
        kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, gs, 4)
        cmds.commit_and_wait()
        outs.append(Y.to_numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, 4, "bf16")
    assert_tol(oracle, outs[0].reshape(m, n), ref, x, k, "bf16", "wide split=4")


def test_qmm_rejects_unaligned_n(device, library):
    W = device.alloc_buffer(40 * 128 // 8, "u32")
    S = device.alloc_buffer(40 * 2, "bf16")
    X = device.alloc_buffer(4 * 128, "bf16")
    Y = device.alloc_buffer(4 * 40, "bf16")
    cmds = device.commands()
    with pytest.raises(_lib.InvalidArgument):
        kqmm.affine_qmm_t_bf16(cmds, library, W, S, S, X, Y, 4, 40, 128, 64, 4)


# ---------------------------------------------------------------------------
# gather_qmm (routed experts)
# ---------------------------------------------------------------------------

def _experts(rng, e, n, k, gs, bits, dtype):
    ws = [make_weight(rng, n, k, gs, bits, dtype) for _ in range(e)]
    return (np.concatenate([w[0] for w in ws]), np.concatenate([w[1] for w in ws]),
            np.concatenate([w[2] for w in ws]))


def run_gather(device, library, x, w_q, s, b, lhs, rhs, n_rows, n, k, e, gs, bits, dtype, sorted_idx):
    X = device.upload(x.reshape(-1), dtype)
    W, S, B = _upload_weight(device, w_q, s, b, dtype)
    L = None if lhs is None else device.upload(lhs, "u32")
    R = device.upload(rhs, "u32")
    Y = device.alloc_buffer(n_rows * n, dtype)
    cmds = device.commands()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L, R, Y, n_rows, n, k, e, gs, bits, sorted_idx,
                         x_rows=x.shape[0])
    cmds.commit_and_wait()
    return Y.to_numpy().reshape(n_rows, n)


@pytest.mark.parametrize("sorted_idx", [False, True])
def test_gather_moe_small(device, library, oracle, sorted_idx):
    rng = np.random.default_rng(21)
    e, n, k, gs, tokens, top = 16, 96, 512, 64, 40, 4
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, tokens, k, "bf16")
    route = make_routing(rng, tokens, top, e).reshape(-1)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), top)
    rhs = route.astype(np.uint32)
    if sorted_idx:
        order = np.argsort(rhs, kind="stable")
        lhs, rhs = lhs[order], rhs[order]
    y = run_gather(device, library, x, w_q, s, b, lhs, rhs, len(rhs), n, k, e, gs, 4, "bf16", sorted_idx)
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, len(rhs), n, k, gs, 4, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", "gather")


def test_gather_config5_full(device, library, oracle):
    """Config 5: 128 experts [768, 2048], 256 tokens, top-8 without replacement."""
    rng = np.random.default_rng(0)
    e, n, k, gs, tokens, top = 128, 768, 2048, 64, 256, 8
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, tokens, k, "bf16")
    rhs = make_routing(rng, tokens, top, e).reshape(-1).astype(np.uint32)
    lhs = np.repeat(np.arange(tokens, dtype=np.uint32), top)
    y = run_gather(device, library, x, w_q, s, b, lhs, rhs, len(rhs), n, k, e, gs, 4, "bf16", False)
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, len(rhs), n, k, gs, 4, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", "gather cfg5")


def test_gather_identity_lhs_and_skewed_routing(device, library, oracle):
    """lhs NULL, one expert receiving 150 rows (several 64-row passes), empty experts."""
    rng = np.random.default_rng(22)
    e, n, k, gs, rows = 6, 64, 256, 32, 170
    w_q, s, b = _experts(rng, e, n, k, gs, 8, "bf16")
    x = make_x(rng, rows, k, "bf16")
    rhs = np.full(rows, 2, np.uint32)
    rhs[:20] = 5
    y = run_gather(device, library, x, w_q, s, b, None, rhs, rows, n, k, e, gs, 8, "bf16", False)
    ref = oracle.gather_qmm_ref(x, None, rhs, w_q, s, b, rows, n, k, gs, 8, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", "gather skewed")


@pytest.mark.parametrize("bits,k,dtype", [(4, 1024, "f16"), (8, 2048, "bf16"), (4, 4096, "bf16")])
def test_gather_expert_kernel_passes(device, library, oracle, bits, k, dtype):
    """Expert-major kernel: experts with 0, a few, and more rows than one pass holds
    (16 * MB rows, MB = 4 / 2 / 1 at K = 1024 / 2048 / 4096), unsorted routing."""
    rng = np.random.default_rng(31 + bits + k)
    e, n, gs, rows = 5, 272, 64, 150
    w_q, s, b = _experts(rng, e, n, k, gs, bits, dtype)
    x = make_x(rng, 40, k, dtype)
    rhs = rng.choice(np.array([0, 1, 1, 3, 3, 3, 3, 3], np.uint32), size=rows)  # experts 2, 4 empty
    lhs = rng.integers(0, 40, size=rows).astype(np.uint32)
    y = run_gather(device, library, x, w_q, s, b, lhs, rhs, rows, n, k, e, gs, bits, dtype, False)
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, rows, n, k, gs, bits, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"gather expert {bits}b K={k}")


def test_gather_unsorted_past_kept_blocks(device, library, oracle):
    """Unsorted routing over 3000 rows (47 blocks of 64): each wave counts
    its first four blocks in one round and keeps their match masks, the
    blocks past 2048 rows take the one-block-at-a-time path; experts with
    many 64-row passes place their rows from both."""
    rng = np.random.default_rng(47)
    e, n, k, gs, rows, xr = 3, 48, 256, 64, 3000, 64
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, xr, k, "bf16")
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    rhs[2500:] = 1  # the tail blocks: one expert only
    lhs = rng.integers(0, xr, size=rows).astype(np.uint32)
    y = run_gather(device, library, x, w_q, s, b, lhs, rhs, rows, n, k, e, gs, 4, "bf16", False)
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, rows, n, k, gs, 4, "bf16")
    assert_tol(oracle, y, ref, x, k, "bf16", "gather unsorted 3000 rows")


@pytest.mark.parametrize("gs,k,dtype,bits,n", [
    (64, 768, "bf16", 4, 512),     # 6 units per slab: scale / bias pairs of steps (8-byte loads)
    (64, 768, "f16", 4, 512),
    (64, 1536, "bf16", 8, 512),    # 12 units: quads of 4 steps (16-byte loads)
    (128, 1024, "bf16", 4, 512),   # quads of 4 steps, gs 128 (8-byte loads)
    (128, 1024, "f16", 4, 512),
    (128, 768, "bf16", 4, 512),    # 6 units at gs 128: per-step loads
    (64, 384, "bf16", 4, 512),     # 3 units: per-step loads
    (32, 1024, "bf16", 4, 512),    # gs 32: per-step loads
    (128, 384, "bf16", 4, 100),    # n G = 300: the vote reads pair by pair; ragged last slab
])
def test_gather_scale_bias_step_groupings(device, library, oracle, gs, k, dtype, bits, n):
    """Every scale / bias load grouping of the expert-major kernel, with
    several slabs per wave (3 experts) and sorted routing (80 rows: past the
    decode kernel's 64)."""
    rng = np.random.default_rng(gs + k + bits + n)
    e, rows = 3, 80
    w_q, s, b = _experts(rng, e, n, k, gs, bits, dtype)
    x = make_x(rng, 30, k, dtype)
    rhs = np.sort(rng.integers(0, e, size=rows)).astype(np.uint32)
    lhs = rng.integers(0, 30, size=rows).astype(np.uint32)
    y = run_gather(device, library, x, w_q, s, b, lhs, rhs, rows, n, k, e, gs, bits, dtype, True)
    ref = oracle.gather_qmm_ref(x, lhs, rhs, w_q, s, b, rows, n, k, gs, bits, dtype)
    assert_tol(oracle, y, ref, x, k, dtype, f"gather gs={gs} K={k} {dtype} {bits}b")


def test_gather_out_of_range_index_reported(device, library, oracle):
    rng = np.random.default_rng(23)
    e, n, k, gs, rows = 4, 32, 128, 64, 8
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, rows, k, "bf16")
    rhs = np.array([0, 1, 2, 3, 9, 1, 0, 2], np.uint32)   # row 4 names expert 9
    X = device.upload(x.reshape(-1), "bf16")
    W, S, B = _upload_weight(device, w_q, s, b, "bf16")
    R = device.upload(rhs, "u32")
    Y = device.upload(np.full(rows * n, 0x3F80, np.uint16), "bf16")
    cmds = device.commands()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, None, R, Y, rows, n, k, e, gs, 4)
    with pytest.raises(_lib.InvalidArgument):
        cmds.commit_and_wait()
    y = Y.to_numpy().reshape(rows, n)
    assert np.all(y[4] == 0)
    ok = np.array([r for r in range(rows) if r != 4])
    ref = oracle.gather_qmm_ref(x[ok], None, rhs[ok], w_q, s, b, len(ok), n, k, gs, 4, "bf16")
    assert_tol(oracle, y[ok], ref, x[ok], k, "bf16", "gather valid rows")
    cmds.commit_and_wait()  # the status word was cleared by the failed wait


@pytest.mark.parametrize("k,gs", [(256, 64), (160, 32)])  # expert-major kernel / per-slab kernel
def test_gather_index_validation_many_rows(device, library, oracle, k, gs):
    """Bad expert and activation indices spread over 1500 rows (checked by
    several workgroups): those rows are zeroed and counted, the others are
    exact; a sorted routing with one descent is reported once."""
    rng = np.random.default_rng(k)
    e, n, rows, xr = 4, 48, 1500, 50
    w_q, s, b = _experts(rng, e, n, k, gs, 4, "bf16")
    x = make_x(rng, xr, k, "bf16")
    rhs = rng.integers(0, e, size=rows).astype(np.uint32)
    lhs = rng.integers(0, xr, size=rows).astype(np.uint32)
    rhs[[0, 700]] = [e, 99]
    lhs[[5, 1499]] = [xr, 0xFFFFFFFF]
    bad = np.array([0, 5, 700, 1499])
    X = device.upload(x.reshape(-1), "bf16")
    W, S, B = _upload_weight(device, w_q, s, b, "bf16")
    L, R = device.upload(lhs, "u32"), device.upload(rhs, "u32")
    Y = device.upload(np.full(rows * n, 0x3F80, np.uint16), "bf16")
    cmds = device.commands()
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L, R, Y, rows, n, k, e, gs, 4, x_rows=xr)
    with pytest.raises(_lib.InvalidArgument, match="affine_gather_qmm: 4 row"):
        cmds.commit_and_wait()
    y = Y.to_numpy().reshape(rows, n)
    assert not y[bad].any()
    ok = np.setdiff1d(np.arange(rows), bad)
    ref = oracle.gather_qmm_ref(x, lhs[ok], rhs[ok], w_q, s, b, len(ok), n, k, gs, 4, "bf16")
    assert_tol(oracle, y[ok], ref, x, k, "bf16", "gather valid rows")

    srt = np.sort(rng.integers(0, e, size=rows)).astype(np.uint32)
    i = int(np.flatnonzero(srt[:-1] < srt[1:])[0])
    srt[i], srt[i + 1] = srt[i + 1], srt[i]  # exactly one descent
    R2 = device.upload(srt, "u32")
    L2 = device.upload(rng.integers(0, xr, size=rows).astype(np.uint32), "u32")
    kg.affine_gather_qmm(cmds, library, X, W, S, B, L2, R2, Y, rows, n, k, e, gs, 4, sorted_indices=True,
                         x_rows=xr)
    with pytest.raises(_lib.InvalidArgument, match="affine_gather_qmm: 1 row"):
        cmds.commit_and_wait()
    cmds.commit_and_wait()


# ---------------------------------------------------------------------------
# Runtime node (QuantizedWeight / Tensor.quantized_matmul / eval)
# ---------------------------------------------------------------------------

def test_runtime_node_qmv_and_qmm(device, oracle):
    from cider_press_amd.runtime import QuantizedWeight, Tensor, q4_gs64

    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmm_qwen2.safetensors"))
    w = QuantizedWeight.from_bytes(device, (896, 896), q4_gs64(), d["w_q"], d["scales"], d["biases"])
    x = Tensor.from_host(device, d["x"])
    y = x.quantized_matmul(w, True)
    assert y.shape() == (8, 896)
    y.eval()
    assert _ref_tol_ok(y.cpu_slice(), d["y_ref"])
    # rank-1 activation = decode (M == 1 -> qmv)
    x1 = Tensor.from_host(device, d["x"][0])
    y1 = x1.quantized_matmul(w).eval()
    assert y1.shape() == (896,)
    assert _ref_tol_ok(y1.cpu_slice(), d["y_ref"][0])
    with pytest.raises(_lib.InvalidArgument):
        x.quantized_matmul(w, False)
    with pytest.raises(_lib.InvalidArgument):
        Tensor.from_host(device, d["x"][:, :640]).quantized_matmul(w)


def test_runtime_k_padded_weight(device, oracle):
    from cider_press_amd.runtime import QuantizedWeight, Tensor, q4_gs64

    rng = np.random.default_rng(31)
    n, k_log, k_pad, gs = 128, 896, 1024, 64
    w_q, s, b = make_weight(rng, n, k_log, gs, 4, "bf16")
    wp = np.zeros((n, k_pad // 8), np.uint32); wp[:, :k_log // 8] = w_q
    sp = np.zeros((n, k_pad // gs), np.uint16); sp[:, :k_log // gs] = s
    bp = np.zeros((n, k_pad // gs), np.uint16); bp[:, :k_log // gs] = b
    w = QuantizedWeight.from_bytes_k_padded(device, (n, k_pad), k_log, q4_gs64(), wp, sp, bp)
    x = make_x(rng, 1, k_log, "bf16")
    y = Tensor.from_host(device, x[0]).quantized_matmul(w).eval().cpu_slice()
    ref = oracle.qmm_ref(x, w_q, s, b, 1, n, k_log, gs, 4, "bf16")
    assert_tol(oracle, y.reshape(1, n), ref, x, k_log, "bf16", "k padded")
    # M > 1 against a padded weight self-rejects (eval.rs:1374-1376)
    xm = Tensor.from_host(device, make_x(rng, 4, k_log, "bf16"))
    with pytest.raises(_lib.InvalidArgument):
        xm.quantized_matmul(w).eval()


def test_runtime_dequantize_node(device, oracle):
    from cider_press_amd.runtime import QuantizedWeight, Quantization, Tensor

    rng = np.random.default_rng(32)
    n, k, gs = 64, 256, 32
    w_q, s, b = make_weight(rng, n, k, gs, 8, "f16")
    w = QuantizedWeight.from_bytes(device, (n, k), Quantization(8, gs), w_q, s, b, dtype="f16")
    out = Tensor.dequantize_affine(w).eval().cpu_slice()
    assert np.array_equal(out, oracle.dequantize(w_q, s, b, n, k, gs, 8, "f16"))
