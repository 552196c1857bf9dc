"""The MLX safetensors loader on the GPU: weights read from disk through
read_quantized_weight (safetensors_io.rs:43-134) give the reference's
committed outputs through the runtime node, the K-padded twin
(qwen2/weights.rs:297-307) gives the unpadded result bit for bit, and the
loaded bytes dequantize exactly as the oracle does.

The reference's fixtures hold the triple under the keys w_q / scales /
biases; the tests repack those arrays under MLX checkpoint keys
({base}.weight / .scales / .biases) with the `safetensors` package.
"""
import os

import numpy as np
import pytest
import torch
import safetensors.torch as stt

from cider_press_amd import _lib
from cider_press_amd import weights as W
from cider_press_amd.runtime import Quantization, Tensor, q4_gs64
from cider_press_amd.synthetic import from_bits, make_weight, make_x

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
BASE = "model.layers.0.mlp.down_proj"


def _ref_tol_ok(got_bits, ref_bits, dtype="bf16"):
    """The reference's own golden tolerance (qmm_parity.rs:80-87)."""
    a = from_bits(got_bits, dtype).astype(np.float64)
    e = from_bits(ref_bits, dtype).astype(np.float64)
    return np.all(np.abs(a - e) <= np.maximum(5e-2, 1e-2 * np.maximum(np.abs(a), np.abs(e))))


def _t(a: np.ndarray, dtype: str) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dtype == "u32":
        return torch.from_numpy(a.view(np.int32)).view(torch.uint32)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16 if dtype == "bf16" else torch.float16)


def _mlx_archive(path, base, w_q, s, b, dtype="bf16", extra=None):
    ents = {f"{base}.weight": _t(w_q, "u32"), f"{base}.scales": _t(s, dtype), f"{base}.biases": _t(b, dtype)}
    ents.update(extra or {})
    stt.save_file(ents, str(path), metadata={"format": "mlx"})
    return W.SafeTensors.open(path)


@pytest.mark.parametrize("fixture,m,k", [("qmv.safetensors", 1, 512), ("qmm_qwen2.safetensors", 8, 896)])
def test_loaded_reference_fixture_matches_reference_output(device, oracle, tmp_path, fixture, m, k):
    d = oracle.read_safetensors(os.path.join(GOLDEN, fixture))
    st = _mlx_archive(tmp_path / "model.safetensors", BASE, d["w_q"], d["scales"], d["biases"],
                      extra={"x": _t(d["x"], "bf16")})
    w = W.read_quantized_weight(st, BASE, q4_gs64(), device)
    assert w.shape() == (d["w_q"].shape[0], k) and w.k_logical() == k and w.dtype == "bf16"
    x = W.read_dense_tensor(st, "x", device)
    y = x.quantized_matmul(w).eval().cpu_slice()
    assert y.shape == d["y_ref"].shape
    assert _ref_tol_ok(y, d["y_ref"])
    ref = oracle.qmm_ref(d["x"].reshape(m, k), d["w_q"], d["scales"], d["biases"], m, d["w_q"].shape[0], k, 64, 4,
                         "bf16")
    rep = oracle.tolerance_report(y.reshape(m, -1), ref, d["x"], k, "bf16")
    assert rep["ok"], rep
    # The loaded bytes are the fixture's bytes: dequantization is bit-exact.
    deq = Tensor.dequantize_affine(w).eval().cpu_slice()
    assert np.array_equal(deq, oracle.dequantize(d["w_q"], d["scales"], d["biases"], d["w_q"].shape[0], k, 64, 4,
                                                 "bf16"))


def test_k_padded_twin_matches_unpadded_bit_for_bit(device, oracle, tmp_path):
    d = oracle.read_safetensors(os.path.join(GOLDEN, "qmm_qwen2.safetensors"))
    st = _mlx_archive(tmp_path / "m.safetensors", BASE, d["w_q"], d["scales"], d["biases"])
    w = W.read_quantized_weight(st, BASE, q4_gs64(), device)
    wp = W.read_quantized_weight_k_padded(st, BASE, q4_gs64(), device, 1024)
    assert wp.shape() == (896, 1024) and wp.k_logical() == 896
    for row in range(3):
        x = Tensor.from_host(device, d["x"][row])
        y = x.quantized_matmul(w).eval().cpu_slice()
        yp = Tensor.from_host(device, d["x"][row]).quantized_matmul(wp).eval().cpu_slice()
        assert np.array_equal(y, yp), f"row {row}"
        assert _ref_tol_ok(yp, d["y_ref"][row])
    # The padded twin's dense form is the padded bytes: zero pad columns.
    deq = Tensor.dequantize_affine(wp).eval().cpu_slice()
    assert np.array_equal(deq[:, :896], oracle.dequantize(d["w_q"], d["scales"], d["biases"], 896, 896, 64, 4, "bf16"))
    assert not deq[:, 896:].any()


@pytest.mark.parametrize("bits,gs,dtype", [(4, 32, "f16"), (8, 64, "bf16"), (4, 128, "bf16")])
def test_loaded_synthetic_weights(device, oracle, tmp_path, bits, gs, dtype):
    rng = np.random.default_rng(bits * 100 + gs)
    m, n, k = 5, 256, 1024
    w_q, s, b = make_weight(rng, n, k, gs, bits, dtype)
    x = make_x(rng, m, k, dtype)
    st = _mlx_archive(tmp_path / "w.safetensors", "lm_head", w_q, s, b, dtype=dtype)
    w = W.read_quantized_weight(st, "lm_head", Quantization(bits, gs), device)
    assert w.dtype == dtype
    y = Tensor.from_host(device, x, dtype).quantized_matmul(w).eval().cpu_slice()
    ref = oracle.qmm_ref(x, w_q, s, b, m, n, k, gs, bits, dtype)
    rep = oracle.tolerance_report(y, ref, x, k, dtype)
    assert rep["ok"], rep
    # A quantization that does not match the packed width is caught on load.
    other = Quantization(8 if bits == 4 else 4, gs)
    with pytest.raises((_lib.ShapeMismatch, _lib.InvalidArgument)):
        W.read_quantized_weight(st, "lm_head", other, device)
