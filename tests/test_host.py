"""Host-side checks of libcpq.so that need no GPU: the C ABI loads and exports
every declared symbol, the quantization descriptor matches the reference's
known answers, and the op validators reject what the reference rejects with
the same error classes (qmv.rs:89-163, qmm.rs:80-119,165-220,
dequantize.rs:66-104, quantization.rs:86-153)."""
import os
import re
import subprocess

import pytest

from cider_press_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "cpq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cpq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 40
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (cpq_\w+)", out))
    assert set(declared) <= exported


def test_version_string():
    assert b"gfx950" in _lib.lib().cpq_version()


# ---------------------------------------------------------------------------
# Quantization (mirrors quantization.rs:156-225)
# ---------------------------------------------------------------------------

def test_quantization_known_answers():
    from cider_press_amd.runtime import Quantization, q4_gs64

    q = q4_gs64()
    assert (q.bits, q.group_size) == (4, 64)
    for bits in (2, 3, 4, 5, 6, 8):
        Quantization(bits, 64)
    assert q.packed_word_count(64) == 8
    assert q.packed_word_count(4096) == 512
    with pytest.raises(_lib.InvalidArgument):
        q.packed_word_count(7)
    assert Quantization(3, 32).packed_word_count(32) == 3
    assert Quantization(3, 32).packed_word_count(64) == 6
    assert Quantization(5, 32).packed_word_count(32) == 5
    assert Quantization(5, 32).packed_word_count(128) == 20
    assert Quantization(6, 32).packed_word_count(32) == 6
    assert Quantization(6, 32).packed_word_count(64) == 12
    assert q.group_count(64) == 1
    assert q.group_count(4096) == 64
    with pytest.raises(_lib.InvalidArgument):
        q.group_count(100)


@pytest.mark.parametrize("bits,gs", [(1, 64), (0, 64), (7, 64), (16, 64), (4, 0), (4, 48), (3, 8)])
def test_quantization_rejects(bits, gs):
    from cider_press_amd.runtime import Quantization

    with pytest.raises(_lib.InvalidArgument):
        Quantization(bits, gs)


# ---------------------------------------------------------------------------
# Validators
# ---------------------------------------------------------------------------

BF16 = _lib.DTYPES["bf16"]
F16 = _lib.DTYPES["f16"]


def qmv_check(w, s, b, xa, y, k, gs=64, bits=4, dt=BF16):
    return _lib.lib().cpq_check_qmv_args(dt, w, s, b, xa, y, k, gs, bits)


def test_qmv_validator():
    n, k = 512, 512
    ok = qmv_check(n * k // 8, n * k // 64, n * k // 64, 2 * k, n, k)
    assert ok == _lib.OK
    # K-padded capacity: allocation smaller than physical K * 2
    assert qmv_check(n * k // 8, n * 8, n * 8, 2 * k - 2, n, k) == _lib.INVALID_ARGUMENT
    assert "K-padded" in _lib.last_error()
    assert qmv_check(0, 0, 0, 0, 0, 0) == _lib.INVALID_ARGUMENT                      # K = N = 0
    assert qmv_check(n * k // 8, n * 8, n * 8, 2 * k, n, k, gs=0) == _lib.INVALID_ARGUMENT
    assert qmv_check(n * 100 // 8, n * 2, n * 2, 200, n, 100) == _lib.INVALID_ARGUMENT  # K % gs
    assert qmv_check(n * k // 8 - 1, n * 8, n * 8, 2 * k, n, k) == _lib.INVALID_ARGUMENT
    assert "w_q.len()" in _lib.last_error()
    assert qmv_check(n * k // 8, n * 8 + 1, n * 8, 2 * k, n, k) == _lib.INVALID_ARGUMENT
    assert qmv_check(n * k // 8, n * 8, n * 8 - 1, 2 * k, n, k) == _lib.INVALID_ARGUMENT
    assert qmv_check(n * k * 7 // 32, n * 8, n * 8, 2 * k, n, k, bits=7) == _lib.KERNEL_NOT_FOUND
    assert "affine_qmv_fast_bfloat16_t_gs_64_b_7" in _lib.last_error()
    assert qmv_check(n * k // 8, n * k // 16, n * k // 16, 2 * k, n, k, gs=16) == _lib.KERNEL_NOT_FOUND
    assert qmv_check(n * k // 8, n * 8, n * 8, 2 * k, n, k, dt=F16) == _lib.OK


def test_qmm_validator():
    L = _lib.lib()
    m, n, k = 8, 896, 896

    def chk(w=n * k // 8, s=n * k // 64, b=n * k // 64, x=m * k, y=m * n, mm=m, nn=n, kk=k, gs=64, bits=4):
        return L.cpq_check_qmm_args(BF16, w, s, b, x, y, mm, nn, kk, gs, bits)

    assert chk() == _lib.OK
    assert chk(mm=0) == _lib.INVALID_ARGUMENT
    assert chk(nn=100, w=100 * k // 8, s=100 * k // 64, b=100 * k // 64, y=m * 100) == _lib.INVALID_ARGUMENT
    assert "multiple of 32" in _lib.last_error()
    assert chk(x=m * k - 1) == _lib.INVALID_ARGUMENT
    assert chk(y=m * n + 1) == _lib.INVALID_ARGUMENT
    assert chk(kk=900) == _lib.INVALID_ARGUMENT
    assert chk(mm=2**31) == _lib.INVALID_ARGUMENT
    assert chk(gs=16, s=n * k // 16, b=n * k // 16) == _lib.KERNEL_NOT_FOUND
    # checked products: N*K*bits that overflows usize must not wrap into a small length
    assert L.cpq_check_qmm_args(BF16, 0, 0, 0, 0, 0, 1, 2**31 - 32, 2**31 - 64, 64, 8) == _lib.INVALID_ARGUMENT


def test_dequantize_validator():
    L = _lib.lib()
    n_out = 128 * 64
    assert L.cpq_check_dequantize_args(BF16, n_out // 8, n_out // 64, n_out // 64, n_out, 64, 4) == _lib.OK
    assert L.cpq_check_dequantize_args(BF16, 0, 0, 0, 0, 64, 4) == _lib.OK  # empty is a no-op
    assert L.cpq_check_dequantize_args(BF16, 1, 1, 1, 63, 64, 4) == _lib.INVALID_ARGUMENT
    assert "pack_factor" in _lib.last_error()
    assert L.cpq_check_dequantize_args(BF16, 12, 1, 1, 96, 64, 4) == _lib.INVALID_ARGUMENT
    assert "group_size" in _lib.last_error()
    assert L.cpq_check_dequantize_args(BF16, n_out // 8, n_out // 64 + 1, n_out // 64, n_out, 64, 4) == \
        _lib.INVALID_ARGUMENT
    assert L.cpq_check_dequantize_args(BF16, n_out // 8 + 1, n_out // 64, n_out // 64, n_out, 64, 4) == \
        _lib.INVALID_ARGUMENT
    assert "w_q length" in _lib.last_error()
    assert L.cpq_check_dequantize_args(BF16, n_out * 3 // 32, n_out // 64, n_out // 64, n_out, 64, 3) == _lib.OK


def test_gather_validator():
    L = _lib.lib()
    e, n, k, rows = 8, 64, 256, 20

    def chk(x_rows=rows, w=e * n * k // 8, s=e * n * k // 64, b=e * n * k // 64, lhs=0, r=rows, y=rows * n,
            ne=e, nn=n, kk=k, gs=64, bits=4):
        return L.cpq_check_gather_args(BF16, x_rows, w, s, b, lhs, r, y, ne, nn, kk, gs, bits)

    assert chk() == _lib.OK
    assert chk(x_rows=5) == _lib.INVALID_ARGUMENT          # no lhs: x must have n_rows rows
    assert chk(x_rows=5, lhs=1) == _lib.OK
    assert chk(ne=0) == _lib.INVALID_ARGUMENT
    assert chk(w=e * n * k // 8 - 1) == _lib.INVALID_ARGUMENT
    assert chk(y=rows * n - 1) == _lib.INVALID_ARGUMENT
    assert chk(kk=250) == _lib.INVALID_ARGUMENT
    assert chk(bits=7, w=e * n * k * 7 // 32) == _lib.KERNEL_NOT_FOUND


def _gpu_visible() -> bool:
    try:
        out = subprocess.run(["rocm-smi", "--showid"], capture_output=True, text=True, timeout=20)
        return "GPU" in out.stdout and "Device" in out.stdout
    except Exception:
        return False


def test_no_device_maps_to_error_kind():
    """Without a GPU the device constructor fails with NoDevice (error.rs:21-23)."""
    if os.path.exists("/dev/kfd") and _gpu_visible():
        pytest.skip("a GPU is visible on this host")
    from cider_press_amd.kernels import Device

    with pytest.raises(_lib.NoDevice):
        Device.system_default()


def test_null_session_is_invalid_argument():
    L = _lib.lib()
    st = L.cpq_affine_qmv(None, BF16, None, 0, None, 0, None, 0, None, 0, None, 0, 0, 64, 4)
    assert st == _lib.INVALID_ARGUMENT


def test_completion_result_maps_stream_status():
    """A finished stream's HIP status maps to the session status the way
    completion_result does (commands.rs:378-400 and its unit tests at
    commands.rs:481-500): success is OK, any failure is CommandBufferFailed
    carrying the runtime's description."""
    L = _lib.lib()
    assert L.cpq_completion_result(0) == _lib.OK
    for code, name in ((700, "hipErrorIllegalAddress"), (719, "hipErrorLaunchFailure")):
        assert L.cpq_completion_result(code) == _lib.COMMAND_BUFFER_FAILED
        msg = L.cpq_last_error_message().decode()
        assert msg.startswith("GPU command stream failed: ") and name in msg, msg
    with pytest.raises(_lib.CommandBufferFailed, match="hipErrorIllegalAddress"):
        _lib.check(L.cpq_completion_result(700))


def test_session_hooks_reject_null_session():
    """The encoder hooks and profiled-session calls validate their session
    before anything else (no GPU needed)."""
    import ctypes

    L = _lib.lib()
    assert L.cpq_commands_record_input(None, 1) == _lib.INVALID_ARGUMENT
    assert L.cpq_commands_record_output(None, 1) == _lib.INVALID_ARGUMENT
    assert L.cpq_commands_record_unresolved_input(None) == _lib.INVALID_ARGUMENT
    assert L.cpq_commands_elide_next_barrier(None) == _lib.INVALID_ARGUMENT
    assert L.cpq_commands_begin_profiled_op(None, b"x") == _lib.INVALID_ARGUMENT
    n = ctypes.c_size_t(7)
    assert L.cpq_commands_commit_wait_resolve(None, None, 0, ctypes.byref(n)) == _lib.INVALID_ARGUMENT
    assert L.cpq_commands_profiled_info(None, None, None) == _lib.INVALID_ARGUMENT
    assert L.cpq_device_supports_stage_boundary_sampling(None) == 0
    h = ctypes.c_void_p()
    assert L.cpq_commands_create_profiled(None, 4, ctypes.byref(h)) == _lib.INVALID_ARGUMENT
