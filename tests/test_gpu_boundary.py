"""Session-level calls of the drop-in boundary on the GPU: the profiled
session (per-op GPU windows; the reference's gpu_sampler.rs tests at
crates/cider-press-kernels/tests/gpu_sampler.rs:9-68 and the
begin_profiled_op / commit_wait_resolve loop of tests/qmv_dispatch_bench.rs:51-79),
the encoder hazard hooks, the allocation slack contract
(tests/alloc_slack_zeroed.rs:33-83) and the QuantizedWeight::from_bytes
rejects (runtime/src/quantized.rs:363-487)."""
import ctypes

import numpy as np
import pytest

from cider_press_amd import _lib
from cider_press_amd.kernels import qmm as kqmm
from cider_press_amd.kernels import qmv as kqmv
from cider_press_amd.runtime import Quantization, QuantizedWeight, q4_gs64
from cider_press_amd.synthetic import make_weight, make_x

pytestmark = pytest.mark.gpu


def _qmv_case(device, rng, n=4096, k=4096, gs=64, bits=4):
    w_q, s, b = make_weight(rng, n, k, gs, bits, "bf16")
    W = device.upload(w_q.reshape(-1), "u32")
    S = device.upload(s.reshape(-1), "bf16")
    B = device.upload(b.reshape(-1), "bf16")
    X = device.upload(make_x(rng, 1, k, "bf16").reshape(-1), "bf16")
    return W, S, B, X


def _plain_qmv(device, library, W, S, B, X, n, k):
    Y = device.alloc_buffer(n, "bf16")
    cmds = device.commands()
    kqmv.affine_qmv(cmds, library, W, S, B, X, Y, k, 64, 4)
    cmds.commit_and_wait()
    return Y.to_numpy()


def test_device_reports_stage_boundary_sampling(device):
    assert device.supports_stage_boundary_sampling()
    period = device.gpu_timestamp_period_ns()
    assert 0.1 <= period <= 10_000.0


def test_profiled_session_capacity_starts_empty(device):
    cmds = device.commands_profiled(4)
    assert cmds.recorded_ops() == 0
    assert cmds.sample_capacity() == 8  # two timestamps per op


def test_profiled_session_times_each_dispatch(device, library):
    """Two labelled qmv dispatches give two ordered, non-overlapping windows,
    and the outputs are bit-equal to an unprofiled session's."""
    rng = np.random.default_rng(11)
    n = k = 4096
    W, S, B, X = _qmv_case(device, rng, n, k)
    want = _plain_qmv(device, library, W, S, B, X, n, k)
    Ya, Yb = device.alloc_buffer(n, "bf16"), device.alloc_buffer(n, "bf16")
    cmds = device.commands_profiled(2)
    cmds.begin_profiled_op("qmv_a")
    kqmv.affine_qmv(cmds, library, W, S, B, X, Ya, k, 64, 4)
    cmds.begin_profiled_op("qmv_b")
    kqmv.affine_qmv(cmds, library, W, S, B, X, Yb, k, 64, 4)
    assert cmds.recorded_ops() == 2
    segs = cmds.commit_wait_resolve()
    print("segments", segs, flush=True)
    assert [s.label for s in segs] == ["qmv_a", "qmv_b"]
    assert segs[0].start_tick == 0
    for s in segs:
        assert s.end_tick >= s.start_tick
        # A 4096 x 4096 4-bit qmv streams 9.4 MB: at least ~1 us at 8 TB/s.
        assert s.ticks() * device.gpu_timestamp_period_ns() > 500
    assert segs[1].start_tick >= segs[0].end_tick
    assert np.array_equal(Ya.to_numpy(), want) and np.array_equal(Yb.to_numpy(), want)
    # The batch is consumed: the session starts a new one.
    assert cmds.recorded_ops() == 0


def test_profiled_session_window_matches_event_timing(device, library):
    """A prefill op's profiled window agrees with HIP events around the
    same launch on an ordinary session (both time one kernel launch)."""
    from cider_press_amd.kernels import Event

    rng = np.random.default_rng(12)
    m, n, k = 512, 4096, 4096
    w_q, s, b = make_weight(rng, n, k, 64, 4, "bf16")
    W, S, B = (device.upload(w_q.reshape(-1), "u32"), device.upload(s.reshape(-1), "bf16"),
               device.upload(b.reshape(-1), "bf16"))
    X = device.upload(make_x(rng, m, k, "bf16").reshape(-1), "bf16")
    Y = device.alloc_buffer(m * n, "bf16")
    plain = device.commands()
    for _ in range(3):
        kqmm.affine_qmm_t(plain, library, W, S, B, X, Y, m, n, k, 64, 4)
    plain.commit_and_wait()
    e0, e1 = Event(), Event()
    reps = 20
    e0.record(plain)
    for _ in range(reps):
        kqmm.affine_qmm_t(plain, library, W, S, B, X, Y, m, n, k, 64, 4)
    e1.record(plain)
    plain.commit_and_wait()
    event_ns = e0.elapsed_ms(e1) * 1e6 / reps
    cmds = device.commands_profiled(reps)
    for _ in range(reps):
        cmds.begin_profiled_op("qmm")
        kqmm.affine_qmm_t(cmds, library, W, S, B, X, Y, m, n, k, 64, 4)
    segs = cmds.commit_wait_resolve()
    per_op = sorted(s.ticks() * device.gpu_timestamp_period_ns() for s in segs)
    median = per_op[len(per_op) // 2]
    print(f"event-timed {event_ns:.0f} ns/op, profiled median {median:.0f} ns", flush=True)
    assert len(segs) == reps
    assert 0.5 * event_ns <= median <= 2.0 * event_ns


def test_profiled_session_past_capacity_stops_timing(device, library):
    """Past op_capacity, further ops run untimed instead of failing
    (commands.rs:172-180)."""
    rng = np.random.default_rng(13)
    n = k = 2048
    W, S, B, X = _qmv_case(device, rng, n, k)
    want = _plain_qmv(device, library, W, S, B, X, n, k)
    ys = [device.alloc_buffer(n, "bf16") for _ in range(3)]
    cmds = device.commands_profiled(2)
    for i, y in enumerate(ys):
        cmds.begin_profiled_op(f"op{i}")
        kqmv.affine_qmv(cmds, library, W, S, B, X, y, k, 64, 4)
    segs = cmds.commit_wait_resolve()
    assert [s.label for s in segs] == ["op0", "op1"]
    for y in ys:
        assert np.array_equal(y.to_numpy(), want)
    # The next batch has the full capacity again.
    cmds.begin_profiled_op("again")
    kqmv.affine_qmv(cmds, library, W, S, B, X, ys[0], k, 64, 4)
    assert [s.label for s in cmds.commit_wait_resolve()] == ["again"]


def test_resolve_needs_room_for_every_segment(device, library):
    rng = np.random.default_rng(14)
    W, S, B, X = _qmv_case(device, rng, 1024, 1024)
    Y = device.alloc_buffer(1024, "bf16")
    cmds = device.commands_profiled(2)
    for label in ("a", "b"):
        cmds.begin_profiled_op(label)
        kqmv.affine_qmv(cmds, library, W, S, B, X, Y, 1024, 64, 4)
    n = ctypes.c_size_t()
    st = _lib.lib().cpq_commands_commit_wait_resolve(cmds.handle, None, 1, ctypes.byref(n))
    assert st == _lib.INVALID_ARGUMENT and n.value == 0
    assert cmds.recorded_ops() == 2  # rejected before waiting: the batch is intact
    assert [s.label for s in cmds.commit_wait_resolve()] == ["a", "b"]


def test_ordinary_session_ignores_profiling_calls(device, library):
    rng = np.random.default_rng(15)
    W, S, B, X = _qmv_case(device, rng, 1024, 1024)
    want = _plain_qmv(device, library, W, S, B, X, 1024, 1024)
    Y = device.alloc_buffer(1024, "bf16")
    cmds = device.commands()
    cmds.begin_profiled_op("ignored")
    kqmv.affine_qmv(cmds, library, W, S, B, X, Y, 1024, 64, 4)
    assert cmds.commit_wait_resolve() == []
    assert np.array_equal(Y.to_numpy(), want)


def test_begin_profiled_op_refused_during_capture(device, library):
    cmds = device.commands_profiled(2)
    cmds.begin_capture()
    try:
        with pytest.raises(_lib.InvalidArgument, match="captured"):
            cmds.begin_profiled_op("x")
    finally:
        cmds.end_capture()
    assert cmds.recorded_ops() == 0


def test_encoder_hooks_leave_results_unchanged(device, library):
    """The evaluator's per-op hooks (eval.rs:280-292) around dependent ops:
    y1 = qmv(x), then a qmv reading y1 after an elided barrier request."""
    rng = np.random.default_rng(16)
    n = k = 2048
    W, S, B, X = _qmv_case(device, rng, n, k)
    y1_want = _plain_qmv(device, library, W, S, B, X, n, k)
    X2 = device.upload(y1_want, "bf16")
    y2_want = _plain_qmv(device, library, W, S, B, X2, n, k)
    Y1, Y2 = device.alloc_buffer(n, "bf16"), device.alloc_buffer(n, "bf16")
    cmds = device.commands()
    cmds.record_output(Y1.ptr)
    cmds.record_input(X.ptr)
    kqmv.affine_qmv(cmds, library, W, S, B, X, Y1, k, 64, 4)
    cmds.elide_next_barrier()
    cmds.record_output(Y2.ptr)
    cmds.record_input(Y1.ptr)
    cmds.record_unresolved_input()
    kqmv.affine_qmv(cmds, library, W, S, B, Y1, Y2, k, 64, 4)
    cmds.commit_and_wait()
    assert np.array_equal(Y1.to_numpy(), y1_want)
    assert np.array_equal(Y2.to_numpy(), y2_want)


@pytest.mark.parametrize("nbytes", [700, 1, 511])
def test_alloc_slack_reads_back_zero(device, nbytes):
    """The allocation is rounded to 512 B and the slack reads back 0 on memory
    that held other data (alloc_slack_zeroed.rs:1-40): blocks of the same
    rounded size are filled with 0xFF and freed, then allocations are made
    until one lands on a dirtied block; its slack must read 0.  The test
    asserts that such a reuse happened, so it cannot pass on fresh memory."""
    L = _lib.lib()
    size = -(-nbytes // 512) * 512
    ff = np.full(size, 0xFF, np.uint8)
    dirtied = set()
    reused = 0
    for _ in range(32):
        d = device.alloc_buffer(size, "u8")
        _lib.check(L.cpq_write_buffer(device.handle, ctypes.c_void_p(d.ptr), ff.ctypes.data_as(ctypes.c_void_p),
                                      size))
        dirtied.add(d.ptr)
        del d  # freed: the next allocation of this size may take the same block
        buf = device.alloc_buffer(nbytes, "u8")
        assert buf.alloc_len == size > nbytes
        raw = buf.read_bytes(buf.alloc_len)
        assert not raw[nbytes:].any(), f"slack of a {nbytes}-byte buffer at {buf.ptr:#x} not zero"
        if buf.ptr in dirtied:
            reused += 1
        del buf
    assert reused > 0, "no allocation reused a dirtied block: the slack check saw only fresh memory"


def test_alloc_qmv_activation_row_slack(device):
    act = device.alloc_buffer(896, "bf16")
    assert act.byte_len == 1792 and act.alloc_len == 2048
    assert not act.read_bytes(2048)[1792:].any()
    exact = device.alloc_buffer(512, "u8")
    assert exact.alloc_len == 512


def _fixture_sizes(n, k, q):
    return n * k * q.bits // 8, n * (k // q.group_size) * 2


def test_from_bytes_constructs_quantized_leaf(device):
    q = q4_gs64()
    wb, ab = _fixture_sizes(64, 64, q)
    w = QuantizedWeight.from_bytes(device, (64, 64), q, bytes(wb), bytes(ab), bytes(ab))
    assert w.shape() == (64, 64)


def test_from_bytes_rejects_wrong_rank(device):
    q = q4_gs64()
    wb, ab = _fixture_sizes(64, 64, q)
    with pytest.raises(_lib.InvalidArgument, match="rank 2"):
        QuantizedWeight.from_bytes(device, (64 * 64,), q, bytes(wb), bytes(ab), bytes(ab))


def test_from_bytes_rejects_size_mismatch(device):
    q = q4_gs64()
    _, ab = _fixture_sizes(64, 64, q)
    with pytest.raises(_lib.InvalidArgument, match="weights byte length"):
        QuantizedWeight.from_bytes(device, (64, 64), q, bytes(17), bytes(ab), bytes(ab))
    wb, _ = _fixture_sizes(64, 64, q)
    with pytest.raises(_lib.InvalidArgument, match="scales byte length"):
        QuantizedWeight.from_bytes(device, (64, 64), q, bytes(wb), bytes(3), bytes(ab))


def test_from_bytes_rejects_k_not_multiple_of_group(device):
    q = q4_gs64()
    wb, ab = 8 * 96 * 4 // 8, 8 * 2 * 2
    with pytest.raises(_lib.InvalidArgument, match="multiple of group_size"):
        QuantizedWeight.from_bytes(device, (8, 96), q, bytes(wb), bytes(ab), bytes(ab))


def test_from_bytes_k_padded_rejects(device):
    q = q4_gs64()
    wb, ab = _fixture_sizes(8, 128, q)
    with pytest.raises(_lib.InvalidArgument, match="k_logical=192 > k_physical=128"):
        QuantizedWeight.from_bytes_k_padded(device, (8, 128), 192, q, bytes(wb), bytes(ab), bytes(ab))
    with pytest.raises(_lib.InvalidArgument, match="k_logical=33 must be a multiple"):
        QuantizedWeight.from_bytes_k_padded(device, (8, 128), 33, q, bytes(wb), bytes(ab), bytes(ab))
    w = QuantizedWeight.from_bytes_k_padded(device, (8, 128), 64, q, bytes(wb), bytes(ab), bytes(ab))
    assert w.k_logical() == 64 and w.shape() == (8, 128)


def test_from_bytes_rejects_bad_quantization(device):
    with pytest.raises(_lib.InvalidArgument):
        QuantizedWeight.from_bytes(device, (8, 64), Quantization(7, 64), bytes(8 * 64 * 7 // 8), bytes(16),
                                   bytes(16))
