"""Kernel dispatch and buffer layer (mirror of the reference's cider-press-kernels
crate, crates/cider-press-kernels/src/lib.rs:35-40), backed by libcpq.so.

    Device.system_default()        -> device.rs:77
    device.alloc_buffer / upload   -> device.rs:167-233 (512-B rounding, zeroed slack)
    device.commands()              -> device.rs:319 (one in-order HIP stream)
    device.commands_profiled(n)    -> device.rs:465-470 (per-op GPU windows, gpu_sampler.rs)
    Commands.commit / wait         -> commands.rs:349-419
    KernelLibrary.quantized(dev)   -> library.rs:230 (kernels are compiled ahead of time)
    kernels.{qmv,qmm,dequantize,gather,embed}.*  -> kernels/{qmv,qmm,dequantize}.rs, nn.rs

Buffers are typed views over device memory; 16-bit float buffers hold raw
uint16 bit patterns on the host side (numpy has no bfloat16).
"""
from __future__ import annotations

import ctypes

import numpy as np

from .. import _lib
from .._lib import (BufferAllocation, BufferTooLarge, CommandBufferFailed, Error, HipApi,  # noqa: F401
                    InvalidArgument, KernelNotFound, NoDevice)

_NP = {"u32": np.uint32, "bf16": np.uint16, "f16": np.uint16, "u16": np.uint16, "u8": np.uint8,
       "f32": np.float32}
_SIZE = {"u32": 4, "bf16": 2, "f16": 2, "u16": 2, "u8": 1, "f32": 4}


class Device:
    def __init__(self, handle):
        self._h = handle
        self._lib = _lib.lib()

    @staticmethod
    def system_default() -> "Device":
        L = _lib.lib()
        h = ctypes.c_void_p()
        _lib.check(L.cpq_device_system_default(ctypes.byref(h)))
        return Device(h)

    @property
    def handle(self):
        return self._h

    def info(self) -> dict:
        name = ctypes.create_string_buffer(256)
        cus, clk = ctypes.c_int(), ctypes.c_int()
        _lib.check(self._lib.cpq_device_info(self._h, name, 256, ctypes.byref(cus), ctypes.byref(clk)))
        return {"name": name.value.decode(), "cu_count": cus.value, "clock_khz": clk.value}

    def alloc_buffer(self, length: int, dtype: str) -> "Buffer":
        ptr, alloc = ctypes.c_void_p(), ctypes.c_size_t()
        _lib.check(self._lib.cpq_alloc_buffer(self._h, length * _SIZE[dtype], ctypes.byref(ptr),
                                              ctypes.byref(alloc)))
        return Buffer(self, ptr.value, length, dtype, alloc.value)

    def upload(self, array: np.ndarray, dtype: str) -> "Buffer":
        a = np.ascontiguousarray(array, dtype=_NP[dtype])
        ptr, alloc = ctypes.c_void_p(), ctypes.c_size_t()
        _lib.check(self._lib.cpq_upload(self._h, a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                                        ctypes.byref(ptr), ctypes.byref(alloc)))
        return Buffer(self, ptr.value, a.size, dtype, alloc.value)

    def commands(self) -> "Commands":
        h = ctypes.c_void_p()
        _lib.check(self._lib.cpq_commands_create(self._h, ctypes.byref(h)))
        return Commands(self, h)

    def wrap_stream(self, hip_stream: int) -> "Commands":
        h = ctypes.c_void_p()
        _lib.check(self._lib.cpq_commands_wrap_stream(self._h, ctypes.c_void_p(hip_stream), ctypes.byref(h)))
        return Commands(self, h)

    def commands_profiled(self, op_capacity: int) -> "Commands":
        """A session that times up to `op_capacity` ops per batch (commands.rs:465-470)."""
        h = ctypes.c_void_p()
        _lib.check(self._lib.cpq_commands_create_profiled(self._h, op_capacity, ctypes.byref(h)))
        return Commands(self, h)

    def supports_stage_boundary_sampling(self) -> bool:
        """device.rs:314-322; always true on an in-order HIP stream."""
        return bool(self._lib.cpq_device_supports_stage_boundary_sampling(self._h))

    def gpu_timestamp_period_ns(self) -> float:
        """Nanoseconds per GpuSegment tick (device.rs:324-368)."""
        v = ctypes.c_double()
        _lib.check(self._lib.cpq_device_gpu_timestamp_period_ns(self._h, ctypes.byref(v)))
        return float(v.value)

    def __del__(self):
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_device_release(self._h)
            self._h = None


class Buffer:
    """A device allocation (Buffer<T>, buffer.rs:62-199)."""

    def __init__(self, device: Device, ptr: int, length: int, dtype: str, alloc_len: int):
        self.device = device
        self.ptr = ptr
        self._len = length
        self.dtype = dtype
        self.alloc_len = alloc_len  # Buffer::metal_alloc_len analogue

    def __len__(self):
        return self._len

    @property
    def byte_len(self) -> int:
        return self._len * _SIZE[self.dtype]

    def to_numpy(self) -> np.ndarray:
        """Host copy (Buffer::as_slice after a wait)."""
        out = np.empty(self._len, _NP[self.dtype])
        _lib.check(_lib.lib().cpq_read_buffer(self.device.handle, ctypes.c_void_p(self.ptr),
                                              out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def read_bytes(self, nbytes: int) -> np.ndarray:
        """Raw bytes of the allocation, including the rounded slack."""
        out = np.empty(nbytes, np.uint8)
        _lib.check(_lib.lib().cpq_read_buffer(self.device.handle, ctypes.c_void_p(self.ptr),
                                              out.ctypes.data_as(ctypes.c_void_p), nbytes))
        return out

    def write(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=_NP[self.dtype])
        if a.size != self._len:
            raise ValueError(f"write: {a.size} elements into a buffer of {self._len}")
        _lib.check(_lib.lib().cpq_write_buffer(self.device.handle, ctypes.c_void_p(self.ptr),
                                               a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def reinterpret_as(self, dtype: str) -> "Buffer":
        """Same allocation viewed with another element type (buffer.rs reinterpret_as)."""
        n = self.byte_len // _SIZE[dtype]
        view = Buffer(self.device, self.ptr, n, dtype, self.alloc_len)
        view._owner = self
        return view

    def __del__(self):
        if getattr(self, "_owner", None) is None and getattr(self, "ptr", None):
            L = _lib._lib
            if L is not None:
                L.cpq_free_buffer(self.device.handle, ctypes.c_void_p(self.ptr))
            self.ptr = None


class _Segment(ctypes.Structure):
    _fields_ = [("label", ctypes.c_char_p), ("start_tick", ctypes.c_uint64), ("end_tick", ctypes.c_uint64)]


class GpuSegment:
    """One timed op: label and GPU window in ticks (gpu_sampler.rs:22-42)."""

    __slots__ = ("label", "start_tick", "end_tick")

    def __init__(self, label: str, start_tick: int, end_tick: int):
        self.label, self.start_tick, self.end_tick = label, start_tick, end_tick

    def ticks(self) -> int:
        """end - start, saturating at 0."""
        return max(0, self.end_tick - self.start_tick)

    def __repr__(self):
        return f"GpuSegment({self.label!r}, {self.start_tick}, {self.end_tick})"


class Commands:
    """A command session on one HIP stream (commands.rs)."""

    def __init__(self, device: Device, handle):
        self.device = device
        self._h = handle
        self._lib = _lib.lib()

    @property
    def handle(self):
        return self._h

    @property
    def stream(self) -> int:
        return self._lib.cpq_commands_stream(self._h) or 0

    def commit(self) -> "Commands":
        _lib.check(self._lib.cpq_commands_commit(self._h))
        return self

    def wait(self) -> None:
        _lib.check(self._lib.cpq_commands_wait(self._h))

    def commit_and_wait(self) -> None:
        _lib.check(self._lib.cpq_commands_commit_and_wait(self._h))

    # Encoder hazard hooks (commands.rs:139-153, 290-296): an in-order stream
    # already orders every launch, so these only validate the session.
    def record_input(self, key: int) -> None:
        _lib.check(self._lib.cpq_commands_record_input(self._h, key))

    def record_output(self, key: int) -> None:
        _lib.check(self._lib.cpq_commands_record_output(self._h, key))

    def record_unresolved_input(self) -> None:
        _lib.check(self._lib.cpq_commands_record_unresolved_input(self._h))

    def elide_next_barrier(self) -> None:
        _lib.check(self._lib.cpq_commands_elide_next_barrier(self._h))

    def begin_profiled_op(self, label: str) -> None:
        """End the open op's window and open one for `label` (commands.rs:163-181)."""
        _lib.check(self._lib.cpq_commands_begin_profiled_op(self._h, label.encode()))

    def recorded_ops(self) -> int:
        n = ctypes.c_size_t()
        _lib.check(self._lib.cpq_commands_profiled_info(self._h, ctypes.byref(n), None))
        return n.value

    def sample_capacity(self) -> int:
        """Timestamp slots: two per op of capacity (gpu_sampler.rs:86-90)."""
        n = ctypes.c_size_t()
        _lib.check(self._lib.cpq_commands_profiled_info(self._h, None, ctypes.byref(n)))
        return n.value

    def commit_wait_resolve(self) -> list:
        """Wait, then one GpuSegment per recorded op (commands.rs:361-374)."""
        cap = self.recorded_ops()
        arr = (_Segment * max(cap, 1))()
        n = ctypes.c_size_t()
        _lib.check(self._lib.cpq_commands_commit_wait_resolve(self._h, arr, cap, ctypes.byref(n)))
        return [GpuSegment(arr[i].label.decode(), arr[i].start_tick, arr[i].end_tick) for i in range(n.value)]

    def begin_capture(self) -> None:
        """Record (not run) everything encoded until end_capture into a HIP graph."""
        _lib.check(self._lib.cpq_commands_begin_capture(self._h))

    def end_capture(self) -> "Graph":
        g = ctypes.c_void_p()
        _lib.check(self._lib.cpq_commands_end_capture(self._h, ctypes.byref(g)))
        return Graph(g, self)

    def __del__(self):
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_commands_release(self._h)
            self._h = None


class Graph:
    """An instantiated HIP graph captured from a session.

    The captured kernels address the capturing session's split-K scratch and
    status word, so the graph keeps that session alive for as long as it
    exists.  Release it (close) only when no replay is in flight."""

    def __init__(self, handle, session: Commands):
        self._h = handle
        self._lib = _lib.lib()
        self._session = session

    def launch(self, cmds: Commands) -> None:
        if not self._h:
            raise ValueError("graph_launch: the graph was released")
        _lib.check(self._lib.cpq_graph_launch(self._h, cmds.handle))

    def close(self) -> None:
        """Release the executable graph now (after its replays completed)."""
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_graph_release(self._h)
        self._h = None
        self._session = None

    def __del__(self):
        self.close()


class Event:
    """GPU timestamp on a session's stream (replaces the reference's GpuSampler)."""

    def __init__(self):
        self._lib = _lib.lib()
        self._h = ctypes.c_void_p()
        _lib.check(self._lib.cpq_event_create(ctypes.byref(self._h)))

    def record(self, cmds: Commands) -> None:
        _lib.check(self._lib.cpq_event_record(self._h, cmds.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _lib.check(self._lib.cpq_event_elapsed_ms(self._h, end._h, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        if getattr(self, "_h", None) and self._lib is not None:
            self._lib.cpq_event_release(self._h)
            self._h = None


class KernelLibrary:
    """The quantized kernel catalogue (library.rs:230); kernels are built ahead of time."""

    def __init__(self, device: Device):
        self.device = device

    @staticmethod
    def quantized(device: Device) -> "KernelLibrary":
        return KernelLibrary(device)

    @staticmethod
    def available(dtype: str, group_size: int, bits: int) -> bool:
        return bool(_lib.lib().cpq_kernel_available(_lib.DTYPES[dtype], group_size, bits))


def _ptr(buf) -> ctypes.c_void_p:
    return ctypes.c_void_p(None if buf is None else buf.ptr)


from . import dequantize, embed, gather, moe, qmm, qmv  # noqa: E402,F401
