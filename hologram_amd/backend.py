"""HipBackend: the reference's `Backend` trait over the C ABI.

    pub trait Backend {
        fn dispatch(&mut self, call: &KernelCall, workspace: &mut Self::WS)
            -> Result<(), BackendError>;
    }                                  (crates/hologram-compute/src/backend.rs:8-15)

`DeviceWorkspace` is the device-resident form of the executor's BufferArena
(crates/hologram-exec/src/buffer.rs:149-207): slots bound to device memory the
pool owns (here torch CUDA tensors, used only as allocations). Every
`dispatch` enqueues on the backend's stream and returns without waiting, as
a device backend must; `synchronize()` is the host-read barrier.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional

from . import _ffi
from .kernel_call import KernelCall


class BackendError(Exception):
    """crates/hologram-compute/src/error.rs:6-20."""
    code = -1


class SlotOutOfRange(BackendError):
    code = _ffi.ERR_SLOT_OUT_OF_RANGE


class ShapeMismatch(BackendError):
    code = _ffi.ERR_SHAPE_MISMATCH


class UnsupportedOp(BackendError):
    code = _ffi.ERR_UNSUPPORTED_OP


class InitError(BackendError):
    code = _ffi.ERR_INIT


class DispatchError(BackendError):
    code = _ffi.ERR_DISPATCH


_ERRORS = {c.code: c for c in (SlotOutOfRange, ShapeMismatch, UnsupportedOp, InitError,
                               DispatchError)}


def check(rc: int) -> None:
    """Raise the BackendError a holo_status stands for (0 = Ok)."""
    if rc != _ffi.OK:
        raise _ERRORS.get(rc, BackendError)(_ffi.last_error())


class DeviceWorkspace:
    """Slot -> device range table (the workspace a dispatch reads and writes).

    Binding keeps a reference to the owning object (e.g. a torch tensor) so the
    memory outlives the binding; the backend never frees pool memory.
    """

    def __init__(self) -> None:
        self._slots: Dict[int, tuple] = {}
        self.generation = 0

    def bind(self, slot: int, tensor=None, *, ptr: Optional[int] = None,
             nbytes: Optional[int] = None) -> None:
        if tensor is not None:
            if not tensor.is_contiguous():
                raise ValueError("slot tensors must be contiguous")
            ptr = tensor.data_ptr()
            nbytes = tensor.numel() * tensor.element_size()
        if ptr is None or nbytes is None:
            raise ValueError("bind needs a tensor or (ptr, nbytes)")
        self._slots[slot] = (int(ptr), int(nbytes), tensor)
        self.generation += 1

    def unbind(self, slot: int) -> None:
        self._slots.pop(slot, None)
        self.generation += 1

    def items(self):
        for slot, (ptr, nbytes, _) in self._slots.items():
            yield slot, ptr, nbytes

    def slot_sizes(self) -> list:
        n = max(self._slots, default=-1) + 1
        sizes = [0] * n
        for slot, (_, nbytes, _) in self._slots.items():
            sizes[slot] = nbytes
        return sizes


class HipBackend:
    """MI355X backend: `dispatch(call, workspace)` as Backend::dispatch."""

    def __init__(self, device: int = 0, stream: Optional[int] = None) -> None:
        lib = _ffi.lib()
        handle = ctypes.c_void_p()
        check(lib.holo_hip_backend_create(device, ctypes.c_void_p(stream or 0),
                                          ctypes.byref(handle)))
        self._h = handle
        self._bound_ws = None
        self._bound_gen = -1

    def close(self) -> None:
        if self._h:
            check(_ffi.lib().holo_hip_backend_destroy(self._h))
            self._h = None

    def __del__(self) -> None:  # best effort; close() is the explicit path
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream: Optional[int]) -> None:
        check(_ffi.lib().holo_hip_set_stream(self._h, ctypes.c_void_p(stream or 0)))

    def _sync_slots(self, ws: DeviceWorkspace) -> None:
        if ws is self._bound_ws and ws.generation == self._bound_gen:
            return
        lib = _ffi.lib()
        if self._bound_ws is not None:
            for slot, _, _ in list(self._bound_ws.items()):
                check(lib.holo_hip_slot_unbind(self._h, slot))
        for slot, ptr, nbytes in ws.items():
            check(lib.holo_hip_slot_bind(self._h, slot, ctypes.c_void_p(ptr), nbytes))
        self._bound_ws, self._bound_gen = ws, ws.generation

    def dispatch(self, call: KernelCall, workspace: DeviceWorkspace) -> None:
        self._sync_slots(workspace)
        kc = call.to_c()
        check(_ffi.lib().holo_hip_dispatch(self._h, ctypes.byref(kc)))

    def dispatch_noalloc(self, call: KernelCall, workspace: DeviceWorkspace) -> None:
        """holo_hip_dispatch_noalloc: decode attention (123 / 125) on the fixed
        per-device scratch, with no device allocation (see include/holo_hip.h)."""
        self._sync_slots(workspace)
        kc = call.to_c()
        check(_ffi.lib().holo_hip_dispatch_noalloc(self._h, ctypes.byref(kc)))

    def dispatch_encoded(self, wire: bytes, workspace: DeviceWorkspace) -> int:
        """Dispatch one call given in the archive wire format; returns its length."""
        self._sync_slots(workspace)
        used = ctypes.c_size_t(0)
        check(_ffi.lib().holo_hip_dispatch_encoded(self._h, wire, len(wire), ctypes.byref(used)))
        return used.value

    def synchronize(self) -> None:
        check(_ffi.lib().holo_hip_synchronize(self._h))


def validate(call: KernelCall, slot_sizes: list) -> None:
    """Host-only check of a call against slot sizes (no device needed)."""
    kc = call.to_c()
    arr = (ctypes.c_uint64 * max(1, len(slot_sizes)))(*slot_sizes)
    check(_ffi.lib().holo_hip_validate(ctypes.byref(kc), arr, len(slot_sizes)))


def decode_call(wire: bytes) -> tuple:
    """Decode one wire-format call with the library's codec: (KernelCallC, length)."""
    out = _ffi.KernelCallC()
    used = ctypes.c_size_t(0)
    check(_ffi.lib().holo_hip_decode_call(wire, len(wire), ctypes.byref(out), ctypes.byref(used)))
    return out, used.value


def lut_table(act: int, dtype: int):
    """The 65536-entry table the backend stages in LDS, as a numpy u16 array."""
    import numpy as np
    t = np.zeros(65536, dtype=np.uint16)
    check(_ffi.lib().holo_hip_lut_table(act, dtype, t.ctypes.data))
    return t
