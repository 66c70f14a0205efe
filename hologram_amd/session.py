"""HipSession: a `.holo` archive executed on the MI355X backend.

The host mirror of InferenceSession (crates/hologram-exec/src/session.rs):
`load` (:399-797), `execute` with host bytes in and out (:846-932), and the
addressed form where inputs are device buffers bound in place (:942-984).
Everything runs in libholo_hip.so (include/holo_hip.h, holo_hip_session_*);
this class only marshals arguments.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _ffi
from .backend import HipBackend, check as _check


@dataclass(frozen=True)
class Port:
    index: int
    slot: int
    element_count: int
    dtype: int
    nbytes: int


# load options (include/holo_hip.h)
NO_EPILOGUE_FUSION = 1   # skip the reference loader's fuse_matmul_epilogue
NO_DEVICE_FUSION = 2     # skip this backend's grouped few-row MatMuls and epilogues
NO_NORM_FUSION = 4       # keep each RmsNorm between few-row MatMuls as its own launch
NO_DEQUANT_FUSION = 8    # skip the loader's fuse_dequant_matmul / fuse_dequant_activation
NO_WEIGHT_PACKING = 16   # keep few-row groups over constant weights on the split-K launches
NO_ATTN_PROLOGUE = 32    # keep the q/k/v group's split-K epilogue out of the decode attention's launch


class HipSession:
    """`backend=None` loads dry: parse, size and validate every call on the host,
    with no device (such a session reports ports and refuses to execute).
    `flags` turns the load-time fusions off (NO_EPILOGUE_FUSION, NO_DEVICE_FUSION,
    NO_NORM_FUSION, NO_DEQUANT_FUSION, NO_WEIGHT_PACKING, NO_ATTN_PROLOGUE);
    fused and unfused walks give the same bits."""

    def __init__(self, backend: HipBackend | None, archive: bytes, flags: int = 0):
        self._lib = _ffi.lib()
        self.backend = backend
        h = ctypes.c_void_p()
        _check(self._lib.holo_hip_session_load_ex(backend._h if backend else None, archive,
                                                  len(archive), flags, ctypes.byref(h)))
        self.handle = h
        ni, no, nc, ns = (ctypes.c_uint32() for _ in range(4))
        _check(self._lib.holo_hip_session_info(self.handle, ctypes.byref(ni), ctypes.byref(no),
                                               ctypes.byref(nc), ctypes.byref(ns)))
        self.n_calls, self.n_slots = nc.value, ns.value
        nn, ng = ctypes.c_uint32(), ctypes.c_uint32()
        _check(self._lib.holo_hip_session_nodes(self.handle, ctypes.byref(nn), ctypes.byref(ng)))
        self.n_nodes, self.n_groups = nn.value, ng.value
        self.last_memo_hit = False
        self.inputs = [self._port(0, i) for i in range(ni.value)]
        self.outputs = [self._port(1, i) for i in range(no.value)]

    def _port(self, is_out: int, i: int) -> Port:
        slot, cnt, dt, nb = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint8(), ctypes.c_uint64()
        _check(self._lib.holo_hip_session_port(self.handle, is_out, i, ctypes.byref(slot),
                                               ctypes.byref(cnt), ctypes.byref(dt),
                                               ctypes.byref(nb)))
        return Port(i, slot.value, cnt.value, dt.value, nb.value)

    def call_tags(self) -> list[int]:
        """The in-memory tag of each loaded call after the loader's passes."""
        tags = []
        for i in range(self.n_calls):
            kc = _ffi.KernelCallC()
            _check(self._lib.holo_hip_session_call(self.handle, i, ctypes.byref(kc)))
            tags.append(kc.tag)
        return tags

    def call(self, index: int) -> _ffi.KernelCallC:
        kc = _ffi.KernelCallC()
        _check(self._lib.holo_hip_session_call(self.handle, index, ctypes.byref(kc)))
        return kc

    def fingerprint(self) -> bytes:
        out = ctypes.create_string_buffer(32)
        _check(self._lib.holo_hip_session_fingerprint(self.handle, out))
        return out.raw

    # ---- the addressed form: device buffers bound in place
    def bind_input(self, index: int, tensor) -> None:
        """Bind input port `index` to a device tensor (torch) or (ptr, nbytes); None unbinds."""
        if tensor is None:
            _check(self._lib.holo_hip_session_bind_input(self.handle, index, None, 0))
            return
        ptr, nbytes = (tensor if isinstance(tensor, tuple)
                       else (tensor.data_ptr(), tensor.numel() * tensor.element_size()))
        _check(self._lib.holo_hip_session_bind_input(self.handle, index, ctypes.c_void_p(ptr),
                                                     nbytes))

    def output_ptr(self, index: int) -> tuple[int, int]:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(self._lib.holo_hip_session_output(self.handle, index, ctypes.byref(p),
                                                 ctypes.byref(n)))
        return p.value or 0, n.value

    def run(self) -> None:
        """One walk, enqueued on the session stream (asynchronous)."""
        _check(self._lib.holo_hip_session_execute(self.handle))

    def capture(self) -> None:
        _check(self._lib.holo_hip_session_capture(self.handle))

    def replay(self) -> None:
        _check(self._lib.holo_hip_session_replay(self.handle))

    def synchronize(self) -> None:
        _check(self._lib.holo_hip_session_synchronize(self.handle))

    def stream(self) -> int:
        s = ctypes.c_void_p()
        _check(self._lib.holo_hip_session_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    # ---- the byte form (execute): host bytes in, host bytes out
    def write_input(self, index: int, data: bytes) -> None:
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        _check(self._lib.holo_hip_session_write_input(self.handle, index, buf, len(data)))

    def read_output(self, index: int) -> bytes:
        n = self.outputs[index].nbytes
        buf = ctypes.create_string_buffer(n)
        _check(self._lib.holo_hip_session_read_output(self.handle, index, buf, n))
        return buf.raw

    def execute(self, inputs: list[bytes]) -> list[bytes]:
        """session.rs execute: bytes per input port in, bytes per output port
        out, with the whole-graph memo (a repeat of the last inputs, nothing
        touched since, skips the walk; `last_memo_hit` says whether it did)."""
        if len(inputs) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs, got {len(inputs)}")
        bufs = [ctypes.create_string_buffer(bytes(b), len(b)) for b in inputs]
        ptrs = (ctypes.c_void_p * max(1, len(bufs)))(*[ctypes.addressof(b) for b in bufs])
        sizes = (ctypes.c_uint64 * max(1, len(bufs)))(*[len(b) for b in inputs])
        hit = ctypes.c_int()
        _check(self._lib.holo_hip_session_execute_bytes(self.handle, ptrs, sizes, len(bufs),
                                                        ctypes.byref(hit)))
        self.last_memo_hit = bool(hit.value)
        self.synchronize()
        return [self.read_output(i) for i in range(len(self.outputs))]

    @property
    def last_walk(self) -> tuple[int, int]:
        """(steps dispatched, steps skipped) of the last walk (session.rs
        last_dispatched / last_skipped): skipped counts the steps bound at
        load (interior Reshape / Slice, repeats of a value the walk holds),
        the steps a memo-on execute found unchanged, and every step of a
        whole-graph memo hit."""
        d, k = ctypes.c_uint32(), ctypes.c_uint32()
        _check(self._lib.holo_hip_session_last_walk(self.handle, ctypes.byref(d), ctypes.byref(k)))
        return d.value, k.value

    @property
    def packed(self) -> tuple[int, int]:
        """(groups run as one launch over packed weights, bytes of the packed
        weight copies)."""
        g, b = ctypes.c_uint32(), ctypes.c_uint64()
        _check(self._lib.holo_hip_session_packed(self.handle, ctypes.byref(g), ctypes.byref(b)))
        return g.value, b.value

    @property
    def attn_prologues(self) -> int:
        """Fused groups whose split-K epilogue runs in the decode attention's
        launch after them (decided at load)."""
        n = ctypes.c_uint32()
        _check(self._lib.holo_hip_session_attn_prologues(self.handle, ctypes.byref(n)))
        return n.value

    def set_memo(self, enabled: bool) -> None:
        """The memo's hits on (default) or off (every execute walks)."""
        _check(self._lib.holo_hip_session_set_memo(self.handle, int(enabled)))

    def output_labels(self, input_labels: list[str]) -> list[str]:
        """The output ports' κ-labels for these input-port labels (works on a
        dry load)."""
        if len(input_labels) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} labels")
        out = ctypes.create_string_buffer(71 * max(1, len(self.outputs)))
        _check(self._lib.holo_hip_session_output_labels(self.handle,
                                                        "".join(input_labels).encode(), out))
        return [out.raw[71 * i:71 * (i + 1)].decode() for i in range(len(self.outputs))]

    def close(self) -> None:
        if self.handle:
            _check(self._lib.holo_hip_session_close(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
