"""κ-labels, the reference's content addresses
(crates/hologram-archive/src/address.rs), over the C ABI: "blake3:" followed
by the 64 hex digits of a BLAKE3 digest.

  address_bytes(data)                     address.rs:96-99
  derive_label(opcode, params, labels)    address.rs:108-116
  derive_label_boundary(op, params, labels)  address.rs:197-221 (an output
                                          port's label)
  op_signature(call)                      KernelCall::op_signature,
                                          kernel_call.rs:1321-1500
"""
from __future__ import annotations

import ctypes

from . import _ffi
from .backend import check as _check

LABEL_LEN = 71


def address_bytes(data: bytes) -> str:
    out = ctypes.create_string_buffer(LABEL_LEN + 1)
    data = bytes(data)
    _check(_ffi.lib().holo_hip_address_bytes(data, len(data), out))
    return out.value.decode()


def derive_label(opcode: int, params: bytes, labels: list[str]) -> str:
    out = ctypes.create_string_buffer(LABEL_LEN + 1)
    joined = "".join(labels).encode()
    if any(len(lbl) != LABEL_LEN for lbl in labels):
        raise ValueError("a κ-label is 71 ASCII bytes")
    params = bytes(params)
    _check(_ffi.lib().holo_hip_derive_label(opcode, params, len(params), joined, len(labels), out))
    return out.value.decode()


def derive_label_boundary(opcode: int, params: bytes, labels: list[str]) -> str:
    out = ctypes.create_string_buffer(LABEL_LEN + 1)
    joined = "".join(labels).encode()
    if any(len(lbl) != LABEL_LEN for lbl in labels):
        raise ValueError("a κ-label is 71 ASCII bytes")
    params = bytes(params)
    _check(_ffi.lib().holo_hip_derive_label_boundary(opcode, params, len(params), joined,
                                                     len(labels), out))
    return out.value.decode()


def op_signature(call) -> tuple[int, bytes]:
    """(opcode, params) of a KernelCall (or its C form)."""
    kc = call.to_c() if hasattr(call, "to_c") else call
    op, n = ctypes.c_uint16(), ctypes.c_uint32()
    buf = ctypes.create_string_buffer(64)
    _check(_ffi.lib().holo_hip_op_signature(ctypes.byref(kc), ctypes.byref(op), buf,
                                            ctypes.byref(n)))
    return op.value, buf.raw[:n.value]
