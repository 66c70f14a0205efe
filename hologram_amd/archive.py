"""`.holo` archive writer: the layout of crates/hologram-archive/src/writer.rs.

    header      "HOLO" | version u16 (3) | flags u16 | section_count u16
    table       per section: kind u8 | pad[7] | offset u64 | length u64
    payloads    in writer order (KernelCalls, Weights, Inputs, Outputs,
                Constants, ExecPlan)
    footer      BLAKE3 over every preceding byte (32 bytes)

Section payloads follow the reference encoders: kernel calls
(kernel_codec.rs encode_calls), ports (writer.rs encode_ports), exec plan
(writer.rs encode_exec_plan), weights (writer.rs encode_weights: count, then
fingerprint[32] | len u64 | body per body, deduplicated by fingerprint) and
constants (constant_codec.rs encode: inline tag 0 or by-reference tag 1).
The fingerprints and the footer are BLAKE3, computed by libholo_hip.so.
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass, field

from . import _ffi
from .kernel_call import KernelCall, encode_calls

MAGIC = b"HOLO"
FORMAT_VERSION = 3     # format.rs:16

# SectionKind, format.rs:24-77
KERNEL_CALLS, SCHEDULE, WEIGHTS, SHAPE_REGISTRY, DTYPE_REGISTRY = 1, 2, 3, 4, 5
CERTIFICATES, TRACE, METADATA, INPUTS, OUTPUTS, CONSTANTS, EXEC_PLAN = 6, 7, 8, 9, 10, 11, 12
WARM_START, EXTENSION = 13, 14


def blake3(data) -> bytes:
    """BLAKE3 digest (32 bytes) of a bytes-like object, via libholo_hip.so."""
    if isinstance(data, bytes):
        buf, n = data, len(data)
    else:
        mv = memoryview(data).cast("B")
        n = len(mv)
        buf = ((ctypes.c_char * n).from_buffer_copy(mv) if mv.readonly
               else (ctypes.c_char * n).from_buffer(mv)) if n else b""
    out = ctypes.create_string_buffer(32)
    rc = _ffi.lib().holo_hip_blake3(ctypes.cast(buf, ctypes.c_char_p) if not isinstance(buf, bytes)
                                    else buf, n, out)
    if rc != 0:
        raise RuntimeError(_ffi.last_error())
    return out.raw


@dataclass
class PortDescriptor:
    """writer.rs PortDescriptor: semantic name, slot, element count, dtype, shape."""
    name: str
    slot: int
    element_count: int
    dtype: int
    shape: list = field(default_factory=list)


@dataclass
class ConstantEntry:
    """constant_codec.rs ConstantEntry: inline bytes, or a reference into Weights."""
    slot: int
    dtype: int
    body: bytes
    by_reference: bool = True


def encode_ports(ports: list[PortDescriptor]) -> bytes:
    out = [struct.pack("<I", len(ports))]
    for p in ports:
        name = p.name.encode()
        out.append(struct.pack("<H", len(name)) + name)
        out.append(struct.pack("<IQBB", p.slot, p.element_count, p.dtype, len(p.shape)))
        out.append(b"".join(struct.pack("<Q", d) for d in p.shape))
    return b"".join(out)


def encode_exec_plan(levels: list[list[int]]) -> bytes:
    out = [struct.pack("<I", len(levels))]
    for lv in levels:
        out.append(struct.pack("<I", len(lv)) + b"".join(struct.pack("<I", i) for i in lv))
    return b"".join(out)


class HoloWriter:
    """writer.rs HoloWriter, for the sections this backend executes."""

    def __init__(self):
        self.kernel_calls: list[KernelCall] = []
        self.inputs: list[PortDescriptor] = []
        self.outputs: list[PortDescriptor] = []
        self.constants: list[ConstantEntry] = []
        self.exec_plan: list[list[int]] = []

    def finish(self) -> bytes:
        weights = {}            # fingerprint -> body, insertion-ordered (WeightStore)
        const_wire = [struct.pack("<I", len(self.constants))]
        for e in self.constants:
            if e.by_reference:
                fp = blake3(e.body)
                weights.setdefault(fp, e.body)
                const_wire.append(struct.pack("<BIB", 1, e.slot, e.dtype) + fp)
            else:
                const_wire.append(struct.pack("<BIBI", 0, e.slot, e.dtype, len(e.body)))
                const_wire.append(bytes(e.body))
        weight_wire = [struct.pack("<I", len(weights))]
        for fp, body in weights.items():
            weight_wire.append(fp + struct.pack("<Q", len(body)))
            weight_wire.append(body)
        payloads = [(KERNEL_CALLS, [encode_calls(self.kernel_calls)]), (WEIGHTS, weight_wire)]
        if self.inputs:
            payloads.append((INPUTS, [encode_ports(self.inputs)]))
        if self.outputs:
            payloads.append((OUTPUTS, [encode_ports(self.outputs)]))
        if self.constants:
            payloads.append((CONSTANTS, const_wire))
        if self.exec_plan:
            payloads.append((EXEC_PLAN, [encode_exec_plan(self.exec_plan)]))
        return assemble(payloads)


def assemble(payloads) -> bytes:
    """writer.rs assemble: header, table, payloads, BLAKE3 footer. Each payload
    is a list of byte chunks (large weight bodies are not concatenated twice)."""
    sizes = [sum(len(c) for c in chunks) for _, chunks in payloads]
    off = 4 + 2 + 2 + 2 + 24 * len(payloads)
    total = off + sum(sizes) + 32
    out = bytearray(total)
    out[0:10] = MAGIC + struct.pack("<HHH", FORMAT_VERSION, 0, len(payloads))
    at = 10
    for (kind, _), n in zip(payloads, sizes):
        out[at:at + 24] = struct.pack("<B7xQQ", kind, off, n)
        at += 24
        off += n
    for _, chunks in payloads:
        for c in chunks:
            out[at:at + len(c)] = c
            at += len(c)
    out[at:at + 32] = blake3(memoryview(out)[:at])
    return bytes(out)
