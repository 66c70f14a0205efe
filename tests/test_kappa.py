"""CPU tests of the κ machinery (crates/hologram-archive/src/address.rs,
KernelCall::op_signature, the session's label derivation): against the
reference's recorded fixture label, its frozen op signatures
(crates/hologram-archive/tests/wire_stability.rs), the pure-Python BLAKE3
of the specification, and the derivation's algebra
(crates/hologram-archive/tests/conformance.rs:88-120). No device work."""
import json
import struct

import numpy as np
import pytest

from conftest import ROOT
from hologram_amd import (DTYPE_BF16, DTYPE_F32, BinaryCall, BufferRef, ConstantEntry, HipSession,
                          HoloWriter, KernelCall, MatMulCall, PortDescriptor, UnaryCall,
                          UnsupportedOp, fused_activation)
from hologram_amd.kappa import address_bytes, derive_label, derive_label_boundary, op_signature
from oracle.blake3_ref import blake3 as blake3_spec
from test_quant import frozen_calls

GOLDEN = ROOT / "tests" / "golden"


def spec_label(data: bytes) -> str:
    return "blake3:" + blake3_spec(data).hex()


def spec_boundary(op: int, params: bytes, labels: list) -> str:
    """derive_label_boundary (address.rs:197-221) stated with the specification's
    BLAKE3: the op's label composed in order with each operand label, a
    composition being the label of the two digests end to end
    (compose_ordered_blake3_address, compose.rs:154-164)."""
    comp = lambda l, r: spec_label(bytes.fromhex(l[7:]) + bytes.fromhex(r[7:]))
    acc = spec_label(struct.pack("<H", op) + params)
    if not labels:
        return comp(acc, acc)
    for lbl in labels:
        acc = comp(acc, lbl)
    return acc


def test_address_bytes_reproduces_the_reference_fixture_label():
    # fixture.holo's one output is the f32 scalar 64.0; the reference engine
    # labelled its bytes with address_bytes (engine.rs:42-51)
    want = (GOLDEN / "reference_fixture.kappa").read_text().strip()
    assert address_bytes(struct.pack("<f", 64.0)) == want
    assert address_bytes(b"") == spec_label(b"")
    assert len(want) == 71


def test_op_signatures_match_the_reference_frozen_params():
    golden = json.loads((GOLDEN / "wire_frozen.json").read_text())["signatures"]
    for name, call in frozen_calls().items():
        op, params = op_signature(call)
        assert (op, params.hex()) == (golden[name][0], golden[name][1]), name


def test_derive_label_is_the_digest_of_opcode_params_and_labels():
    a, b = address_bytes(b"A" * 100), address_bytes(b"B" * 3000)
    got = derive_label(45, bytes([1, 2, 3]), [a, b])
    assert got == spec_label(struct.pack("<H", 45) + bytes([1, 2, 3]) + a.encode() + b.encode())
    # the algebra the reference's conformance test states (:88-120)
    assert derive_label(45, b"\x07", [a, b]) == derive_label(45, b"\x07", [a, b])
    assert derive_label(45, b"\x07", [a, b]) != derive_label(45, b"\x07", [b, a])
    assert derive_label(45, b"\x07", [a, b]) != derive_label(46, b"\x07", [a, b])
    assert derive_label(45, b"\x07", [a, b]) != derive_label(45, b"\x08", [a, b])
    assert derive_label(45, b"", []) == spec_label(struct.pack("<H", 45))


def test_derive_label_boundary_composes_the_op_label_with_each_operand():
    a, b = address_bytes(b"A" * 100), address_bytes(b"B" * 3000)
    for op, params, labels in ((45, bytes([1, 2, 3]), [a, b]), (13, b"\x07", [a]),
                               (4, b"", []), (59, struct.pack("<QB", 77, DTYPE_F32), [b])):
        assert derive_label_boundary(op, params, labels) == spec_boundary(op, params, labels)
    # ordered, and a different address from the plain derivation of the same call
    assert derive_label_boundary(45, b"\x07", [a, b]) != derive_label_boundary(45, b"\x07", [b, a])
    assert derive_label_boundary(45, b"\x07", [a, b]) != derive_label(45, b"\x07", [a, b])
    with pytest.raises(Exception):       # an operand label of another axis cannot compose
        derive_label_boundary(45, b"", ["sha256:" + "0" * 64])


def test_op_signature_of_the_served_families():
    u = UnaryCall(BufferRef(0), BufferRef(1), 1000, 16, DTYPE_BF16)
    unary_params = struct.pack("<QHB", 1000, 16, DTYPE_BF16)
    for ctor, op in ((KernelCall.Relu, 10), (KernelCall.Sigmoid, 11), (KernelCall.Tanh, 12),
                     (KernelCall.Gelu, 13), (KernelCall.Silu, 14), (KernelCall.Elu, 15),
                     (KernelCall.Selu, 16), (KernelCall.Exp, 17), (KernelCall.Erf, 31)):
        assert op_signature(ctor(u)) == (op, unary_params)
    bn = BinaryCall(BufferRef(0), BufferRef(1), BufferRef(2), 7, 32, DTYPE_F32)
    assert op_signature(KernelCall.Add(bn)) == (4, struct.pack("<QHB", 7, 32, DTYPE_F32))
    assert op_signature(KernelCall.Mul(bn))[0] == 6
    # b_packed is layout: the packed and row-major products share a signature
    mm = lambda packed: KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), 2,
                                                     8, 4, DTYPE_F32, packed))
    assert op_signature(mm(False)) == op_signature(mm(True))


# ---- the session's derivation (dry loads) ----------------------------------------

def archive(calls, inputs, outputs, constants=()):
    w = HoloWriter()
    w.kernel_calls = list(calls)
    for s, n, dt in inputs:
        w.inputs.append(PortDescriptor(f"in{s}", s, n, dt, [n]))
    for s, n, dt in outputs:
        w.outputs.append(PortDescriptor(f"out{s}", s, n, dt, [n]))
    w.constants = list(constants)
    return w.finish()


N = 16


def add(a, b, o):
    return KernelCall.Add(BinaryCall(BufferRef(a, 0, N * 4), BufferRef(b, 0, N * 4),
                                     BufferRef(o, 0, N * 4), N, 32, DTYPE_F32))


def test_session_labels_a_commutative_op_by_sorted_operands():
    la, lb = address_bytes(b"a" * 64), address_bytes(b"b" * 64)
    sess = HipSession(None, archive([add(0, 1, 2)], [(0, N, 8), (1, N, 8)], [(2, N, 8)]))
    params = struct.pack("<QHB", N, 32, DTYPE_F32)
    # the call writing an output port gives it the boundary label (session.rs:1236-1250)
    want = spec_boundary(4, params, sorted([la, lb]))
    assert sess.output_labels([la, lb]) == [want]
    assert sess.output_labels([lb, la]) == [want]          # a+b and b+a: one label


def test_session_labels_chain_constants_and_fused_calls():
    m, k, n = 2, 8, 4
    w = np.arange(k * n, dtype=np.float32).tobytes()
    calls = [KernelCall.MatMul(MatMulCall(BufferRef(0, 0, m * k * 4), BufferRef(5, 0, k * n * 4),
                                          BufferRef(6, 0, m * n * 4), m, k, n, DTYPE_F32)),
             KernelCall.Gelu(UnaryCall(BufferRef(6, 0, m * n * 4), BufferRef(7, 0, m * n * 4),
                                       m * n, 32, DTYPE_F32))]
    for by_ref in (True, False):
        a = archive(calls, [(0, m * k, 8)], [(7, m * n, 8)],
                    [ConstantEntry(5, DTYPE_F32, w, by_reference=by_ref)])
        sess = HipSession(None, a)
        assert sess.n_calls == 1                            # MatMul -> Gelu fused (106)
        lx = address_bytes(b"x" * (m * k * 4))
        mm_params = struct.pack("<IIIB", m, k, n, DTYPE_F32)
        # the fused call carries one derivation: MatMulActivation's signature
        want = spec_boundary(105, mm_params + bytes([fused_activation.GELU]),
                             [lx, address_bytes(w)])
        assert sess.output_labels([lx]) == [want]
    # with the fusion off, the two calls derive in sequence
    from hologram_amd.session import NO_EPILOGUE_FUSION
    sess = HipSession(None, archive(calls, [(0, m * k, 8)], [(7, m * n, 8)],
                                    [ConstantEntry(5, DTYPE_F32, w)]), flags=NO_EPILOGUE_FUSION)
    inner = derive_label(45, mm_params, [lx, address_bytes(w)])
    want = spec_boundary(13, struct.pack("<QHB", m * n, 32, DTYPE_F32), [inner])
    assert sess.output_labels([lx]) == [want]


def test_output_labels_refuse_a_wrong_count():
    sess = HipSession(None, archive([add(0, 1, 2)], [(0, N, 8), (1, N, 8)], [(2, N, 8)]))
    with pytest.raises(ValueError):
        sess.output_labels([address_bytes(b"")])


def test_op_signature_refuses_an_unserved_call():
    import ctypes
    from hologram_amd import _ffi
    kc = _ffi.KernelCallC()
    kc.tag = 64   # Softmax
    with pytest.raises(UnsupportedOp):
        op_signature(kc)
