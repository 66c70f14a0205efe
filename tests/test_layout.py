"""Reshape (wire 60) and Slice (wire 63), CPU side: the wire form
(kernel_codec.rs:681-686 put_layout), the op signatures (kernel_call.rs:1385,
1388: opcodes 59 and 62 over element_count and dtype), the refusals of the
reference kernels (layout_float, float_kernels.rs:2939-2954; layout_copy,
kernels.rs:688-701; f64, kernels.rs:1611-1615), and how a session treats
them (session.rs compute_and_label :1106-1150), checked on dry loads: an
interior Reshape or Slice is bound, not run, and a Reshape carries its input's
κ-label; one that writes an output port is a copy step whose port takes the
boundary label; a step that recomputes a value the walk already holds is bound
to it (resident reuse, :1121-1131). The oracle walk's copies are checked
against numpy slicing."""
import struct

import numpy as np
import pytest

from hologram_amd import (DTYPE_BF16, DTYPE_F32, DTYPE_I32, BinaryCall, BufferRef, ConstantEntry,
                          HipSession, HoloWriter, KernelCall, LayoutCall, MatMulCall,
                          PortDescriptor, SlotOutOfRange, UnaryCall, UnsupportedOp, decode_call,
                          validate)
from hologram_amd.kappa import address_bytes, derive_label, op_signature
from oracle.graph import OracleSession
from test_kappa import spec_boundary


def reshape(i, o, n, dt=DTYPE_F32):
    return KernelCall.Reshape(LayoutCall(i, o, n, dt))


def slice_(i, o, n, dt=DTYPE_F32):
    return KernelCall.Slice(LayoutCall(i, o, n, dt))


def test_wire_form_and_signature():
    c = slice_(BufferRef(3, 64, 128), BufferRef(4, 0, 128), 32, DTYPE_F32)
    wire = c.encode()
    assert wire == struct.pack("<H", 63) + struct.pack("<IQQIQQQB", 3, 64, 128, 4, 0, 128, 32, 8)
    kc, used = decode_call(wire)
    assert used == len(wire) and kc.tag == 63
    assert (kc.u.layout.input.slot, kc.u.layout.input.offset, kc.u.layout.element_count) == (3, 64, 32)
    assert op_signature(c) == (62, struct.pack("<QB", 32, DTYPE_F32))
    assert op_signature(reshape(BufferRef(0), BufferRef(1), 9, DTYPE_BF16)) == \
        (59, struct.pack("<QB", 9, DTYPE_BF16))


def test_refusals_follow_the_reference_kernels():
    ok = reshape(BufferRef(0), BufferRef(1), 16, DTYPE_F32)
    validate(ok, [64, 64])
    with pytest.raises(SlotOutOfRange):                     # input shorter than 16 f32
        validate(reshape(BufferRef(0, 0, 32), BufferRef(1), 16, DTYPE_F32), [64, 64])
    with pytest.raises(SlotOutOfRange):                     # output shorter
        validate(reshape(BufferRef(0), BufferRef(1, 0, 60), 16, DTYPE_F32), [64, 64])
    with pytest.raises(SlotOutOfRange):                     # read overlaps the write
        validate(reshape(BufferRef(0, 0, 64), BufferRef(0, 32, 64), 8, DTYPE_F32), [128])
    with pytest.raises(UnsupportedOp):                      # f64 is no compute dtype
        validate(reshape(BufferRef(0), BufferRef(1), 4, 9), [64, 64])
    # the byte domain: an i32 layout call copies element_count bytes (layout_copy)
    validate(reshape(BufferRef(0, 0, 16), BufferRef(1, 0, 16), 16, DTYPE_I32), [64, 64])


N = 16


def port(s, n, dt=DTYPE_F32):
    return PortDescriptor(f"p{s}", s, n, dt, [n])


def build(calls, inputs, outputs, constants=()):
    w = HoloWriter()
    w.kernel_calls = list(calls)
    w.inputs = [port(*p) for p in inputs]
    w.outputs = [port(*p) for p in outputs]
    w.constants = list(constants)
    return w.finish()


def add(a, b, o, n=N):
    return KernelCall.Add(BinaryCall(a, b, o, n, 32, DTYPE_F32))


def bf16(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def chain_archive(dt=DTYPE_BF16):
    """x (slot 0, 2 x 16) -> Reshape -> [slot 2] -> Add c (const slot 1) ->
    [slot 3] -> Slice of the second row -> [slot 4] -> Gelu -> out (slot 5);
    the Reshape and the Slice are interior."""
    es = 2 if dt == DTYPE_BF16 else 4
    c = np.arange(2 * N, dtype=np.float32) * 0.25
    cb = bf16(c) if dt == DTYPE_BF16 else c
    nb = 2 * N * es
    calls = [reshape(BufferRef(0, 0, nb), BufferRef(2, 0, nb), 2 * N, dt),
             KernelCall.Add(BinaryCall(BufferRef(2, 0, nb), BufferRef(1, 0, nb), BufferRef(3, 0, nb),
                                       2 * N, 16, dt)),
             slice_(BufferRef(3, N * es, N * es), BufferRef(4, 0, N * es), N, dt),
             KernelCall.Gelu(UnaryCall(BufferRef(4, 0, N * es), BufferRef(5, 0, N * es), N, 16, dt))]
    return build(calls, [(0, 2 * N, dt)], [(5, N, dt)], [ConstantEntry(1, dt, cb.tobytes())]), cb


def test_interior_reshape_and_slice_are_bound_not_run():
    arch, c = chain_archive()
    sess = HipSession(None, arch)
    assert sess.n_calls == 4 and sess.n_nodes == 2         # Add and Gelu run; the rest is bound
    lx = address_bytes(b"x" * (2 * N * 2))
    lc = address_bytes(c.tobytes())
    # Reshape re-addresses: the Add derives from x's own label
    l_add = derive_label(4, struct.pack("<QHB", 2 * N, 16, DTYPE_BF16), sorted([lx, lc]))
    l_slice = derive_label(62, struct.pack("<QB", N, DTYPE_BF16), [l_add])
    want = spec_boundary(13, struct.pack("<QHB", N, 16, DTYPE_BF16), [l_slice])
    assert sess.output_labels([lx]) == [want]


def test_oracle_walk_of_the_chain():
    """The walk's value: widen, add in f32, truncate (binary_float), the second
    row, then the GELU table."""
    import oracle
    arch, c = chain_archive()
    x = bf16(np.linspace(-3, 3, 2 * N, dtype=np.float32))
    o = OracleSession(arch)
    o.set_input(0, x.tobytes())
    o.run()
    wide = lambda u: (u.astype(np.uint32) << 16).view(np.float32)
    s = bf16(wide(x) + wide(c))[N:]
    want = oracle.build_table(2, DTYPE_BF16)[s]
    assert np.array_equal(o.output(0).view(np.uint16), want)


def test_output_port_reshape_is_a_copy_with_a_boundary_label():
    calls = [add(BufferRef(0, 0, N * 4), BufferRef(1, 0, N * 4), BufferRef(2, 0, N * 4)),
             reshape(BufferRef(2, 0, N * 4), BufferRef(3, 0, N * 4), N)]
    sess = HipSession(None, build(calls, [(0, N), (1, N)], [(3, N)]))
    assert sess.n_nodes == 2                                # the port's Reshape copies
    la, lb = address_bytes(b"a"), address_bytes(b"b")
    l_add = derive_label(4, struct.pack("<QHB", N, 32, DTYPE_F32), sorted([la, lb]))
    assert sess.output_labels([la, lb]) == [spec_boundary(59, struct.pack("<QB", N, DTYPE_F32),
                                                          [l_add])]


def test_a_port_no_call_writes_carries_its_input_label():
    calls = [add(BufferRef(0, 0, N * 4), BufferRef(0, 0, N * 4), BufferRef(2, 0, N * 4))]
    sess = HipSession(None, build(calls, [(0, N)], [(2, N), (0, N)]))
    la = address_bytes(b"a")
    got = sess.output_labels([la])
    assert got[1] == la
    assert got[0] == spec_boundary(4, struct.pack("<QHB", N, 32, DTYPE_F32), [la, la])


def dup_archive():
    """Two MatMuls of the same operands and params (the second a repeat of the
    first), added; a third product over a different weight is not a repeat."""
    m, k, n = 4, 8, 16
    w1 = np.arange(k * n, dtype=np.float32).tobytes()
    w2 = (np.arange(k * n, dtype=np.float32) + 1).tobytes()
    mm = lambda b, o: KernelCall.MatMul(MatMulCall(BufferRef(0, 0, m * k * 4), BufferRef(b, 0, k * n * 4),
                                                   BufferRef(o, 0, m * n * 4), m, k, n, DTYPE_F32))
    calls = [mm(1, 3), mm(1, 4), mm(2, 5), add(BufferRef(3, 0, m * n * 4), BufferRef(4, 0, m * n * 4),
                                               BufferRef(6, 0, m * n * 4), m * n),
             add(BufferRef(6, 0, m * n * 4), BufferRef(5, 0, m * n * 4), BufferRef(7, 0, m * n * 4),
                 m * n)]
    return build(calls, [(0, m * k)], [(7, m * n)],
                 [ConstantEntry(1, DTYPE_F32, w1), ConstantEntry(2, DTYPE_F32, w2)]), (m, k, n)


def test_a_repeated_value_is_bound_to_its_first_computation():
    arch, _ = dup_archive()
    from hologram_amd.session import NO_DEVICE_FUSION
    sess = HipSession(None, arch, flags=NO_DEVICE_FUSION)
    assert sess.n_calls == 5 and sess.n_nodes == 4          # the second product is bound


def test_an_output_port_value_is_never_bound_to_a_repeat():
    m = N
    calls = [add(BufferRef(0, 0, m * 4), BufferRef(1, 0, m * 4), BufferRef(2, 0, m * 4)),
             add(BufferRef(0, 0, m * 4), BufferRef(1, 0, m * 4), BufferRef(3, 0, m * 4))]
    sess = HipSession(None, build(calls, [(0, m), (1, m)], [(2, m), (3, m)]))
    assert sess.n_nodes == 2


def test_oracle_layout_copy_semantics():
    """The oracle walk's Reshape/Slice: a float dtype copies element_count
    elements, the byte domain element_count bytes, f64 is refused."""
    data = np.arange(64, dtype=np.uint8)
    for dt, n, want in ((DTYPE_F32, 4, data[16:32]), (DTYPE_BF16, 4, data[16:24]),
                        (DTYPE_I32, 4, data[16:20])):
        arch = build([slice_(BufferRef(0, 16, 32), BufferRef(1, 0, 16), n, dt)], [(0, 16, 1)],
                     [(1, 16, 1)])
        o = OracleSession(arch)
        o.set_input(0, data.tobytes())
        o.run()
        assert np.array_equal(o.slots[1][:len(want)], want), dt
    arch = build([reshape(BufferRef(0), BufferRef(1), 2, 9)], [(0, 16, 1)], [(1, 16, 1)])
    o = OracleSession(arch)
    o.set_input(0, data.tobytes())
    with pytest.raises(ValueError):
        o.run()
