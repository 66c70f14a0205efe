"""CPU tests of the quantized-weight row: the oracle's Dequantize and
DequantActivation pinned against the reference's known answers
(crates/hologram-compute/tests/conformance.rs:934-1015,
tests/dequant_activation.rs) and against exact arithmetic; the wire codec of
tags 105 / 118 / 111 / 116 / 117 / 113 against the reference's frozen bytes
(crates/hologram-archive/tests/wire_stability.rs); the host-side refusals of
dispatch; and the loader's fuse_dequant_matmul / fuse_dequant_activation
(crates/hologram-exec/src/session.rs:1853-2148) through dry loads. No device
work."""
import json
import struct

import numpy as np
import pytest

import oracle
from conftest import ROOT
from hologram_amd import (DTYPE_BF16, DTYPE_E8CB, DTYPE_F16, DTYPE_F32, DTYPE_I4, DTYPE_I8,
                          DTYPE_U8, NO_BUFFER, BinaryCall, BufferRef, DequantActivationCall,
                          DequantizeCall, DispatchError, HipSession, HoloWriter, KernelCall,
                          MatMulCall, MatMulDequantCall, PortDescriptor, SlotOutOfRange,
                          UnaryCall, UnsupportedOp, decode_call, encode_calls, fused_activation,
                          lut_act, validate)
from hologram_amd.session import NO_DEQUANT_FUSION, NO_EPILOGUE_FUSION


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def exact_dequant(q: np.ndarray, zp, scale) -> np.ndarray:
    """(q - zp) is a small integer and scale an f32: their product is exact in
    f64, so rounding it once to f32 is the f32 product."""
    return ((q.astype(np.float64) - np.asarray(zp, np.float64))
            * np.asarray(scale, np.float32).astype(np.float64)).astype(np.float32)


# ---- oracle pins: Dequantize ---------------------------------------------------

def test_dequantize_reference_known_answer_per_tensor():
    # conformance.rs:936-967 (kc9): all 256 i8 values, scale 0.0125, zp 7
    q = (np.arange(256) - 128).astype(np.int8)
    got = oracle.dequantize(q, 256, DTYPE_I8, scale=0.0125, zp=7)
    assert np.array_equal(got, exact_dequant(q, 7, np.float32(0.0125)))


def test_dequantize_reference_known_answer_per_channel():
    # conformance.rs:970-1009 (kc9b): [O=4, I=8] per output channel, inner 8
    o, i = 4, 8
    scales = np.array([0.0125, 0.05, 0.2, 0.0033], np.float32)
    zps = np.array([7, -3, 0, 11], np.int32)
    q = (np.arange(o * i) % 200 - 100).astype(np.int8)
    got = oracle.dequantize(q, o * i, DTYPE_I8, scales=scales, zps=zps, channels=o, inner=i)
    want = exact_dequant(q.reshape(o, i), zps[:, None], scales[:, None]).ravel()
    assert np.array_equal(got, want)


def test_dequantize_channel_index_wraps_over_outer():
    # channel = (i / inner) % channels: a [2, 3, 4] tensor with the channel on axis 1
    outer, ch, inner = 2, 3, 4
    scales = np.array([0.5, 0.25, 2.0], np.float32)
    zps = np.array([1, -2, 3], np.int32)
    q = np.arange(outer * ch * inner, dtype=np.int8)
    got = oracle.dequantize(q, q.size, DTYPE_I8, scales=scales, zps=zps, channels=ch, inner=inner)
    want = exact_dequant(q.reshape(outer, ch, inner), zps[None, :, None], scales[None, :, None])
    assert np.array_equal(got, want.ravel())
    # a plausible mistake (channel = i % channels) disagrees
    wrong = exact_dequant(q, zps[np.arange(q.size) % ch], scales[np.arange(q.size) % ch])
    assert not np.array_equal(got, wrong)


def test_dequantize_i4_nibble_order_and_u8():
    # kernels.rs:256-268: element 2k is the low nibble, sign-extended from bit 3
    packed = np.array([0x8F, 0x71, 0x0A], np.uint8)
    got = oracle.dequantize(packed, 5, DTYPE_I4, scale=1.0, zp=0)
    assert got.tolist() == [-1.0, -8.0, 1.0, 7.0, -6.0]
    u8 = np.array([0, 128, 255], np.uint8)
    got = oracle.dequantize(u8, 3, DTYPE_U8, scale=0.5, zp=128)
    assert got.tolist() == [-64.0, 0.0, 63.5]


def test_dequantize_zero_point_subtraction_wraps_like_i32():
    q = np.array([-128], np.int8)
    got = oracle.dequantize(q, 1, DTYPE_I8, scale=1.0, zp=2 ** 31 - 1)
    # -128 - (2^31 - 1) wraps to 2^31 - 127 in two's complement
    assert got[0] == np.float32(2 ** 31 - 127)


def test_dequantize_narrowings():
    q = np.arange(-128, 128, dtype=np.int8)
    f = oracle.dequantize(q, 256, DTYPE_I8, scale=0.0371, zp=-5)
    bf = oracle.dequantize(q, 256, DTYPE_I8, DTYPE_BF16, scale=0.0371, zp=-5)
    assert np.array_equal(bf, (f.view(np.uint32) >> 16).astype(np.uint16))   # truncation
    h = oracle.dequantize(q, 256, DTYPE_I8, DTYPE_F16, scale=0.0371, zp=-5)
    L = oracle.lib()
    assert h.tolist() == [L.or_f32_to_f16(float(v)) for v in f]


def test_dequantize_refuses_unknown_dtypes():
    with pytest.raises(ValueError):
        oracle.dequantize(np.zeros(8, np.uint8), 8, DTYPE_E8CB)
    with pytest.raises(ValueError):
        oracle.dequantize(np.zeros(8, np.uint8), 8, DTYPE_I8, dtype=DTYPE_I8)


# ---- oracle pins: DequantActivation -----------------------------------------------

def gelu_f64(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978846 * (x + 0.044715 * x ** 3)))


@pytest.mark.parametrize("quant,scale,zp", [(DTYPE_I8, 0.05, -7), (DTYPE_U8, 0.03, 128)])
def test_dequant_gelu_tracks_the_f64_function(quant, scale, zp):
    # dequant_activation.rs:68-148 and :150-233: every level, within 1e-5 abs +
    # 1e-5 rel of gelu evaluated in f64 on the dequantized input
    raw = np.arange(256, dtype=np.uint8)
    got = oracle.dequant_activation(raw, 256, quant, lut_act.GELU, scale, zp)
    q = raw.astype(np.int8).astype(np.int64) if quant == DTYPE_I8 else raw.astype(np.int64)
    want = gelu_f64((q - zp) * np.float64(np.float32(scale)))
    assert np.all(np.abs(got - want) <= 1e-5 + 1e-5 * np.abs(want))


FA_OF_LUT = {lut_act.SIGMOID: fused_activation.SIGMOID, lut_act.TANH: fused_activation.TANH,
             lut_act.GELU: fused_activation.GELU, lut_act.SILU: fused_activation.SILU,
             lut_act.EXP: fused_activation.EXP}


@pytest.mark.parametrize("act", sorted(FA_OF_LUT))
@pytest.mark.parametrize("quant", [DTYPE_I8, DTYPE_U8, DTYPE_I4])
def test_dequant_activation_is_the_unfused_pair(act, quant):
    # the densified table equals Dequantize (f32) then the f32 activation,
    # bit for bit (the reference's contract, kernels.rs:305-310)
    rng = np.random.default_rng(act * 7 + quant)
    n = 999
    raw = rng.integers(0, 256, (n + 1) // 2 if quant == DTYPE_I4 else n).astype(np.uint8)
    fused = oracle.dequant_activation(raw, n, quant, act, 0.0417, 3)
    x = oracle.dequantize(raw, n, quant, scale=0.0417, zp=3)
    assert np.array_equal(fused.view(np.uint32), oracle.fused_act_f32(FA_OF_LUT[act], x).view(np.uint32))


@pytest.mark.parametrize("act", [lut_act.ERF, 9])
def test_dequant_activation_erf_is_the_unfused_pair(act):
    # lut_act_ref maps Erf, and any id past it, to libm erff (float_kernels.rs:3628-3638)
    raw = np.arange(256, dtype=np.uint8)
    fused = oracle.dequant_activation(raw, 256, DTYPE_I8, act, 0.021, -4)
    x = oracle.dequantize(raw, 256, DTYPE_I8, scale=0.021, zp=-4)
    L = oracle.lib()
    assert np.array_equal(fused, np.array([L.or_libm_erff(float(v)) for v in x], np.float32))


# ---- W8A32 reference ----------------------------------------------------------

def test_w8a32_reference_is_dequantize_then_f64_product():
    # float_kernels.rs:629-716: the [k, n] weight dequantized, then A . W; the
    # small-m fused path factors the scale to the writeback: (A . Q) * s
    rng = np.random.default_rng(3)
    m, k, n = 3, 40, 24
    a = rng.standard_normal(m * k).astype(np.float32)
    q = rng.integers(-127, 128, k * n).astype(np.int8)
    s = rng.uniform(0.001, 0.02, n).astype(np.float32)
    w = oracle.dequantize(q, k * n, DTYPE_I8, scales=s, zps=np.zeros(n, np.int32), channels=n,
                          inner=1)
    prod = oracle.matmul_f64_blas(a, w, m, k, n)
    factored = (a.reshape(m, k).astype(np.float64) @ q.reshape(k, n).astype(np.float64)
                * s.astype(np.float64)).ravel()
    assert oracle.max_rel_err(prod, factored.astype(np.float32)) < 1e-6


# ---- wire codec ---------------------------------------------------------------

def frozen_calls():
    b = lambda s: BufferRef(s, 0, 64)          # wire_stability.rs:24-30
    plain = MatMulDequantCall(b(0), b(1), b(2), b(3), b(4), 2, 8, 4, channels=4, inner=1,
                              quant_dtype=DTYPE_I8, dtype=DTYPE_F32)

    def omajor(q):
        return MatMulDequantCall(b(0), b(1), b(2), b(3), b(4), 1, 8, 4, channels=4, inner=1,
                                 quant_dtype=q, dtype=DTYPE_F32, bq_omajor=True, act_quant=1)
    return {"mmdq_plain": KernelCall.MatMulDequant(plain),
            "mmdq_omajor_i8": KernelCall.MatMulDequant(omajor(DTYPE_I8)),
            "mmdq_omajor_i4": KernelCall.MatMulDequant(omajor(DTYPE_I4)),
            "plain_matmul": KernelCall.MatMul(MatMulCall(b(0), b(1), b(2), 2, 8, 4, DTYPE_F32))}


def test_wire_bytes_match_the_reference_frozen_encodings():
    golden = json.loads((ROOT / "tests" / "golden" / "wire_frozen.json").read_text())["calls"]
    calls = frozen_calls()
    assert set(golden) == set(calls)
    for name, call in calls.items():
        wire = encode_calls([call])
        assert wire.hex() == golden[name], name
        kc, used = decode_call(wire[4:])
        assert used == len(wire) - 4
        assert bytes(kc) == bytes(call.to_c()), name


def qcalls():
    r = [BufferRef(i, 8 * i, 16 + i) for i in range(8)]
    return [
        KernelCall.Dequantize(DequantizeCall(r[0], r[1], r[2], r[3], 77, 4, 3, DTYPE_I4, DTYPE_BF16,
                                             f32_bits(0.25), -9)),
        KernelCall.Dequantize(DequantizeCall(r[0], NO_BUFFER, NO_BUFFER, r[3], 77,
                                             quant_dtype=DTYPE_E8CB, codebook=r[5],
                                             weight_layout=1, act_quant=1)),
        KernelCall.MatMulDequant(MatMulDequantCall(r[0], r[1], r[2], r[3], r[4], 5, 6, 7, 7, 1,
                                                   DTYPE_U8, DTYPE_F32, f32_bits(0.5), 3)),
        KernelCall.MatMulDequant(MatMulDequantCall(r[0], r[1], r[2], r[3], r[4], 5, 64, 7, 7, 1,
                                                   act=fused_activation.SILU, residual=r[6])),
        KernelCall.MatMulDequant(MatMulDequantCall(r[0], r[1], r[2], r[3], r[4], 1, 64, 7, 7, 1,
                                                   DTYPE_E8CB, bq_omajor=True, act_quant=1,
                                                   codebook=r[7])),
        KernelCall.DequantActivation(DequantActivationCall(r[0], r[1], 123, DTYPE_U8, lut_act.TANH,
                                                           DTYPE_F32, f32_bits(0.1), 128)),
        KernelCall.Relu(UnaryCall(r[0], r[1], 9, 32, DTYPE_F32)),
        KernelCall.Elu(UnaryCall(r[0], r[1], 9, 16, DTYPE_BF16)),
        KernelCall.Selu(UnaryCall(r[0], r[1], 9, 16, DTYPE_F16)),
    ]


@pytest.mark.parametrize("i", range(9))
def test_quant_codec_round_trip(i):
    call = qcalls()[i]
    wire = call.encode()
    kc, used = decode_call(wire + b"\x00\x01")
    assert used == len(wire)
    assert bytes(kc) == bytes(call.to_c())


def test_quant_wire_discriminants():
    tags = [struct.unpack_from("<H", c.encode())[0] for c in qcalls()]
    assert tags == [105, 118, 111, 116, 117, 113, 11, 16, 17]
    # 105 carries no tail; 118 adds layout, act quant and a codebook ref
    assert len(qcalls()[1].encode()) - len(qcalls()[0].encode()) == 2 + 20


def test_quant_codec_truncated():
    for c in qcalls()[:6]:
        with pytest.raises(DispatchError):
            decode_call(c.encode()[:-1])


# ---- refusals (dispatch's host checks) --------------------------------------------

def dq(n=16, quant=DTYPE_I8, dtype=DTYPE_F32, per_ch=False, channels=4, inner=4):
    if per_ch:
        return KernelCall.Dequantize(DequantizeCall(BufferRef(0), BufferRef(1), BufferRef(2),
                                                    BufferRef(3), n, channels, inner, quant,
                                                    dtype))
    return KernelCall.Dequantize(DequantizeCall(BufferRef(0), NO_BUFFER, NO_BUFFER, BufferRef(3),
                                                n, 0, 1, quant, dtype))


def test_dequantize_refusals():
    validate(dq(), [16, 0, 0, 64])
    validate(dq(17, DTYPE_I4), [9, 0, 0, 68])
    with pytest.raises(SlotOutOfRange):
        validate(dq(17, DTYPE_I4), [8, 0, 0, 68])            # input short
    with pytest.raises(SlotOutOfRange):
        validate(dq(dtype=DTYPE_BF16), [16, 0, 0, 31])       # output short
    with pytest.raises(SlotOutOfRange):
        validate(dq(quant=DTYPE_E8CB), [16, 0, 0, 64])       # kernels.rs:188-191
    with pytest.raises(SlotOutOfRange):
        validate(dq(dtype=DTYPE_I8), [16, 0, 0, 64])         # unknown output dtype
    with pytest.raises(UnsupportedOp):
        validate(dq(dtype=9), [16, 0, 0, 128])               # f64: not served here
    validate(dq(per_ch=True), [16, 16, 16, 64])
    with pytest.raises(SlotOutOfRange):
        validate(dq(per_ch=True), [16, 12, 16, 64])          # scales short


def test_dequant_activation_refusals():
    da = lambda act=lut_act.GELU, quant=DTYPE_I8: KernelCall.DequantActivation(
        DequantActivationCall(BufferRef(0), BufferRef(1), 10, quant, act))
    validate(da(), [10, 40])
    with pytest.raises(SlotOutOfRange):
        validate(da(), [10, 39])
    with pytest.raises(SlotOutOfRange):
        validate(da(quant=DTYPE_E8CB), [10, 40])
    validate(da(lut_act.ERF), [10, 40])


def mmd(m=2, k=16, n=8, **kw):
    per_ch = kw.pop("per_ch", True)
    sc, zp = (BufferRef(2), BufferRef(3)) if per_ch else (NO_BUFFER, NO_BUFFER)
    kw.setdefault("channels", n if per_ch else 0)
    return KernelCall.MatMulDequant(MatMulDequantCall(BufferRef(0), BufferRef(1), sc, zp,
                                                      BufferRef(4), m, k, n, **kw))


def test_matmul_dequant_refusals():
    sizes = [2 * 16 * 4, 16 * 8, 8 * 4, 8 * 4, 2 * 8 * 4, 0, 2048]
    validate(mmd(), sizes)
    validate(mmd(m=0), [])
    with pytest.raises(UnsupportedOp):
        validate(mmd(dtype=DTYPE_BF16), sizes)                       # f32 output only
    with pytest.raises(UnsupportedOp):
        validate(mmd(quant_dtype=9), sizes)                          # unknown tier
    with pytest.raises(UnsupportedOp):                               # VQ tier without codebook
        validate(mmd(quant_dtype=DTYPE_E8CB, bq_omajor=True, act_quant=1), sizes)
    with pytest.raises(UnsupportedOp):                               # codebook on a scalar tier
        validate(mmd(codebook=BufferRef(6)), sizes)
    with pytest.raises(UnsupportedOp):                               # omajor without W8A8
        validate(mmd(bq_omajor=True), sizes)
    with pytest.raises(UnsupportedOp):                               # W8A8 on u8
        validate(mmd(quant_dtype=DTYPE_U8, bq_omajor=True, act_quant=1), sizes)
    with pytest.raises(UnsupportedOp):                               # i4 W8A8 with odd k
        validate(mmd(k=15, quant_dtype=DTYPE_I4, bq_omajor=True, act_quant=1), sizes)
    with pytest.raises(UnsupportedOp):                               # per-tensor W8A8
        validate(mmd(per_ch=False, bq_omajor=True, act_quant=1), sizes)
    with pytest.raises(UnsupportedOp):                               # beyond the exact-i32 k
        validate(mmd(m=1, k=133145, n=1, bq_omajor=True, act_quant=1),
                 [133145 * 4, 133145, 4, 4, 4])
    validate(mmd(m=1, k=133144, n=1, bq_omajor=True, act_quant=1), [133144 * 4, 133144, 4, 4, 4])
    validate(mmd(quant_dtype=DTYPE_E8CB, bq_omajor=True, act_quant=1, codebook=BufferRef(6)),
             sizes)
    with pytest.raises(SlotOutOfRange):                              # codebook short
        validate(mmd(quant_dtype=DTYPE_E8CB, bq_omajor=True, act_quant=1, codebook=BufferRef(6)),
                 sizes[:6] + [2047])
    with pytest.raises(UnsupportedOp):                               # e8cb W8A32
        validate(mmd(quant_dtype=DTYPE_E8CB, codebook=BufferRef(6)), sizes)
    with pytest.raises(SlotOutOfRange):
        validate(mmd(), [2 * 16 * 4, 16 * 8 - 1] + sizes[2:])       # bq short
    with pytest.raises(SlotOutOfRange):
        validate(mmd(residual=BufferRef(5)), sizes)                  # residual slot empty
    validate(mmd(residual=BufferRef(5), act=fused_activation.GELU), sizes[:5] + [64] + sizes[6:])
    validate(mmd(act=200), sizes)                                    # past the table: identity


# ---- the loader's dequant passes (dry loads) ----------------------------------------

def archive(calls, inputs, outputs, plan=None):
    w = HoloWriter()
    w.kernel_calls = list(calls)
    for s, n, dt in inputs:
        w.inputs.append(PortDescriptor(f"in{s}", s, n, dt, [n]))
    for s, n, dt in outputs:
        w.outputs.append(PortDescriptor(f"out{s}", s, n, dt, [n]))
    if plan:
        w.exec_plan = plan
    return w.finish()


M, K, N = 2, 64, 32


def dq_weight(out_slot=10, per_ch=True, quant=DTYPE_I8, layout=0, aq=0, codebook=NO_BUFFER,
              n=N, k=K):
    wb = k * n if quant in (DTYPE_I8, DTYPE_U8) else (k * n + 1) // 2 if quant == DTYPE_I4 \
        else k * n // 8
    sc, zp = (BufferRef(2, 0, n * 4), BufferRef(3, 0, n * 4)) if per_ch else (NO_BUFFER, NO_BUFFER)
    return KernelCall.Dequantize(DequantizeCall(
        BufferRef(1, 0, wb), sc, zp, BufferRef(out_slot, 0, k * n * 4), k * n,
        n if per_ch else 0, 1, quant, DTYPE_F32, f32_bits(0.01), 0, codebook, layout, aq))


def f32mm(a, b, o, m=M, k=K, n=N):
    return KernelCall.MatMul(MatMulCall(BufferRef(a, 0, m * k * 4), BufferRef(b, 0, k * n * 4),
                                        BufferRef(o, 0, m * n * 4), m, k, n, DTYPE_F32))


def f32u(ctor, x, o, n=M * N):
    return ctor(UnaryCall(BufferRef(x, 0, n * 4), BufferRef(o, 0, n * 4), n, 32, DTYPE_F32))


def f32add(a, b, o, n=M * N):
    return KernelCall.Add(BinaryCall(BufferRef(a, 0, n * 4), BufferRef(b, 0, n * 4),
                                     BufferRef(o, 0, n * 4), n, 32, DTYPE_F32))


QIN = [(0, M * K, DTYPE_F32), (1, K * N, DTYPE_I8), (2, N, DTYPE_F32), (3, N, 4)]


def test_dequant_matmul_fuses_and_absorbs_the_epilogue():
    a = archive([dq_weight(), f32mm(0, 10, 11), f32add(11, 5, 12), f32u(KernelCall.Gelu, 12, 13)],
                QIN + [(5, M * N, DTYPE_F32)], [(13, M * N, DTYPE_F32)])
    s = HipSession(None, a)
    assert s.call_tags() == [111]
    c = s.call(0).u.matmul_dequant
    assert (c.bq.slot, c.output.slot, c.residual.slot, c.act) == (1, 13, 5, fused_activation.GELU)
    assert (c.bq_omajor, c.act_quant, c.codebook.slot) == (0, 0, 0xFFFFFFFF)
    # each pass alone
    assert HipSession(None, a, flags=NO_EPILOGUE_FUSION).call_tags() == [111, 5, 14]
    assert HipSession(None, a, flags=NO_DEQUANT_FUSION).call_tags() == [105, 108]


def test_dequant_matmul_conditions():
    # the dequantized weight must be the B operand of an unpacked f32 MatMul
    a = archive([dq_weight(), f32mm(10, 0, 11, m=K, k=K, n=K)],
                [(0, K * K, DTYPE_F32), (1, K * N, DTYPE_I8), (2, N, 8), (3, N, 4)],
                [(11, K * K, DTYPE_F32)])
    assert HipSession(None, a).call_tags() == [105, 46]
    # a second reader of the dense weight blocks the fusion
    a = archive([dq_weight(), f32mm(0, 10, 11), f32u(KernelCall.Relu, 10, 12, n=K * N)], QIN,
                [(11, M * N, DTYPE_F32), (12, K * N, DTYPE_F32)])
    assert HipSession(None, a).call_tags() == [105, 46, 11]
    # the dense weight as an output port blocks it
    a = archive([dq_weight(), f32mm(0, 10, 11)], QIN,
                [(10, K * N, DTYPE_F32), (11, M * N, DTYPE_F32)])
    assert HipSession(None, a).call_tags() == [105, 46]


def test_output_major_declaration_fuses_as_w8a8():
    a = archive([dq_weight(layout=1, aq=1), f32mm(0, 10, 11)], QIN, [(11, M * N, DTYPE_F32)])
    s = HipSession(None, a)
    assert s.call_tags() == [111]
    c = s.call(0).u.matmul_dequant
    assert (c.bq_omajor, c.act_quant) == (1, 1)


def test_unreadable_output_major_declaration_refuses_the_load():
    # session.rs:1944-1946 / 1995-2006: [n, k] bytes that only the W8A8 GEMV reads
    lonely = archive([dq_weight(layout=1, aq=1)], QIN[:4], [(10, K * N, DTYPE_F32)])
    with pytest.raises(DispatchError):
        HipSession(None, lonely)
    per_tensor = archive([dq_weight(per_ch=False, layout=1, aq=1), f32mm(0, 10, 11)], QIN[:2],
                         [(11, M * N, DTYPE_F32)])
    with pytest.raises(DispatchError):
        HipSession(None, per_tensor)
    with pytest.raises(DispatchError):      # the declaration stands with the pass off
        HipSession(None, archive([dq_weight(layout=1, aq=1), f32mm(0, 10, 11)], QIN,
                                 [(11, M * N, DTYPE_F32)]), flags=NO_DEQUANT_FUSION)


def test_e8cb_without_the_w8a8_form_stays_unfused():
    # not scalar-decodable: the pass leaves it, and the standalone Dequantize refuses it
    a = archive([dq_weight(quant=DTYPE_E8CB), f32mm(0, 10, 11)],
                [(0, M * K, 8), (1, K * N // 8, 1), (2, N, 8), (3, N, 4)],
                [(11, M * N, DTYPE_F32)])
    with pytest.raises(SlotOutOfRange):
        HipSession(None, a)


def test_dequant_activation_fuses_per_tensor_f32_only():
    n = K * N
    one = lambda ctor, per_ch=False: archive(
        [dq_weight(per_ch=per_ch), f32u(ctor, 10, 11, n=n)],
        QIN[:2] + (QIN[2:] if per_ch else []), [(11, n, DTYPE_F32)])
    for ctor in (KernelCall.Sigmoid, KernelCall.Tanh, KernelCall.Gelu, KernelCall.Silu,
                 KernelCall.Exp, KernelCall.Erf):
        s = HipSession(None, one(ctor))
        assert s.call_tags() == [113]
    assert HipSession(None, one(KernelCall.Erf)).call(0).u.dequant_act.act == lut_act.ERF
    assert HipSession(None, one(KernelCall.Gelu)).call(0).u.dequant_act.act == lut_act.GELU
    assert HipSession(None, one(KernelCall.Relu)).call_tags() == [105, 11]    # no table form
    assert HipSession(None, one(KernelCall.Gelu, per_ch=True)).call_tags() == [105, 14]
    assert HipSession(None, one(KernelCall.Gelu), flags=NO_DEQUANT_FUSION).call_tags() == [105, 14]


def test_dequant_matmul_wins_over_the_epilogue_pass():
    # the reference runs fuse_dequant_matmul before fuse_matmul_epilogue
    # (session.rs:474-497): the MatMul becomes a MatMulDequant, which then takes
    # the activation in its own epilogue
    a = archive([dq_weight(), f32mm(0, 10, 11), f32u(KernelCall.Silu, 11, 12)], QIN,
                [(12, M * N, DTYPE_F32)])
    s = HipSession(None, a)
    assert s.call_tags() == [111]
    assert s.call(0).u.matmul_dequant.act == fused_activation.SILU
