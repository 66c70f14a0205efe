"""GPU parity of the quantized-weight row and the computed f32 activations.

- MatMulDequant, output-major W8A8 (i8 / i4 / e8cb): bit-exact against the
  oracle's restatement of matmul_{i8,i4,e8cb}_omajor (exact int32 dots, the
  reference's writeback), with the epilogue (residual, activation) as the
  reference's matmul_dequant_epilogue (float_kernels.rs:727-764).
- MatMulDequant, W8A32 (i8 / u8 / i4, per-channel or per-tensor): within
  1e-5 (normalized max error) of the f64 product of A and the oracle's
  dequantized weight.
- Dequantize and DequantActivation: bit-exact against the oracle.
- f32 Relu / Sigmoid / Tanh / Gelu / Silu / Elu / Selu / Exp / Erf: bit-exact
  against the oracle's scalar functions; 16-bit Relu / Elu / Selu / Erf:
  bit-exact on all 65536 patterns (unary_float's widen, f, narrow; the LUT).
- Sessions: the loader's dequant fusions give the unfused walk's bits.
"""
import struct

import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_E8CB, DTYPE_F16, DTYPE_F32, DTYPE_I4, DTYPE_I8,
                          DTYPE_U8, NO_BUFFER, BinaryCall, BufferRef, DequantActivationCall,
                          DequantizeCall, DeviceWorkspace, HipSession, HoloWriter, KernelCall,
                          MatMulCall, MatMulDequantCall, PortDescriptor, UnaryCall, UnsupportedOp,
                          fused_activation, lut_act)
from hologram_amd.session import NO_DEQUANT_FUSION, NO_EPILOGUE_FUSION

pytestmark = pytest.mark.gpu
FA = fused_activation


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def weight_bytes(quant, count):
    return {DTYPE_I8: count, DTYPE_U8: count, DTYPE_I4: (count + 1) // 2,
            DTYPE_E8CB: count // 8}[quant]


def same_bits(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    both_nan = np.isnan(got) & np.isnan(want)
    return bool(np.all((got.view(np.uint32) == want.view(np.uint32)) | both_nan))


def run_mmd(torch, backend, call_kw, a, bq, scales, zps, residual=None, codebook=None):
    m, n = call_kw["m"], call_kw["n"]
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch, a))
    ws.bind(1, to_dev(torch, bq))
    if scales is not None:
        ws.bind(2, to_dev(torch, scales))
        ws.bind(3, to_dev(torch, zps))
    out = torch.zeros(m * n * 4, dtype=torch.uint8, device="cuda")
    ws.bind(4, out)
    extra = {}
    if residual is not None:
        ws.bind(5, to_dev(torch, residual))
        extra["residual"] = BufferRef(5)
    if codebook is not None:
        ws.bind(6, to_dev(torch, codebook))
        extra["codebook"] = BufferRef(6)
    per_ch = scales is not None
    call = KernelCall.MatMulDequant(MatMulDequantCall(
        BufferRef(0), BufferRef(1), BufferRef(2) if per_ch else NO_BUFFER,
        BufferRef(3) if per_ch else NO_BUFFER, BufferRef(4), **call_kw, **extra))
    backend.dispatch(call, ws)
    backend.synchronize()
    return from_dev(out, np.float32)


def w8a8_operands(rng, tier, m, k, n):
    a = rng.standard_normal(m * k).astype(np.float32) * 3
    if m > 2:
        a[k:2 * k] = 0.0                           # an all-zero row: scale 0, output 0
    bq = rng.integers(0, 256, weight_bytes(tier, k * n)).astype(np.uint8)
    scales = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    cb = rng.integers(-127, 128, 256 * 8).astype(np.int8) if tier == DTYPE_E8CB else None
    return a, bq, scales, cb


# m <= 4 with whole chunks (k a multiple of 16 / 32 / 64 per tier) takes the
# dot4 GEMV; the rest the MFMA GEMM
W8A8_SHAPES = [(1, 896, 4864), (1, 4096, 64), (3, 64, 17), (16, 128, 16), (17, 256, 33),
               (64, 512, 48), (70, 1024, 100), (5, 8, 3), (2, 2048, 1000), (4, 1024, 33),
               (1, 64, 1), (1, 2048, 16385)]


@pytest.mark.parametrize("tier", [DTYPE_I8, DTYPE_I4, DTYPE_E8CB])
@pytest.mark.parametrize("m,k,n", W8A8_SHAPES)
def test_w8a8_omajor_bit_exact(torch_cuda, backend, tier, m, k, n):
    rng = np.random.default_rng(m * 131 + k + n + tier)
    a, bq, scales, cb = w8a8_operands(rng, tier, m, k, n)
    kw = dict(m=m, k=k, n=n, channels=n, inner=1, quant_dtype=tier, bq_omajor=True, act_quant=1)
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, np.zeros(n, np.int32), codebook=cb)
    want = oracle.matmul_q_omajor(tier, a, bq, scales, m, k, n, codebook=cb)
    assert same_bits(got, want)
    if m > 2:
        assert not np.any(got.reshape(m, n)[1])


@pytest.mark.parametrize("tier", [DTYPE_I8, DTYPE_I4])
def test_w8a8_i8_unaligned_k(torch_cuda, backend, tier):
    # k not a multiple of 16: the byte-wise fragment path, ragged last step
    k = 200 if tier == DTYPE_I4 else 201
    rng = np.random.default_rng(k)
    a, bq, scales, cb = w8a8_operands(rng, tier, 4, k, 21)
    kw = dict(m=4, k=k, n=21, channels=21, inner=1, quant_dtype=tier, bq_omajor=True,
              act_quant=1)
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, np.zeros(21, np.int32))
    assert same_bits(got, oracle.matmul_q_omajor(tier, a, bq, scales, 4, k, 21))


@pytest.mark.parametrize("act,res", [(FA.GELU, True), (FA.SILU, False), (0, True),
                                     (FA.SELU, True), (FA.EXP, False)])
def test_w8a8_epilogue_bit_exact(torch_cuda, backend, act, res):
    m, k, n = 3, 256, 40
    rng = np.random.default_rng(act + 10 * res)
    a, bq, scales, cb = w8a8_operands(rng, DTYPE_I8, m, k, n)
    r = rng.standard_normal(m * n).astype(np.float32) if res else None
    kw = dict(m=m, k=k, n=n, channels=n, inner=1, quant_dtype=DTYPE_I8, bq_omajor=True,
              act_quant=1, act=act)
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, np.zeros(n, np.int32), residual=r)
    base = oracle.matmul_q_omajor(DTYPE_I8, a, bq, scales, m, k, n)
    if res:
        base = (base + r).astype(np.float32)
    want = oracle.fused_act_f32(act, base) if act else base
    assert same_bits(got, want)


def test_w8a8_exact_i32_bound(torch_cuda, backend):
    # k = i32::MAX // 127^2: the extreme dot 127 * 127 * k still fits in i32
    k, n = 133144, 16
    a = np.ones(k, np.float32)
    bq = np.full(n * k, 127, np.int8).view(np.uint8)
    bq[k:2 * k] = np.uint8(0x81)                     # -127
    scales = np.full(n, 1e-6, np.float32)
    kw = dict(m=1, k=k, n=n, channels=n, inner=1, quant_dtype=DTYPE_I8, bq_omajor=True,
              act_quant=1)
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, np.zeros(n, np.int32))
    want = oracle.matmul_q_omajor(DTYPE_I8, a, bq, scales, 1, k, n)
    assert same_bits(got, want)
    # a row of ones quantizes to 127 with scale 1/127; the dots are +-127*127*k
    acc = np.float32(127 * 127 * k)
    assert acc == 2147479576 and want[0] == acc * (np.float32(1.0) / np.float32(127) * np.float32(1e-6))
    assert want[1] == -want[0] and np.all(want[2:] == want[0])


def test_w8a8_nonzero_zero_point_is_reported(torch_cuda, backend):
    m, k, n = 1, 64, 16
    rng = np.random.default_rng(1)
    a, bq, scales, _ = w8a8_operands(rng, DTYPE_I8, m, k, n)
    zps = np.zeros(n, np.int32)
    zps[7] = 3
    kw = dict(m=m, k=k, n=n, channels=n, inner=1, quant_dtype=DTYPE_I8, bq_omajor=True,
              act_quant=1)
    with pytest.raises(UnsupportedOp):
        run_mmd(torch_cuda, backend, kw, a, bq, scales, zps)
    # the report is cleared: the next symmetric call runs
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, np.zeros(n, np.int32))
    assert same_bits(got, oracle.matmul_q_omajor(DTYPE_I8, a, bq, scales, m, k, n))


W8A32_CASES = [  # quant, m, k, n, mode
    (DTYPE_I8, 1, 896, 256, "col"), (DTYPE_I8, 3, 64, 40, "tensor"),
    (DTYPE_U8, 5, 128, 48, "col"), (DTYPE_I4, 2, 100, 33, "row"),
    (DTYPE_I4, 70, 256, 130, "col"), (DTYPE_U8, 200, 96, 64, "tensor"),
]


@pytest.mark.parametrize("quant,m,k,n,mode", W8A32_CASES)
def test_w8a32_within_1e5_of_f64(torch_cuda, backend, quant, m, k, n, mode):
    rng = np.random.default_rng(m + k + n + quant)
    a = rng.standard_normal(m * k).astype(np.float32)
    bq = rng.integers(0, 256, weight_bytes(quant, k * n)).astype(np.uint8)
    lo, hi = (-8, 8) if quant == DTYPE_I4 else (-128, 128) if quant == DTYPE_I8 else (0, 256)
    if mode == "tensor":
        scales = zps = None
        kw = dict(channels=0, inner=1, scale_bits=f32_bits(0.0123), zero_point=int(lo // 4))
        w = oracle.dequantize(bq, k * n, quant, scale=0.0123, zp=int(lo // 4))
    else:
        ch, inner = (n, 1) if mode == "col" else (k, n)     # per column, or per input row
        scales = rng.uniform(1e-3, 3e-2, ch).astype(np.float32)
        zps = rng.integers(lo // 2, hi // 2, ch).astype(np.int32)
        kw = dict(channels=ch, inner=inner)
        w = oracle.dequantize(bq, k * n, quant, scales=scales, zps=zps, channels=ch, inner=inner)
    res = rng.standard_normal(m * n).astype(np.float32)
    kw.update(m=m, k=k, n=n, quant_dtype=quant, act=FA.GELU)
    got = run_mmd(torch_cuda, backend, kw, a, bq, scales, zps, residual=res)
    prod = oracle.matmul_f64_blas(a, w, m, k, n)
    want = oracle.fused_act_f32(FA.GELU, (prod + res).astype(np.float32))
    assert oracle.max_rel_err(got, want) <= 1e-5


DQ_N = 100003


@pytest.mark.parametrize("quant", [DTYPE_I8, DTYPE_U8, DTYPE_I4])
@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_BF16, DTYPE_F16])
@pytest.mark.parametrize("per_ch", [False, True])
def test_dequantize_bit_exact(torch_cuda, backend, quant, dtype, per_ch):
    rng = np.random.default_rng(quant * 100 + dtype * 10 + per_ch)
    q = rng.integers(0, 256, weight_bytes(quant, DQ_N)).astype(np.uint8)
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, q))
    es = 4 if dtype == DTYPE_F32 else 2
    out = torch_cuda.zeros(DQ_N * es, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(3, out)
    if per_ch:
        ch, inner = 7, 13
        scales = rng.uniform(1e-3, 5.0, ch).astype(np.float32)
        zps = rng.integers(-300, 300, ch).astype(np.int32)
        ws.bind(1, to_dev(torch_cuda, scales))
        ws.bind(2, to_dev(torch_cuda, zps))
        call = DequantizeCall(BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), DQ_N, ch,
                              inner, quant, dtype)
        want = oracle.dequantize(q, DQ_N, quant, dtype, scales=scales, zps=zps, channels=ch,
                                 inner=inner)
    else:
        call = DequantizeCall(BufferRef(0), NO_BUFFER, NO_BUFFER, BufferRef(3), DQ_N, 0, 1, quant,
                              dtype, f32_bits(0.0371), -5)
        want = oracle.dequantize(q, DQ_N, quant, dtype, scale=0.0371, zp=-5)
    backend.dispatch(KernelCall.Dequantize(call), ws)
    backend.synchronize()
    got = from_dev(out, np.float32 if es == 4 else np.uint16)
    assert np.array_equal(got.view(np.uint32 if es == 4 else np.uint16),
                          want.view(np.uint32 if es == 4 else np.uint16))


@pytest.mark.parametrize("quant", [DTYPE_I8, DTYPE_U8, DTYPE_I4])
@pytest.mark.parametrize("act", [lut_act.SIGMOID, lut_act.TANH, lut_act.GELU, lut_act.SILU,
                                 lut_act.EXP, lut_act.ERF])
def test_dequant_activation_bit_exact(torch_cuda, backend, quant, act):
    rng = np.random.default_rng(quant * 10 + act)
    n = 100001
    q = rng.integers(0, 256, weight_bytes(quant, n)).astype(np.uint8)
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, q))
    out = torch_cuda.zeros(n * 4, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    zp = 128 if quant == DTYPE_U8 else -3
    backend.dispatch(KernelCall.DequantActivation(DequantActivationCall(
        BufferRef(0), BufferRef(1), n, quant, act, DTYPE_F32, f32_bits(0.047), zp)), ws)
    backend.synchronize()
    assert same_bits(from_dev(out, np.float32),
                     oracle.dequant_activation(q, n, quant, act, 0.047, zp))


UNARY = {"Relu": FA.RELU, "Sigmoid": FA.SIGMOID, "Tanh": FA.TANH, "Gelu": FA.GELU,
         "Silu": FA.SILU, "Elu": FA.ELU, "Selu": FA.SELU, "Exp": FA.EXP}
SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72, 88.73, -87.3, -103.9, -104.0,
                     1e-40, -1e-40, 1e-7, -1e-7, 9.0, -9.0, 15.0, -15.0], np.float32)


@pytest.mark.parametrize("name", sorted(UNARY))
def test_f32_unary_bit_exact(torch_cuda, backend, name):
    rng = np.random.default_rng(len(name))
    x = np.concatenate([SPECIALS, (rng.standard_normal(200000) * 6).astype(np.float32),
                        rng.uniform(-120, 90, 50000).astype(np.float32)])
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, x))
    out = torch_cuda.zeros(x.size * 4, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    ctor = getattr(KernelCall, name)
    backend.dispatch(ctor(UnaryCall(BufferRef(0), BufferRef(1), x.size, 32, DTYPE_F32)), ws)
    backend.synchronize()
    assert same_bits(from_dev(out, np.float32), oracle.fused_act_f32(UNARY[name], x))


def test_f32_erf_bit_exact(torch_cuda, backend):
    rng = np.random.default_rng(32)
    x = np.concatenate([SPECIALS, rng.uniform(-7, 7, 100000).astype(np.float32),
                        rng.uniform(-1.3, 1.3, 50000).astype(np.float32),
                        (np.float32(2.0) ** rng.uniform(-40, 0, 20000)).astype(np.float32)])
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, x))
    out = torch_cuda.zeros(x.size * 4, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    backend.dispatch(KernelCall.Erf(UnaryCall(BufferRef(0), BufferRef(1), x.size, 32, DTYPE_F32)),
                     ws)
    backend.synchronize()
    L = oracle.lib()
    want = np.array([L.or_libm_erff(float(v)) for v in x], np.float32)
    assert same_bits(from_dev(out, np.float32), want)


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16])
def test_16bit_erf_every_pattern(torch_cuda, backend, dtype):
    bits = np.arange(65536, dtype=np.uint16)
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, bits))
    out = torch_cuda.zeros(65536 * 2, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    backend.dispatch(KernelCall.Erf(UnaryCall(BufferRef(0), BufferRef(1), 65536, 16, dtype)), ws)
    backend.synchronize()
    assert np.array_equal(from_dev(out, np.uint16), oracle.build_table(lut_act.ERF, dtype))


@pytest.mark.parametrize("name", ["Relu", "Elu", "Selu"])
@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16])
def test_16bit_relu_elu_selu_every_pattern(torch_cuda, backend, name, dtype):
    bits = np.arange(65536, dtype=np.uint16)
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, bits))
    out = torch_cuda.zeros(65536 * 2, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    ctor = getattr(KernelCall, name)
    backend.dispatch(ctor(UnaryCall(BufferRef(0), BufferRef(1), 65536, 16, dtype)), ws)
    backend.synchronize()
    L = oracle.lib()
    if dtype == DTYPE_BF16:
        x = (bits.astype(np.uint32) << 16).view(np.float32)
        want = (oracle.fused_act_f32(UNARY[name], x).view(np.uint32) >> 16).astype(np.uint16)
    else:
        x = np.array([L.or_f16_to_f32(int(b)) for b in bits], np.float32)
        y = oracle.fused_act_f32(UNARY[name], x)
        want = np.array([L.or_f32_to_f16(float(v)) for v in y], np.uint16)
    assert np.array_equal(from_dev(out, np.uint16), want)


# ---- sessions: the loader's dequant fusions ---------------------------------------

M, K, N = 3, 128, 48


def archive(calls, inputs, outputs):
    w = HoloWriter()
    w.kernel_calls = list(calls)
    for s, n, dt in inputs:
        w.inputs.append(PortDescriptor(f"in{s}", s, n, dt, [n]))
    for s, n, dt in outputs:
        w.outputs.append(PortDescriptor(f"out{s}", s, n, dt, [n]))
    return w.finish()


def dq_call(quant, per_ch, layout=0, aq=0, zp=0):
    wb = weight_bytes(quant, K * N)
    sc, zr = (BufferRef(2, 0, N * 4), BufferRef(3, 0, N * 4)) if per_ch else (NO_BUFFER, NO_BUFFER)
    return KernelCall.Dequantize(DequantizeCall(
        BufferRef(1, 0, wb), sc, zr, BufferRef(10, 0, K * N * 4), K * N, N if per_ch else 0, 1,
        quant, DTYPE_F32, f32_bits(0.02), zp, NO_BUFFER, layout, aq))


def chain(quant, per_ch, layout=0, aq=0):
    ref = lambda s, n: BufferRef(s, 0, n * 4)
    calls = [dq_call(quant, per_ch, layout, aq),
             KernelCall.MatMul(MatMulCall(ref(0, M * K), ref(10, K * N), ref(11, M * N), M, K, N,
                                          DTYPE_F32)),
             KernelCall.Add(BinaryCall(ref(11, M * N), ref(5, M * N), ref(12, M * N), M * N, 32,
                                       DTYPE_F32)),
             KernelCall.Silu(UnaryCall(ref(12, M * N), ref(13, M * N), M * N, 32, DTYPE_F32))]
    ins = [(0, M * K, DTYPE_F32), (1, weight_bytes(quant, K * N), 1)]
    if per_ch:
        ins += [(2, N, DTYPE_F32), (3, N, 4)]
    ins += [(5, M * N, DTYPE_F32)]
    return archive(calls, ins, [(13, M * N, DTYPE_F32)])


@pytest.mark.parametrize("quant,per_ch", [(DTYPE_I8, True), (DTYPE_U8, False), (DTYPE_I4, True)])
def test_session_dequant_matmul_epilogue_matches_unfused(torch_cuda, backend, quant, per_ch):
    rng = np.random.default_rng(quant)
    a = rng.standard_normal(M * K).astype(np.float32)
    bq = rng.integers(0, 256, weight_bytes(quant, K * N)).astype(np.uint8)
    res = rng.standard_normal(M * N).astype(np.float32)
    ins = [a.tobytes(), bq.tobytes()]
    if per_ch:
        ins += [rng.uniform(1e-3, 3e-2, N).astype(np.float32).tobytes(),
                rng.integers(-3, 4, N).astype(np.int32).tobytes()]
    ins.append(res.tobytes())
    arch = chain(quant, per_ch)
    fused = HipSession(backend, arch)
    assert fused.call_tags() == [111]
    plain = HipSession(backend, arch, flags=NO_DEQUANT_FUSION | NO_EPILOGUE_FUSION)
    assert plain.call_tags() == [105, 46, 5, 15]
    got, want = fused.execute(ins)[0], plain.execute(ins)[0]
    assert got == want
    fused.close()
    plain.close()


@pytest.mark.parametrize("tier", [DTYPE_I8, DTYPE_I4])
def test_session_declared_output_major_runs_w8a8(torch_cuda, backend, tier):
    rng = np.random.default_rng(tier + 1)
    a = rng.standard_normal(M * K).astype(np.float32)
    bq = rng.integers(0, 256, weight_bytes(tier, K * N)).astype(np.uint8)
    scales = rng.uniform(1e-3, 3e-2, N).astype(np.float32)
    res = rng.standard_normal(M * N).astype(np.float32)
    sess = HipSession(backend, chain(tier, True, layout=1, aq=1))
    assert sess.call_tags() == [111]
    c = sess.call(0).u.matmul_dequant
    assert (c.bq_omajor, c.act_quant, c.act, c.residual.slot) == (1, 1, FA.SILU, 5)
    got = np.frombuffer(sess.execute([a.tobytes(), bq.tobytes(), scales.tobytes(),
                                      np.zeros(N, np.int32).tobytes(), res.tobytes()])[0],
                        np.float32)
    base = oracle.matmul_q_omajor(tier, a, bq, scales, M, K, N)
    assert same_bits(got, oracle.fused_act_f32(FA.SILU, (base + res).astype(np.float32)))
    sess.close()


def test_session_dequant_activation_matches_unfused(torch_cuda, backend):
    n = K * N
    ref = lambda s: BufferRef(s, 0, n * 4)
    arch = archive([dq_call(DTYPE_I8, False, zp=-2),
                    KernelCall.Tanh(UnaryCall(ref(10), ref(11), n, 32, DTYPE_F32))],
                   [(1, n, 1)], [(11, n, DTYPE_F32)])
    q = np.random.default_rng(9).integers(0, 256, n).astype(np.uint8)
    fused = HipSession(backend, arch)
    assert fused.call_tags() == [113]
    plain = HipSession(backend, arch, flags=NO_DEQUANT_FUSION)
    assert plain.call_tags() == [105, 13]
    got, want = fused.execute([q.tobytes()])[0], plain.execute([q.tobytes()])[0]
    assert got == want
    assert same_bits(np.frombuffer(got, np.float32),
                     oracle.dequant_activation(q, n, DTYPE_I8, lut_act.TANH, 0.02, -2))
    fused.close()
    plain.close()
