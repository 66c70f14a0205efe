"""GPU parity of the fused MatMul epilogues and of the fused session walk.

The fused ops (MatMulActivation, MatMulAdd, MatMulAddActivation,
src/cpu/float_kernels.rs:816-935) apply their epilogue to the product the
unfused MatMul gives. So the check is bit for bit: the device's fused output
equals the oracle's epilogue applied to the device's own unfused product. The
product's accuracy is pinned separately (test_gpu_matmul.py).

Both MatMul paths are covered: few rows, where the product is finished in the
epilogue launch, and the tiled path, where the epilogue runs in place.

The session is checked by stepping the same decoder archive with the fusions
on and off. The load-time fusions must not change a single bit of any output
(tokens, logits, int8 caches and scales).
"""
import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BinaryCall, BufferRef, DeviceWorkspace,
                          HipSession, HoloWriter, KernelCall, MatMulActivationCall,
                          MatMulAddActivationCall, MatMulAddCall, MatMulCall, NormCall,
                          PortDescriptor, fused_activation)
from hologram_amd.decoder_graph import DecoderConfig, build_decode_step, init_weights, rope_tables
from hologram_amd.session import NO_DEVICE_FUSION, NO_EPILOGUE_FUSION, NO_NORM_FUSION

pytestmark = pytest.mark.gpu

FA = fused_activation


def widen(bits, dtype):
    if dtype == DTYPE_BF16:
        return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == DTYPE_F16:
        return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(bits).view(np.float32)


def narrow(x, dtype):
    x = np.ascontiguousarray(x, np.float32)
    if dtype == DTYPE_F16:   # the reference's rounding (dtype.rs:121-153), the oracle's codec
        return np.array([oracle.lib().or_f32_to_f16(float(v)) for v in x.ravel()], np.uint16)
    return (x.view(np.uint32) >> 16).astype(np.uint16) if dtype == DTYPE_BF16 else x.view(np.uint32)


CASES = [("act", FA.SILU, DTYPE_BF16), ("act", FA.GELU, DTYPE_BF16), ("act", FA.EXP, DTYPE_BF16),
         ("act", FA.SIGMOID, DTYPE_F32), ("act", FA.TANH, DTYPE_F32), ("act", FA.SILU, DTYPE_F32),
         ("add", 0, DTYPE_BF16), ("add", 0, DTYPE_F32),
         ("addact", FA.GELU, DTYPE_F32), ("addact", FA.SILU, DTYPE_BF16),
         # Relu/Elu/Selu/Exp: tables of narrow(f(widen)) for bf16, f32 computed
         ("act", FA.RELU, DTYPE_BF16), ("act", FA.ELU, DTYPE_BF16), ("act", FA.SELU, DTYPE_BF16),
         ("act", FA.RELU, DTYPE_F32), ("act", FA.ELU, DTYPE_F32), ("act", FA.SELU, DTYPE_F32),
         ("act", FA.EXP, DTYPE_F32), ("addact", FA.EXP, DTYPE_F32), ("addact", FA.SELU, DTYPE_BF16),
         ("addact", FA.RELU, DTYPE_F32),
         # f16: the product narrowed with the reference's rounding, the scalar
         # activation on its widened value (or on the f32 sum), one narrowing
         ("act", FA.GELU, DTYPE_F16), ("act", FA.RELU, DTYPE_F16), ("add", 0, DTYPE_F16),
         ("addact", FA.SILU, DTYPE_F16)]


@pytest.mark.parametrize("m", [8, 100])
@pytest.mark.parametrize("kind,act,dtype", CASES)
def test_fused_matmul_bit_exact(torch_cuda, backend, m, kind, act, dtype):
    k, n = 512, 384
    rng = np.random.default_rng(m * 31 + act)
    a32 = (rng.standard_normal(m * k) * (3 / np.sqrt(k))).astype(np.float32)
    b32 = rng.standard_normal(k * n).astype(np.float32)
    r32 = rng.standard_normal(m * n).astype(np.float32)
    a, b, r = (narrow(x, dtype) for x in (a32, b32, r32))
    es = 4 if dtype == DTYPE_F32 else 2
    ws = DeviceWorkspace()
    keep = [to_dev(torch_cuda, x) for x in (a, b, r)]
    for s, t in enumerate(keep):
        ws.bind(s, t)
    prod = torch_cuda.zeros(m * n * es, dtype=torch_cuda.uint8, device="cuda")
    fused = torch_cuda.zeros(m * n * es, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(3, prod)
    ws.bind(4, fused)
    mm = MatMulCall(BufferRef(0), BufferRef(1), BufferRef(3), m, k, n, dtype)
    backend.dispatch(KernelCall.MatMul(mm), ws)
    mmf = MatMulCall(BufferRef(0), BufferRef(1), BufferRef(4), m, k, n, dtype)
    if kind == "act":
        call = KernelCall.MatMulActivation(MatMulActivationCall(mmf, act))
    elif kind == "add":
        call = KernelCall.MatMulAdd(MatMulAddCall(mmf, BufferRef(2)))
    else:
        call = KernelCall.MatMulAddActivation(MatMulAddActivationCall(mmf, BufferRef(2), act))
    backend.dispatch(call, ws)
    backend.synchronize()
    bits_t = np.uint32 if dtype == DTYPE_F32 else np.uint16
    p = from_dev(prod, bits_t)
    got = from_dev(fused, bits_t)
    v = widen(p, dtype)
    if kind == "act" and dtype == DTYPE_BF16 and act in oracle.FUSED_TO_LUT:
        want = oracle.build_table(oracle.FUSED_TO_LUT[act], dtype)[p]
    elif kind == "act" and dtype == DTYPE_BF16:
        want = narrow(oracle.fused_act_f32(act, v), dtype)
    elif kind == "act":
        want = narrow(oracle.fused_act_f32(act, v), dtype)
    elif kind == "add":
        want = narrow(v + widen(r, dtype), dtype)
    else:
        want = narrow(oracle.fused_act_f32(act, v + widen(r, dtype)), dtype)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:4]}: {got[bad[:4]]} vs {want[bad[:4]]}"


@pytest.mark.parametrize("m,k,n", [(1024, 512, 2048), (4096, 256, 4096), (512, 1024, 4096)])
def test_fused_add_large_m_bit_exact(torch_cuda, backend, m, k, n):
    """bf16 MatMulAdd at large M adds the residual in the tiled kernel's store
    (256x128 tiles for the first and last shapes, 256x256 for the second):
    each element is the plain product narrowed, plus the residual in f32,
    narrowed again."""
    rng = np.random.default_rng(m + k + n)
    a = narrow((rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float32), DTYPE_BF16)
    b = narrow(rng.standard_normal(k * n).astype(np.float32), DTYPE_BF16)
    r = narrow(rng.standard_normal(m * n).astype(np.float32), DTYPE_BF16)
    ws = DeviceWorkspace()
    keep = [to_dev(torch_cuda, x) for x in (a, b, r)]
    for s, t in enumerate(keep):
        ws.bind(s, t)
    prod = torch_cuda.zeros(m * n * 2, dtype=torch_cuda.uint8, device="cuda")
    fused = torch_cuda.zeros(m * n * 2, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(3, prod)
    ws.bind(4, fused)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(3), m, k, n,
                                                  DTYPE_BF16)), ws)
    mmf = MatMulCall(BufferRef(0), BufferRef(1), BufferRef(4), m, k, n, DTYPE_BF16)
    backend.dispatch(KernelCall.MatMulAdd(MatMulAddCall(mmf, BufferRef(2))), ws)
    backend.synchronize()
    p = from_dev(prod, np.uint16)
    got = from_dev(fused, np.uint16)
    want = narrow(widen(p, DTYPE_BF16) + widen(r, DTYPE_BF16), DTYPE_BF16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:4]}: {got[bad[:4]]} vs {want[bad[:4]]}"


CFG = DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                    batch=3, bucket=64)


def step_inputs(cfg, step, tokens):
    cq, sq = rope_tables(cfg, np.array([step]), cfg.heads)
    ck, sk = rope_tables(cfg, np.array([step]), cfg.kv_heads)
    return [np.asarray(tokens, np.int32).tobytes(), np.uint32(step).tobytes(),
            np.full(cfg.batch, step + 1, np.uint32).tobytes(), cq, sq, ck, sk]


def walk(backend, archive, flags, steps, graph=False):
    cfg = CFG
    sess = HipSession(backend, archive, flags=flags)
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    for layer in range(cfg.layers):
        for j, z in enumerate([bytes(P * S * Dh), bytes(P * S * 4)] * 2):
            sess.write_input(7 + 4 * layer + j, z)
    tokens = np.arange(cfg.batch) * 11 + 5
    record = []
    for step in range(steps):
        for i, b in enumerate(step_inputs(cfg, step, tokens)):
            sess.write_input(i, b)
        if graph and step == 0:
            sess.capture()            # step 0 runs eagerly, then the walk is recorded
        elif graph:
            sess.replay()
        else:
            sess.run()
        sess.synchronize()
        record.append([sess.read_output(o) for o in range(len(sess.outputs))])
        tokens = np.frombuffer(record[-1][0], np.int32)
    counts = (sess.n_calls, sess.n_nodes, sess.n_groups)
    sess.close()
    return record, counts


def test_session_fusion_is_bit_identical(torch_cuda, backend):
    archive = build_decode_step(CFG, init_weights(CFG, seed=21))
    base, base_counts = walk(backend, archive, NO_EPILOGUE_FUSION | NO_DEVICE_FUSION, 5)
    assert base_counts[2] == 0
    for flags in (NO_DEVICE_FUSION, NO_EPILOGUE_FUSION, NO_NORM_FUSION, 0):
        rec, counts = walk(backend, archive, flags, 5)
        if not flags & NO_DEVICE_FUSION:
            assert counts[2] > 0 and counts[1] < base_counts[1]
        for step, (x, y) in enumerate(zip(rec, base)):
            for o, (u, v) in enumerate(zip(x, y)):
                assert u == v, f"flags {flags}: step {step}, output {o} differs"


def test_fused_session_graph_replay_matches_eager(torch_cuda, backend):
    archive = build_decode_step(CFG, init_weights(CFG, seed=23))
    eager, _ = walk(backend, archive, 0, 6)
    graph, _ = walk(backend, archive, 0, 6, graph=True)
    for step, (x, y) in enumerate(zip(eager, graph)):
        assert x == y, f"step {step}"


def norm_archive(m, k0, feat, n, gamma, residual):
    """h = A*B (+ R); y = RmsNorm(h) (gamma or none); z = y*W. A, B, W and gamma
    are doubled in-graph, so the MatMuls' operands are session memory. Outputs
    z and h."""
    bf = DTYPE_BF16

    def r(slot, elems):
        return BufferRef(slot, 0, 2 * elems)

    def add(a, b, o, elems):
        return KernelCall.Add(BinaryCall(r(a, elems), r(b, elems), r(o, elems), elems, 16, bf))

    calls = [add(20, 20, 0, m * k0), add(21, 21, 1, k0 * feat), add(22, 22, 3, feat * n)]
    if gamma:
        calls.append(add(23, 23, 5, feat))
    if residual:
        calls.append(add(24, 24, 9, m * feat))
    calls.append(KernelCall.MatMul(MatMulCall(r(0, m * k0), r(1, k0 * feat), r(2, m * feat),
                                              m, k0, feat, bf)))
    h = 2
    if residual:
        calls.append(add(2, 9, 8, m * feat))
        h = 8
    calls.append(KernelCall.RmsNorm(NormCall(r(h, m * feat),
                                             r(5, feat) if gamma else BufferRef(0xFFFFFFFF),
                                             r(4, m * feat), m, feat, dtype=bf)))
    calls.append(KernelCall.MatMul(MatMulCall(r(4, m * feat), r(3, feat * n), r(6, m * n),
                                              m, feat, n, bf)))
    w = HoloWriter()
    w.kernel_calls = calls
    w.exec_plan = [[i] for i in range(len(calls))]   # the residual is ready before the MatMul
    for s, e in ((20, m * k0), (21, k0 * feat), (22, feat * n), (23, feat), (24, m * feat)):
        w.inputs.append(PortDescriptor(f"in{s}", s, e, bf, [e]))
    for s, e in ((6, m * n), (h, m * feat)):
        w.outputs.append(PortDescriptor(f"out{s}", s, e, bf, [e]))
    return w.finish()


@pytest.mark.parametrize("m,feat,gamma,residual", [
    (8, 2048, True, True), (3, 1056, True, True), (40, 4096, False, True),
    (1, 8192, True, False), (17, 256, True, True)])
def test_split_norm_is_bit_identical(torch_cuda, backend, m, feat, gamma, residual):
    """The norm split between its producer's epilogue (row statistics) and its
    reader's A load gives the standalone RmsNorm's bits: same z, same h.
    Features cover one to four vectors per lane and partly filled waves."""
    k0, n = 512, 384
    rng = np.random.default_rng(m * 7 + feat)
    data = [rng.standard_normal(m * k0) / np.sqrt(k0), rng.standard_normal(k0 * feat) * 0.5,
            rng.standard_normal(feat * n) / np.sqrt(feat), 1 + 0.25 * rng.standard_normal(feat),
            rng.standard_normal(m * feat)]
    inputs = [narrow(x.astype(np.float32), DTYPE_BF16).tobytes() for x in data]
    arch = norm_archive(m, k0, feat, n, gamma, residual)
    got = {}
    for flags in (0, NO_NORM_FUSION):
        sess = HipSession(backend, arch, flags=flags)
        for i, b in enumerate(inputs):
            sess.write_input(i, b)
        sess.run()
        sess.synchronize()
        got[flags] = ([sess.read_output(o) for o in range(len(sess.outputs))], sess.n_nodes)
        sess.close()
    (fused, n_fused), (plain, n_plain) = got[0], got[NO_NORM_FUSION]
    assert n_fused == n_plain - 1, "the norm was not fused"
    for o, (u, v) in enumerate(zip(fused, plain)):
        a, b = np.frombuffer(u, np.uint16), np.frombuffer(v, np.uint16)
        bad = np.flatnonzero(a != b)
        assert bad.size == 0, f"output {o}: {bad.size} of {a.size} differ, first at {bad[:4]}"


def two_residual_products_archive(res_offset):
    """Two large-M bf16 MatMulAdds sharing A, their residuals at a byte offset
    of one constant slot: device fusion groups them into one tiled launch."""
    m, k, n = 2048, 512, 1024
    rng = np.random.default_rng(41)
    a = narrow(rng.standard_normal(m * k) / np.sqrt(k), DTYPE_BF16)
    b1, b2 = (narrow(rng.standard_normal(k * n), DTYPE_BF16) for _ in range(2))
    res = narrow(rng.standard_normal(2 * m * n + 8), DTYPE_BF16)
    from hologram_amd import ConstantEntry
    w = HoloWriter()
    w.outputs = [PortDescriptor("y1", 4, m * n, DTYPE_BF16, [m, n]),
                 PortDescriptor("y2", 5, m * n, DTYPE_BF16, [m, n])]
    w.constants = [ConstantEntry(s, DTYPE_BF16, x.tobytes()) for s, x in
                   ((0, a), (1, b1), (2, b2), (3, res))]
    mn2 = m * n * 2
    w.kernel_calls = [
        KernelCall.MatMulAdd(MatMulAddCall(
            MatMulCall(BufferRef(0), BufferRef(1), BufferRef(4), m, k, n, DTYPE_BF16),
            BufferRef(3, res_offset, mn2))),
        KernelCall.MatMulAdd(MatMulAddCall(
            MatMulCall(BufferRef(0), BufferRef(2), BufferRef(5), m, k, n, DTYPE_BF16),
            BufferRef(3, res_offset + mn2, mn2))),
    ]
    w.exec_plan = [[0, 1]]
    return w.finish()


@pytest.mark.parametrize("res_offset", [0, 2])
def test_grouped_tiled_products_with_any_residual_alignment(torch_cuda, backend, res_offset):
    """A residual the grouped kernel's 16-byte loads cannot take (2-byte offset)
    is added in place after the product instead; either way the grouped walk
    equals the unfused one bit for bit."""
    arch = two_residual_products_archive(res_offset)
    outs = []
    for flags in (0, NO_DEVICE_FUSION):
        s = HipSession(backend, arch, flags=flags)
        if flags == 0:
            assert s.n_groups == 1
        s.run()
        s.synchronize()
        outs.append([s.read_output(0), s.read_output(1)])
        s.close()
    assert outs[0] == outs[1]
