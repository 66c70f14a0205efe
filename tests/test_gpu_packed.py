"""GPU: few-row bf16 groups over constant weights run as one launch over
weights packed into the matrix cores' operand order (gemv_packed.hip).

The few-row product's summation order is fixed by K alone (64 chains of
32-deep steps, 16 groups of four chains, gemm_skinny.hip), so the packed
launch must give the bits of the split-K launches it replaces, for every
epilogue: the plain product, + residual (MatMulAdd, float_kernels.rs:846-888),
a table activation (MatMulActivation, :816-844), an f32 activation of the
sum (MatMulAddActivation, :890-935), the SwiGLU product (binary_float Mul,
:238-300), rotary embedding (rope_float, :3123-3186), the int8 append
(quantize_row_i8, simd.rs:4755-4785) and a fused RmsNorm of A (rms_norm,
float_kernels.rs:1683-1755), whose statistics the packed launch takes itself.
Each archive is walked three ways — packed, split-K fused (NO_WEIGHT_PACKING)
and unfused (NO_DEVICE_FUSION) — and all outputs must agree bit for bit; the
plain product is also held to a float64 product within bf16 rounding."""
import numpy as np
import pytest

from hologram_amd import (DTYPE_BF16, BinaryCall, BufferRef, ConstantEntry, HipSession, HoloWriter,
                          KernelCall, MatMulActivationCall, MatMulAddActivationCall, MatMulAddCall,
                          MatMulCall, NormCall, PortDescriptor, fused_activation)
from hologram_amd.decoder_graph import DecoderConfig, build_decode_step, init_weights, rope_tables
from hologram_amd.session import NO_DEVICE_FUSION, NO_WEIGHT_PACKING

pytestmark = pytest.mark.gpu
FA = fused_activation
BF = DTYPE_BF16


def bf16(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def widen(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


def r(slot, elems):
    return BufferRef(slot, 0, 2 * elems)


def run3(backend, arch, inputs, expect_packed):
    """Outputs of the packed, split-K fused and unfused walks (asserting the
    packed session really packed `expect_packed` groups)."""
    outs = {}
    for flags in (0, NO_WEIGHT_PACKING, NO_DEVICE_FUSION):
        s = HipSession(backend, arch, flags=flags)
        if flags == 0:
            assert s.packed[0] == expect_packed, s.packed
        elif flags == NO_WEIGHT_PACKING:
            assert s.packed[0] == 0
        outs[flags] = s.execute(inputs)
        s.close()
    for flags in (NO_WEIGHT_PACKING, NO_DEVICE_FUSION):
        for o, (u, v) in enumerate(zip(outs[0], outs[flags])):
            a, b = np.frombuffer(u, np.uint16), np.frombuffer(v, np.uint16)
            bad = np.flatnonzero(a != b)
            assert bad.size == 0, f"flags {flags}, output {o}: {bad.size} of {a.size} differ at {bad[:4]}"
    return outs[0]


def product_archive(m, k, n, kind, act, w, res):
    """y = 2x * W (W a constant [k, n]) with the fused epilogue `kind`; 2x is
    computed in-graph, so A is session memory."""
    mm = MatMulCall(r(4, m * k), r(1, k * n), r(2, m * n), m, k, n, BF)
    if kind == "store":
        call = KernelCall.MatMul(mm)
    elif kind == "act":
        call = KernelCall.MatMulActivation(MatMulActivationCall(mm, act))
    elif kind == "add":
        call = KernelCall.MatMulAdd(MatMulAddCall(mm, r(3, m * n)))
    else:
        call = KernelCall.MatMulAddActivation(MatMulAddActivationCall(mm, r(3, m * n), act))
    wr = HoloWriter()
    wr.kernel_calls = [KernelCall.Add(BinaryCall(r(0, m * k), r(0, m * k), r(4, m * k), m * k, 16, BF)),
                       call]
    wr.constants = [ConstantEntry(1, BF, w.tobytes()), ConstantEntry(3, BF, res.tobytes())]
    wr.inputs = [PortDescriptor("x", 0, m * k, BF, [m, k])]
    wr.outputs = [PortDescriptor("y", 2, m * n, BF, [m, n])]
    return wr.finish()


@pytest.mark.parametrize("m,k,n", [(8, 2048, 2048), (1, 32, 16), (5, 96, 48), (16, 4096, 384),
                                   (8, 8192, 256), (3, 2080, 64), (16, 512, 1040), (4, 256, 8192),
                                   (8, 256, 16384), (2, 128, 1000), (8, 256, 16400)])
@pytest.mark.parametrize("kind,act", [("store", 0), ("add", 0), ("act", FA.GELU), ("addact", FA.SILU)])
def test_packed_product_and_epilogues(torch_cuda, backend, m, k, n, kind, act):
    """Every K shape class: one step a chain and several, chains and groups
    left empty (K = 32, 96), a last group partly filled (K = 2080); rows 1 to
    16; 8-column tiles (few tiles, or a width not a multiple of 16: 1040,
    1000), 16-column tiles (8192) and several tiles a workgroup (16384). K =
    8192 and more than 1024 tiles (16400 columns) stay split-K (measured
    faster there): all three walks still agree."""
    rng = np.random.default_rng(m * 1000 + k + n)
    x = bf16(rng.standard_normal(m * k) / np.sqrt(k))
    w = bf16(rng.standard_normal(k * n))
    res = bf16(rng.standard_normal(m * n))
    expect = 1 if k <= 4096 and n <= 16384 else 0
    out = run3(backend, product_archive(m, k, n, kind, act, w, res), [x.tobytes()], expect)
    if kind == "store":
        want = 2 * widen(x).reshape(m, k).astype(np.float64) @ widen(w).reshape(k, n).astype(np.float64)
        got = widen(np.frombuffer(out[0], np.uint16)).reshape(m, n)
        err = np.abs(got - want) / (np.abs(want) + 1.0)
        assert err.max() <= 2 ** -7, err.max()       # bf16 truncation of an fp32 sum


def swiglu_archive(m, k, f, norm):
    """h = silu(x' Wg) * (x' Wu); x' = RmsNorm(2x) when `norm` (gamma a constant), else 2x."""
    rng = np.random.default_rng(m + k + f)
    wg, wu = (bf16(rng.standard_normal(k * f) / np.sqrt(k)) for _ in range(2))
    gam = bf16(1 + 0.25 * rng.standard_normal(k))
    # A = 2x, or RmsNorm(2x) (session memory; the norm has no producer group)
    calls = [KernelCall.Add(BinaryCall(r(0, m * k), r(0, m * k), r(7, m * k), m * k, 16, BF))]
    a = 7
    if norm:
        calls.append(KernelCall.RmsNorm(NormCall(r(7, m * k), r(9, k), r(8, m * k), m, k, dtype=BF)))
        a = 8
    calls += [KernelCall.MatMulActivation(MatMulActivationCall(
                  MatMulCall(r(a, m * k), r(1, k * f), r(3, m * f), m, k, f, BF), FA.SILU)),
              KernelCall.MatMul(MatMulCall(r(a, m * k), r(2, k * f), r(4, m * f), m, k, f, BF)),
              KernelCall.Mul(BinaryCall(r(3, m * f), r(4, m * f), r(5, m * f), m * f, 16, BF))]
    wr = HoloWriter()
    wr.kernel_calls = calls
    wr.constants = [ConstantEntry(1, BF, wg.tobytes()), ConstantEntry(2, BF, wu.tobytes()),
                    ConstantEntry(9, BF, gam.tobytes())]
    wr.inputs = [PortDescriptor("x", 0, m * k, BF, [m, k])]
    wr.outputs = [PortDescriptor("h", 5, m * f, BF, [m, f])]
    return wr.finish()


@pytest.mark.parametrize("m,k,f", [(8, 2048, 1024), (1, 256, 48), (16, 4096, 256), (8, 256, 8192)])
def test_packed_swiglu_pair(torch_cuda, backend, m, k, f):
    """Gate and up as tile pairs of one workgroup (one pair, or two at f =
    8192), SiLU(gate) * up in its epilogue."""
    x = bf16(np.random.default_rng(m).standard_normal(m * k))
    run3(backend, swiglu_archive(m, k, f, False), [x.tobytes()], 1)


CFGS = [DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1024,
                      batch=8, bucket=64),
        # head_dim 128 at K = 256: q/k/v stays split-K (eight tiles a head), so
        # layer 0's Wd keeps writing layer 1's input-norm statistics; vocab
        # 1000 runs in 8-column tiles
        DecoderConfig(layers=2, hidden=256, heads=2, kv_heads=1, head_dim=128, ffn=512, vocab=1000,
                      batch=3, bucket=64),
        DecoderConfig(layers=1, hidden=512, heads=16, kv_heads=4, head_dim=32, ffn=1024, vocab=512,
                      batch=16, bucket=32),
        DecoderConfig(layers=1, hidden=128, heads=8, kv_heads=8, head_dim=16, ffn=256, vocab=256,
                      batch=1, bucket=16)]


def decode_steps(backend, cfg, archive, flags, steps):
    sess = HipSession(backend, archive, flags=flags)
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    for layer in range(cfg.layers):
        for j, z in enumerate([bytes(P * S * Dh), bytes(P * S * 4)] * 2):
            sess.write_input(7 + 4 * layer + j, z)
    tokens = np.arange(cfg.batch) * 7 + 3
    rec = []
    for step in range(steps):
        cq, sq = rope_tables(cfg, np.array([step]), cfg.heads)
        ck, sk = rope_tables(cfg, np.array([step]), cfg.kv_heads)
        for i, b in enumerate([np.asarray(tokens, np.int32).tobytes(), np.uint32(step).tobytes(),
                               np.full(cfg.batch, step + 1, np.uint32).tobytes(), cq, sq, ck, sk]):
            sess.write_input(i, b)
        sess.run()
        sess.synchronize()
        rec.append([sess.read_output(o) for o in range(len(sess.outputs))])
        tokens = np.frombuffer(rec[-1][0], np.int32)[:cfg.batch]
    packed = sess.packed[0]
    sess.close()
    return rec, packed


@pytest.mark.parametrize("ci", range(len(CFGS)))
def test_packed_decode_steps_bit_identical(torch_cuda, backend, ci):
    """A decode step (fused norms, q/k/v with RoPE and int8 appends per head,
    attention, Wo + residual, SwiGLU, Wd + residual, LM head) walked packed,
    split-K and unfused: every output of every step (tokens, logits, caches,
    scales) equal."""
    cfg = CFGS[ci]
    archive = build_decode_step(cfg, init_weights(cfg, seed=40 + ci))
    packed, n_packed = decode_steps(backend, cfg, archive, 0, 4)
    assert n_packed >= 2 * cfg.layers + 1
    for flags in (NO_WEIGHT_PACKING, NO_DEVICE_FUSION):
        other, n = decode_steps(backend, cfg, archive, flags, 4)
        assert n == 0
        for step, (x, y) in enumerate(zip(packed, other)):
            for o, (u, v) in enumerate(zip(x, y)):
                assert u == v, f"config {ci}, flags {flags}: step {step}, output {o} differs"


def test_packed_group_graph_replays(torch_cuda, backend):
    """A captured walk of packed groups replays to the eager walk's bits, with
    new inputs between replays."""
    m, k, f = 8, 1024, 512
    arch = swiglu_archive(m, k, f, True)
    rng = np.random.default_rng(5)
    xs = [bf16(rng.standard_normal(m * k)).tobytes() for _ in range(3)]
    eager = HipSession(backend, arch)
    assert eager.packed[0] == 1
    want = [eager.execute([x])[0] for x in xs]
    eager.close()
    s = HipSession(backend, arch)
    s.write_input(0, xs[0])
    s.capture()
    s.synchronize()
    assert s.read_output(0) == want[0]
    for x, w in zip(xs[1:] + xs[:1], want[1:] + want[:1]):
        s.write_input(0, x)
        s.replay()
        s.synchronize()
        assert s.read_output(0) == w
    s.close()


def norm_archive(m, k, n, gamma):
    """z = RmsNorm(2x) * W, gamma a constant or absent, W a constant."""
    rng = np.random.default_rng(m + k + n)
    w = bf16(rng.standard_normal(k * n) / np.sqrt(k))
    gam = bf16(1 + 0.25 * rng.standard_normal(k))
    wr = HoloWriter()
    wr.kernel_calls = [
        KernelCall.Add(BinaryCall(r(0, m * k), r(0, m * k), r(7, m * k), m * k, 16, BF)),
        KernelCall.RmsNorm(NormCall(r(7, m * k), r(9, k) if gamma else BufferRef(0xFFFFFFFF),
                                    r(8, m * k), m, k, dtype=BF)),
        KernelCall.MatMul(MatMulCall(r(8, m * k), r(1, k * n), r(2, m * n), m, k, n, BF))]
    wr.constants = [ConstantEntry(1, BF, w.tobytes())]
    if gamma:
        wr.constants.append(ConstantEntry(9, BF, gam.tobytes()))
    wr.inputs = [PortDescriptor("x", 0, m * k, BF, [m, k])]
    wr.outputs = [PortDescriptor("z", 2, m * n, BF, [m, n])]
    return wr.finish()


@pytest.mark.parametrize("m,k,n,gamma,folds", [
    (8, 2048, 512, True, True), (3, 1056, 64, True, True), (8, 4064, 64, True, True),
    (16, 2016, 128, False, True), (1, 32, 16, False, True),
    # K = 8192: split-K, the norm stays on its own
    (16, 8192, 64, True, False)])
def test_packed_norm_statistics_in_launch(torch_cuda, backend, m, k, n, gamma, folds):
    """A fused RmsNorm with no producer group of its own: the packed reader
    takes the row statistics itself from its LDS copy of A (one or two
    vectors a thread, partly filled waves, gamma or the identity); bits equal
    the standalone RmsNorm's walk."""
    x = bf16(np.random.default_rng(k).standard_normal(m * k))
    arch = norm_archive(m, k, n, gamma)
    run3(backend, arch, [x.tobytes()], 1 if k <= 4096 else 0)
    packed = HipSession(None, arch)
    split = HipSession(None, arch, flags=NO_WEIGHT_PACKING)
    assert packed.n_nodes == split.n_nodes - (1 if folds else 0)


def rope_archive(m, k, heads, hd, with_add):
    """q = 2x * Wq (+ R), then RoPE(q) over heads of hd (cos/sin inputs): a
    rotary-only head-wise group, run in rope tiles."""
    from hologram_amd import RoPECall
    n = heads * hd
    rng = np.random.default_rng(heads * hd + k)
    wq = bf16(rng.standard_normal(k * n) / np.sqrt(k))
    res = bf16(rng.standard_normal(m * n))
    mm = MatMulCall(r(7, m * k), r(1, k * n), r(3, m * n), m, k, n, BF)
    prod = KernelCall.MatMulAdd(MatMulAddCall(mm, r(2, m * n))) if with_add else KernelCall.MatMul(mm)
    wr = HoloWriter()
    wr.kernel_calls = [KernelCall.Add(BinaryCall(r(0, m * k), r(0, m * k), r(7, m * k), m * k, 16, BF)), prod,
                       KernelCall.RotaryEmbedding(RoPECall(r(3, m * n), r(4, m * n), r(5, m * n), r(6, m * n),
                                                          hd, m * n, BF))]
    wr.constants = [ConstantEntry(1, BF, wq.tobytes()), ConstantEntry(2, BF, res.tobytes())]
    wr.inputs = [PortDescriptor("x", 0, m * k, BF, [m, k]), PortDescriptor("cos", 4, m * n, BF, [m, n]),
                 PortDescriptor("sin", 5, m * n, BF, [m, n])]
    wr.outputs = [PortDescriptor("q", 6, m * n, BF, [m, n])]
    return wr.finish()


@pytest.mark.parametrize("m,k,heads,hd,with_add", [(8, 2048, 32, 64, False), (3, 256, 4, 128, True),
                                                   (16, 512, 8, 16, False), (1, 96, 2, 32, True)])
def test_packed_rope_tiles(torch_cuda, backend, m, k, heads, hd, with_add):
    """A rotary-only head-wise product runs in rope tiles: its weights packed
    so each 16-column tile holds 8 rotate-half pairs, the pair meeting in
    lanes q and q ^ 8; the rotated values equal the standalone RoPE's."""
    from hologram_amd.decoder_graph import DecoderConfig
    n = heads * hd
    rng = np.random.default_rng(m + hd)
    x = bf16(rng.standard_normal(m * k))
    ang = rng.uniform(-3, 3, m * n).astype(np.float32)
    cos, sin = bf16(np.cos(ang)), bf16(np.sin(ang))
    arch = rope_archive(m, k, heads, hd, with_add)
    assert HipSession(None, arch).n_nodes == 2       # the 2x, then one group
    run3(backend, arch, [x.tobytes(), cos.tobytes(), sin.tobytes()], 1)
