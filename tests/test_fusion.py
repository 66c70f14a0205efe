"""CPU tests of the load-time fusions, with no device.

The reference loader's epilogue fusion (fuse_matmul_epilogue,
crates/hologram-exec/src/session.rs:2150-2373) is restated in the session.
Its conditions are checked through the call count of dry loads:
- one producer and one reader of the product;
- the product is not an output port;
- the residual is ready no later than the MatMul's level;
- the three-op chain is f32 only.
This backend's device fusion (grouped few-row MatMuls and their epilogues) is
checked through the walk's node and group counts. Also covered: the fused
MatMul calls' wire codec (kernel_codec.rs:509-524) and their refusals.
"""
import pytest

from hologram_amd import (DTYPE_BF16, DTYPE_F32, BinaryCall, BufferRef, HipSession, HoloWriter,
                          KernelCall, MatMulActivationCall, MatMulAddActivationCall,
                          MatMulAddCall, MatMulCall, NormCall, PortDescriptor, SlotOutOfRange, UnaryCall,
                          UnsupportedOp, decode_call, fused_activation, validate)
from hologram_amd.decoder_graph import DecoderConfig, build_decode_step, init_weights
from hologram_amd.session import (NO_ATTN_PROLOGUE, NO_DEVICE_FUSION, NO_EPILOGUE_FUSION, NO_NORM_FUSION,
                                  NO_WEIGHT_PACKING)

M, K, N = 4, 64, 32


def ref(slot, elems, es):
    return BufferRef(slot, 0, elems * es)


def archive(calls, inputs, outputs, plan=None):
    """inputs / outputs: (slot, elements, dtype); calls: KernelCalls."""
    w = HoloWriter()
    w.kernel_calls = list(calls)
    for s, n, dt in inputs:
        w.inputs.append(PortDescriptor(f"in{s}", s, n, dt, [n]))
    for s, n, dt in outputs:
        w.outputs.append(PortDescriptor(f"out{s}", s, n, dt, [n]))
    if plan:
        w.exec_plan = plan
    return w.finish()


def mm(a, b, o, dt, m=M, k=K, n=N):
    es = 2 if dt == DTYPE_BF16 else 4
    return KernelCall.MatMul(MatMulCall(ref(a, m * k, es), ref(b, k * n, es), ref(o, m * n, es),
                                        m, k, n, dt))


def unary(ctor, x, o, dt, n=M * N):
    es = 2 if dt == DTYPE_BF16 else 4
    return ctor(UnaryCall(ref(x, n, es), ref(o, n, es), n, 16, dt))


def add(a, b, o, dt, n=M * N):
    es = 2 if dt == DTYPE_BF16 else 4
    return KernelCall.Add(BinaryCall(ref(a, n, es), ref(b, n, es), ref(o, n, es), n, 16, dt))


def ins(dt, extra=()):
    return [(0, M * K, dt), (1, K * N, dt)] + [(s, M * N, dt) for s in extra]


def n_calls(a, flags=0):
    return HipSession(None, a, flags=flags).n_calls


def test_matmul_activation_fuses():
    a = archive([mm(0, 1, 2, DTYPE_BF16), unary(KernelCall.Silu, 2, 3, DTYPE_BF16)],
                ins(DTYPE_BF16), [(3, M * N, DTYPE_BF16)])
    assert n_calls(a) == 1
    assert n_calls(a, NO_EPILOGUE_FUSION) == 2


def test_second_reader_blocks_fusion():
    a = archive([mm(0, 1, 2, DTYPE_BF16), unary(KernelCall.Silu, 2, 3, DTYPE_BF16),
                 add(2, 3, 4, DTYPE_BF16)],
                ins(DTYPE_BF16), [(4, M * N, DTYPE_BF16)])
    assert n_calls(a) == 3


def test_output_port_product_is_not_fused():
    a = archive([mm(0, 1, 2, DTYPE_BF16), unary(KernelCall.Gelu, 2, 3, DTYPE_BF16)],
                ins(DTYPE_BF16), [(2, M * N, DTYPE_BF16), (3, M * N, DTYPE_BF16)])
    assert n_calls(a) == 2


def test_residual_readiness():
    # residual is a graph input: ready, fused
    a = archive([mm(0, 1, 2, DTYPE_F32), add(2, 5, 6, DTYPE_F32)], ins(DTYPE_F32, [5]),
                [(6, M * N, DTYPE_F32)])
    assert n_calls(a) == 1
    # residual produced at the MatMul's own level or later: not fused
    calls = [mm(0, 1, 2, DTYPE_F32), unary(KernelCall.Gelu, 7, 5, DTYPE_BF16),
             add(2, 5, 6, DTYPE_F32)]
    inputs = ins(DTYPE_F32) + [(7, M * N, DTYPE_BF16)]
    for plan in ([[0, 1], [2]], [[0], [1], [2]]):
        a = archive(calls, inputs, [(6, M * N, DTYPE_F32)], plan)
        assert n_calls(a) == 3, plan
    # produced at an earlier level: fused
    a = archive(calls, inputs, [(6, M * N, DTYPE_F32)], [[1], [0], [2]])
    assert n_calls(a) == 2


def test_three_op_chain_is_f32_only():
    for dt, want in ((DTYPE_F32, 1), (DTYPE_BF16, 2)):
        a = archive([mm(0, 1, 2, dt), add(2, 5, 6, dt), unary(KernelCall.Gelu, 6, 7, dt)],
                    ins(dt, [5]), [(7, M * N, dt)])
        assert n_calls(a) == want, dt


@pytest.mark.parametrize("dt", [DTYPE_F32, DTYPE_BF16])
def test_every_activation_is_fused(dt):
    """Every fused_activation the reference loader absorbs (kernel_call.rs:
    861-870) has a device form, so matmul -> activation is always one call:
    the table of narrow(f(widen(x))) for 16-bit products, f computed in f32
    otherwise (f32 Exp through libm's expf restated, Relu/Elu/Selu too)."""
    for ctor in (KernelCall.Exp, KernelCall.Gelu, KernelCall.Silu):
        a = archive([mm(0, 1, 2, dt), unary(ctor, 2, 3, dt)], ins(dt), [(3, M * N, dt)])
        assert n_calls(a) == 1, (ctor, dt)


def decoder(layers=2):
    cfg = DecoderConfig(layers=layers, hidden=128, heads=4, kv_heads=2, head_dim=64, ffn=256,
                        vocab=304, batch=2, bucket=64)
    return cfg, build_decode_step(cfg, init_weights(cfg, seed=3))


def test_decoder_walk_counts():
    cfg, a = decoder()
    L = cfg.layers
    plain = HipSession(None, a, flags=NO_EPILOGUE_FUSION | NO_DEVICE_FUSION)
    assert plain.n_calls == plain.n_nodes == 1 + 18 * L + 3 and plain.n_groups == 0
    ref = HipSession(None, a, flags=NO_DEVICE_FUSION)
    assert ref.n_calls == ref.n_nodes == 1 + 15 * L + 3      # Silu, two Adds absorbed
    full = HipSession(None, a)
    # per layer: RmsNorm, {q,k,v + 2 RoPE + 2 appends}, attention, Wo+Add, RmsNorm,
    # {gate+Silu, up, Mul}, Wd+Add
    assert full.n_calls == 1 + 15 * L + 3
    grouped = HipSession(None, a, flags=NO_NORM_FUSION | NO_WEIGHT_PACKING)
    assert grouped.n_nodes == 1 + 7 * L + 3 and grouped.n_groups == 2 * L
    # with packing, the plain few-row MatMuls over constant weights (Wo+Add,
    # Wd+Add, the LM head) run as groups of one; every group but q/k/v (the
    # int8 appends need whole heads) runs packed
    packed = HipSession(None, a, flags=NO_NORM_FUSION)
    assert packed.n_nodes == 1 + 7 * L + 3 and packed.n_groups == 4 * L + 1
    assert packed.packed[0] == 3 * L + 1
    # the norms after Wo+Add and Wd+Add (the next layer's, or the final one)
    # split between producer and reader: Wo+Add, Wd+Add and the LM head become
    # groups of one; layer 0's input norm (after the embedding) stays on its
    # own when the weights are not packed
    split = HipSession(None, a, flags=NO_WEIGHT_PACKING)
    assert split.n_nodes == 1 + 5 * L + 3 and split.n_groups == 4 * L + 1
    assert split.packed[0] == 0
    # packed: Wo and gate/up per layer, the last Wd and the LM head; the
    # other Wd + Add steps write the statistics a split-K q/k/v group reads
    assert full.n_nodes == 1 + 5 * L + 3 and full.n_groups == 4 * L + 1
    assert full.packed[0] == 2 * L + 2
    # each layer's q/k/v group leaves its split-K epilogue (RoPE, int8 appends)
    # to the decode attention after it; the node count does not change
    assert full.attn_prologues == L and split.attn_prologues == L
    off = HipSession(None, a, flags=NO_ATTN_PROLOGUE)
    assert off.attn_prologues == 0 and off.n_nodes == full.n_nodes
    assert ref.attn_prologues == 0 and plain.attn_prologues == 0


def norm(x, g, o, rows, feat, dt=DTYPE_BF16):
    es = 2 if dt == DTYPE_BF16 else 4
    return KernelCall.RmsNorm(NormCall(ref(x, rows * feat, es), ref(g, feat, es),
                                       ref(o, rows * feat, es), rows, feat, dtype=dt))


def norm_chain(dt=DTYPE_BF16, out_y=False, extra_reader=False, feat=K, clobber=False):
    """X = A*B (slot 2); Y = RmsNorm(X) (slot 4, gamma slot 5); Z = Y*W (slot 6).
    A, B, W and gamma are computed in-graph (sums of inputs), so no operand of
    the MatMuls or the norm is caller-bound."""
    calls = [add(10, 10, 0, dt, M * K), add(11, 11, 1, dt, K * feat),
             add(12, 12, 3, dt, feat * N), add(13, 13, 5, dt, feat),
             mm(0, 1, 2, dt, n=feat), norm(2, 5, 4, M, feat, dt)]
    if clobber:
        calls.append(add(10, 10, 2, dt, M * feat))
    calls.append(mm(4, 3, 6, dt, k=feat))
    outs = [(6, M * N, dt)]
    if extra_reader:
        calls.append(add(4, 4, 7, dt, M * feat))
        outs.append((7, M * feat, dt))
    if out_y:
        outs.append((4, M * feat, dt))
    inputs = [(10, M * K, dt), (11, K * feat, dt), (12, feat * N, dt), (13, feat, dt)]
    return archive(calls, inputs, outs)


def test_norm_between_few_row_matmuls_is_split():
    s = HipSession(None, norm_chain())
    assert s.n_calls == 7 and s.n_nodes == 6 and s.n_groups == 2
    assert HipSession(None, norm_chain(), flags=NO_NORM_FUSION).n_nodes == 7


@pytest.mark.parametrize("kw", [dict(dt=DTYPE_F32), dict(out_y=True), dict(extra_reader=True),
                                dict(feat=K + 4), dict(clobber=True)])
def test_norm_fusion_conditions(kw):
    # f32; the norm's output a graph output or read twice; a feature that is
    # not a multiple of 8; the input overwritten before the reader: standalone
    s = HipSession(None, norm_chain(**kw))
    assert s.n_nodes == s.n_calls, kw


def test_members_that_depend_on_each_other_are_not_grouped():
    dt = DTYPE_BF16
    # X = A*B1; Z = A*X: the second product reads the first's output
    a = archive([mm(0, 1, 2, dt, m=M, k=K, n=K), mm(0, 2, 3, dt, m=M, k=K, n=N)],
                [(0, M * K, dt), (1, K * K, dt)], [(3, M * N, dt)])
    s = HipSession(None, a)
    assert s.n_groups == 0 and s.n_nodes == 2


@pytest.mark.parametrize("call", [
    KernelCall.MatMulActivation(MatMulActivationCall(
        MatMulCall(BufferRef(1, 16, 64), BufferRef(2), BufferRef(3), 4, 8, 16, DTYPE_BF16),
        fused_activation.SILU)),
    KernelCall.MatMulAdd(MatMulAddCall(
        MatMulCall(BufferRef(1), BufferRef(2, 32), BufferRef(3), 4, 8, 16, DTYPE_F32),
        BufferRef(5, 8, 256))),
    KernelCall.MatMulAddActivation(MatMulAddActivationCall(
        MatMulCall(BufferRef(1), BufferRef(2), BufferRef(3), 2, 3, 4, DTYPE_F32),
        BufferRef(6), fused_activation.GELU)),
])
def test_fused_codec_round_trip(call):
    wire = call.encode()
    kc, used = decode_call(wire + b"\x01\x02")
    assert used == len(wire) and kc.tag == call.tag in (106, 107, 108)
    assert bytes(kc) == bytes(call.to_c())


def test_fused_refusals():
    sizes = [1 << 16] * 8
    base = MatMulCall(BufferRef(1), BufferRef(2), BufferRef(3), 8, 64, 64, DTYPE_BF16)
    f32 = MatMulCall(BufferRef(1), BufferRef(2), BufferRef(3), 8, 64, 64, DTYPE_F32)
    for act in range(1, 9):                  # every fused_activation has a device form
        validate(KernelCall.MatMulActivation(MatMulActivationCall(base, act)), sizes)
        validate(KernelCall.MatMulActivation(MatMulActivationCall(f32, act)), sizes)
        validate(KernelCall.MatMulAddActivation(MatMulAddActivationCall(base, BufferRef(4), act)),
                 sizes)
    with pytest.raises(UnsupportedOp):       # no such activation id
        validate(KernelCall.MatMulActivation(MatMulActivationCall(f32, 9)), sizes)
    with pytest.raises(SlotOutOfRange):      # residual overlaps the output (split_borrow)
        validate(KernelCall.MatMulAdd(MatMulAddCall(base, BufferRef(3))), sizes)
    with pytest.raises(SlotOutOfRange):      # short residual
        validate(KernelCall.MatMulAdd(MatMulAddCall(base, BufferRef(4, 0, 64))), sizes)
    validate(KernelCall.MatMulAdd(MatMulAddCall(base, BufferRef(4))), sizes)
    validate(KernelCall.MatMulActivation(MatMulActivationCall(base, fused_activation.EXP)), sizes)
