"""The tiled SwiGLU pair (the prompt pass's gate/up at large M) looks gate's
activation up in its 65536-entry table, staged in LDS once the main loop is
done. Every finite bf16 pattern goes through it here: A is a 0/1 row selector
(row i holds its one 1 at column i mod 256), so gate's product row i is
exactly B_gate's row i mod 256, and B_gate holds every finite pattern (twice);
B_up is all ones, so up is exactly 1. The fused output must equal the walk
without device fusion (the MatMuls, the activation, the Mul) bit for bit, and,
for the unary ops' tables, the table entry of every normal pattern. All eight
fused activations are covered (Relu, Elu and Selu through the fused
epilogues' own tables)."""
import numpy as np
import pytest

import oracle
from hologram_amd import (DTYPE_BF16, BinaryCall, BufferRef, ConstantEntry, HipSession,
                          HoloWriter, KernelCall, MatMulCall, PortDescriptor, UnaryCall, lut_act)
from hologram_amd.session import NO_DEVICE_FUSION

pytestmark = pytest.mark.gpu

M, K, N = 4096, 256, 512          # 16 x 4 tiles of 256 x 128: the tiled pair applies


def pair_archive(act_call):
    sel = np.zeros((M, K), np.float32)
    sel[np.arange(M), np.arange(M) % K] = 1.0
    pat = np.arange(65536, dtype=np.uint32)
    finite = ((pat >> 7) & 0xFF) != 0xFF
    bg = np.where(finite, pat, 0).astype(np.uint16).reshape(K, 256)
    bg = np.concatenate([bg, bg], axis=1)                   # [K, N]: every finite pattern, twice
    bu = np.full(K * N, 0x3F80, np.uint16)                   # 1.0
    a = (sel.view(np.uint32) >> 16).astype(np.uint16)
    bf = 2
    w = HoloWriter()
    # every operand a constant (an input port could be rebound to memory of
    # any alignment, so the session groups no product over one)
    w.constants = [ConstantEntry(0, DTYPE_BF16, a.tobytes()), ConstantEntry(1, DTYPE_BF16, bg.tobytes()),
                   ConstantEntry(2, DTYPE_BF16, bu.tobytes())]
    w.outputs = [PortDescriptor("y", 6, M * N, DTYPE_BF16, [M, N])]
    mn = M * N * bf
    w.kernel_calls = [
        KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(3, 0, mn), M, K, N, DTYPE_BF16)),
        KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(2), BufferRef(4, 0, mn), M, K, N, DTYPE_BF16)),
        act_call(UnaryCall(BufferRef(3, 0, mn), BufferRef(5, 0, mn), M * N, 16, DTYPE_BF16)),
        KernelCall.Mul(BinaryCall(BufferRef(5, 0, mn), BufferRef(4, 0, mn), BufferRef(6, 0, mn),
                                  M * N, 16, DTYPE_BF16)),
    ]
    w.exec_plan = [[i] for i in range(len(w.kernel_calls))]
    return w.finish(), bg, finite


ACTS = [("silu", KernelCall.Silu, lut_act.SILU), ("gelu", KernelCall.Gelu, lut_act.GELU),
        ("exp", KernelCall.Exp, lut_act.EXP), ("sigmoid", KernelCall.Sigmoid, lut_act.SIGMOID),
        ("tanh", KernelCall.Tanh, lut_act.TANH),
        # the fused epilogues' own tables (the loader fuses these unary ops
        # into the MatMul as MatMulActivation)
        ("relu", KernelCall.Relu, None), ("elu", KernelCall.Elu, None),
        ("selu", KernelCall.Selu, None)]


@pytest.mark.parametrize("name,call,act", ACTS, ids=[a[0] for a in ACTS])
def test_pair_table_every_finite_pattern(torch_cuda, backend, name, call, act):
    print(f"pair table {name}", flush=True)
    archive, bg, finite = pair_archive(call)
    outs, groups = {}, {}
    for flags in (0, NO_DEVICE_FUSION):
        sess = HipSession(backend, archive, flags=flags)
        sess.run()
        sess.synchronize()
        outs[flags] = np.frombuffer(sess.read_output(0), np.uint16).copy()
        groups[flags] = sess.n_groups
        sess.close()
    assert groups[0] == 1, "gate/up did not run as one group"
    fused, plain = outs[0], outs[NO_DEVICE_FUSION]
    bad = np.flatnonzero(fused != plain)
    assert bad.size == 0, f"{name}: {bad.size} of {fused.size} differ from the unfused walk, first at {bad[:4]}"
    if act is None:
        return
    # rows 0..255 hold each pattern once: the table entry times 1.0 (normal
    # patterns: a zero's sign and a subnormal depend on how the product sums
    # its zero terms, which both walks share)
    table = oracle.build_table(act, DTYPE_BF16).astype(np.uint16)
    got = fused.reshape(M, N)[:K, :256].ravel()
    want = table[bg[:, :256].ravel()]
    normal = finite & (((np.arange(65536) >> 7) & 0xFF) != 0)
    keep = normal & ~np.isnan((want.astype(np.uint32) << 16).view(np.float32))
    mism = np.flatnonzero((got != want) & keep)
    assert mism.size == 0, f"{name}: {mism.size} patterns differ from the table, first {mism[:4]}"
