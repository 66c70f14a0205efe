"""GPU parity: LUT activations (bf16/f16) through HipBackend.dispatch vs the
oracle's restatement of build_table/unary_lut (src/cpu/lut.rs:43-98). Bit-exact."""
import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev, u16_patterns
from hologram_amd import (DTYPE_BF16, DTYPE_F16, BufferRef, DeviceWorkspace, KernelCall,
                          UnaryCall, lut_act)

pytestmark = pytest.mark.gpu

ACTS = [("Gelu", lut_act.GELU), ("Silu", lut_act.SILU), ("Exp", lut_act.EXP),
        ("Sigmoid", lut_act.SIGMOID), ("Tanh", lut_act.TANH)]


def run_lut(torch, backend, name, x: np.ndarray, dtype, in_off=0, out_off=0):
    n = x.size
    src = to_dev(torch, np.concatenate([np.zeros(in_off // 2, np.uint16), x]))
    dst = torch.zeros(out_off + 2 * n + 64, dtype=torch.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, src)
    ws.bind(1, dst)
    call = getattr(KernelCall, name)(UnaryCall(BufferRef(0, in_off), BufferRef(1, out_off), n,
                                               16, dtype))
    backend.dispatch(call, ws)
    backend.synchronize()
    return from_dev(dst, np.uint8)[out_off:out_off + 2 * n].view(np.uint16)


@pytest.mark.parametrize("name,act", ACTS)
@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16])
def test_every_pattern(torch_cuda, backend, name, act, dtype):
    x = np.arange(65536, dtype=np.uint16)
    got = run_lut(torch_cuda, backend, name, x, dtype)
    want = oracle.build_table(act, dtype)
    assert np.array_equal(got, want), f"{name} dtype {dtype}: {(got != want).sum()} mismatches"


@pytest.mark.parametrize("name,act", [("Gelu", lut_act.GELU), ("Silu", lut_act.SILU),
                                      ("Exp", lut_act.EXP)])
def test_config_size_seeded(torch_cuda, backend, name, act):
    n = 16_777_216
    x = u16_patterns(n, seed=0xC1 + act)
    got = run_lut(torch_cuda, backend, name, x, DTYPE_BF16)
    want = oracle.unary_lut(oracle.build_table(act, DTYPE_BF16), x)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n,in_off,out_off", [(1, 0, 0), (7, 0, 0), (9, 0, 0), (1000003, 0, 0),
                                              (4099, 2, 0), (4099, 0, 6), (8, 16, 32)])
def test_ragged_and_unaligned(torch_cuda, backend, n, in_off, out_off):
    x = u16_patterns(n, seed=n)
    got = run_lut(torch_cuda, backend, "Gelu", x, DTYPE_BF16, in_off, out_off)
    want = oracle.unary_lut(oracle.build_table(lut_act.GELU, DTYPE_BF16), x)
    assert np.array_equal(got, want)


def test_empty_is_noop(torch_cuda, backend):
    dst = torch_cuda.full((16,), 7, dtype=torch_cuda.uint8, device="cuda")
    src = torch_cuda.zeros(16, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, src)
    ws.bind(1, dst)
    backend.dispatch(KernelCall.Gelu(UnaryCall(BufferRef(0), BufferRef(1), 0)), ws)
    backend.synchronize()
    assert (dst.cpu().numpy() == 7).all()


def test_wire_encoded_dispatch(torch_cuda, backend):
    x = u16_patterns(5000, seed=3)
    src, dst = to_dev(torch_cuda, x), torch_cuda.zeros(10000, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(4, src)
    ws.bind(9, dst)
    call = KernelCall.Silu(UnaryCall(BufferRef(4), BufferRef(9), 5000, 16, DTYPE_BF16))
    used = backend.dispatch_encoded(call.encode(), ws)
    backend.synchronize()
    assert used == len(call.encode())
    want = oracle.unary_lut(oracle.build_table(lut_act.SILU, DTYPE_BF16), x)
    assert np.array_equal(from_dev(dst, np.uint16), want)


@pytest.mark.parametrize("n,out_off", [(3_000_001, 0), (20_000_003, 0), (2_100_007, 16),
                                       (1000003, 0)])
def test_partial_spans_store_nothing_past_the_output(torch_cuda, backend, n, out_off):
    """The gather's last span is a partial one: its lanes' stores past the
    output are dropped by the buffer range (the per-unroll offset sits in the
    instruction's scalar offset). Every byte before and after the output, over
    more than one 128 KiB workgroup span, keeps its canary value; the partial
    span of the grid's second pass (20,000,003 elements) is covered too."""
    x = u16_patterns(n, seed=n + 1)
    guard = 256 << 10
    src = to_dev(torch_cuda, np.concatenate([x, np.zeros(guard // 2, np.uint16)]))
    dst = torch_cuda.full((out_off + 2 * n + guard,), 0xA5, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, src)
    ws.bind(1, dst)
    backend.dispatch(KernelCall.Gelu(UnaryCall(BufferRef(0, 0, 2 * n), BufferRef(1, out_off, 2 * n),
                                               n, 16, DTYPE_BF16)), ws)
    backend.synchronize()
    raw = from_dev(dst, np.uint8)
    assert (raw[:out_off] == 0xA5).all()
    assert (raw[out_off + 2 * n:] == 0xA5).all(), "a store landed past the output"
    want = oracle.unary_lut(oracle.build_table(lut_act.GELU, DTYPE_BF16), x)
    assert np.array_equal(raw[out_off:out_off + 2 * n].view(np.uint16), want)
