"""The allocation-free entry point, holo_hip_dispatch_noalloc: decode attention
on the fixed per-device scratch gives the bits of holo_hip_dispatch, on two
calls in a row (the second smaller, so the array keeps the first call's
contents), for the single-row (123) and multi-row (125) forms; a call needing
more scratch than the array holds is refused before any launch."""
import numpy as np
import pytest

from conftest import to_dev
from hologram_amd import (DTYPE_BF16, AttentionI8RowsCall, BufferRef, DecodeAttentionI8Call,
                          DeviceWorkspace, KernelCall, UnsupportedOp)

pytestmark = pytest.mark.gpu


def cache_setup(torch, B, Hkv, bucket, D, rng):
    planes = B * Hkv
    kq = rng.integers(-127, 128, planes * bucket * D, dtype=np.int8)
    vq = rng.integers(-127, 128, planes * bucket * D, dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, planes * bucket).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, planes * bucket).astype(np.float32)
    return [to_dev(torch, x) for x in (kq, vq, ks, vs)]


def both_forms(torch, backend, B, H, Hkv, bucket, D, lens, q_rows, seed):
    rng = np.random.default_rng(seed)
    kq, vq, ks, vs = cache_setup(torch, B, Hkv, bucket, D, rng)
    q = to_dev(torch, (rng.standard_normal(B * q_rows * H * D).astype(np.float32)
                       .view(np.uint32) >> 16).astype(np.uint16))
    lens_t = to_dev(torch, np.asarray(lens, np.uint32))
    outs = []
    for noalloc in (False, True):
        out = torch.full((B * q_rows * H * D * 2,), 0x5A, dtype=torch.uint8, device="cuda")
        ws = DeviceWorkspace()
        for s, t in enumerate([q, kq, vq, ks, vs, lens_t, out]):
            ws.bind(s, t)
        attn = DecodeAttentionI8Call(*[BufferRef(s) for s in range(7)], B, H, Hkv, bucket, D, 0,
                                     DTYPE_BF16)
        call = (KernelCall.DecodeAttentionI8(attn) if q_rows == 1
                else KernelCall.AttentionI8Rows(AttentionI8RowsCall(attn, q_rows)))
        (backend.dispatch_noalloc if noalloc else backend.dispatch)(call, ws)
        backend.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def test_noalloc_equals_dispatch_on_two_calls_second_smaller(torch_cuda, backend):
    # config 4's shape at a shorter bucket: the balanced split over every CU
    rng = np.random.default_rng(3)
    lens1 = rng.integers(512, 8193, 32)
    a, b = both_forms(torch_cuda, backend, 32, 32, 8, 8192, 128, lens1, 1, seed=4)
    assert np.array_equal(a, b)
    # a smaller call second: the array still holds the first call's partials
    a, b = both_forms(torch_cuda, backend, 3, 16, 4, 1000, 64, [1000, 17, 500], 1, seed=5)
    assert np.array_equal(a, b)


def test_noalloc_multi_row_form(torch_cuda, backend):
    a, b = both_forms(torch_cuda, backend, 2, 8, 2, 4096, 128, [4096, 300], 4, seed=6)
    assert np.array_equal(a, b)
    a, b = both_forms(torch_cuda, backend, 1, 8, 2, 256, 64, [40], 3, seed=7)
    assert np.array_equal(a, b)


def test_noalloc_refuses_beyond_its_scratch(torch_cuda, backend):
    B, H, Hkv, bucket, D, q_rows = 1, 32, 8, 2048, 128, 2048   # about 34 MB of partials
    ws = DeviceWorkspace()
    sizes = [B * q_rows * H * D * 2, B * Hkv * bucket * D, B * Hkv * bucket * D,
             B * Hkv * bucket * 4, B * Hkv * bucket * 4, 4, B * q_rows * H * D * 2]
    for s, n in enumerate(sizes):
        ws.bind(s, torch_cuda.zeros(n, dtype=torch_cuda.uint8, device="cuda"))
    call = KernelCall.AttentionI8Rows(AttentionI8RowsCall(DecodeAttentionI8Call(
        *[BufferRef(s) for s in range(7)], B, H, Hkv, bucket, D, 0, DTYPE_BF16), q_rows))
    with pytest.raises(UnsupportedOp):
        backend.dispatch_noalloc(call, ws)
    backend.synchronize()


def test_noalloc_serves_attention_only(torch_cuda, backend):
    from hologram_amd import MatMulCall
    ws = DeviceWorkspace()
    for s in range(3):
        ws.bind(s, torch_cuda.zeros(64, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):
        backend.dispatch_noalloc(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1),
                                                              BufferRef(2), 2, 2, 2, 8)), ws)
