"""GPU parity: int8 KV quantize+append (new op 122) and KvCacheWrite (120) vs the
oracle (quantize_row_i8, src/cpu/simd.rs:4755-4785; kv_cache_write,
src/cpu/kernels.rs:455-501). Bit-exact int8 bytes and f32 scale bits."""
import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BufferRef, DeviceWorkspace,
                          KernelCall, KvCacheWriteCall, KvQuantAppendCall, UnsupportedOp)

pytestmark = pytest.mark.gpu


def kv_rows(rng, planes, new_rows, d, dtype, outlier_frac=0.02):
    """N(0,1) rows with a fixed set of outlier channels scaled x20 (config 3)."""
    x = rng.standard_normal((planes, new_rows, d)).astype(np.float32)
    nout = max(1, int(np.ceil(outlier_frac * d)))
    ch = rng.choice(d, size=nout, replace=False)
    x[..., ch] *= 20.0
    if dtype == DTYPE_BF16:
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    if dtype == DTYPE_F16:
        return x.astype(np.float16).view(np.uint16)
    return x


def run_append(torch, backend, new, dtype, pos, cq, cs, planes, bucket, new_rows, d, in_place):
    ws = DeviceWorkspace()
    t_new, t_pos = to_dev(torch, new), to_dev(torch, np.array([pos], np.uint32))
    t_cq, t_cs = to_dev(torch, cq), to_dev(torch, cs)
    ws.bind(0, t_new)
    ws.bind(1, t_pos)
    ws.bind(2, t_cq)
    ws.bind(3, t_cs)
    if in_place:
        out_q, out_s = BufferRef(2), BufferRef(3)
    else:
        t_oq = torch.full((cq.size,), 0x55, dtype=torch.uint8, device="cuda")
        t_os = torch.full((cs.size * 4,), 0x55, dtype=torch.uint8, device="cuda")
        ws.bind(4, t_oq)
        ws.bind(5, t_os)
        out_q, out_s = BufferRef(4), BufferRef(5)
    call = KernelCall.KvQuantAppend(KvQuantAppendCall(
        BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), out_q, out_s, planes, bucket,
        new_rows, d, dtype))
    backend.dispatch(call, ws)
    backend.synchronize()
    if in_place:
        return from_dev(t_cq, np.int8), from_dev(t_cs, np.float32)
    return from_dev(t_oq, np.int8), from_dev(t_os, np.float32)


@pytest.mark.parametrize("pos", [4095, 4096, 7, 2**32 - 1])
@pytest.mark.parametrize("in_place", [False, True])
def test_config3_shape(torch_cuda, backend, pos, in_place):
    planes, bucket, d, new_rows = 16 * 8, 4096, 128, 1
    rng = np.random.default_rng(pos & 0xFFFF)
    cq = rng.integers(-127, 128, size=planes * bucket * d, dtype=np.int8)
    cs = rng.random(planes * bucket, dtype=np.float32)
    new = kv_rows(rng, planes, new_rows, d, DTYPE_BF16)
    gq, gs = run_append(torch_cuda, backend, new, DTYPE_BF16, pos, cq, cs, planes, bucket,
                        new_rows, d, in_place)
    wq, ws_ = oracle.kv_quant_append(new, DTYPE_BF16, pos, cq, cs, planes, bucket, new_rows, d)
    assert np.array_equal(gq, wq)
    assert np.array_equal(gs.view(np.uint32), ws_.view(np.uint32))


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("d", [64, 128, 96, 300])
@pytest.mark.parametrize("bucket", [10, 12])
def test_dtypes_dims_and_wrap(torch_cuda, backend, dtype, d, bucket):
    """Rows bucket-2, bucket-1, 0, 1: the append wraps the ring. A bucket of 12
    with d a multiple of 16 takes the one-launch copy form (copy everything but
    the appended rows, whose 16-byte scale vectors are shared with copied
    rows); a bucket of 10 or d = 300 the copy-then-append launches."""
    planes, new_rows, pos = 6, 4, bucket - 2
    rng = np.random.default_rng(d + dtype + bucket)
    cq = rng.integers(-127, 128, size=planes * bucket * d, dtype=np.int8)
    cs = rng.random(planes * bucket, dtype=np.float32)
    new = kv_rows(rng, planes, new_rows, d, dtype)
    gq, gs = run_append(torch_cuda, backend, new, dtype, pos, cq, cs, planes, bucket, new_rows,
                        d, False)
    wq, ws_ = oracle.kv_quant_append(new, dtype, pos, cq, cs, planes, bucket, new_rows, d)
    assert np.array_equal(gq, wq)
    assert np.array_equal(gs.view(np.uint32), ws_.view(np.uint32))


@pytest.mark.parametrize("dtype,d", [(DTYPE_F32, 128), (DTYPE_BF16, 128), (DTYPE_BF16, 64),
                                     (DTYPE_F16, 64)])
def test_special_rows(torch_cuda, backend, dtype, d):
    """all-zero row -> q 0, scale 0; NaN ignored by the max and quantized to 0;
    an Inf row gives scale Inf; subnormal-only rows; half-way ties. The 16-bit
    cases (rows narrowed from the same f32 values) take the eight-a-lane kernel."""
    planes, bucket = 8, 4
    rows = np.zeros((planes, d), np.float32)
    rows[1, :] = np.float32(1e-40)                       # subnormal
    rows[2, :5] = [np.nan, 1.0, -2.0, 0.5, -0.0]
    rows[3, 0] = np.inf
    rows[3, 1] = 3.0
    rows[4, :] = np.linspace(-127.5, 127.5, d, dtype=np.float32)  # exact .5 ties
    rows[5, :] = -0.0
    rows[6, 0] = -np.inf
    rows[7, :] = np.float32(3.4e38)
    if dtype == DTYPE_BF16:
        rows = (rows.view(np.uint32) >> 16).astype(np.uint16)
    elif dtype == DTYPE_F16:
        with np.errstate(over="ignore"):
            rows = rows.astype(np.float16).view(np.uint16)
    cq = np.full(planes * bucket * d, 9, np.int8)
    cs = np.full(planes * bucket, 2.0, np.float32)
    gq, gs = run_append(torch_cuda, backend, rows, dtype, 2, cq, cs, planes, bucket, 1, d,
                        False)
    wq, ws_ = oracle.kv_quant_append(rows, dtype, 2, cq, cs, planes, bucket, 1, d)
    assert np.array_equal(gq, wq)
    assert np.array_equal(gs.view(np.uint32), ws_.view(np.uint32))


@pytest.mark.parametrize("new_rows,pos", [(0, 3), (16, 5), (16, 0), (7, 13)])
def test_copy_form_all_or_no_rows_appended(torch_cuda, backend, new_rows, pos):
    """The one-launch copy form at its edges: no new row (a pure copy of both
    planes), every row of the bucket replaced (nothing copied), and a wrapping
    run that ends on a 16-byte scale vector boundary."""
    planes, bucket, d = 33, 16, 128
    rng = np.random.default_rng(new_rows * 100 + pos)
    cq = rng.integers(-127, 128, size=planes * bucket * d, dtype=np.int8)
    cs = rng.random(planes * bucket, dtype=np.float32)
    new = kv_rows(rng, planes, new_rows, d, DTYPE_BF16) if new_rows else np.zeros(8, np.uint16)
    gq, gs = run_append(torch_cuda, backend, new, DTYPE_BF16, pos, cq, cs, planes, bucket,
                        new_rows, d, False)
    wq, ws_ = oracle.kv_quant_append(new, DTYPE_BF16, pos, cq, cs, planes, bucket, new_rows, d)
    assert np.array_equal(gq, wq)
    assert np.array_equal(gs.view(np.uint32), ws_.view(np.uint32))


@pytest.mark.parametrize("pos,new_rows", [(0, 1), (4094, 3), (5, 0)])
def test_kv_cache_write_bytes(torch_cuda, backend, pos, new_rows):
    planes, bucket, row = 16, 4096 // 16, 128
    rng = np.random.default_rng(pos)
    cache = rng.integers(0, 256, size=planes * bucket * row, dtype=np.uint8)
    new = rng.integers(0, 256, size=planes * new_rows * row, dtype=np.uint8)
    ws = DeviceWorkspace()
    t_out = torch_cuda.zeros(cache.size, dtype=torch_cuda.uint8, device="cuda")
    for s, t in enumerate([to_dev(torch_cuda, cache), to_dev(torch_cuda, new),
                           to_dev(torch_cuda, np.array([pos], np.uint32)), t_out]):
        ws.bind(s, t)
    backend.dispatch(KernelCall.KvCacheWrite(KvCacheWriteCall(
        BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), planes, bucket, new_rows, row)), ws)
    backend.synchronize()
    want = oracle.kv_cache_write(cache, new, pos, planes, bucket, new_rows, row)
    assert np.array_equal(from_dev(t_out, np.uint8), want)


def test_refusals_on_device(torch_cuda, backend):
    ws = DeviceWorkspace()
    for s in range(6):
        ws.bind(s, torch_cuda.zeros(4096, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):
        backend.dispatch(KernelCall.KvQuantAppend(KvQuantAppendCall(
            BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), BufferRef(4), BufferRef(5),
            1, 2, 3, 8, DTYPE_BF16)), ws)
