"""GPU parity: MatMul (f32, bf16) vs the f64 reference of tests/conformance.rs:100-144
on the same (bf16-quantized) inputs. Normalized error bound: 1e-5 (f32), 1e-2 (bf16)."""
import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BufferRef, DeviceWorkspace, KernelCall,
                          MatMulCall, UnsupportedOp)

pytestmark = pytest.mark.gpu


def run_mm(torch, backend, m, k, n, dtype, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    if dtype == DTYPE_BF16:
        ab = (a.view(np.uint32) >> 16).astype(np.uint16)
        bb = (b.view(np.uint32) >> 16).astype(np.uint16)
        a = (ab.astype(np.uint32) << 16).view(np.float32)
        b = (bb.astype(np.uint32) << 16).view(np.float32)
        da, db, es = ab, bb, 2
    else:
        da, db, es = a, b, 4
    out = torch.zeros(m * n * es, dtype=torch.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch, da))
    ws.bind(1, to_dev(torch, db))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), m, k,
                                                  n, dtype)), ws)
    backend.synchronize()
    if dtype == DTYPE_BF16:
        got = (from_dev(out, np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        got = from_dev(out, np.float32)
    return got, oracle.matmul_ref_f64(a, b, m, k, n)


@pytest.mark.parametrize("dtype,tol", [(DTYPE_F32, 1e-5), (DTYPE_BF16, 1e-2)])
@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (16, 4096, 4096), (128, 64, 128),
                                   (1, 1, 1), (77, 131, 45), (300, 1000, 257), (16, 4096, 1000)])
def test_matmul_parity(torch_cuda, backend, m, k, n, dtype, tol):
    got, want = run_mm(torch_cuda, backend, m, k, n, dtype, seed=m * 7 + n)
    err = oracle.max_rel_err(got, want)
    assert err <= tol, f"normalized error {err:.3g}"


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (16, 4096, 4096), (77, 131, 45),
                                   (300, 1000, 257), (1, 1, 1), (4096, 512, 1000), (5, 64, 24)])
def test_matmul_f16_parity(torch_cuda, backend, m, k, n):
    """f16 MatMul (the reference's lowp path serves f16 as bf16,
    float_kernels.rs:356-392): f16 operands, f32 accumulation, each result
    narrowed with the reference's rounding; within 1e-2 of the f64 product of
    the same f16 values."""
    rng = np.random.default_rng(m * 5 + n)
    a = (rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float16)
    b = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float16)
    out = torch_cuda.zeros(m * n * 2, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, a.view(np.uint16)))
    ws.bind(1, to_dev(torch_cuda, b.view(np.uint16)))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), m, k,
                                                  n, DTYPE_F16)), ws)
    backend.synchronize()
    got = from_dev(out, np.uint16).view(np.float16).astype(np.float32)
    want = oracle.matmul_ref_f64(a.astype(np.float32), b.astype(np.float32), m, k, n)
    err = oracle.max_rel_err(got, want)
    assert err <= 1e-2, f"normalized error {err:.3g}"


@pytest.mark.parametrize("m,k,n", [(64, 512, 64), (192, 1024, 320), (1024, 2048, 512),
                                   (512, 4096, 64), (960, 512, 1984)])
def test_matmul_bf16_dma64_parity(torch_cuda, backend, m, k, n):
    """Mid-size bf16 shapes taken by the 64x64-tile DMA kernel (m, n multiples of
    64, k a multiple of 512, fewer than 256 128x128 tiles), including tile
    counts that are not a multiple of the 8 XCDs and the shortest K (8 slabs)."""
    got, want = run_mm(torch_cuda, backend, m, k, n, DTYPE_BF16, seed=m + 3 * n + k)
    err = oracle.max_rel_err(got, want)
    assert err <= 1e-2, f"normalized error {err:.3g}"


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_BF16])
@pytest.mark.parametrize("m,k,n", [(7, 65, 40), (16, 4096, 4096), (300, 1000, 257), (1024, 1024, 1024),
                                   (77, 131, 45), (4096, 512, 1000), (4096, 4096, 4096)])
def test_matmul_row_bytes_independent_of_row_index(torch_cuda, backend, m, k, n, dtype):
    """simd.rs:8369 on the device: two rows of A with the same values, one in the
    first tile and one in the last (ragged) tile, give the same output bytes."""
    rng = np.random.default_rng(m + k + n)
    a = (rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float32).reshape(m, k)
    a[m - 1] = a[0]
    b = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    if dtype == DTYPE_BF16:
        da, db, es, view = (a.view(np.uint32) >> 16).astype(np.uint16), \
            (b.view(np.uint32) >> 16).astype(np.uint16), 2, np.uint16
    else:
        da, db, es, view = a, b, 4, np.float32
    out = torch_cuda.zeros(m * n * es, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, da.ravel()))
    ws.bind(1, to_dev(torch_cuda, db))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), m, k,
                                                  n, dtype)), ws)
    backend.synchronize()
    c = from_dev(out, view).reshape(m, n)
    assert np.array_equal(c[0], c[m - 1])


def test_bf16_truncates(torch_cuda, backend):
    """bf16 narrowing is truncation (write_bf16, src/cpu/dtype.rs:75-79): the single
    exact product (1 + 2^-7) * 1.5 = 0x3FC18000 narrows to 0x3FC1, where rounding to
    nearest-even would give 0x3FC2."""
    k = 64
    ab = np.zeros(k, np.uint16)
    bb = np.zeros(k, np.uint16)
    ab[5], bb[5] = 0x3F81, 0x3FC0
    out = torch_cuda.zeros(2, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, ab))
    ws.bind(1, to_dev(torch_cuda, bb))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), 1, k,
                                                  1, DTYPE_BF16)), ws)
    backend.synchronize()
    assert int(from_dev(out, np.uint16)[0]) == 0x3FC1


@pytest.mark.parametrize("m,k,n", [(1, 64, 17), (16, 4096, 4096), (300, 1000, 257),
                                   (1024, 1024, 1024), (77, 131, 45), (4096, 512, 1000)])
def test_packed_b_matmul_parity(torch_cuda, backend, m, k, n):
    """f32 MatMul with B panel-packed as the reference compiler packs constant
    weights (src/layout.rs:16-45, compiler.rs:590-613): within 1e-5 of the f64
    product of the unpacked weight."""
    rng = np.random.default_rng(m + k + n)
    a = (rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    bp = oracle.pack_b_panels(b, k, n)
    out = torch_cuda.zeros(m * n * 4, dtype=torch_cuda.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, a))
    ws.bind(1, to_dev(torch_cuda, bp))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), m, k,
                                                  n, DTYPE_F32, True)), ws)
    backend.synchronize()
    err = oracle.max_rel_err(from_dev(out, np.float32), oracle.matmul_ref_f64(a, b, m, k, n))
    assert err <= 1e-5, f"normalized error {err:.3g}"


def test_packed_b_refused_for_bf16(torch_cuda, backend):
    ws = DeviceWorkspace()
    for s in range(3):
        ws.bind(s, torch_cuda.zeros(4096, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):
        backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2),
                                                      4, 4, 4, DTYPE_BF16, True)), ws)


def packed_archive(m, k, n, weight_also_added):
    """y = relu-free MatMulAdd(x, W_packed, r); with weight_also_added the
    packed constant is also an Add operand, so it stays packed on the device."""
    from hologram_amd import (BinaryCall, ConstantEntry, HoloWriter, MatMulAddCall,
                              PortDescriptor)
    rng = np.random.default_rng(9)
    w = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    r = rng.standard_normal(m * n).astype(np.float32)
    wp = oracle.pack_b_panels(w, k, n)
    wr = HoloWriter()
    wr.inputs = [PortDescriptor("x", 0, m * k, DTYPE_F32, [m, k])]
    wr.outputs = [PortDescriptor("y", 3, m * n, DTYPE_F32, [m, n])]
    wr.constants = [ConstantEntry(1, DTYPE_F32, wp.tobytes()), ConstantEntry(2, DTYPE_F32, r.tobytes())]
    calls = [KernelCall.MatMulAdd(MatMulAddCall(
        MatMulCall(BufferRef(0), BufferRef(1, 0, wp.nbytes), BufferRef(3), m, k, n, DTYPE_F32,
                   True), BufferRef(2)))]
    if weight_also_added:
        wr.outputs.append(PortDescriptor("w2", 4, 16, DTYPE_F32, [16]))
        calls.append(KernelCall.Add(BinaryCall(BufferRef(1, 0, 64), BufferRef(1, 64, 64),
                                               BufferRef(4), 16, 32, DTYPE_F32)))
    wr.kernel_calls = calls
    wr.exec_plan = [list(range(len(calls)))]
    return wr.finish()


@pytest.mark.parametrize("m", [4, 256])
@pytest.mark.parametrize("also_added", [False, True])
def test_packed_weight_session_matches_oracle(torch_cuda, backend, m, also_added):
    """A reference-style archive whose f32 weight is panel-packed: unpacked at
    load when the MatMul is its only reader (the device's own kernels then run,
    few-row included), the packed kernel otherwise; both within 1e-5 of the
    oracle walk, which unpacks the weight itself."""
    from hologram_amd import HipSession
    from oracle.graph import OracleSession
    k, n = 512, 272
    arch = packed_archive(m, k, n, also_added)
    x = np.random.default_rng(10).standard_normal(m * k).astype(np.float32)
    sess = HipSession(backend, arch)
    ref = OracleSession(arch)
    sess.write_input(0, x.tobytes())
    ref.set_input(0, x.tobytes())
    sess.run()
    sess.synchronize()
    ref.run()
    got = np.frombuffer(sess.read_output(0), np.float32)
    err = oracle.max_rel_err(got, ref.output(0).view(np.float32))
    assert err <= 1e-5, err
    if also_added:
        assert sess.read_output(1) == ref.output(1).tobytes()
    sess.close()


def run_mm_rows(torch, backend, m, k, n, seed, rows, dtype=DTYPE_BF16):
    """MatMul on the device; f64 reference only on the sampled rows."""
    g = torch.Generator().manual_seed(seed)
    tdt = torch.bfloat16 if dtype == DTYPE_BF16 else torch.float32
    a = (torch.randn(m, k, generator=g) / np.sqrt(k)).to(tdt)
    b = (torch.randn(k, n, generator=g) / np.sqrt(k)).to(tdt)
    ad, bd = a.cuda(), b.cuda()
    out = torch.zeros(m, n, dtype=tdt, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, ad)
    ws.bind(1, bd)
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2), m, k, n,
                                                  dtype)), ws)
    backend.synchronize()
    got = out[rows].float().cpu().numpy().reshape(-1)
    a32 = a[rows].float().numpy().reshape(-1).copy()
    b32 = b.float().numpy().reshape(-1).copy()
    want = oracle.matmul_ref_f64(a32, b32, len(rows), k, n)
    return got, want


@pytest.mark.parametrize("m,k,n", [(4096, 256, 4096), (4096, 384, 4096), (4096, 320, 4096),
                                   (4096, 4096, 4096), (8192, 8192, 8192), (2048, 1024, 8192),
                                   (4096, 2048, 2048),
                                   (4096, 8192, 2048), (4096, 2048, 512), (2048, 2048, 2048)])
def test_matmul_large_tiles_sampled_rows(torch_cuda, backend, m, k, n):
    """The large-tile paths (256x256 tiles from 256 of them up, 256x128 tiles
    from 32): every 256-row tile and every row residue mod 32 appears among
    the sampled rows, and every column is checked."""
    rows = sorted({(t * 256 + (t * 37) % 256) % m for t in range(m // 256)} | set(range(0, 64)))
    got, want = run_mm_rows(torch_cuda, backend, m, k, n, seed=m + n + k, rows=rows)
    err = oracle.max_rel_err(got, want)
    assert err <= 1e-2, f"normalized error {err:.3g}"


@pytest.mark.parametrize("m,k,n", [(4096, 4096, 4096), (8192, 8192, 8192), (1024, 1024, 1024)])
def test_matmul_f32_config_shapes_sampled_rows(torch_cuda, backend, m, k, n):
    """Config 2's f32 squares at full size (the 128-tile kernel the bench times
    at 4096^3 and 8192^3): every 128-row tile is sampled once at a varying
    residue, plus the first 64 rows; every column is checked, bound 1e-5."""
    rows = sorted({(t * 128 + (t * 37) % 128) % m for t in range(m // 128)} | set(range(0, 64)))
    got, want = run_mm_rows(torch_cuda, backend, m, k, n, seed=m + 3, rows=rows, dtype=DTYPE_F32)
    err = oracle.max_rel_err(got, want)
    assert err <= 1e-5, f"normalized error {err:.3g}"


SKINNY = [(1, 4096, 4096), (7, 96, 136), (16, 512, 256), (16, 544, 264), (17, 1024, 512),
          (33, 2048, 384), (64, 4096, 1024), (5, 48, 68)]


def run_mm_guarded(torch, backend, m, k, n, dtype, a, b):
    """MatMul into an output slot followed by 256 guard bytes; returns (C, guard)."""
    es = 2 if dtype == DTYPE_BF16 else 4
    out = torch.full((m * n * es + 256,), 0xAB, dtype=torch.uint8, device="cuda")
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch, a))
    ws.bind(1, to_dev(torch, b))
    ws.bind(2, out)
    backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1),
                                                  BufferRef(2, 0, m * n * es), m, k, n, dtype)), ws)
    backend.synchronize()
    raw = out.cpu().numpy()
    body = raw[:m * n * es]
    if dtype == DTYPE_BF16:
        got = (body.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        got = body.view(np.float32).copy()
    return got, raw[m * n * es:]


def inputs(m, k, n, dtype, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(m * k) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    if dtype == DTYPE_BF16:
        ab = (a.view(np.uint32) >> 16).astype(np.uint16)
        bb = (b.view(np.uint32) >> 16).astype(np.uint16)
        return ab, bb, (ab.astype(np.uint32) << 16).view(np.float32), \
            (bb.astype(np.uint32) << 16).view(np.float32)
    return a, b, a, b


@pytest.mark.parametrize("dtype,tol", [(DTYPE_F32, 1e-5), (DTYPE_BF16, 1e-2)])
@pytest.mark.parametrize("m,k,n", SKINNY)
def test_matmul_skinny(torch_cuda, backend, m, k, n, dtype, tol):
    """The few-row path (m <= 64): 1, 2 and 4 row tiles, partial column strips,
    one K range (direct store) and several (partials + ordered sum); nothing is
    written past the output."""
    da, db, a, b = inputs(m, k, n, dtype, seed=m * 31 + k + n)
    got, guard = run_mm_guarded(torch_cuda, backend, m, k, n, dtype, da, db)
    assert (guard == 0xAB).all()
    err = oracle.max_rel_err(got, oracle.matmul_ref_f64(a, b, m, k, n))
    assert err <= tol, f"normalized error {err:.3g}"


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_BF16])
def test_matmul_skinny_nonfinite_row_isolated(torch_cuda, backend, dtype):
    """An Inf in one row of A makes that row non-finite (B has no zeros) and
    leaves every other row exact to tolerance; rows past m inside the last
    16-row tile are computed but never stored."""
    m, k, n = 7, 1024, 256
    da, db, a, b = inputs(m, k, n, dtype, seed=5)
    if dtype == DTYPE_BF16:
        da = da.copy()
        da[3 * k + 17] = 0x7F80
    else:
        da = da.copy()
        da[3 * k + 17] = np.inf
    a = a.copy()
    a[3 * k + 17] = np.inf
    got, guard = run_mm_guarded(torch_cuda, backend, m, k, n, dtype, da, db)
    assert (guard == 0xAB).all()
    got = got.reshape(m, n)
    assert not np.isfinite(got[3]).any()
    keep = [r for r in range(m) if r != 3]
    want = oracle.matmul_ref_f64(a.reshape(m, k)[keep].reshape(-1).copy(), b, len(keep), k, n)
    assert oracle.max_rel_err(got[keep].reshape(-1).copy(), want) <= (1e-2 if dtype == DTYPE_BF16 else 1e-5)


def test_matmul_skinny_deterministic_and_scratch_growth(torch_cuda, backend):
    """Split-K partials are summed in a fixed order: repeated calls agree
    bitwise, also after the scratch has grown for a larger call in between."""
    m, k, n = 16, 2048, 512
    da, db, _, _ = inputs(m, k, n, DTYPE_BF16, seed=9)
    first, _ = run_mm_guarded(torch_cuda, backend, m, k, n, DTYPE_BF16, da, db)
    ea, eb, _, _ = inputs(64, 8192, 1024, DTYPE_F32, seed=10)   # larger scratch
    run_mm_guarded(torch_cuda, backend, 64, 8192, 1024, DTYPE_F32, ea, eb)
    again, _ = run_mm_guarded(torch_cuda, backend, m, k, n, DTYPE_BF16, da, db)
    assert first.view(np.uint32).tolist() == again.view(np.uint32).tolist()
