"""GPU parity: int8-KV GQA decode attention (new op 123) vs the oracle's
per-sequence DecodeAttentionValid over dequantized rows
(src/cpu/float_kernels.rs:3834-3957). Tolerance: normalized max error
max|got - want| / max|want| <= 1e-2 (bf16 output is narrowed by truncation)."""
import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F32, BufferRef, DecodeAttentionI8Call,
                          DeviceWorkspace, KernelCall, UnsupportedOp)

pytestmark = pytest.mark.gpu
TOL = 1e-2


def make_cache(rng, B, Hkv, bucket, D):
    """Fill every row through the oracle quantizer (config 3's scheme)."""
    planes = B * Hkv
    x = rng.standard_normal((planes, bucket, D)).astype(np.float32)
    ch = rng.choice(D, size=max(1, int(np.ceil(0.02 * D))), replace=False)
    x[..., ch] *= 20.0
    cq = np.zeros(planes * bucket * D, np.int8)
    cs = np.zeros(planes * bucket, np.float32)
    return oracle.kv_quant_append(x, DTYPE_F32, 0, cq, cs, planes, bucket, bucket, D)


def run_case(torch, backend, B, H, Hkv, D, bucket, lens, dtype, seed, scale_bits=0):
    rng = np.random.default_rng(seed)
    kq, ks = make_cache(rng, B, Hkv, bucket, D)
    vq, vs = make_cache(rng, B, Hkv, bucket, D)
    q32 = rng.standard_normal(B * H * D).astype(np.float32)
    if dtype == DTYPE_BF16:
        qbits = (q32.view(np.uint32) >> 16).astype(np.uint16)
        q32 = (qbits.astype(np.uint32) << 16).view(np.float32)
        qdev = qbits
    else:
        qdev = q32
    lens = np.asarray(lens, np.uint32)
    es = 2 if dtype == DTYPE_BF16 else 4
    out = torch.zeros(B * H * D * es, dtype=torch.uint8, device="cuda")
    ws = DeviceWorkspace()
    for s, arr in enumerate([qdev, kq, vq, ks, vs, lens]):
        ws.bind(s, to_dev(torch, arr))
    ws.bind(6, out)
    call = KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
        *[BufferRef(s) for s in range(7)], B, H, Hkv, bucket, D, scale_bits, dtype))
    backend.dispatch(call, ws)
    backend.synchronize()
    if dtype == DTYPE_BF16:
        got = (from_dev(out, np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        got = from_dev(out, np.float32)
    want = oracle.decode_attention_i8(q32, kq, ks, vq, vs, lens, B, H, Hkv, bucket, D,
                                      oracle.attn_scale(D, scale_bits))
    return got.reshape(B, H, D), want.reshape(B, H, D), lens


def norm_err(got, want):
    return float(np.max(np.abs(got - want)) / (np.max(np.abs(want)) + 1e-9))


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F32])
@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (8, 8, 128), (16, 8, 64), (16, 2, 128),
                                     (8, 1, 64)])
def test_ragged_gqa(torch_cuda, backend, H, Hkv, D, dtype):
    B, bucket = 5, 1300
    lens = [1, 256, 257, 1299, 5000]          # last one clamps to the bucket
    got, want, _ = run_case(torch_cuda, backend, B, H, Hkv, D, bucket, lens, dtype, seed=H * D)
    assert np.all(np.isfinite(got))
    for b in range(B):
        assert norm_err(got[b], want[b]) <= TOL, f"sequence {b} (len {lens[b]})"


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F32])
@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 96), (16, 8, 256), (8, 2, 80), (32, 1, 64),
                                     (4, 4, 32), (64, 2, 128)])
def test_any_head_dim_and_group(torch_cuda, backend, H, Hkv, D, dtype):
    """Shapes the MFMA kernels do not take (head_dim other than 64 / 128, or
    more than 16 query heads per kv head) run the generic blocked kernel, to
    the same bound, ragged lengths and a length past the bucket included."""
    B, bucket = 4, 700
    lens = [0, 1, 699, 5000]
    got, want, _ = run_case(torch_cuda, backend, B, H, Hkv, D, bucket, lens, dtype, seed=H + D)
    assert np.all(np.isfinite(got))
    assert np.all(got[0] == 0)
    for b in range(1, B):
        assert norm_err(got[b], want[b]) <= TOL, f"sequence {b} (len {lens[b]})"


def test_zero_length_is_exact_zero(torch_cuda, backend):
    got, want, _ = run_case(torch_cuda, backend, 3, 8, 2, 128, 64, [0, 64, 0], DTYPE_F32, seed=1)
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert norm_err(got[1], want[1]) <= TOL


def test_scale_bits(torch_cuda, backend):
    sb = int(np.float32(0.05).view(np.uint32))
    got, want, _ = run_case(torch_cuda, backend, 2, 8, 2, 128, 600, [600, 333], DTYPE_F32,
                            seed=7, scale_bits=sb)
    assert norm_err(got, want) <= TOL


def test_config4_shape_subset(torch_cuda, backend):
    """B=8 of config 4's 32, H=32/8, D=128, ragged L up to 8192."""
    rng = np.random.default_rng(44)
    lens = rng.integers(512, 8193, size=8)
    got, want, _ = run_case(torch_cuda, backend, 8, 32, 8, 128, 8192, lens, DTYPE_BF16, seed=4)
    for b in range(8):
        assert norm_err(got[b], want[b]) <= TOL


def test_refusals(torch_cuda, backend):
    ws = DeviceWorkspace()
    for s in range(7):
        ws.bind(s, torch_cuda.zeros(1 << 16, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):   # heads not a multiple of kv_heads
        backend.dispatch(KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
            *[BufferRef(s) for s in range(7)], 1, 6, 4, 16, 128)), ws)


def test_repeat_calls_are_bitwise_identical(torch_cuda, backend):
    """The split-K merge order is fixed (a plane's partials merged in index
    order): back-to-back calls, and a call on a different batch shape in
    between (which reuses the scratch), give identical bits."""
    B, H, Hkv, D, bucket = 4, 16, 4, 128, 5000
    rng = np.random.default_rng(9)
    kq, ks = make_cache(rng, B, Hkv, bucket, D)
    vq, vs = make_cache(rng, B, Hkv, bucket, D)
    q = (rng.standard_normal(B * H * D).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    lens = np.array([4999, 1025, 3000, 17], np.uint32)
    ws = DeviceWorkspace()
    for s, arr in enumerate([q, kq, vq, ks, vs, lens]):
        ws.bind(s, to_dev(torch_cuda, arr))
    out = torch_cuda.zeros(B * H * D * 2, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(6, out)
    call = KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
        *[BufferRef(s) for s in range(7)], B, H, Hkv, bucket, D, 0, DTYPE_BF16))
    runs = []
    for i in range(3):
        backend.dispatch(call, ws)
        backend.synchronize()
        runs.append(from_dev(out, np.uint16).copy())
        if i == 1:   # a differently shaped call in between reuses the scratch
            run_case(torch_cuda, backend, 2, 8, 8, 64, 3000, [2999, 1500], DTYPE_F32, seed=3)
    assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2])


def test_shares_cross_planes(torch_cuda, backend):
    """Lengths that make the balanced split cut planes at odd places: single-key
    planes, a plane of exactly one 128-key quad, zero-length sequences between
    long ones, and lengths beyond the bucket."""
    lens = [3000, 0, 1, 128, 129, 0, 0, 2047, 4096, 5000, 7, 0]
    B, H, Hkv, D, bucket = len(lens), 16, 4, 128, 4096
    got, want, _ = run_case(torch_cuda, backend, B, H, Hkv, D, bucket, lens, DTYPE_F32, seed=21)
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0), f"sequence {b} must be exact zeros"
        else:
            assert norm_err(got[b], want[b]) <= TOL, f"sequence {b} (len {lens[b]})"


def test_large_batch_grid_form(torch_cuda, backend):
    """More sequences than the balanced form scans in LDS (1024): the grid form."""
    B, H, Hkv, D, bucket = 1030, 4, 2, 64, 96
    rng = np.random.default_rng(5)
    lens = rng.integers(0, 120, size=B)
    got, want, _ = run_case(torch_cuda, backend, B, H, Hkv, D, bucket, lens, DTYPE_BF16, seed=6)
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0)
        else:
            assert norm_err(got[b], want[b]) <= TOL, f"sequence {b} (len {lens[b]})"


@pytest.mark.parametrize("D", [64, 128])
def test_short_contexts_one_chunk_per_plane(torch_cuda, backend, D):
    """Many planes whose bucket fits one chunk (a decode step's shape: 8 sequences
    x 8 kv heads, bucket 1024): one workgroup per plane, no merge launch."""
    B, H, Hkv, bucket = 8, 32, 8, 1024
    lens = [0, 1, 31, 128, 513, 767, 1024, 4000]
    got, want, _ = run_case(torch_cuda, backend, B, H, Hkv, D, bucket, lens, DTYPE_BF16,
                            seed=D + 1)
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0)
        else:
            assert norm_err(got[b], want[b]) <= TOL, f"sequence {b} (len {lens[b]})"


@pytest.mark.parametrize("out_dtype", [DTYPE_BF16, DTYPE_F32])
def test_config4_full_shape_every_sequence(torch_cuda, backend, out_dtype):
    """Config 4 as the bench runs it: B=32, H=32/8, D=128, a 32,768-row bucket
    (two 1 GiB int8 caches), lengths L ~ U[512, 32768] from the bench's seed,
    so the balanced split over 512+ workgroups and its cross-plane merge run
    exactly as timed. The caches are filled on the device with seeded bf16
    N(0,1) rows (2% of channels x20) through the int8 append op; every one of
    the 32 sequences is compared with the oracle over the same cache bytes.
    With an f32 output the error is the kernel's own arithmetic (Q as a
    15-bit integer, P in f16); a bf16 output adds its truncation. The worst
    and mean normalized errors are printed (pytest -s)."""
    import math
    from hologram_amd import KvQuantAppendCall
    torch = torch_cuda
    B, H, Hkv, D, bucket = 32, 32, 8, 128, 32768
    lens = np.random.default_rng(1234).integers(512, 32769, size=B).astype(np.uint32)
    planes = B * Hkv
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    kq = torch.empty(planes * bucket * D, dtype=torch.int8, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty(planes * bucket, dtype=torch.float32, device="cuda")
    vs = torch.empty_like(ks)
    pos0 = torch.zeros(1, dtype=torch.int32, device="cuda")
    ch_n = math.ceil(0.02 * D)
    for cq, cs in ((kq, ks), (vq, vs)):
        for p0 in range(0, planes, 32):
            x = torch.randn((32, bucket, D), generator=gen, device="cuda")
            x[..., torch.randperm(D, generator=gen, device="cuda")[:ch_n]] *= 20.0
            src = x.to(torch.bfloat16)
            del x
            ws = DeviceWorkspace()
            for s, t in enumerate([src, pos0, cq, cs]):
                ws.bind(s, t)
            oq, os_ = p0 * bucket * D, p0 * bucket * 4
            rq, rs = BufferRef(2, oq, 32 * bucket * D), BufferRef(3, os_, 32 * bucket * 4)
            backend.dispatch(KernelCall.KvQuantAppend(KvQuantAppendCall(
                BufferRef(0), BufferRef(1), rq, rs, rq, rs, 32, bucket, bucket, D, DTYPE_BF16)), ws)
            backend.synchronize()
            del src
    q = torch.randn(B * H * D, generator=gen, device="cuda").to(torch.bfloat16)
    if out_dtype == DTYPE_F32:                    # the op's dtype is Q's and the output's
        q = q.float()
    out = torch.zeros(B * H * D, dtype=torch.bfloat16 if out_dtype == DTYPE_BF16 else
                      torch.float32, device="cuda")
    lens_t = torch.from_numpy(lens.astype(np.int32)).cuda()
    ws = DeviceWorkspace()
    for s, t in enumerate([q, kq, vq, ks, vs, lens_t, out]):
        ws.bind(s, t)
    backend.dispatch(KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
        *[BufferRef(s) for s in range(7)], B, H, Hkv, bucket, D, 0, out_dtype)), ws)
    backend.synchronize()
    got = out.float().cpu().numpy().reshape(B, H, D)
    want = oracle.decode_attention_i8(q.float().cpu().numpy(), kq.cpu().numpy(), ks.cpu().numpy(),
                                      vq.cpu().numpy(), vs.cpu().numpy(), lens, B, H, Hkv, bucket,
                                      D, oracle.attn_scale(D)).reshape(B, H, D)
    del kq, vq
    torch.cuda.empty_cache()
    errs = [norm_err(got[b], want[b]) for b in range(B)]
    print(f"\nconfig 4 full shape, {'bf16' if out_dtype == DTYPE_BF16 else 'f32'} output: "
          f"normalized error worst {max(errs):.3g} (sequence {int(np.argmax(errs))}), "
          f"mean {float(np.mean(errs)):.3g}")
    assert max(errs) <= TOL, f"worst sequence {int(np.argmax(errs))}: {max(errs):.3g}"
