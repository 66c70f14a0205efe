"""GPU parity: DecodeAttentionValid (discriminant 121, the reference's own
decode attention, kernel_call.rs:691-716) over bf16, f16 and f32 K/V, against
the oracle's restatement of decode_attention_valid_float
(src/cpu/float_kernels.rs:4192-4307). Bounds (normalized max error, per
query row): 1e-2 for bf16/f16, 1e-5 for f32. Unrealized past rows hold NaN:
the device must never read them (the op reads only min(valid_len, past) rows)."""
import numpy as np
import pytest

import oracle
from conftest import to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BufferRef, DecodeAttentionValidCall,
                          DeviceWorkspace, KernelCall, UnsupportedOp)

pytestmark = pytest.mark.gpu
TOL = {DTYPE_BF16: 1e-2, DTYPE_F16: 1e-2, DTYPE_F32: 1e-5}


def enc(x, dtype):
    x = np.ascontiguousarray(x, np.float32)
    if dtype == DTYPE_BF16:
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    if dtype == DTYPE_F16:
        return x.astype(np.float16).view(np.uint16)
    return x


def dec(u, dtype):
    if dtype == DTYPE_BF16:
        return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == DTYPE_F16:
        return np.asarray(u, np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(u, np.float32)


def law_f64(ops, valid, b, h, hkv, m, past, d, scale_bits, dtype):
    """The op's law in f64 on the same (widened) operands, per plane with numpy."""
    hk = h if hkv == 0 else hkv
    q, kp, vp, kn, vn = (dec(x, dtype).astype(np.float64) for x in ops)
    q = q.reshape(b, h, m, d)
    kp, vp = kp.reshape(b, hk, past, d), vp.reshape(b, hk, past, d)
    kn, vn = kn.reshape(b, hk, m, d), vn.reshape(b, hk, m, d)
    scale = 1.0 / float(np.uint32(scale_bits).view(np.float32)) if scale_bits else max(np.sqrt(np.float32(d)), 1.0)
    vis = min(valid, past)
    out = np.zeros((b, h, m, d))
    for bi in range(b):
        for hi in range(h):
            kv = hi // (h // hk)
            for qi in range(m):
                K = np.concatenate([kp[bi, kv, :vis], kn[bi, kv, :qi + 1]])
                V = np.concatenate([vp[bi, kv, :vis], vn[bi, kv, :qi + 1]])
                s_ = K @ q[bi, hi, qi] / scale
                e = np.exp(s_ - s_.max())
                out[bi, hi, qi] = (e / e.sum()) @ V
    return out.reshape(b * h * m, d)


def row_err(got, want):
    scale = np.max(np.abs(want), axis=1, keepdims=True) + 1e-9
    return float(np.max(np.abs(got - want) / scale))


def run_valid(torch, backend, b, h, hkv, m, past, valid, d, dtype, seed, scale_bits=0,
              with_law=False):
    rng = np.random.default_rng(seed)
    hk = h if hkv == 0 else hkv
    vis = min(valid, past)
    q = enc(rng.standard_normal(b * h * m * d), dtype)
    kp = rng.standard_normal((b, hk, past, d)).astype(np.float32)
    vp = rng.standard_normal((b, hk, past, d)).astype(np.float32)
    kp[:, :, vis:] = np.nan                       # unrealized rows: never read
    vp[:, :, vis:] = np.nan
    kn = rng.standard_normal(b * hk * m * d)
    vn = rng.standard_normal(b * hk * m * d)
    ops = [q, enc(kp.ravel(), dtype), enc(vp.ravel(), dtype), enc(kn, dtype), enc(vn, dtype)]
    es = 4 if dtype == DTYPE_F32 else 2
    ws = DeviceWorkspace()
    for s, x in enumerate(ops + [np.array([valid], np.uint32)]):
        ws.bind(s, to_dev(torch, x) if x.size else torch.zeros(64, dtype=torch.uint8, device="cuda"))
    out = torch.zeros(b * h * m * d * es, dtype=torch.uint8, device="cuda")
    ws.bind(6, out)
    call = KernelCall.DecodeAttentionValid(DecodeAttentionValidCall(
        *[BufferRef(s) for s in range(7)], b, h, hkv, m, past, m, d, scale_bits, dtype))
    backend.dispatch(call, ws)
    backend.synchronize()
    got = dec(out.cpu().numpy().view(np.float32 if es == 4 else np.uint16), dtype)
    want = dec(oracle.decode_attention_valid(*ops, valid, b, h, hkv, m, past, m, d, scale_bits,
                                             dtype), dtype)
    law = law_f64(ops, valid, b, h, hkv, m, past, d, scale_bits, dtype) if with_law else None
    return got.reshape(b * h * m, d), want.reshape(b * h * m, d), law


CASES = [
    (2, 32, 8, 1, 4096, 3000, 128),    # decode over a partly realized bucket (split + merge)
    (1, 8, 2, 4, 256, 100, 64),        # chunked prefill: four causal new rows
    (3, 4, 4, 1, 50, 77, 80),          # valid_len beyond the bucket clamps; head_dim 80
    (1, 2, 1, 16, 0, 0, 256),          # no past; sixteen rows; head_dim 256
    (2, 6, 0, 2, 33, 33, 40),          # kv_heads 0 = heads
    (4, 16, 4, 1, 32768, 32768, 128),  # a full 32K bucket
]


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("b,h,hkv,m,past,valid,d", CASES)
def test_decode_attention_valid_parity(torch_cuda, backend, b, h, hkv, m, past, valid, d, dtype):
    """bf16/f16: within 1e-2 of the oracle. f32: within 1e-5 of the exact (f64)
    law, and of the oracle within 1e-5 plus the oracle's own distance from the
    law: over tens of thousands of keys the reference's sequential f32 sums
    are themselves about sqrt(L) * 2^-24 ~ 1e-5 from exact."""
    f32 = dtype == DTYPE_F32
    got, want, law = run_valid(torch_cuda, backend, b, h, hkv, m, past, valid, d, dtype,
                               seed=b + h + m + d + past, with_law=f32)
    assert np.all(np.isfinite(got))
    err = row_err(got, want)
    if not f32:
        assert err <= TOL[dtype], f"normalized error {err:.3g}"
        return
    e_law, o_law = row_err(got, law), row_err(want, law)
    assert e_law <= 1e-5 and err <= 1e-5 + o_law, (err, e_law, o_law)


def test_decode_attention_valid_scale_bits_and_head_dim_1000(torch_cuda, backend):
    sb = int(np.float32(0.07).view(np.uint32))
    got, want, law = run_valid(torch_cuda, backend, 1, 4, 2, 2, 300, 200, 1000, DTYPE_F32, 5, sb,
                               with_law=True)
    assert row_err(got, law) <= 1e-5 and row_err(got, want) <= 1e-5 + row_err(want, law)


def test_decode_attention_valid_refuses_unpaired_rows(torch_cuda, backend):
    ws = DeviceWorkspace()
    for s in range(7):
        ws.bind(s, torch_cuda.zeros(1 << 16, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):            # q_rows != new_len (float_kernels.rs:4205)
        backend.dispatch(KernelCall.DecodeAttentionValid(DecodeAttentionValidCall(
            *[BufferRef(s) for s in range(7)], 1, 4, 2, 2, 16, 1, 64, 0, DTYPE_F32)), ws)


@pytest.mark.parametrize("b,h,hkv,m,past,valid,d", [
    (64, 8, 8, 4, 16, 16, 32),      # 512 planes: one share, no merge
    (1, 8, 2, 4, 256, 100, 64),     # split + merge
])
def test_decode_attention_valid_non_finite_v_past_the_causal_limit(torch_cuda, backend, b, h, hkv,
                                                                   m, past, valid, d):
    """A new row past a query row's causal limit is not in that row's key list
    (float_kernels.rs:3899-3957), so NaN and Inf in its v row reach only the
    rows that see it, exactly where the oracle puts them."""
    dtype = DTYPE_F32
    rng = np.random.default_rng(9)
    hk = h if hkv == 0 else hkv
    q = rng.standard_normal(b * h * m * d).astype(np.float32)
    kp = rng.standard_normal(b * hk * past * d).astype(np.float32)
    vp = rng.standard_normal(b * hk * past * d).astype(np.float32)
    kn = rng.standard_normal(b * hk * m * d).astype(np.float32)
    vn = rng.standard_normal((b, hk, m, d)).astype(np.float32)
    vn[:, :, m - 1, ::2] = np.nan                # the last new row: only row m-1 sees it
    vn[:, :, m - 1, 1::2] = np.inf
    ops = [q, kp, vp, kn, vn.ravel()]
    ws = DeviceWorkspace()
    for s, x in enumerate(ops + [np.array([valid], np.uint32)]):
        ws.bind(s, to_dev(torch_cuda, x))
    out = torch_cuda.zeros(b * h * m * d * 4, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(6, out)
    backend.dispatch(KernelCall.DecodeAttentionValid(DecodeAttentionValidCall(
        *[BufferRef(s) for s in range(7)], b, h, hkv, m, past, m, d, 0, dtype)), ws)
    backend.synchronize()
    got = out.cpu().numpy().view(np.float32).reshape(b, h, m, d)
    want = oracle.decode_attention_valid(*ops, valid, b, h, hkv, m, past, m, d, 0,
                                         dtype).reshape(b, h, m, d)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    assert not np.isnan(got[:, :, :m - 1]).any()
    assert row_err(got[:, :, :m - 1].reshape(-1, d), want[:, :, :m - 1].reshape(-1, d)) <= 1e-5
