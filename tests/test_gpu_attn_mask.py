"""GPU parity: DecodeAttention (discriminant 119, the mask form,
kernel_call.rs:600-656) over bf16, f16 and f32 K/V, against the oracle's
restatement of decode_attention_float (src/cpu/float_kernels.rs:2420-2660).
Every past row, then every new row, is a key; query row qi adds
mask[qi][j] (f32 [q_rows, past + new]) to the score of key j. Bounds
(normalized max error per query row): 1e-2 for bf16/f16; for f32 1e-5 of the
f64 law and of the oracle within 1e-5 plus the oracle's own distance from the
law. A row whose every key is erased must be exactly zero."""
import numpy as np
import pytest

import oracle
from conftest import to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BufferRef, DecodeAttentionCall,
                          DeviceWorkspace, KernelCall, UnsupportedOp)
from test_gpu_attn_valid import TOL, dec, enc, row_err

pytestmark = pytest.mark.gpu


def law_f64(ops, mask, b, h, hkv, m, past, new, d, dtype):
    """The mask form's law in f64 on the same (widened) operands."""
    hk = h if hkv == 0 else hkv
    q, kp, vp, kn, vn = (dec(x, dtype).astype(np.float64) for x in ops)
    q = q.reshape(b, h, m, d)
    K = np.concatenate([kp.reshape(b, hk, past, d), kn.reshape(b, hk, new, d)], 2)
    V = np.concatenate([vp.reshape(b, hk, past, d), vn.reshape(b, hk, new, d)], 2)
    scale = max(np.sqrt(np.float32(d)), 1.0)
    out = np.zeros((b, h, m, d))
    for bi in range(b):
        for hi in range(h):
            kv = hi // (h // hk)
            for qi in range(m):
                s_ = K[bi, kv] @ q[bi, hi, qi] / scale + mask[qi].astype(np.float64)
                fin = np.isfinite(s_)
                if not fin.any():
                    continue
                e = np.exp(s_ - s_[fin].max())
                out[bi, hi, qi] = (e / e.sum()) @ V[bi, kv]
    return out.reshape(b * h * m, d)


def make_mask(rng, m, past, new, kind):
    L = past + new
    if kind == "realized":   # a realized prefix of 3/4 of the bucket, causal new rows
        mask = np.full((m, L), -np.inf, np.float32)
        for qi in range(m):
            mask[qi, :(3 * past) // 4] = 0.0
            mask[qi, past:past + min(qi + 1, new)] = 0.0
        return mask
    mask = (rng.standard_normal((m, L)) * 2).astype(np.float32)
    mask[rng.random((m, L)) < 0.3] = -np.inf
    mask[m - 1, :] = -np.inf                 # one fully erased query row
    return mask


def run_mask(torch, backend, b, h, hkv, m, past, new, d, dtype, kind, seed):
    rng = np.random.default_rng(seed)
    hk = h if hkv == 0 else hkv
    ops = [enc(rng.standard_normal(n), dtype) for n in
           (b * h * m * d, b * hk * past * d, b * hk * past * d, b * hk * new * d,
            b * hk * new * d)]
    mask = make_mask(rng, m, past, new, kind)
    es = 4 if dtype == DTYPE_F32 else 2
    ws = DeviceWorkspace()
    for s, x in enumerate(ops + [mask.ravel()]):
        ws.bind(s, to_dev(torch, x) if x.size else torch.zeros(64, dtype=torch.uint8, device="cuda"))
    out = torch.full((b * h * m * d * es,), 0x55, dtype=torch.uint8, device="cuda")
    ws.bind(6, out)
    backend.dispatch(KernelCall.DecodeAttention(DecodeAttentionCall(
        *[BufferRef(s) for s in range(7)], b, h, hkv, m, past, new, d, 0, dtype)), ws)
    backend.synchronize()
    got = dec(out.cpu().numpy().view(np.float32 if es == 4 else np.uint16), dtype)
    want = dec(oracle.decode_attention(*ops, mask, b, h, hkv, m, past, new, d, 0, dtype), dtype)
    law = law_f64(ops, mask, b, h, hkv, m, past, new, d, dtype)
    return got.reshape(-1, d), want.reshape(-1, d), law, mask


CASES = [
    (2, 32, 8, 1, 4096, 1, 128, "realized"),   # decode over a bucket, split + merge
    (1, 8, 2, 4, 256, 4, 64, "realized"),      # chunked prefill, causal new rows
    (1, 8, 2, 4, 256, 4, 64, "random"),        # arbitrary additive mask, one erased row
    (1, 4, 2, 3, 100, 0, 80, "random"),        # frozen cache: no new rows, q_rows 3
    (2, 2, 0, 2, 0, 5, 32, "random"),          # no past; q_rows != new_len
    (1, 8, 8, 1, 32768, 1, 128, "realized"),   # a 32K bucket
]


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("b,h,hkv,m,past,new,d,kind", CASES)
def test_decode_attention_mask_parity(torch_cuda, backend, b, h, hkv, m, past, new, d, kind,
                                      dtype):
    got, want, law, mask = run_mask(torch_cuda, backend, b, h, hkv, m, past, new, d, dtype, kind,
                                    seed=b + h + m + d + past + new)
    assert np.all(np.isfinite(got))
    erased = ~np.isfinite(mask).any(axis=1)            # [m] rows with no visible key
    rows = got.reshape(b, h, m, d)
    if erased.any():
        assert np.array_equal(rows[:, :, erased], np.zeros_like(rows[:, :, erased]))
    if dtype != DTYPE_F32:
        err = row_err(got, want)
        assert err <= TOL[dtype], f"normalized error {err:.3g}"
        return
    err, e_law, o_law = row_err(got, want), row_err(got, law), row_err(want, law)
    assert e_law <= 1e-5 and err <= 1e-5 + o_law, (err, e_law, o_law)


def test_decode_attention_mask_refuses_empty_key_list(torch_cuda, backend):
    ws = DeviceWorkspace()
    for s in range(7):
        ws.bind(s, torch_cuda.zeros(1 << 12, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):            # past_len + new_len == 0 (float_kernels.rs:2496)
        backend.dispatch(KernelCall.DecodeAttention(DecodeAttentionCall(
            *[BufferRef(s) for s in range(7)], 1, 4, 2, 1, 0, 0, 64, 0, DTYPE_F32)), ws)


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F32])
def test_mask_form_archive_session_matches_oracle_walk(torch_cuda, backend, dtype):
    """A .holo archive holding a DecodeAttention call (wire 119, put_decattn)
    walks on the device to within the op's bound of the oracle's walk of the
    same archive (oracle/graph.py, the reference engine's arithmetic)."""
    from hologram_amd import HipSession, HoloWriter, PortDescriptor
    from oracle.graph import OracleSession
    b, h, hkv, m, past, new, d = 2, 8, 2, 2, 96, 2, 64
    es = 4 if dtype == DTYPE_F32 else 2
    rng = np.random.default_rng(5)
    ops = [enc(rng.standard_normal(n), dtype) for n in
           (b * h * m * d, b * hkv * past * d, b * hkv * past * d, b * hkv * new * d,
            b * hkv * new * d)]
    mask = make_mask(rng, m, past, new, "random")
    names = ["q", "k_past", "v_past", "k_new", "v_new"]
    w = HoloWriter()
    w.inputs = [PortDescriptor(nm, s, x.size, dtype, [x.size]) for s, (nm, x) in
                enumerate(zip(names, ops))]
    w.inputs.append(PortDescriptor("mask", 5, mask.size, DTYPE_F32, [m, past + new]))
    w.outputs = [PortDescriptor("out", 6, b * h * m * d, dtype, [b, h, m, d])]
    w.kernel_calls = [KernelCall.DecodeAttention(DecodeAttentionCall(
        *[BufferRef(s, 0, n) for s, n in enumerate(
            [x.nbytes for x in ops] + [mask.nbytes, b * h * m * d * es])],
        b, h, hkv, m, past, new, d, 0, dtype))]
    arch = w.finish()
    sess = HipSession(backend, arch)
    ref = OracleSession(arch)
    ins = [x.tobytes() for x in ops] + [mask.tobytes()]
    got = sess.execute(ins)[0]
    for i, x in enumerate(ins):
        ref.set_input(i, x)
    ref.run()
    g = dec(np.frombuffer(got, np.float32 if es == 4 else np.uint16), dtype).reshape(-1, d)
    r = dec(ref.output(0).view(np.float32 if es == 4 else np.uint16), dtype).reshape(-1, d)
    assert row_err(g, r) <= TOL[dtype]
    sess.close()


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F32])
def test_mask_form_split_equals_precatenated_on_device(torch_cuda, backend, dtype):
    """tests/decode_attention.rs:5-9 on the device, bit for bit: the same keys
    split past || new, or precatenated as past with no new rows, give the same
    bytes (the key list, its order and the work split depend on past + new
    only)."""
    b, h, hkv, m, past, new, d = 2, 8, 2, 2, 700, 3, 64
    rng = np.random.default_rng(33)
    es = 4 if dtype == DTYPE_F32 else 2
    q = enc(rng.standard_normal(b * h * m * d), dtype)
    kp, vp = (rng.standard_normal((b, hkv, past, d)) for _ in range(2))
    kn, vn = (rng.standard_normal((b, hkv, new, d)) for _ in range(2))
    mask = make_mask(rng, m, past, new, "random").ravel()

    def run(kp_, vp_, kn_, vn_, p_, n_):
        ws = DeviceWorkspace()
        ops = [q, enc(kp_.ravel(), dtype), enc(vp_.ravel(), dtype), enc(kn_.ravel(), dtype),
               enc(vn_.ravel(), dtype), mask]
        for s_, x in enumerate(ops):
            ws.bind(s_, to_dev(torch_cuda, x) if x.size else
                    torch_cuda.zeros(64, dtype=torch_cuda.uint8, device="cuda"))
        out = torch_cuda.zeros(b * h * m * d * es, dtype=torch_cuda.uint8, device="cuda")
        ws.bind(6, out)
        backend.dispatch(KernelCall.DecodeAttention(DecodeAttentionCall(
            *[BufferRef(s_) for s_ in range(7)], b, h, hkv, m, p_, n_, d, 0, dtype)), ws)
        backend.synchronize()
        return out.cpu().numpy()

    split = run(kp, vp, kn, vn, past, new)
    cat = run(np.concatenate([kp, kn], 2), np.concatenate([vp, vn], 2), kn[:, :, :0],
              vn[:, :, :0], past + new, 0)
    assert np.array_equal(split, cat)


@pytest.mark.parametrize("b,h,hkv,m,past,new,d", [
    (2, 2, 0, 2, 0, 5, 32),          # one share, no merge
    (2, 32, 8, 1, 4096, 1, 128),     # split + merge
])
def test_mask_form_erased_row_is_zero_over_non_finite_v(torch_cuda, backend, b, h, hkv, m, past,
                                                        new, d):
    """A query row whose mask erases every key is the exact zero row
    (float_kernels.rs:2446-2453) even where the v rows hold NaN and Inf; a row
    that sees any key passes an erased key's NaN on as 0 * NaN, as the
    reference's axpy does, and the oracle marks the same elements NaN."""
    dtype = DTYPE_F32
    rng = np.random.default_rng(21)
    hk = h if hkv == 0 else hkv
    L = past + new
    q = rng.standard_normal(b * h * m * d).astype(np.float32)
    kp, vp = (rng.standard_normal((b, hk, past, d)).astype(np.float32) for _ in range(2))
    kn, vn = (rng.standard_normal((b, hk, new, d)).astype(np.float32) for _ in range(2))
    mask = np.zeros((m, L), np.float32)
    mask[:, L // 2] = -np.inf                    # erased for every row; its v is non-finite
    mask[m - 1, :] = -np.inf                     # the last row sees nothing
    vrow = L // 2
    tgt = vp if vrow < past else vn
    j = vrow if vrow < past else vrow - past
    tgt[:, :, j, ::2] = np.nan
    tgt[:, :, j, 1::2] = np.inf
    ops = [q, kp.ravel(), vp.ravel(), kn.ravel(), vn.ravel()]
    ws = DeviceWorkspace()
    for s, x in enumerate(ops + [mask.ravel()]):
        ws.bind(s, to_dev(torch_cuda, x) if x.size else
                torch_cuda.zeros(64, dtype=torch_cuda.uint8, device="cuda"))
    out = torch_cuda.full((b * h * m * d * 4,), 0x55, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(6, out)
    backend.dispatch(KernelCall.DecodeAttention(DecodeAttentionCall(
        *[BufferRef(s) for s in range(7)], b, h, hkv, m, past, new, d, 0, dtype)), ws)
    backend.synchronize()
    got = out.cpu().numpy().view(np.float32).reshape(b, h, m, d)
    want = oracle.decode_attention(*ops, mask.ravel(), b, h, hkv, m, past, new, d, 0,
                                   dtype).reshape(b, h, m, d)
    assert np.array_equal(got[:, :, m - 1], np.zeros_like(got[:, :, m - 1]))
    assert np.array_equal(want[:, :, m - 1], np.zeros_like(want[:, :, m - 1]))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
