"""Pins of the oracle's decode-step ops (oracle/holo_oracle.c) against what
the mathematics fixes, independently of the restatement's own code:
  or_binary   numpy float32 add/mul then bf16 truncation (exact)
  or_rms_norm f64 closed form; a constant row maps to gamma exactly
  or_add_rms_norm RmsNorm without a residual; bf16 = f32 RmsNorm of the
              unnarrowed sum, truncated; f64 closed form
  or_rope     f64 rotation; angle 0 is the identity; norms are preserved
  or_gather   brute-force indexing with negative wrap; range refusal
  or_argmax   numpy argmax on NaN-free rows; lowest index on ties; NaN skipped
"""
import numpy as np

import oracle
from oracle import _p, lib

BF16, F32 = 7, 8


def bf(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def unbf(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def test_binary_is_f32_op_then_truncation():
    rng = np.random.default_rng(0)
    a = bf(rng.standard_normal(4099) * 3)
    b = bf(rng.standard_normal(4099) * 3)
    for op, f in ((0, np.add), (1, np.multiply)):
        out = np.zeros_like(a)
        lib().or_binary(op, _p(a), _p(b), _p(out), a.size, BF16)
        want = bf(f(unbf(a), unbf(b)))
        assert np.array_equal(out, want)
        a32, b32 = unbf(a), unbf(b)
        o32 = np.zeros_like(a32)
        lib().or_binary(op, _p(a32), _p(b32), _p(o32), a.size, F32)
        assert np.array_equal(o32, f(a32, b32))


def test_rms_norm_closed_form():
    rng = np.random.default_rng(1)
    B, F = 5, 384
    x = rng.standard_normal((B, F)).astype(np.float32)
    g = rng.standard_normal(F).astype(np.float32)
    out = np.zeros_like(x)
    assert lib().or_rms_norm(_p(x), _p(g), _p(out), B, F, 0, F32) == 0
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-9) * g
    assert np.max(np.abs(out - want)) <= 1e-5 * np.max(np.abs(want))
    # a constant row c: x / |c| * gamma = sign(c) * gamma (up to rounding)
    c = np.full((1, F), -2.5, np.float32)
    o = np.zeros_like(c)
    lib().or_rms_norm(_p(c), _p(g), _p(o), 1, F, 0, F32)
    assert np.allclose(o[0], -g, rtol=1e-6)
    # invalid epsilon is refused (float_kernels.rs:1324-1336)
    assert lib().or_rms_norm(_p(c), None, _p(o), 1, F, 0xBF800000, F32) == -1


def test_add_rms_norm_laws():
    """or_add_rms_norm (float_kernels.rs:1566-1672): without a residual it is
    RmsNorm bit for bit; a bf16 row is the f32 RmsNorm of the unnarrowed f32
    sum x + r, truncated; f32 rows with a residual follow the f64 closed form."""
    rng = np.random.default_rng(7)
    B, F = 4, 520
    x = rng.standard_normal((B, F)).astype(np.float32) * 2
    r = rng.standard_normal((B, F)).astype(np.float32)
    g = rng.standard_normal(F).astype(np.float32)
    eps = int(np.float32(1e-5).view(np.uint32))
    o1, o2 = np.zeros_like(x), np.zeros_like(x)
    assert lib().or_add_rms_norm(_p(x), None, _p(g), _p(o1), B, F, eps, F32) == 0
    lib().or_rms_norm(_p(x), _p(g), _p(o2), B, F, eps, F32)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    # bf16: v = widen(x) + widen(r) in f32, never narrowed before the norm
    xb, rb, gb = bf(x), bf(r), bf(g)
    ob = np.zeros_like(xb)
    assert lib().or_add_rms_norm(_p(xb), _p(rb), _p(gb), _p(ob), B, F, eps, BF16) == 0
    v = (unbf(xb) + unbf(rb)).astype(np.float32)
    g32 = unbf(gb)                    # held: _p() takes no reference to its array
    of = np.zeros_like(v)
    lib().or_rms_norm(_p(v), _p(g32), _p(of), B, F, eps, F32)
    assert np.array_equal(ob, bf(of))
    # narrowing the sum first (Add then RmsNorm) is a different function
    vn = unbf(bf(v))
    lib().or_rms_norm(_p(vn), _p(g32), _p(of), B, F, eps, F32)
    assert not np.array_equal(ob, bf(of))
    # f32 with a residual: the f64 closed form
    o3 = np.zeros_like(x)
    lib().or_add_rms_norm(_p(x), _p(r), _p(g), _p(o3), B, F, eps, F32)
    vd = x.astype(np.float64) + r
    want = vd / np.sqrt((vd * vd).mean(axis=1, keepdims=True) + 1e-5) * g
    assert np.max(np.abs(o3 - want)) <= 2e-6 * np.max(np.abs(want))
    assert lib().or_add_rms_norm(_p(x), _p(r), None, _p(o3), B, F, 0xBF800000, F32) == -1


def test_rope_is_a_rotation():
    rng = np.random.default_rng(2)
    heads, D = 6, 64
    x = rng.standard_normal((heads, D)).astype(np.float32)
    theta = rng.uniform(-3, 3, (heads, D // 2)).astype(np.float32)
    cs = np.concatenate([np.cos(theta), np.cos(theta)], 1).astype(np.float32)
    sn = np.concatenate([np.sin(theta), np.sin(theta)], 1).astype(np.float32)
    out = np.zeros_like(x)
    assert lib().or_rope(_p(x), _p(cs), _p(sn), _p(out), D, x.size, F32) == 0
    x1, x2 = x[:, :D // 2].astype(np.float64), x[:, D // 2:].astype(np.float64)
    t = theta.astype(np.float64)
    want = np.concatenate([x1 * np.cos(t) - x2 * np.sin(t), x2 * np.cos(t) + x1 * np.sin(t)], 1)
    assert np.max(np.abs(out - want)) <= 1e-5
    n_in = x1 ** 2 + x2 ** 2
    n_out = out[:, :D // 2].astype(np.float64) ** 2 + out[:, D // 2:].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)
    ident, one, zero = np.zeros_like(x), np.ones_like(x), np.zeros_like(x)
    lib().or_rope(_p(x), _p(one), _p(zero), _p(ident), D, x.size, F32)
    assert np.array_equal(ident, x)
    assert lib().or_rope(_p(x), _p(cs), _p(sn), _p(out), 63, x.size, F32) == -1


def test_gather_brute_force():
    rng = np.random.default_rng(3)
    outer, axis, inner = 3, 11, 5
    data = rng.integers(0, 255, (outer, axis, inner * 2), dtype=np.uint8)
    idx = np.array([0, -1, 10, -11, 4], np.int32)
    out = np.zeros((outer, idx.size, inner * 2), np.uint8)
    assert lib().or_gather(_p(data), _p(idx), _p(out), outer, axis, inner * 2, idx.size, 0) == 0
    for o in range(outer):
        for k, i in enumerate(idx):
            assert np.array_equal(out[o, k], data[o, i % axis])
    idx64 = idx.astype(np.int64)
    out2 = np.zeros_like(out)
    lib().or_gather(_p(data), _p(idx64), _p(out2), outer, axis, inner * 2, idx.size, 1)
    assert np.array_equal(out, out2)
    bad = np.array([11], np.int32)
    assert lib().or_gather(_p(data), _p(bad), _p(out), outer, axis, inner * 2, 1, 0) == -1


def test_argmax_rules():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 1000)).astype(np.float32)
    out = np.zeros(7, np.int32)
    lib().or_argmax(_p(x), _p(out), 7, 1000, F32)
    assert np.array_equal(out, np.argmax(x, axis=1))
    t = np.array([[1, 3, 3, 2], [np.nan, -1, np.nan, -1], [np.nan] * 4], np.float32)
    o = np.zeros(3, np.int32)
    lib().or_argmax(_p(t), _p(o), 3, 4, F32)
    assert list(o) == [1, 1, 0]


F16 = 6


def f16_narrow(x):
    """The reference's f32 -> f16 rule (dtype.rs:121-153), through the pinned
    scalar codec (test_oracle_pins.py checks it exhaustively)."""
    return np.array([lib().or_f32_to_f16(float(v)) for v in np.ravel(x)], np.uint16)


def unf16(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def test_f16_element_ops_widen_compute_in_f32_and_narrow_by_the_reference_rule():
    """or_binary / or_rope / or_rms_norm over f16 (read_float / write_float,
    dtype.rs:94-153): each element widened exactly, the f32 arithmetic of the
    f32 path, then the reference's f16 narrowing."""
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(2051) * 40).astype(np.float16).view(np.uint16)
    b = (rng.standard_normal(2051) * 40).astype(np.float16).view(np.uint16)
    for op, f in ((0, np.add), (1, np.multiply)):
        out = np.zeros_like(a)
        lib().or_binary(op, _p(a), _p(b), _p(out), a.size, F16)
        assert np.array_equal(out, f16_narrow(f(unf16(a), unf16(b))))
    heads, D = 5, 32
    x = (rng.standard_normal(heads * D)).astype(np.float16).view(np.uint16)
    th = rng.uniform(-3, 3, (heads, D // 2))
    cs = np.concatenate([np.cos(th), np.cos(th)], 1).astype(np.float16).view(np.uint16).ravel()
    sn = np.concatenate([np.sin(th), np.sin(th)], 1).astype(np.float16).view(np.uint16).ravel()
    o16 = np.zeros_like(x)
    assert lib().or_rope(_p(x), _p(cs), _p(sn), _p(o16), D, x.size, F16) == 0
    x32, c32, s32 = unf16(x), unf16(cs), unf16(sn)
    o32 = np.zeros_like(x32)
    lib().or_rope(_p(x32), _p(c32), _p(s32), _p(o32), D, x.size, F32)
    assert np.array_equal(o16, f16_narrow(o32))
    B, F = 3, 96
    xr = (rng.standard_normal(B * F) * 3).astype(np.float16).view(np.uint16)
    g = rng.standard_normal(F).astype(np.float16).view(np.uint16)
    o16 = np.zeros_like(xr)
    assert lib().or_rms_norm(_p(xr), _p(g), _p(o16), B, F, 0, F16) == 0
    xr32, g32 = unf16(xr), unf16(g)
    o32 = np.zeros_like(xr32)
    lib().or_rms_norm(_p(xr32), _p(g32), _p(o32), B, F, 0, F32)
    assert np.array_equal(o16, f16_narrow(o32))
