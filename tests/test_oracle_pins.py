"""CPU tests that pin the oracle (oracle/holo_oracle.c) to the reference.

Each oracle function is checked against something other than its own formula:
the reference's golden vector, the reference's own test tolerances, a closed
form or a brute force on tiny inputs. Where a plausible mistake would slip
through one check, a second check is chosen to catch it (a planted mistake is
computed here on the CPU and shown to fail).
"""
import math

import numpy as np
import pytest

import oracle

BF16, F16, F32 = oracle.DTYPE_BF16, oracle.DTYPE_F16, oracle.DTYPE_F32
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = BF16, F16, F32
L = oracle.lib()


def bf16_values():
    bits = np.arange(65536, dtype=np.uint32) << 16
    return bits.view(np.float32)


def golden_inputs():
    """The generators of integer_gemv_bits_are_the_cross_lane_golden (simd.rs:8247-8256)."""
    m, k, n = 3, 64, 24
    a = (np.array([(i * 37) % 91 for i in range(m * k)], np.float32) - np.float32(45.0)) * np.float32(0.031)
    scales = (np.float32(0.011) + np.arange(n, dtype=np.float32) * np.float32(0.0007)).astype(np.float32)
    bq = np.array([((i * 31) % 255) - 127 for i in range(k * n)], dtype=np.int8)
    return a.astype(np.float32), bq, scales, m, k, n


# ---------------------------------------------------------------- golden ----

def test_int8_quantizer_reproduces_reference_golden():
    """FNV-1a of matmul_i8_pc_omajor(3, 64, 24) == 0x787ccdc172029f9b (simd.rs:8259)."""
    a, bq, scales, m, k, n = golden_inputs()
    out = oracle.matmul_i8_pc_omajor(a, bq, scales, m, k, n)
    assert oracle.fnv1a_f32(out) == 0x787CCDC172029F9B


def test_packed_i4_and_e8cb_gemvs_reproduce_reference_goldens():
    """The same test's other two tiers (simd.rs:8261-8283): packed i4 (W4A8)
    FNV 0x4c5123c024af97ae and e8cb (W1A8, an 8-D codebook block per index)
    FNV 0x88ac55a91dd5aa0d, over the same activations and scales; and the i8
    golden through the generic entry."""
    a, bq, scales, m, k, n = golden_inputs()
    o8 = oracle.matmul_q_omajor(2, a, bq, scales, m, k, n)
    assert oracle.fnv1a_f32(o8) == 0x787CCDC172029F9B
    bq4 = np.array([(i * 53 + 9) % 251 for i in range(k * n // 2)], np.uint8)
    o4 = oracle.matmul_q_omajor(10, a, bq4, scales, m, k, n)
    assert oracle.fnv1a_f32(o4) == 0x4C5123C024AF97AE
    cb = np.array([(i * 37 + 11) % 255 - 127 for i in range(256 * 8)], np.int8)
    bq8 = np.array([(i * 17 + 3) % 256 for i in range(n * (k // 8))], np.uint8)
    oe = oracle.matmul_q_omajor(11, a, bq8, scales, m, k, n, codebook=cb)
    assert oracle.fnv1a_f32(oe) == 0x88AC55A91DD5AA0D
    # a nibble-order mistake (high nibble first) breaks the i4 golden
    swapped = ((bq4 & 0x0F) << 4) | (bq4 >> 4)
    assert oracle.fnv1a_f32(oracle.matmul_q_omajor(10, a, swapped, scales, m, k, n)) != \
        0x4C5123C024AF97AE


def _golden_with(quantize):
    """The golden's arithmetic with a substitute quantizer (numpy, CPU only)."""
    a, bq, scales, m, k, n = golden_inputs()
    out = np.zeros(m * n, np.float32)
    for i in range(m):
        row = a[i * k:(i + 1) * k]
        q, s = quantize(row)
        for j in range(n):
            acc = int(np.dot(q.astype(np.int64), bq[j * k:(j + 1) * k].astype(np.int64)))
            out[i * n + j] = np.float32(acc) * (np.float32(s) * scales[j])
    return oracle.fnv1a_f32(out)


def test_golden_discriminates_quantizer_mistakes():
    """The golden catches a truncating quantizer and a scale computed as 1/inv
    instead of amax/127. Its inputs never hit an exact .5 tie, so it does NOT
    tell half-away-from-zero from half-to-even: the tie rule is pinned by the
    exact-tie closed form in test_quantizer_closed_forms."""
    def quant(row, rnd, scale_from_inv=False):
        amax = np.float32(np.max(np.abs(row)))
        inv = np.float32(127.0) / amax
        t = (row * inv).astype(np.float32)
        q = np.clip(rnd(t), -127, 127).astype(np.int8)
        s = np.float32(1.0) / inv if scale_from_inv else amax / np.float32(127.0)
        return q, s

    away = lambda t: np.where(t >= 0, np.trunc(t + np.float32(0.5)), np.trunc(t - np.float32(0.5)))
    assert _golden_with(lambda r: quant(r, away)) == 0x787CCDC172029F9B
    assert _golden_with(lambda r: quant(r, np.rint)) == 0x787CCDC172029F9B   # no ties here
    assert _golden_with(lambda r: quant(r, np.trunc)) != 0x787CCDC172029F9B
    assert _golden_with(lambda r: quant(r, away, scale_from_inv=True)) != 0x787CCDC172029F9B


def test_quantizer_closed_forms():
    # all-zero row: scale 0 and q untouched (the oracle's caller zeroes q)
    q, s = oracle.quantize_row_i8(np.zeros(8, np.float32))
    assert s == 0.0 and not q.any()
    # amax = 127 makes inv exactly 1, so x.5 values are exact ties: they round
    # away from zero (half-to-even would give 2, -2, 0, 0)
    row = np.array([127.0, 2.5, -2.5, 0.5, -0.5, -127.0], np.float32)
    q, s = oracle.quantize_row_i8(row)
    assert s == np.float32(1.0)
    assert list(q) == [127, 3, -3, 1, -1, -127]
    # NaN is ignored by the max and quantizes to 0; Inf gives scale Inf, q 0 / NaN -> 0
    q, s = oracle.quantize_row_i8(np.array([np.nan, 1.0, -0.5], np.float32))
    assert q[0] == 0 and q[1] == 127 and s == np.float32(1.0) / np.float32(127.0)
    q, s = oracle.quantize_row_i8(np.array([np.inf, 3.0], np.float32))
    assert math.isinf(s) and not q.any()


# ---------------------------------------------------------------- exp -------

def test_exp_det_error_bound_and_cutoffs():
    xs = np.linspace(-87.3, 88.0, 200_001, dtype=np.float32)
    got = np.array([L.or_exp_f32_det(float(x)) for x in xs[::50]], np.float64)
    want = np.exp(xs[::50].astype(np.longdouble)).astype(np.float64)
    rel = np.abs(got - want) / want
    assert rel.max() <= 2e-6
    assert L.or_exp_f32_det(0.0) == 1.0
    assert L.or_exp_f32_det(-100.0) == 0.0
    assert L.or_exp_f32_det(float("nan")) == 0.0
    big = L.or_exp_f32_det(float("inf"))
    assert big == L.or_exp_f32_det(88.0) and 1.6e38 < big < 1.7e38


def test_libm_expf_within_one_ulp_of_correctly_rounded_on_every_bf16_input():
    xs = bf16_values()
    fin = np.isfinite(xs)
    got = np.array([L.or_libm_expf(float(x)) for x in xs], np.float32)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        cr = np.exp(xs.astype(np.longdouble)).astype(np.float32)
    gu, cu = got.view(np.uint32).astype(np.int64), cr.view(np.uint32).astype(np.int64)
    assert np.abs(gu - cu)[fin].max() <= 1
    # the bf16 Exp table equals the truncated correctly rounded value everywhere
    assert np.array_equal((gu >> 16)[fin], (cu >> 16)[fin])
    assert int(np.float32(L.or_libm_expf(1.0)).view(np.uint32)) == 0x402DF854
    assert L.or_libm_expf(float("-inf")) == 0.0 and math.isinf(L.or_libm_expf(100.0))


def signed_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in units in the last place between f32 arrays (sign-aware)."""
    def key(v):
        i = v.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7fffffff), i)
    return np.abs(key(np.asarray(a, np.float32)) - key(np.asarray(b, np.float32)))


def test_libm_erff_within_one_ulp_of_correctly_rounded():
    """or_libm_erff restates libm 0.2.16 erff (musl erff.c from FreeBSD
    s_erff.c), whose published error bound is under one ulp: on every finite
    bf16 input and on 450,000 sampled f32 inputs it is within one ulp of erf
    computed in double and rounded once."""
    rng = np.random.default_rng(5)
    b = bf16_values()
    xs = np.concatenate([b[np.isfinite(b)], rng.uniform(-7, 7, 200000),
                         rng.uniform(-1.3, 1.3, 200000),
                         np.float32(2.0) ** rng.uniform(-40, 0, 50000)]).astype(np.float32)
    xs = xs[np.isfinite(xs)]
    got = np.array([L.or_libm_erff(float(x)) for x in xs], np.float32)
    cr = np.array([math.erf(float(x)) for x in xs]).astype(np.float32)
    assert signed_ulps(got, cr).max() <= 1
    # each of the four ranges is exercised, and odd symmetry holds
    for lo, hi in ((0, 0.84375), (0.84375, 1.25), (1.25, 1 / 0.35), (1 / 0.35, 6)):
        assert np.any((np.abs(xs) >= lo) & (np.abs(xs) < hi))
    neg = np.array([L.or_libm_erff(float(-x)) for x in xs[:5000]], np.float32)
    assert np.array_equal(neg, -got[:5000])
    # special values: signed zeros, infinities, NaN, the saturated tail
    assert math.copysign(1.0, L.or_libm_erff(-0.0)) == -1.0 and L.or_libm_erff(0.0) == 0.0
    assert L.or_libm_erff(float("inf")) == 1.0 and L.or_libm_erff(float("-inf")) == -1.0
    assert math.isnan(L.or_libm_erff(float("nan")))
    assert L.or_libm_erff(6.0) == 1.0 and L.or_libm_erff(-1e30) == -1.0
    # the Erf table is that function narrowed (lut.rs:43-67)
    t = oracle.build_table(oracle.ACT_ERF, BF16)
    fin = np.isfinite(bf16_values())
    want = (np.array([L.or_libm_erff(float(x)) for x in bf16_values()], np.float32)
            .view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(t[fin], want[fin])


# ---------------------------------------------------------------- tables ----

def gelu_f64(x):
    c = math.sqrt(2.0 / math.pi)
    return 0.5 * x * (1.0 + math.tanh(c * (x + 0.044715 * x ** 3)))


def test_reference_lut_tests_hold():
    """tests/lut.rs:67-132: GELU within 0.02 + 0.02|want|, Sigmoid within 0.01."""
    tg = oracle.build_table(oracle.ACT_GELU, BF16)
    ts = oracle.build_table(oracle.ACT_SIGMOID, BF16)
    to_bits = lambda v: int(np.float32(v).view(np.uint32)) >> 16
    widen = lambda b: float((np.uint32(b) << np.uint32(16)).view(np.float32))
    for i in range(64):
        b = to_bits(i * 0.25 - 8.0)
        x, got = widen(b), widen(tg[b])
        assert abs(got - gelu_f64(x)) <= 0.02 + 0.02 * abs(gelu_f64(x))
    for i in range(48):
        b = to_bits(i * 0.4 - 9.0)
        x, got = widen(b), widen(ts[b])
        assert abs(got - 1.0 / (1.0 + math.exp(-x))) <= 0.01


@pytest.mark.parametrize("act,ref,floor", [
    (oracle.ACT_GELU, gelu_f64, 0.0),
    (oracle.ACT_SILU, lambda x: x / (1.0 + math.exp(-x)) if x > -700 else 0.0, 0.0),
    (oracle.ACT_SIGMOID, lambda x: 1.0 / (1.0 + math.exp(-x)) if x > -700 else 0.0, 0.0),
    # tanh_f = (e - 1)/(e + 1): e - 1 cancels, an absolute error of ~ulp(1)/2
    (oracle.ACT_TANH, math.tanh, 2.0 ** -23),
])
def test_tables_track_the_f64_function_on_every_finite_pattern(act, ref, floor):
    """Each bf16 entry is within one bf16 ulp (truncation) of the f64 function,
    plus the f32 rounding of the cancelling term 1 + tanh/exp (|x| * 2^-22, or
    the absolute floor of tanh's e - 1)."""
    t = oracle.build_table(act, BF16)
    xs = bf16_values()
    got = (t.astype(np.uint32) << 16).view(np.float32)
    for b in range(0, 65536, 7):
        x = float(xs[b])
        if not math.isfinite(x) or abs(x) > 80:
            continue
        want = ref(x)
        tol = abs(want) * 2.0 ** -7 + abs(x) * 2.0 ** -22 + floor + 1e-38
        assert abs(float(got[b]) - want) <= tol, (hex(b), x, float(got[b]), want)


def test_table_special_values_follow_x86_semantics():
    g = oracle.build_table(oracle.ACT_GELU, BF16)
    s = oracle.build_table(oracle.ACT_SILU, BF16)
    assert g[0xFF80] == 0xFFC0          # GELU(-Inf) = (-Inf) * 0: x86 default NaN
    assert g[0x7F80] == 0x7F80          # GELU(+Inf) = +Inf
    assert s[0x7F80] == 0x7F80 and s[0xFF80] == 0xFF80
    assert g[0x7FC1] == 0x7FC1          # quiet NaN input propagates
    assert s[0x7F81] == 0x7FC1          # signaling NaN is quieted (IEEE arithmetic on it)
    e = oracle.build_table(oracle.ACT_EXP, BF16)
    assert e[0x0000] == 0x3F80 and e[0x8000] == 0x3F80   # exp(+-0) = 1
    assert e[0x7F81] == 0x7F81          # libm returns a NaN input unchanged


# ---------------------------------------------------------------- codecs ----

def test_f16_codec_round_trip_and_rounding_rule():
    for b in range(65536):
        if (b & 0x7C00) == 0x7C00 and (b & 0x3FF):
            continue   # NaNs
        assert L.or_f32_to_f16(L.or_f16_to_f32(b)) == b
    # ties: the reference adds half an ulp and truncates (half-up), not RNE
    assert L.or_f32_to_f16(1.0 + 2.0 ** -11) == 0x3C01            # RNE would give 0x3C00
    assert L.or_f32_to_f16(70000.0) == 0x7C00                      # overflow -> Inf
    assert L.or_f32_to_f16(float("nan")) in (0x7E00, 0xFE00)
    # bf16 narrowing is truncation
    assert L.or_f32_to_bf16(float(np.float32(1.0 + 2.0 ** -8 + 2.0 ** -9))) == 0x3F80


# ---------------------------------------------------------------- KV write --

@pytest.mark.parametrize("pos,new_rows", [(0, 1), (3, 2), (4, 3), (2**32 - 1, 5), (7, 5)])
def test_kv_cache_write_ring_placement_brute_force(pos, new_rows):
    planes, bucket, row = 3, 5, 4
    rng = np.random.default_rng(pos % 1000)
    cache = rng.integers(0, 256, size=planes * bucket * row, dtype=np.uint8)
    new = rng.integers(0, 256, size=planes * new_rows * row, dtype=np.uint8)
    got = oracle.kv_cache_write(cache, new, pos, planes, bucket, new_rows, row)
    want = cache.reshape(planes, bucket, row).copy()
    for p in range(planes):
        for j in range(new_rows):
            want[p, (pos + j) % bucket] = new.reshape(planes, new_rows, row)[p, j]
    assert np.array_equal(got, want.reshape(-1))


def _widen_independently(bits, dtype):
    """bf16 = bits << 16, f16 through numpy's IEEE half, f32 as is."""
    if dtype == DTYPE_BF16:
        return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == DTYPE_F16:
        return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(bits, np.float32)


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("pos,new_rows", [(0, 1), (6, 1), (7, 1), (5, 3), (2**32 - 1, 4), (13, 8)])
def test_kv_quant_append_is_quantizer_plus_ring_placement(dtype, pos, new_rows):
    """or_kv_quant_append = the golden-pinned row quantizer (quantize_row_i8,
    simd.rs:4755-4785) applied to each new row, placed as KvCacheWrite places
    rows (kernels.rs:489-499): new row j of plane p, laid out [planes][new_rows][D],
    lands at ring row (pos + j) % bucket; every other row is untouched; an
    all-zero row writes q = 0 and scale 0 over whatever the slot held. Checked
    against a brute-force placement and against the composition of the two
    pinned oracle functions (quantizer, then kv_cache_write on bytes and scales)."""
    planes, bucket, D = 3, 8, 32
    rng = np.random.default_rng(pos % 997 + 31 * new_rows + dtype)
    x = rng.standard_normal((planes, new_rows, D)).astype(np.float32) * 4
    x[1, 0] = 0.0                                     # an all-zero row
    x[2, new_rows - 1, 5] *= 40                       # an outlier channel
    if dtype == DTYPE_BF16:
        new = (x.view(np.uint32) >> 16).astype(np.uint16)
    elif dtype == DTYPE_F16:
        new = x.astype(np.float16).view(np.uint16)
    else:
        new = x
    old_q = rng.integers(-127, 128, planes * bucket * D).astype(np.int8)
    old_s = rng.uniform(0.01, 1, planes * bucket).astype(np.float32)
    got_q, got_s = oracle.kv_quant_append(new, dtype, pos, old_q, old_s, planes, bucket, new_rows, D)
    vals = _widen_independently(new, dtype).reshape(planes, new_rows, D)
    want_q = old_q.reshape(planes, bucket, D).copy()
    want_s = old_s.reshape(planes, bucket).copy()
    rows_q = np.zeros((planes, new_rows, D), np.int8)
    rows_s = np.zeros((planes, new_rows), np.float32)
    for p in range(planes):
        for j in range(new_rows):
            q, sc = oracle.quantize_row_i8(vals[p, j])
            rows_q[p, j], rows_s[p, j] = q, sc
            want_q[p, (pos + j) % bucket] = q
            want_s[p, (pos + j) % bucket] = sc
    assert np.array_equal(got_q, want_q.ravel())
    assert np.array_equal(got_s.view(np.uint32), want_s.ravel().view(np.uint32))
    # the zero row: q = 0, scale 0, regardless of the slot's old contents
    zr = (pos + 0) % bucket
    assert np.all(got_q.reshape(planes, bucket, D)[1, zr] == 0) and got_s.reshape(planes, bucket)[1, zr] == 0
    # composition of the two pinned functions, byte for byte
    cq = oracle.kv_cache_write(old_q.view(np.uint8), rows_q.view(np.uint8).ravel(), pos, planes,
                               bucket, new_rows, D)
    cs = oracle.kv_cache_write(old_s.view(np.uint8), rows_s.view(np.uint8).ravel(), pos, planes,
                               bucket, new_rows, 4)
    assert np.array_equal(got_q.view(np.uint8), cq) and np.array_equal(got_s.view(np.uint8), cs)


def test_kv_quant_append_catches_a_placement_mistake():
    """The brute force above discriminates: placing row j at (pos - j) or
    reading the new rows [new_rows][planes] would not match."""
    planes, bucket, D, pos, nr = 2, 8, 16, 6, 3
    rng = np.random.default_rng(5)
    x = rng.standard_normal((planes, nr, D)).astype(np.float32)
    got_q, _ = oracle.kv_quant_append(x, DTYPE_F32, pos, np.zeros(planes * bucket * D, np.int8),
                                      np.zeros(planes * bucket, np.float32), planes, bucket, nr, D)
    got = got_q.reshape(planes, bucket, D)
    swapped = x.reshape(nr, planes, D)                # the transposed reading of the new rows
    q_wrong, _ = oracle.quantize_row_i8(swapped[1, 0])
    q_right, _ = oracle.quantize_row_i8(x[0, 1])
    assert np.array_equal(got[0, (pos + 1) % bucket], q_right)
    assert not np.array_equal(got[0, (pos + 1) % bucket], q_wrong)
    assert not np.array_equal(got[0, (pos - 1) % bucket], q_right)


def test_kv_cache_write_refusals():
    with pytest.raises(ValueError):
        oracle.kv_cache_write(np.zeros(8, np.uint8), np.zeros(48, np.uint8), 0, 1, 2, 3, 4)


# ---------------------------------------------------------------- attention -

def softmax_attention_f64(q, k, v, scale):
    s = (k.astype(np.float64) @ q.astype(np.float64)) / scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ v.astype(np.float64)


def test_decode_attention_matches_f64_softmax_and_gqa_map():
    rng = np.random.default_rng(0)
    B, H, Hkv, D, bucket = 2, 4, 2, 16, 37
    lens = np.array([37, 5], np.uint32)
    x = rng.standard_normal((B * Hkv, bucket, D)).astype(np.float32)
    kq, ks = oracle.kv_quant_append(x, F32, 0, np.zeros(x.size, np.int8),
                                    np.zeros(B * Hkv * bucket, np.float32), B * Hkv, bucket,
                                    bucket, D)
    y = rng.standard_normal((B * Hkv, bucket, D)).astype(np.float32)
    vq, vs = oracle.kv_quant_append(y, F32, 0, np.zeros(y.size, np.int8),
                                    np.zeros(B * Hkv * bucket, np.float32), B * Hkv, bucket,
                                    bucket, D)
    q = rng.standard_normal(B * H * D).astype(np.float32)
    scale = oracle.attn_scale(D)
    assert scale == np.float32(4.0)
    got = oracle.decode_attention_i8(q, kq, ks, vq, vs, lens, B, H, Hkv, bucket, D, scale)
    kd = oracle.dequant_i8(kq, ks, D).reshape(B * Hkv, bucket, D)
    vd = oracle.dequant_i8(vq, vs, D).reshape(B * Hkv, bucket, D)
    for b in range(B):
        for h in range(H):
            plane = b * Hkv + h // (H // Hkv)          # GQA: kv head h / group
            Lb = int(lens[b])
            want = softmax_attention_f64(q[(b * H + h) * D:(b * H + h + 1) * D],
                                         kd[plane, :Lb], vd[plane, :Lb], scale)
            np.testing.assert_allclose(got[(b * H + h) * D:(b * H + h + 1) * D], want,
                                       rtol=1e-5, atol=1e-6)


def test_decode_attention_zero_and_single_key():
    D, bucket = 8, 4
    kq = np.ones(bucket * D, np.int8)
    ks = np.ones(bucket, np.float32)
    vq = np.arange(bucket * D, dtype=np.int8)
    vs = np.full(bucket, 0.5, np.float32)
    q = np.ones(D, np.float32)
    out0 = oracle.decode_attention_i8(q, kq, ks, vq, vs, np.array([0], np.uint32), 1, 1, 1,
                                      bucket, D, 1.0)
    assert not out0.any()
    out1 = oracle.decode_attention_i8(q, kq, ks, vq, vs, np.array([1], np.uint32), 1, 1, 1,
                                      bucket, D, 1.0)
    np.testing.assert_array_equal(out1, vq[:D].astype(np.float32) * 0.5)


# ---------------------------------------------------------------- matmul ----

def test_matmul_reference_closed_forms():
    rng = np.random.default_rng(3)
    m, k = 5, 7
    a = rng.standard_normal(m * k).astype(np.float32)
    eye = np.eye(k, dtype=np.float32).reshape(-1)
    assert np.array_equal(oracle.matmul_ref_f64(a, eye, m, k, k), a)
    perm = np.eye(k, dtype=np.float32)[::-1].copy().reshape(-1)
    assert np.array_equal(oracle.matmul_ref_f64(a, perm, m, k, k),
                          a.reshape(m, k)[:, ::-1].reshape(-1))
    b = rng.standard_normal(k * 3).astype(np.float32)
    want = a.reshape(m, k).astype(np.float64) @ b.reshape(k, 3).astype(np.float64)
    np.testing.assert_allclose(oracle.matmul_ref_f64(a, b, m, k, 3),
                               want.astype(np.float32).reshape(-1), rtol=1e-6)
    assert oracle.max_rel_err(np.array([1.0, 2.0], np.float32),
                              np.array([1.0, 4.0], np.float32)) == pytest.approx(0.5)


def test_blas_f64_product_is_the_f64_reference():
    """The graph oracle's large products go through numpy's f64 BLAS: the same
    f64 products and sums as or_matmul_ref_f64, in another order, so the f32
    results agree to f64 rounding (well under one f32 ulp)."""
    rng = np.random.default_rng(17)
    m, k, n = 37, 1500, 70
    a = rng.standard_normal(m * k).astype(np.float32)
    b = rng.standard_normal(k * n).astype(np.float32)
    x = oracle.matmul_ref_f64(a, b, m, k, n)
    y = oracle.matmul_f64_blas(a, b, m, k, n)
    ulps = np.abs(x.view(np.int32).astype(np.int64) - y.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and np.mean(ulps != 0) < 0.01


# ------------------------------------------------- DecodeAttentionValid ----

def _valid_attention_f64(q, kp, vp, kn, vn, valid, b, h, hkv, m, past, new, d, scale):
    """The op's law in f64 (kernel_call.rs:691-716, float_kernels.rs:3834-3957):
    row qi of head hi sees past rows [0, min(valid, past)) then new rows
    [0, min(qi + 1, new)) of kv head hi // (h // hkv); softmax(q.k / scale) . v."""
    q = q.reshape(b, h, m, d).astype(np.float64)
    kp, vp = (x.reshape(b, hkv, past, d).astype(np.float64) for x in (kp, vp))
    kn, vn = (x.reshape(b, hkv, new, d).astype(np.float64) for x in (kn, vn))
    vis = min(valid, past)
    out = np.zeros((b, h, m, d))
    for bi in range(b):
        for hi in range(h):
            kv = hi // (h // hkv)
            for qi in range(m):
                K = np.concatenate([kp[bi, kv, :vis], kn[bi, kv, :min(qi + 1, new)]])
                V = np.concatenate([vp[bi, kv, :vis], vn[bi, kv, :min(qi + 1, new)]])
                if len(K) == 0:
                    continue
                s = K @ q[bi, hi, qi] / scale
                p = np.exp(s - s.max())
                out[bi, hi, qi] = (p / p.sum()) @ V
    return out.ravel()


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("b,h,hkv,m,past,valid,d", [
    (2, 4, 2, 1, 9, 5, 16),       # decode: a realized prefix of the bucket
    (1, 6, 3, 3, 7, 7, 8),        # chunked prefill: 3 causal new rows, GQA group 2
    (2, 2, 0, 2, 5, 99, 12),      # kv_heads 0 = heads; valid_len beyond past clamps
    (1, 4, 1, 1, 0, 0, 32),       # no past at all: the new row only
])
def test_decode_attention_valid_oracle_matches_f64_law(dtype, b, h, hkv, m, past, valid, d):
    rng = np.random.default_rng(b * 100 + h * 10 + m + d)
    hk = h if hkv == 0 else hkv
    q, kp, vp, kn, vn = (rng.standard_normal(n).astype(np.float32) for n in
                         (b * h * m * d, b * hk * past * d, b * hk * past * d,
                          b * hk * m * d, b * hk * m * d))
    if dtype == BF16:
        enc = lambda x: (x.view(np.uint32) >> 16).astype(np.uint16)
        dec = lambda u: (u.astype(np.uint32) << 16).view(np.float32)
        tol = 2 ** -7
    elif dtype == F16:
        enc = lambda x: x.astype(np.float16).view(np.uint16)
        dec = lambda u: u.view(np.float16).astype(np.float32)
        tol = 2 ** -10
    else:
        enc = dec = lambda x: x
        tol = 1e-6
    ops = [enc(x) for x in (q, kp, vp, kn, vn)]
    # unrealized past rows hold NaN: the op must never read them
    if past > min(valid, past):
        for i in (1, 2):
            t = ops[i].reshape(b, hk, past, d).copy()
            t[:, :, min(valid, past):] = enc(np.full(1, np.nan, np.float32))[0]
            ops[i] = t.ravel()
    got = dec(oracle.decode_attention_valid(*ops, valid, b, h, hkv, m, past, m, d, 0, dtype))
    want = _valid_attention_f64(*[dec(x) for x in ops[:3]], *[dec(x) for x in ops[3:]], valid,
                                b, h, hk, m, past, m, d, max(math.sqrt(d), 1.0))
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) <= tol * (np.max(np.abs(want)) + 1e-6) * 2


def test_decode_attention_valid_oracle_refusals_and_scale_bits():
    z = np.zeros(64, np.float32)
    with pytest.raises(ValueError):     # q_rows != new_len (float_kernels.rs:4205-4209)
        oracle.decode_attention_valid(z, z, z, z, z, 0, 1, 2, 2, 2, 1, 1, 4, 0, F32)
    with pytest.raises(ValueError):     # heads % kv_heads (:4216)
        oracle.decode_attention_valid(z, z, z, z, z, 0, 1, 3, 2, 1, 1, 1, 4, 0, F32)
    # scale_bits: the multiplier; a one-key row returns that key's V row exactly
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal(8).astype(np.float32) for _ in range(3))
    sb = int(np.float32(0.25).view(np.uint32))
    out = oracle.decode_attention_valid(q, z[:0], z[:0], k, v, 0, 1, 1, 1, 1, 0, 1, 8, sb, F32)
    assert np.array_equal(out, v)


def _visibility_mask(m, past, new, valid):
    """The valid form's law as an additive mask [m, past + new]: 0 on the
    realized prefix and the causal new rows, -inf elsewhere."""
    mask = np.full((m, past + new), -np.inf, np.float32)
    for qi in range(m):
        mask[qi, :min(valid, past)] = 0.0
        mask[qi, past:past + min(qi + 1, new)] = 0.0
    return mask


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("b,h,hkv,m,past,valid,d", [
    (2, 4, 2, 1, 9, 5, 16), (1, 6, 3, 3, 7, 7, 8), (2, 2, 0, 2, 5, 3, 12), (1, 4, 1, 1, 0, 0, 32)])
def test_decode_attention_mask_form_equals_valid_form(dtype, b, h, hkv, m, past, valid, d):
    """The reference's witness (tests/decode_attention_valid.rs:1-13): with
    finite bytes in the erased rows, the mask form over the mask that states
    the valid form's visibility is bit-identical to the valid form (an erased
    key's exp is exactly 0 and its context term an exact no-op)."""
    rng = np.random.default_rng(7 * b + h + m + d)
    hk = h if hkv == 0 else hkv
    raw = [rng.standard_normal(n).astype(np.float32) for n in
           (b * h * m * d, b * hk * past * d, b * hk * past * d, b * hk * m * d, b * hk * m * d)]
    if dtype == BF16:
        ops = [(x.view(np.uint32) >> 16).astype(np.uint16) for x in raw]
    elif dtype == F16:
        ops = [x.astype(np.float16).view(np.uint16) for x in raw]
    else:
        ops = raw
    mask = _visibility_mask(m, past, m, valid)
    got = oracle.decode_attention(*ops, mask, b, h, hkv, m, past, m, d, 0, dtype)
    want = oracle.decode_attention_valid(*ops, valid, b, h, hkv, m, past, m, d, 0, dtype)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def _mask_attention_f64(q, kp, vp, kn, vn, mask, b, h, hkv, m, past, new, d, scale):
    """The mask form's law in f64 (kernel_call.rs:600-656): every past row then
    every new row of kv head hi // (h // hkv), score q.k / scale + mask[qi][j],
    softmax over the finite scores; no finite score gives the zero row."""
    q = q.reshape(b, h, m, d).astype(np.float64)
    K = np.concatenate([kp.reshape(b, hkv, past, d), kn.reshape(b, hkv, new, d)], 2).astype(np.float64)
    V = np.concatenate([vp.reshape(b, hkv, past, d), vn.reshape(b, hkv, new, d)], 2).astype(np.float64)
    out = np.zeros((b, h, m, d))
    for bi in range(b):
        for hi in range(h):
            kv = hi // (h // hkv)
            for qi in range(m):
                s = K[bi, kv] @ q[bi, hi, qi] / scale + mask[qi].astype(np.float64)
                if not np.isfinite(s).any():
                    continue
                p = np.exp(s - s[np.isfinite(s)].max())
                out[bi, hi, qi] = (p / p.sum()) @ V[bi, kv]
    return out.ravel()


@pytest.mark.parametrize("b,h,hkv,m,past,new,d", [
    (2, 4, 2, 1, 9, 1, 16), (1, 6, 3, 3, 7, 2, 8), (1, 2, 1, 4, 5, 0, 12), (2, 4, 4, 2, 0, 3, 8)])
def test_decode_attention_mask_form_matches_f64_law(b, h, hkv, m, past, new, d):
    """Any q_rows / new_len pairing (decode, frozen cache, no past), a finite
    additive bias on every key plus erased (-inf) entries; one row fully
    erased, which the law pins to exact zeros."""
    rng = np.random.default_rng(b + h * 3 + m * 5 + new)
    q, kp, vp, kn, vn = (rng.standard_normal(n).astype(np.float32) for n in
                         (b * h * m * d, b * hkv * past * d, b * hkv * past * d,
                          b * hkv * new * d, b * hkv * new * d))
    L = past + new
    mask = (rng.standard_normal((m, L)) * 2).astype(np.float32)
    mask[rng.random((m, L)) < 0.3] = -np.inf
    mask[0, :] = -np.inf
    got = oracle.decode_attention(q, kp, vp, kn, vn, mask, b, h, hkv, m, past, new, d, 0, F32)
    want = _mask_attention_f64(q, kp, vp, kn, vn, mask, b, h, hkv, m, past, new, d,
                               max(math.sqrt(d), 1.0))
    assert np.max(np.abs(got - want)) <= 1e-6 * (np.max(np.abs(want)) + 1e-6) * 4
    rows = got.reshape(b, h, m, d)
    assert np.array_equal(rows[:, :, 0], np.zeros_like(rows[:, :, 0]))


def test_decode_attention_mask_form_split_and_padding_witnesses():
    """The reference's witnesses for the mask form (tests/decode_attention.rs:
    1-18), bit for bit on the oracle: keys split past || new equal the same
    keys precatenated as past; and a bucket padded with finite rows the mask
    erases (-inf) equals the tight call over the realized rows only."""
    rng = np.random.default_rng(21)
    b, h, hkv, m, d = 2, 4, 2, 3, 16
    past, new, pad = 11, 3, 9
    q = rng.standard_normal(b * h * m * d).astype(np.float32)
    kp, vp = (rng.standard_normal((b, hkv, past, d)).astype(np.float32) for _ in range(2))
    kn, vn = (rng.standard_normal((b, hkv, new, d)).astype(np.float32) for _ in range(2))
    mask = (rng.standard_normal((m, past + new)) * 0.5).astype(np.float32)
    mask[rng.random((m, past + new)) < 0.25] = -np.inf
    split = oracle.decode_attention(q, kp.ravel(), vp.ravel(), kn.ravel(), vn.ravel(), mask, b, h,
                                    hkv, m, past, new, d, 0, F32)
    kc = np.concatenate([kp, kn], 2).ravel()
    vc = np.concatenate([vp, vn], 2).ravel()
    cat = oracle.decode_attention(q, kc, vc, kc[:0], vc[:0], mask, b, h, hkv, m, past + new, 0,
                                  d, 0, F32)
    assert np.array_equal(split.view(np.uint32), cat.view(np.uint32))
    # padded bucket: pad extra finite past rows, erased by -inf in the mask
    kpad = np.concatenate([kp, rng.standard_normal((b, hkv, pad, d)).astype(np.float32)], 2)
    vpad = np.concatenate([vp, rng.standard_normal((b, hkv, pad, d)).astype(np.float32)], 2)
    mpad = np.concatenate([mask[:, :past], np.full((m, pad), -np.inf, np.float32),
                           mask[:, past:]], 1)
    padded = oracle.decode_attention(q, kpad.ravel(), vpad.ravel(), kn.ravel(), vn.ravel(), mpad,
                                     b, h, hkv, m, past + pad, new, d, 0, F32)
    assert np.array_equal(padded.view(np.uint32), split.view(np.uint32))


def test_decode_attention_mask_form_reads_every_row_and_refuses():
    """The mask form reads the erased rows (a NaN in an erased V row reaches
    the output through 0 * NaN, kernel_call.rs:682-685), and refuses an empty
    key list, a kv_heads that does not divide heads, and integer dtypes."""
    d = 8
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal(n).astype(np.float32) for n in (d, 2 * d, 2 * d))
    v[d:] = np.nan
    mask = np.array([[0.0, -np.inf]], np.float32)
    out = oracle.decode_attention(q, k, v, k[:0], v[:0], mask, 1, 1, 1, 1, 2, 0, d, 0, F32)
    assert np.isnan(out).all()
    v[d:] = 0.5
    out = oracle.decode_attention(q, k, v, k[:0], v[:0], mask, 1, 1, 1, 1, 2, 0, d, 0, F32)
    assert np.array_equal(out, v[:d])
    z = np.zeros(64, np.float32)
    with pytest.raises(ValueError):
        oracle.decode_attention(z, z, z, z, z, z, 1, 2, 2, 1, 0, 0, 4, 0, F32)
    with pytest.raises(ValueError):
        oracle.decode_attention(z, z, z, z, z, z, 1, 3, 2, 1, 1, 1, 4, 0, F32)
    with pytest.raises(ValueError):
        oracle.decode_attention(z, z, z, z, z, z, 1, 2, 2, 1, 1, 1, 4, 0, 2)


@pytest.mark.parametrize("k,n", [(1, 1), (3, 16), (5, 17), (7, 40), (64, 100)])
def test_panel_packing_follows_the_layout_formula(k, n):
    """layout.rs:16-45, element by element: packed[(p*k + kk)*16 + c] is
    b[kk*n + p*16 + c], zero where p*16 + c >= n; packed_len = ceil(n/16)*k*16;
    unpacking returns the weight."""
    b = np.arange(1, k * n + 1, dtype=np.float32)
    pk = oracle.pack_b_panels(b, k, n)
    assert pk.size == oracle.packed_len(k, n) == -(-n // 16) * k * 16
    for p in range(-(-n // 16)):
        for kk in range(k):
            for c in range(16):
                want = b[kk * n + p * 16 + c] if p * 16 + c < n else 0.0
                assert pk[(p * k + kk) * 16 + c] == want
    assert np.array_equal(oracle.unpack_b_panels(pk, k, n), b)


def test_relu_elu_selu_exp_closed_forms():
    """relu_f / elu_f / selu_f / exp_f (float_kernels.rs:3448, 3641-3656,
    3498-3500) in the oracle against f64 closed forms on a dense sweep, and
    their special values: relu(NaN) = relu(-0) = +0, elu(-inf) = -1,
    selu(+inf) = +inf, elu and selu continuous at 0."""
    x = np.concatenate([np.linspace(-30, 30, 20001), [-0.0, 0.0, 1e-30, -1e-30]]).astype(np.float32)
    f = lambda act: oracle.fused_act_f32(act, x).astype(np.float64)
    x64 = x.astype(np.float64)
    assert np.array_equal(f(1), np.maximum(x64, 0.0))
    elu = np.where(x64 >= 0, x64, np.expm1(x64))
    assert np.max(np.abs(f(6) - elu)) <= 2e-7
    a, s = float(np.float32(1.6732632)), float(np.float32(1.050701))
    selu = np.where(x64 >= 0, s * x64, s * a * np.expm1(x64))
    assert np.max(np.abs(f(7) - selu)) <= 5e-7 * np.maximum(1, np.abs(selu)).max()
    e = f(8)
    assert np.max(np.abs(e - np.exp(x64)) / np.exp(x64)) <= 2 ** -23
    sp = np.array([np.nan, -0.0, -np.inf, np.inf], np.float32)
    r = oracle.fused_act_f32(1, sp)
    assert r[0] == 0 and r[1] == 0 and not np.signbit(r[0]) and not np.signbit(r[1])
    assert oracle.fused_act_f32(6, sp)[2] == -1.0
    assert oracle.fused_act_f32(7, sp)[3] == np.inf
