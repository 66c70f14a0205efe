"""CPU tests of the prompt pass (prefill), with no device.

Two new pieces of oracle are pinned here:
- Transpose (transpose_float, src/cpu/float_kernels.rs:2980-3028), against a
  brute-force restatement of the reference's coordinate loop.
- The multi-row int8 attention (op 125), against the reference's multi-row
  DecodeAttentionValid restated in the C oracle
  (or_decode_attention_valid_f32: new rows causal, float_kernels.rs:3899-3957)
  on the dequantized cache.

Also covered: the wire codec and refusals of both ops, and the prompt-pass
archive (dry load, ports, call counts).
"""
import itertools

import numpy as np
import pytest

import oracle
from hologram_amd import (DTYPE_BF16, DTYPE_F32, AttentionI8RowsCall, BufferRef,
                          DecodeAttentionI8Call, HipSession, KernelCall, SlotOutOfRange,
                          TransposeCall, UnsupportedOp, decode_call, validate)
from hologram_amd.decoder_graph import DecoderConfig, build_prefill, init_weights


def transpose_loop(x, dims, perm):
    """The reference loop: decompose each output index over the permuted extents,
    gather from the input position (float_kernels.rs:3006-3025)."""
    rank = len(dims)
    in_strides = [int(np.prod(dims[i + 1:])) for i in range(rank)]
    out_dims = [dims[perm[i]] for i in range(rank)]
    out = np.empty_like(x)
    for o in range(x.size):
        rem, coord = o, [0] * rank
        for i in reversed(range(rank)):
            coord[i] = rem % out_dims[i]
            rem //= out_dims[i]
        out[o] = x[sum(coord[i] * in_strides[perm[i]] for i in range(rank))]
    return out


@pytest.mark.parametrize("dims", [(2, 3, 4, 5), (3, 1, 7), (6,), (2, 2, 2, 2, 2, 3)])
def test_transpose_oracle_matches_reference_loop(dims):
    x = np.arange(int(np.prod(dims)), dtype=np.uint16)
    for perm in itertools.islice(itertools.permutations(range(len(dims))), 12):
        assert np.array_equal(oracle.transpose(x, dims, perm), transpose_loop(x, dims, perm)), perm


def make_cache(rng, planes, bucket, D):
    x = rng.standard_normal((planes, bucket, D)).astype(np.float32)
    cq = np.zeros(planes * bucket * D, np.int8)
    cs = np.zeros(planes * bucket, np.float32)
    return oracle.kv_quant_append(x, DTYPE_F32, 0, cq, cs, planes, bucket, bucket, D)


def test_attention_rows_oracle_is_the_valid_form():
    """Row t of a T-row prompt over a cache of lens[b] rows equals the reference's
    DecodeAttentionValid with past = lens[b] - T and the last T rows as new rows."""
    rng = np.random.default_rng(3)
    B, T, H, Hkv, D, S = 2, 5, 4, 2, 64, 32
    kq, ks = make_cache(rng, B * Hkv, S, D)
    vq, vs = make_cache(rng, B * Hkv, S, D)
    lens = np.array([5, 23], np.uint32)
    q = rng.standard_normal(B * T * H * D).astype(np.float32)
    scale = oracle.attn_scale(D)
    got = oracle.attention_i8_rows(q, kq, ks, vq, vs, lens, B, T, H, Hkv, S, D, scale)
    got = got.reshape(B, T, H, D)
    kd = np.zeros(B * Hkv * S * D, np.float32)
    vd = np.zeros_like(kd)
    oracle.lib().or_dequant_i8(oracle._p(kq), oracle._p(ks), oracle._p(kd), B * Hkv * S, D)
    oracle.lib().or_dequant_i8(oracle._p(vq), oracle._p(vs), oracle._p(vd), B * Hkv * S, D)
    kd, vd = kd.reshape(B, Hkv, S, D), vd.reshape(B, Hkv, S, D)
    for b in range(B):
        L = int(lens[b])
        past = L - T
        qb = np.ascontiguousarray(q.reshape(B, T, H, D)[b].transpose(1, 0, 2))   # [H, M, D]
        want = oracle.decode_attention_valid_f32(
            qb, np.ascontiguousarray(kd[b, :, :past]), np.ascontiguousarray(vd[b, :, :past]),
            np.ascontiguousarray(kd[b, :, past:L]), np.ascontiguousarray(vd[b, :, past:L]),
            1, H, Hkv, T, past, T, D, scale, past).reshape(H, T, D).transpose(1, 0, 2)
        assert np.allclose(got[b], want, rtol=1e-5, atol=1e-6), b


def test_attention_rows_oracle_brute_force_causal():
    """Brute force in f64 over the dequantized, unwrapped positions: row t of a
    T-row prompt ending at position lens[b] - 1 attends to positions
    0 .. lens[b] - T + t, nothing later; a wrapped ring (lens > bucket) is refused."""
    rng = np.random.default_rng(8)
    B, T, H, Hkv, D, S = 2, 4, 4, 2, 64, 16
    kq, ks = make_cache(rng, B * Hkv, S, D)
    vq, vs = make_cache(rng, B * Hkv, S, D)
    lens = np.array([16, 9], np.uint32)           # a full bucket and a partial one
    q = rng.standard_normal(B * T * H * D).astype(np.float32)
    scale = oracle.attn_scale(D)
    got = oracle.attention_i8_rows(q, kq, ks, vq, vs, lens, B, T, H, Hkv, S, D, scale)
    got = got.reshape(B, T, H, D)
    kd = (kq.reshape(B, Hkv, S, D).astype(np.float64) * ks.reshape(B, Hkv, S, 1))
    vd = (vq.reshape(B, Hkv, S, D).astype(np.float64) * vs.reshape(B, Hkv, S, 1))
    qq = q.reshape(B, T, H, D).astype(np.float64)
    for b in range(B):
        for t in range(T):
            last = int(lens[b]) - T + t           # the row's own position
            for h in range(H):
                kv = h // (H // Hkv)
                s_ = kd[b, kv, :last + 1] @ qq[b, t, h] / scale
                p = np.exp(s_ - s_.max())
                want = (p / p.sum()) @ vd[b, kv, :last + 1]
                assert np.allclose(got[b, t, h], want, rtol=1e-4, atol=1e-5), (b, t, h)
    with pytest.raises(ValueError):
        oracle.attention_i8_rows(q, kq, ks, vq, vs, np.array([17, 9], np.uint32), B, T, H, Hkv,
                                 S, D, scale)


def test_attention_rows_short_sequence_rows_are_zero():
    rng = np.random.default_rng(4)
    B, T, H, Hkv, D, S = 1, 6, 2, 1, 64, 16
    kq, ks = make_cache(rng, B * Hkv, S, D)
    vq, vs = make_cache(rng, B * Hkv, S, D)
    q = rng.standard_normal(B * T * H * D).astype(np.float32)
    got = oracle.attention_i8_rows(q, kq, ks, vq, vs, np.array([3], np.uint32), B, T, H, Hkv, S,
                                   D, oracle.attn_scale(D)).reshape(T, H, D)
    assert np.all(got[:3] == 0) and np.all(np.abs(got[3:]).sum(axis=(1, 2)) > 0)


@pytest.mark.parametrize("call", [
    KernelCall.Transpose(TransposeCall(BufferRef(1, 8, 96), BufferRef(2), (2, 3, 4), (2, 0, 1),
                                       DTYPE_F32)),
    KernelCall.AttentionI8Rows(AttentionI8RowsCall(DecodeAttentionI8Call(
        *[BufferRef(i) for i in range(7)], 8, 32, 8, 1024, 64, 0, DTYPE_BF16), 512)),
])
def test_codec_round_trip(call):
    wire = call.encode()
    kc, used = decode_call(wire + b"\x07")
    assert used == len(wire) and kc.tag == call.tag
    assert bytes(kc) == bytes(call.to_c())


def test_refusals():
    sizes = [1 << 20] * 10
    with pytest.raises(UnsupportedOp):       # not a permutation
        validate(KernelCall.Transpose(TransposeCall(BufferRef(1), BufferRef(2), (2, 3), (0, 0))),
                 sizes)
    with pytest.raises(UnsupportedOp):       # rank 0 (rank must be 1..=8)
        validate(KernelCall.Transpose(TransposeCall(BufferRef(1), BufferRef(2), (), ())), sizes)
    with pytest.raises(SlotOutOfRange):      # short input
        validate(KernelCall.Transpose(TransposeCall(BufferRef(1, 0, 10), BufferRef(2), (4, 4),
                                                    (1, 0))), sizes)
    attn = DecodeAttentionI8Call(*[BufferRef(i) for i in range(7)], 2, 8, 2, 64, 64, 0, DTYPE_BF16)
    with pytest.raises(UnsupportedOp):       # no rows
        validate(KernelCall.AttentionI8Rows(AttentionI8RowsCall(attn, 0)), sizes)
    with pytest.raises(UnsupportedOp):       # grid rows above 65535
        validate(KernelCall.AttentionI8Rows(AttentionI8RowsCall(attn, 40000)),
                 [1 << 34] * 10)
    validate(KernelCall.AttentionI8Rows(AttentionI8RowsCall(attn, 16)), sizes)


def test_prefill_archive_loads_dry():
    cfg = DecoderConfig(layers=2, hidden=128, heads=4, kv_heads=2, head_dim=64, ffn=256,
                        vocab=304, batch=2, bucket=64)
    a = build_prefill(cfg, init_weights(cfg, seed=2), 16)
    s = HipSession(None, a)
    assert [p.element_count for p in s.inputs[:3]] == [2 * 16, 1, 2]
    assert len(s.outputs) == 2 + 4 * cfg.layers
    # per layer 18 calls + 2 transposes, minus the loader's three fusions; then
    # gather, last-row gather, norm, head, argmax
    assert s.n_calls == 1 + 17 * cfg.layers + 4
    with pytest.raises(ValueError):
        build_prefill(cfg, init_weights(cfg, seed=2), 1)
