"""`.holo` archives on the host: BLAKE3, the writer, the library's reader
(dry session load) and the oracle's independent reader, and the wire codec
of the decode-step ops (crates/hologram-archive/src/{writer,loader,
kernel_codec,constant_codec}.rs). No GPU needed."""
import struct

import numpy as np
import pytest

from hologram_amd import (DTYPE_BF16, DTYPE_F32, DTYPE_I32, ArgMaxCall, BinaryCall, BufferRef,
                          DecodeAttentionValidCall,
                          ConstantEntry, GatherCall, HipSession, HoloWriter, KernelCall,
                          MatMulCall, NormCall, PortDescriptor, RoPECall, UnsupportedOp,
                          DispatchError, SlotOutOfRange, blake3, decode_call, validate)
from hologram_amd.decoder_graph import DecoderConfig, build_decode_step, init_weights
from hologram_amd.session import NO_EPILOGUE_FUSION
from oracle.blake3_ref import blake3 as blake3_py
from oracle.graph import OracleSession

# Known-answer vectors of the BLAKE3 specification (default hash, 32 bytes):
# the empty input, "abc", and the official test-vector inputs (byte i = i % 251)
# of lengths 1, 1024 (one full chunk), 1025 and 2048 (two chunks).
KAT = {
    b"": "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262",
    b"abc": "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85",
}
KAT_TV = {
    1: "2d3adedff11b61f14c886e35afa036736dcd87a74d27b5c1510225d0f592e213",
    1024: "42214739f095a406f3fc83deb889744ac00df831c10daa55189b5d121c855af7",
    1025: "d00278ae47eb27b34faecf67b4fe263f82d5412916c1ffd97c8cb7fb814b8444",
    2048: "e776b6028c7cd22a4d0ba182a8bf62205d2ef576467e838ed6f2529b85fba24a",
}


def tv(n):
    return bytes((np.arange(n) % 251).astype(np.uint8))


def test_blake3_known_answers():
    for msg, hexd in KAT.items():
        assert blake3(msg).hex() == hexd and blake3_py(msg).hex() == hexd
    for n, hexd in KAT_TV.items():
        assert blake3(tv(n)).hex() == hexd and blake3_py(tv(n)).hex() == hexd


def test_blake3_tree_fold_matches_recursive_definition():
    """The library folds chunk values with the incremental stack (and threads);
    the restatement uses the recursive left-complete tree. Lengths cover 1..17
    chunks and a deep tree; a one-byte change flips the digest."""
    rng = np.random.default_rng(3)
    for n in list(range(0, 64 * 1024 + 1, 1024 - 7)) + [1023, 3073, 8193, 100003]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert blake3(data) == blake3_py(data), n
    big = rng.integers(0, 256, (4 << 20) + 1000, dtype=np.uint8)   # threaded path
    digest = blake3(big)
    assert digest == blake3_py(big.tobytes())
    big[123457] ^= 1
    assert blake3(big) != digest


def small_archive():
    w = HoloWriter()
    w.inputs = [PortDescriptor("a", 0, 16, DTYPE_F32, [16])]
    w.outputs = [PortDescriptor("out", 2, 16, DTYPE_F32, [16])]
    body = np.arange(16, dtype=np.float32).tobytes()
    w.constants = [ConstantEntry(1, DTYPE_F32, body, by_reference=True),
                   ConstantEntry(3, DTYPE_F32, body, by_reference=False)]
    w.kernel_calls = [KernelCall.Add(BinaryCall(BufferRef(0, 0, 64), BufferRef(1, 0, 64),
                                                BufferRef(2, 0, 64), 16, 32, DTYPE_F32))]
    w.exec_plan = [[0]]
    return w.finish()


def test_writer_layout_and_footer():
    a = small_archive()
    assert a[:4] == b"HOLO" and struct.unpack_from("<HHH", a, 4)[0] == 3
    assert blake3(a[:-32]) == a[-32:]
    o = OracleSession(a)
    assert [p["name"] for p in o.inputs] == ["a"] and o.outputs[0]["slot"] == 2
    assert o.plan == [[0]] and o.calls[0][0] == 5
    s = HipSession(None, a)                       # the library's reader, dry
    assert len(s.inputs) == 1 and s.outputs[0].slot == 2 and s.n_calls == 1
    assert s.fingerprint() == a[-32:]
    bad = bytearray(a)
    bad[40] ^= 1
    with pytest.raises(DispatchError):
        HipSession(None, bytes(bad))
    with pytest.raises(ValueError):
        OracleSession(bytes(bad))


def test_weights_are_deduplicated_and_checked():
    w = HoloWriter()
    body = bytes(range(256))
    w.constants = [ConstantEntry(0, DTYPE_F32, body), ConstantEntry(1, DTYPE_F32, body)]
    w.kernel_calls = [KernelCall.Add(BinaryCall(BufferRef(0, 0, 256), BufferRef(1, 0, 256),
                                                BufferRef(2, 0, 256), 64, 32, DTYPE_F32))]
    a = w.finish()
    assert a.count(body) == 1                    # one Weights entry for both constants
    HipSession(None, a)
    # corrupt the weight body and re-seal the footer: the fingerprint check refuses
    bad = bytearray(a[:-32])
    i = bytes(bad).index(body)
    bad[i] ^= 0xFF
    with pytest.raises(DispatchError):
        HipSession(None, bytes(bad) + blake3(bytes(bad)))


def test_dry_session_refuses_execute():
    s = HipSession(None, small_archive())
    from hologram_amd import InitError
    with pytest.raises(InitError):
        s.run()


def decode_step_cfg():
    return DecoderConfig(layers=2, hidden=128, heads=4, kv_heads=2, head_dim=64, ffn=256,
                         vocab=300, batch=2, bucket=64)


def test_decoder_archive_loads_dry_with_in_place_caches():
    cfg = decode_step_cfg()
    a = build_decode_step(cfg, init_weights(cfg, seed=1))
    s = HipSession(None, a)
    assert len(s.inputs) == 7 + 4 * cfg.layers and len(s.outputs) == 2 + 4 * cfg.layers
    o = OracleSession(a)
    assert len(o.calls) == 1 + 18 * cfg.layers + 3
    assert HipSession(None, a, flags=NO_EPILOGUE_FUSION).n_calls == len(o.calls)


@pytest.mark.parametrize("call", [
    KernelCall.DecodeAttentionValid(DecodeAttentionValidCall(
        *[BufferRef(i, 4 * i, 0) for i in range(7)], 2, 32, 8, 1, 4096, 1, 128, 0x3E000000,
        DTYPE_BF16)),
    KernelCall.Add(BinaryCall(BufferRef(1, 8, 24), BufferRef(2), BufferRef(3), 7, 16, DTYPE_BF16)),
    KernelCall.Mul(BinaryCall(BufferRef(1), BufferRef(2), BufferRef(3), 9, 32, DTYPE_F32)),
    KernelCall.RmsNorm(NormCall(BufferRef(1), BufferRef(2), BufferRef(3), 4, 64, 0x3727C5AC,
                                DTYPE_BF16)),
    KernelCall.RotaryEmbedding(RoPECall(BufferRef(1), BufferRef(2), BufferRef(3), BufferRef(4),
                                        64, 640, DTYPE_BF16)),
    KernelCall.Gather(GatherCall(BufferRef(1), BufferRef(2), BufferRef(3), 1, 300, 128, 2,
                                 DTYPE_I32, DTYPE_BF16)),
    KernelCall.ArgMax(ArgMaxCall(BufferRef(1), BufferRef(2), 2, 300, DTYPE_BF16)),
])
def test_wire_codec_round_trip(call):
    wire = call.encode()
    c, used = decode_call(wire + b"\xAA\xBB")
    assert used == len(wire) and c.tag == call.tag
    kc = call.to_c()
    assert bytes(c) == bytes(kc)


def test_decode_step_refusals():
    sizes = [1 << 20] * 8
    with pytest.raises(UnsupportedOp):           # odd head_dim (float_kernels.rs:3126-3131)
        validate(KernelCall.RotaryEmbedding(RoPECall(BufferRef(1), BufferRef(2), BufferRef(3),
                                                     BufferRef(4), 63, 630, DTYPE_BF16)), sizes)
    with pytest.raises(UnsupportedOp):           # negative epsilon (:1324-1336)
        validate(KernelCall.RmsNorm(NormCall(BufferRef(1), BufferRef(2), BufferRef(3), 1, 8,
                                             0xBF800000, DTYPE_F32)), sizes)
    with pytest.raises(SlotOutOfRange):          # index dtype (kernels.rs:399-403)
        validate(KernelCall.Gather(GatherCall(BufferRef(1), BufferRef(2), BufferRef(3), 1, 10, 4,
                                              2, 8, DTYPE_F32)), sizes)
    with pytest.raises(SlotOutOfRange):          # output overlaps an input
        validate(KernelCall.Add(BinaryCall(BufferRef(1), BufferRef(2), BufferRef(1), 8, 32,
                                           DTYPE_F32)), sizes)
    with pytest.raises(SlotOutOfRange):          # short operand
        validate(KernelCall.MatMul(MatMulCall(BufferRef(1, 0, 64), BufferRef(2), BufferRef(3),
                                              8, 8, 8, DTYPE_F32)), sizes)


def _one_add_archive(out_slot=2, in_port_slot=0, const_slot=1):
    w = HoloWriter()
    w.inputs = [PortDescriptor("a", in_port_slot, 16, DTYPE_F32, [16])]
    w.outputs = [PortDescriptor("out", 2, 16, DTYPE_F32, [16])]
    w.constants = [ConstantEntry(const_slot, DTYPE_F32, np.arange(16, dtype=np.float32).tobytes())]
    w.kernel_calls = [KernelCall.Add(BinaryCall(BufferRef(0, 0, 64), BufferRef(1, 0, 64),
                                                BufferRef(out_slot, 0, 64), 16, 32, DTYPE_F32))]
    w.exec_plan = [[0]]
    return w.finish()


ABSENT = 0xFFFFFFFF


@pytest.mark.parametrize("where", ["output", "port", "constant"])
def test_dry_load_refuses_the_absent_slot(where):
    """Slot ids from the archive index host tables at load: an absent write
    operand, port or constant is a malformed archive and comes back as an
    error, never as an out-of-range index."""
    kw = {"output": dict(out_slot=ABSENT), "port": dict(in_port_slot=ABSENT),
          "constant": dict(const_slot=ABSENT)}[where]
    HipSession(None, _one_add_archive())          # the well-formed twin loads
    with pytest.raises(SlotOutOfRange):
        HipSession(None, _one_add_archive(**kw))


def test_view_length_past_the_slot_saturates():
    """buf_range clamps the end of a view to its slot (buffer.rs:312-335). A
    length near 2^64 must clamp, not wrap round to a huge view that passes the
    size check: 16 f32 at offset 8 of a 64-byte slot have only 56 bytes."""
    sizes = [64] * 4
    call = KernelCall.Add(BinaryCall(BufferRef(1, 8, (1 << 64) - 4), BufferRef(2), BufferRef(3),
                                     16, 32, DTYPE_F32))
    with pytest.raises(SlotOutOfRange):
        validate(call, sizes)
    ok = KernelCall.Add(BinaryCall(BufferRef(1, 8, (1 << 64) - 4), BufferRef(2), BufferRef(3),
                                   14, 32, DTYPE_F32))
    validate(ok, sizes)                           # 14 f32 = 56 bytes fit


def test_decode_attention_valid_refusals():
    """decode_attention_valid_float's refusals (float_kernels.rs:4199-4240)."""
    sizes = [1 << 20] * 8
    mk = lambda m, new, h=4, hkv=2, q_len=0, dtype=DTYPE_BF16: KernelCall.DecodeAttentionValid(
        DecodeAttentionValidCall(BufferRef(0, 0, q_len), *[BufferRef(i) for i in range(1, 7)], 1,
                                 h, hkv, m, 64, new, 64, 0, dtype))
    validate(mk(1, 1), sizes)
    with pytest.raises(UnsupportedOp):
        validate(mk(2, 1), sizes)                # q_rows != new_len
    with pytest.raises(UnsupportedOp):
        validate(mk(0, 0), sizes)                # q_rows == 0
    with pytest.raises(UnsupportedOp):
        validate(mk(1, 1, h=6, hkv=4), sizes)    # heads % kv_heads
    with pytest.raises(UnsupportedOp):
        validate(mk(1, 1, dtype=2), sizes)       # int8 is no compute dtype here
    with pytest.raises(SlotOutOfRange):
        validate(mk(1, 1, q_len=16), sizes)      # q shorter than 4 x 64 bf16


GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def kappa_of(data: bytes) -> str:
    """address_bytes (address.rs:96-99): blake3:<lowercase hex digest>."""
    return "blake3:" + blake3(data).hex()


def test_reference_compiled_fixture_loads_and_labels():
    """The reference compiler's own archive (tests/golden/README.md): the
    library's reader verifies its BLAKE3 footer and loads it dry; the oracle
    walk's output carries the κ the reference's engine recorded."""
    arch = (GOLDEN / "reference_fixture.holo").read_bytes()
    want = (GOLDEN / "reference_fixture.kappa").read_text().strip()
    s = HipSession(None, arch)
    assert s.fingerprint() == arch[-32:] == blake3(arch[:-32])
    assert len(s.outputs) == 1 and s.outputs[0].dtype == DTYPE_F32
    o = OracleSession(arch)
    o.run()
    assert kappa_of(o.output(0).tobytes()) == want
