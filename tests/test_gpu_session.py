"""GPU parity of the decode-step ops and of the `.holo` session walk.

Ops (vs the C oracle, oracle/holo_oracle.c): Add, Mul, RoPE, Gather and
ArgMax bit-exact; RmsNorm and AddRmsNorm within 1e-2 (bf16) / 1e-5 (f32)
normalized error (the sum of squares is a tree here, sequential in the
reference).
Session (vs oracle/graph.py, the reference walk over the same archive on the
CPU): a small Llama-style decoder stepped several tokens. Every op of the walk
narrows to bf16 by truncation, so a value near a bf16 boundary can land one ulp
(2^-8 relative) apart in the two walks, and those flips compound through the
layers: the logits bound is 2e-2 normalized max error per step (the per-op bf16
bound, 1e-2, composed over the two layers and the head), with the mean error
held to 2e-3 so a systematic error cannot hide under it; greedy tokens are
equal up to near-ties.
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_I32, DTYPE_I64, ArgMaxCall, BinaryCall,
                          BufferRef, DeviceWorkspace, DispatchError, GatherCall, HipSession,
                          KernelCall, NormCall, RoPECall, SlotOutOfRange)
from hologram_amd.decoder_graph import (DecoderConfig, build_decode_step, f32_bits,
                                        init_weights, rope_tables)
from oracle import _p, lib
from oracle.graph import OracleSession

pytestmark = pytest.mark.gpu


def bf(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def unbf(b):
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)


def run(torch, backend, call, arrays, out_bytes, out_slot):
    ws = DeviceWorkspace()
    keep = []
    for s, a in arrays.items():
        t = to_dev(torch, a)
        keep.append(t)
        ws.bind(s, t)
    out = torch.zeros(out_bytes, dtype=torch.uint8, device="cuda")
    ws.bind(out_slot, out)
    backend.dispatch(call, ws)
    backend.synchronize()
    return out.cpu().numpy()


def enc16(x32, dtype):
    """f32 values as the operand dtype's array: bf16 / f16 bits, or f32."""
    if dtype == DTYPE_BF16:
        return bf(x32)
    if dtype == DTYPE_F16:
        return np.asarray(x32, np.float32).astype(np.float16).view(np.uint16)
    return np.asarray(x32, np.float32)


def dec16(raw, dtype):
    """Output bytes of the dtype as f32 values."""
    if dtype == DTYPE_BF16:
        return unbf(raw.view(np.uint16))
    if dtype == DTYPE_F16:
        return raw.view(np.float16).astype(np.float32)
    return raw.view(np.float32)


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_add_mul_bit_exact(torch_cuda, backend, dtype, n):
    rng = np.random.default_rng(n)
    a32 = (rng.standard_normal(n) * 5).astype(np.float32)
    b32 = (rng.standard_normal(n) * 5).astype(np.float32)
    a, b = enc16(a32, dtype), enc16(b32, dtype)
    es = a.itemsize
    for tag, op in ((KernelCall.Add, 0), (KernelCall.Mul, 1)):
        # an offset view of slot 1 exercises the unaligned path
        a_pad = np.concatenate([np.zeros(1, a.dtype), a])
        call = tag(BinaryCall(BufferRef(1, es, n * es), BufferRef(2), BufferRef(3), n, 16, dtype))
        got = run(torch_cuda, backend, call, {1: a_pad, 2: b}, n * es, 3)
        want = np.zeros(n * es, np.uint8)
        lib().or_binary(op, _p(a), _p(b), _p(want), n, dtype)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,tol", [(DTYPE_BF16, 1e-2), (DTYPE_F16, 1e-2), (DTYPE_F32, 1e-5)])
@pytest.mark.parametrize("batch,feature", [(1, 64), (8, 2048), (3, 1000)])
def test_rms_norm(torch_cuda, backend, dtype, tol, batch, feature):
    rng = np.random.default_rng(feature)
    x32 = rng.standard_normal((batch, feature)).astype(np.float32) * 3
    g32 = rng.standard_normal(feature).astype(np.float32)
    x, g = enc16(x32, dtype), enc16(g32, dtype)
    es = x.itemsize
    eps = f32_bits(1e-5)
    for with_g in (True, False):
        gref = BufferRef(2) if with_g else BufferRef(0xFFFFFFFF)
        call = KernelCall.RmsNorm(NormCall(BufferRef(1), gref, BufferRef(3), batch, feature, eps,
                                           dtype))
        got = run(torch_cuda, backend, call, {1: x, 2: g}, x.size * es, 3)
        want = np.zeros(x.size * es, np.uint8)
        lib().or_rms_norm(_p(x), _p(g) if with_g else None, _p(want), batch, feature, eps, dtype)
        got_f, want_f = dec16(got, dtype), dec16(want, dtype)
        assert oracle.max_rel_err(got_f, want_f) <= tol


@pytest.mark.parametrize("dtype,tol", [(DTYPE_BF16, 1e-2), (DTYPE_F16, 1e-2), (DTYPE_F32, 1e-5)])
@pytest.mark.parametrize("batch,feature", [(1, 64), (8, 2048), (3, 1000)])
def test_add_rms_norm(torch_cuda, backend, dtype, tol, batch, feature):
    """AddRmsNorm (54): rms_norm(x + residual), the sum in f32; with and
    without the residual and gamma, against or_add_rms_norm."""
    rng = np.random.default_rng(feature + 1)
    x32 = rng.standard_normal((batch, feature)).astype(np.float32) * 3
    r32 = rng.standard_normal((batch, feature)).astype(np.float32)
    g32 = rng.standard_normal(feature).astype(np.float32)
    x, r, g = enc16(x32, dtype), enc16(r32, dtype), enc16(g32, dtype)
    es = x.itemsize
    eps = f32_bits(1e-5)
    absent = BufferRef(0xFFFFFFFF)
    for with_r in (True, False):
        for with_g in (True, False):
            call = KernelCall.AddRmsNorm(NormCall(
                BufferRef(1), BufferRef(2) if with_g else absent, BufferRef(3), batch, feature,
                eps, dtype, residual=BufferRef(4) if with_r else absent))
            got = run(torch_cuda, backend, call, {1: x, 2: g, 4: r}, x.size * es, 3)
            want = np.zeros(x.size * es, np.uint8)
            lib().or_add_rms_norm(_p(x), _p(r) if with_r else None, _p(g) if with_g else None,
                                  _p(want), batch, feature, eps, dtype)
            got_f, want_f = dec16(got, dtype), dec16(want, dtype)
            assert oracle.max_rel_err(got_f, want_f) <= tol, (with_r, with_g)


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("heads,D", [(37, 64), (5, 40), (80000, 128)])
def test_rope_bit_exact(torch_cuda, backend, dtype, heads, D):
    """bf16 with head_dim a multiple of 16 takes the eight-a-lane kernel (the
    largest case also its grid-stride loop); head_dim 40 the scalar one."""
    rng = np.random.default_rng(5 + heads)
    x32 = rng.standard_normal(heads * D).astype(np.float32)
    th = rng.uniform(-3, 3, (heads, D // 2))
    c32 = np.concatenate([np.cos(th), np.cos(th)], 1).astype(np.float32).ravel()
    s32 = np.concatenate([np.sin(th), np.sin(th)], 1).astype(np.float32).ravel()
    x, c, s = enc16(x32, dtype), enc16(c32, dtype), enc16(s32, dtype)
    es = x.itemsize
    call = KernelCall.RotaryEmbedding(RoPECall(BufferRef(1), BufferRef(2), BufferRef(3),
                                               BufferRef(4), D, x.size, dtype))
    got = run(torch_cuda, backend, call, {1: x, 2: c, 3: s}, x.size * es, 4)
    want = np.zeros(x.size * es, np.uint8)
    lib().or_rope(_p(x), _p(c), _p(s), _p(want), D, x.size, dtype)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("idx_dtype", [DTYPE_I32, DTYPE_I64])
def test_gather_rows(torch_cuda, backend, idx_dtype):
    rng = np.random.default_rng(6)
    V, D = 1000, 96
    table = bf(rng.standard_normal((V, D)))
    idx = np.array([0, 999, -1, 17, -1000, 512, 3], np.int32 if idx_dtype == DTYPE_I32 else np.int64)
    call = KernelCall.Gather(GatherCall(BufferRef(1), BufferRef(2), BufferRef(3), 1, V, D, idx.size,
                                        idx_dtype, DTYPE_BF16))
    got = run(torch_cuda, backend, call, {1: table, 2: idx}, idx.size * D * 2, 3)
    want = np.zeros(idx.size * D * 2, np.uint8)
    assert lib().or_gather(_p(table), _p(idx), _p(want), 1, V, D * 2, idx.size,
                           int(idx_dtype == DTYPE_I64)) == 0
    assert np.array_equal(got, want)


def test_gather_out_of_range_is_reported(torch_cuda, backend):
    table = np.arange(40, dtype=np.float32)
    idx = np.array([1, 10], np.int32)            # 10 >= axis_dim 10
    call = KernelCall.Gather(GatherCall(BufferRef(1), BufferRef(2), BufferRef(3), 1, 10, 4, 2,
                                        DTYPE_I32, DTYPE_F32))
    ws = DeviceWorkspace()
    keep = [to_dev(torch_cuda, table), to_dev(torch_cuda, idx)]
    ws.bind(1, keep[0])
    ws.bind(2, keep[1])
    out = torch_cuda.full((32,), 7, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(3, out)
    backend.dispatch(call, ws)
    with pytest.raises(SlotOutOfRange):
        backend.synchronize()
    o = out.cpu().numpy().view(np.float32)
    assert np.array_equal(o[:4], table[4:8]) and np.all(o[4:] == 0)
    backend.synchronize()                        # the flag was cleared


@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F32])
@pytest.mark.parametrize("cols", [32000, 100003, 131072])
def test_argmax(torch_cuda, backend, dtype, cols):
    """Rows of one to several rounds of the kernel's four vectors a thread
    (32768 bf16 / 16384 f32 elements a round), odd lengths whose later rows
    start unaligned (the element loop), ties across rounds, NaN rows."""
    rng = np.random.default_rng(7)
    rows = 9
    x32 = rng.standard_normal((rows, cols)).astype(np.float32)
    x32[3, :] = 1.0                              # all equal: index 0
    x32[4, 100] = x32[4, 20000] = 50.0           # a tie: the lower index
    x32[5, :] = np.nan
    x32[6, 10] = np.nan
    x32[6, 11] = 60.0
    x32[7, cols - 1] = x32[7, cols // 2 + 1] = 70.0   # a tie in later rounds
    x32[8, cols - 1] = 80.0                      # the last element
    x = bf(x32) if dtype == DTYPE_BF16 else x32
    call = KernelCall.ArgMax(ArgMaxCall(BufferRef(1), BufferRef(2), rows, cols, dtype))
    got = run(torch_cuda, backend, call, {1: x}, rows * 4, 2).view(np.int32)
    want = np.zeros(rows, np.int32)
    lib().or_argmax(_p(x), _p(want), rows, cols, dtype)
    assert np.array_equal(got, want) and got[3] == 0 and got[4] == 100 and got[6] == 11
    assert got[7] == cols // 2 + 1 and got[8] == cols - 1


# ------------------------------------------------------------- session -----
CFG = DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                    batch=3, bucket=64)


def step_inputs(cfg, step, tokens):
    cq, sq = rope_tables(cfg, np.array([step]), cfg.heads)
    ck, sk = rope_tables(cfg, np.array([step]), cfg.kv_heads)
    return [np.asarray(tokens, np.int32).tobytes(), np.uint32(step).tobytes(),
            np.full(cfg.batch, step + 1, np.uint32).tobytes(), cq, sq, ck, sk]


def test_session_decoder_matches_oracle_walk(torch_cuda, backend):
    cfg = CFG
    archive = build_decode_step(cfg, init_weights(cfg, seed=11))
    sess = HipSession(backend, archive)
    ref = OracleSession(archive)
    assert sess.fingerprint() == archive[-32:]
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    zero_caches = [bytes(P * S * Dh), bytes(P * S * 4), bytes(P * S * Dh), bytes(P * S * 4)]
    for layer in range(cfg.layers):
        for j, z in enumerate(zero_caches):
            sess.write_input(7 + 4 * layer + j, z)
            ref.set_input(7 + 4 * layer + j, z)
    rng = np.random.default_rng(12)
    tokens = rng.integers(0, cfg.vocab, cfg.batch)
    for step in range(6):
        ins = step_inputs(cfg, step, tokens)
        for i, b in enumerate(ins):
            sess.write_input(i, b)
            ref.set_input(i, b)
        sess.run()
        sess.synchronize()
        ref.run()
        got_logits = unbf(np.frombuffer(sess.read_output(1), np.uint16)).reshape(cfg.batch, -1)
        want_logits = unbf(ref.output(1).view(np.uint16)).reshape(cfg.batch, -1)
        err = oracle.max_rel_err(got_logits, want_logits)
        scale = np.max(np.abs(want_logits))
        mean_err = float(np.mean(np.abs(got_logits - want_logits)) / scale)
        assert err <= 2e-2 and mean_err <= 2e-3, f"step {step}: logits error {err}, {mean_err}"
        nxt = np.frombuffer(sess.read_output(0), np.int32)
        for b in range(cfg.batch):    # greedy pick equal, up to a near-tie in the oracle
            assert want_logits[b, nxt[b]] >= want_logits[b].max() - 2e-2 * scale, (step, b)
        # caches: the oracle carries its outputs back as the next inputs; the
        # session's output ports alias its input buffers (the in-place move)
        for layer in range(cfg.layers):
            for j in range(4):
                ref.set_input(7 + 4 * layer + j, ref.output(2 + 4 * layer + j).tobytes())
        kq_dev = np.frombuffer(sess.read_output(2), np.int8)
        kq_ref = ref.output(2).view(np.int8)
        assert np.mean(kq_dev != kq_ref) < 0.02   # int8 K rows agree (rounding of k upstream)
        tokens = nxt
    p_in = sess.output_ptr(2)[0]
    assert p_in != 0
    sess.close()


def test_session_capture_replay_matches_eager(torch_cuda, backend):
    cfg = CFG
    archive = build_decode_step(cfg, init_weights(cfg, seed=13))
    outs = []
    for mode in ("eager", "graph"):
        sess = HipSession(backend, archive)
        P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
        for layer in range(cfg.layers):
            for j, z in enumerate([bytes(P * S * Dh), bytes(P * S * 4)] * 2):
                sess.write_input(7 + 4 * layer + j, z)
        tokens = np.arange(cfg.batch) * 7
        logits = []
        if mode == "graph":
            for i, b in enumerate(step_inputs(cfg, 0, tokens)):
                sess.write_input(i, b)
            sess.capture()      # one eager walk (step 0) + the recording
            sess.synchronize()
            logits.append(sess.read_output(1))
            tokens = np.frombuffer(sess.read_output(0), np.int32)
        for step in range(len(logits), 5):
            for i, b in enumerate(step_inputs(cfg, step, tokens)):
                sess.write_input(i, b)
            sess.replay() if mode == "graph" else sess.run()
            sess.synchronize()
            logits.append(sess.read_output(1))
            tokens = np.frombuffer(sess.read_output(0), np.int32)
        outs.append(logits)
        if mode == "graph":
            t = torch_cuda.zeros(64, dtype=torch_cuda.uint8, device="cuda")
            sess.bind_input(0, t)
            with pytest.raises(DispatchError):
                sess.replay()
        sess.close()
    for a, b in zip(*outs):
        assert a == b


def test_captured_walk_survives_other_work_on_its_backend(torch_cuda, backend):
    """A captured walk keeps the split-K scratch it was recorded with: a larger
    session and a large direct few-row MatMul on the same backend in between
    (each needing more scratch than the first session) must not move or free
    it. Every replay equals the eager walk of the same inputs."""
    from hologram_amd import MatMulCall
    cfg = CFG
    archive = build_decode_step(cfg, init_weights(cfg, seed=21))
    big = DecoderConfig(layers=1, hidden=1024, heads=8, kv_heads=2, head_dim=128, ffn=4096,
                        vocab=4000, batch=4, bucket=128)
    big_archive = build_decode_step(big, init_weights(big, seed=22))

    def fresh(c, arch):
        s = HipSession(backend, arch)
        P, S, Dh = c.planes, c.bucket, c.head_dim
        for layer in range(c.layers):
            for j, z in enumerate([bytes(P * S * Dh), bytes(P * S * 4)] * 2):
                s.write_input(7 + 4 * layer + j, z)
        for i, b in enumerate(step_inputs(c, 0, np.arange(c.batch) * 5)):
            s.write_input(i, b)
        return s

    eager = fresh(cfg, archive)
    eager.run()
    eager.synchronize()
    want = eager.read_output(1)
    eager.close()

    sess = fresh(cfg, archive)
    sess.capture()
    sess.synchronize()
    for rnd in range(3):
        other = fresh(big, big_archive)          # larger few-row products, own scratch
        other.run()
        other.synchronize()
        other.close()
        m, k, n = 16, 8192, 8192                 # a direct call that grows the backend's scratch
        a = to_dev(torch_cuda, bf(np.ones(m * k, np.float32)))
        b = to_dev(torch_cuda, bf(np.full(k * n, 2 ** -13, np.float32)))
        c = torch_cuda.zeros(m * n * 2, dtype=torch_cuda.uint8, device="cuda")
        ws = DeviceWorkspace()
        ws.bind(1, a), ws.bind(2, b), ws.bind(3, c)
        backend.dispatch(KernelCall.MatMul(MatMulCall(BufferRef(1), BufferRef(2), BufferRef(3),
                                                      m, k, n, DTYPE_BF16)), ws)
        backend.synchronize()
        assert np.all(unbf(c.cpu().numpy().view(np.uint16)) == 1.0)
        # the same step's inputs again: the caches were appended at the same ring row
        for i, bb in enumerate(step_inputs(cfg, 0, np.arange(cfg.batch) * 5)):
            sess.write_input(i, bb)
        sess.replay()
        sess.synchronize()
        assert sess.read_output(1) == want, rnd
    sess.close()


def test_reference_compiled_fixture_runs_to_its_kappa(torch_cuda, backend):
    """The reference's compiled fixture.holo (tests/golden/) through the device
    session: the output's κ (blake3 of its bytes, address.rs:96-99) equals the
    reference engine's recorded fixture.kappa."""
    from pathlib import Path
    from hologram_amd import blake3
    golden = Path(__file__).resolve().parent / "golden"
    arch = (golden / "reference_fixture.holo").read_bytes()
    want = (golden / "reference_fixture.kappa").read_text().strip()
    sess = HipSession(backend, arch)
    sess.run()
    sess.synchronize()
    assert "blake3:" + blake3(sess.read_output(0)).hex() == want
    sess.close()


def test_session_memo_skips_a_repeated_walk(torch_cuda, backend):
    """The whole-graph memo (session.rs:841-905): the same input bytes again,
    nothing touched in between, skip the walk and leave the same outputs; new
    bytes, a direct write, or the memo switched off walk again."""
    from hologram_amd import HoloWriter, PortDescriptor
    n = 4099
    w = HoloWriter()
    w.kernel_calls = [KernelCall.Add(BinaryCall(BufferRef(0, 0, n * 4), BufferRef(1, 0, n * 4),
                                                BufferRef(2, 0, n * 4), n, 32, DTYPE_F32))]
    w.inputs = [PortDescriptor("a", 0, n, DTYPE_F32, [n]), PortDescriptor("b", 1, n, DTYPE_F32, [n])]
    w.outputs = [PortDescriptor("y", 2, n, DTYPE_F32, [n])]
    sess = HipSession(backend, w.finish())
    rng = np.random.default_rng(3)
    a, b, c = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    y1 = sess.execute([a.tobytes(), b.tobytes()])[0]
    assert not sess.last_memo_hit
    assert np.array_equal(np.frombuffer(y1, np.float32), a + b)
    assert sess.execute([a.tobytes(), b.tobytes()])[0] == y1 and sess.last_memo_hit
    y2 = sess.execute([a.tobytes(), c.tobytes()])[0]
    assert not sess.last_memo_hit and np.array_equal(np.frombuffer(y2, np.float32), a + c)
    sess.write_input(1, b.tobytes())          # touched directly: the next call walks
    assert sess.execute([a.tobytes(), c.tobytes()])[0] == y2 and not sess.last_memo_hit
    sess.set_memo(False)
    sess.execute([a.tobytes(), c.tobytes()])
    assert not sess.last_memo_hit
    sess.set_memo(True)
    sess.execute([a.tobytes(), c.tobytes()])
    assert not sess.last_memo_hit
    assert sess.execute([a.tobytes(), c.tobytes()])[0] == y2 and sess.last_memo_hit
    sess.close()


def test_session_memo_with_in_place_caches(torch_cuda, backend):
    """A decode step whose caches move in place: a memo hit leaves the outputs
    of the last walk (its caches included) exactly as a fresh walk of the
    same inputs produces them."""
    cfg = CFG
    archive = build_decode_step(cfg, init_weights(cfg, seed=11))
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    caches = [bytes(P * S * Dh), bytes(P * S * 4), bytes(P * S * Dh), bytes(P * S * 4)] * cfg.layers
    ins = step_inputs(cfg, 0, np.arange(cfg.batch) * 7) + caches
    sess = HipSession(backend, archive)
    first = sess.execute(ins)
    again = sess.execute(ins)
    assert sess.last_memo_hit and again == first
    fresh = HipSession(backend, archive)
    fresh.set_memo(False)
    assert fresh.execute(ins) == first
    sess.close()
    fresh.close()
