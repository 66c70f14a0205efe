"""GPU: Reshape (wire 60) and Slice (wire 63) through dispatch and through the
session walk, and the walk's per-step reuse (session.rs compute_and_label
:1106-1150 and :1121-1131), against the oracle walk (oracle/graph.py).

- Direct dispatch copies the input view's first element_count elements (float
  dtypes) or bytes (the byte domain), nothing past them.
- A session binds an interior Reshape / Slice to its input's memory and runs
  a port-writing one as a copy; the walk equals the oracle's bit for bit
  (the chain's ops are bit-exact), eagerly and as a replayed graph.
- A repeated computation is bound to its first result; the walk still equals
  the oracle.
- With the memo on, a step whose operands did not change since the last walk
  is skipped, and the outputs equal a fresh walk of the same inputs; a decode
  step with in-place caches and a changing token stays equal to a memo-off
  session step after step."""
import numpy as np
import pytest

from conftest import from_dev, to_dev
from hologram_amd import (DTYPE_BF16, DTYPE_F32, DTYPE_I32, BinaryCall, BufferRef, DeviceWorkspace,
                          HipSession, KernelCall, LayoutCall, UnaryCall, UnsupportedOp)
from oracle.graph import OracleSession
from test_layout import bf16, build, chain_archive, dup_archive, port

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tag,dt,n,es", [("Reshape", DTYPE_F32, 1000, 4), ("Slice", DTYPE_BF16, 777, 2),
                                         ("Slice", DTYPE_I32, 777, 1), ("Reshape", 2, 4099, 1)])
def test_direct_dispatch_copies_the_view(torch_cuda, backend, tag, dt, n, es):
    rng = np.random.default_rng(n)
    src = rng.integers(0, 256, size=8192, dtype=np.uint8)
    off = 48
    ws = DeviceWorkspace()
    ws.bind(0, to_dev(torch_cuda, src))
    out = torch_cuda.full((8192,), 0xA5, dtype=torch_cuda.uint8, device="cuda")
    ws.bind(1, out)
    call = getattr(KernelCall, tag)(LayoutCall(BufferRef(0, off, 0), BufferRef(1, 16), n, dt))
    backend.dispatch(call, ws)
    backend.synchronize()
    got = from_dev(out, np.uint8)
    nb = n * es
    assert np.array_equal(got[16:16 + nb], src[off:off + nb])
    assert (got[:16] == 0xA5).all() and (got[16 + nb:] == 0xA5).all()


def test_direct_dispatch_refuses_f64(torch_cuda, backend):
    ws = DeviceWorkspace()
    ws.bind(0, torch_cuda.zeros(256, dtype=torch_cuda.uint8, device="cuda"))
    ws.bind(1, torch_cuda.zeros(256, dtype=torch_cuda.uint8, device="cuda"))
    with pytest.raises(UnsupportedOp):
        backend.dispatch(KernelCall.Reshape(LayoutCall(BufferRef(0), BufferRef(1), 8, 9)), ws)


def test_chain_with_bound_reshape_and_slice_matches_oracle(torch_cuda, backend):
    arch, _ = chain_archive()
    sess = HipSession(backend, arch)
    assert sess.n_nodes == 2
    rng = np.random.default_rng(4)
    for rnd in range(3):
        x = bf16(rng.standard_normal(32).astype(np.float32) * 2)
        got = sess.execute([x.tobytes()])[0]
        o = OracleSession(arch)
        o.set_input(0, x.tobytes())
        o.run()
        assert got == o.output(0).tobytes(), rnd
        assert sess.last_walk == (2, 2)
    sess.capture()
    sess.replay()
    sess.synchronize()
    assert sess.read_output(0) == got
    sess.close()


def test_port_writing_reshape_and_slice_copy_on_device(torch_cuda, backend):
    n = 3000
    calls = [KernelCall.Add(BinaryCall(BufferRef(0, 0, n * 4), BufferRef(1, 0, n * 4),
                                       BufferRef(2, 0, n * 4), n, 32, DTYPE_F32)),
             KernelCall.Reshape(LayoutCall(BufferRef(2, 0, n * 4), BufferRef(3, 0, n * 4), n,
                                           DTYPE_F32)),
             KernelCall.Slice(LayoutCall(BufferRef(2, 400, 1000 * 4), BufferRef(4, 0, 1000 * 4),
                                         1000, DTYPE_F32))]
    arch = build(calls, [(0, n), (1, n)], [(3, n), (4, 1000)])
    sess = HipSession(backend, arch)
    assert sess.n_nodes == 3
    rng = np.random.default_rng(6)
    a, b = (rng.standard_normal(n).astype(np.float32) for _ in range(2))
    y, z = sess.execute([a.tobytes(), b.tobytes()])
    s = a + b
    assert np.array_equal(np.frombuffer(y, np.float32), s)
    assert np.array_equal(np.frombuffer(z, np.float32), s[100:1100])
    sess.close()


def test_repeated_value_bound_on_device_matches_oracle(torch_cuda, backend):
    from hologram_amd.session import NO_DEVICE_FUSION
    import oracle
    arch, (m, k, n) = dup_archive()
    for flags in (0, NO_DEVICE_FUSION):
        sess = HipSession(backend, arch, flags=flags)
        x = np.random.default_rng(8).standard_normal(m * k).astype(np.float32)
        got = np.frombuffer(sess.execute([x.tobytes()])[0], np.float32)
        o = OracleSession(arch)
        o.set_input(0, x.tobytes())
        o.run()
        want = o.output(0).view(np.float32)
        assert oracle.max_rel_err(got, want) <= 1e-5
        sess.close()


def two_chain_archive(n=4096):
    """x -> Gelu -> a;  y -> Silu -> b;  out = a + b (bf16)."""
    nb = 2 * n
    calls = [KernelCall.Gelu(UnaryCall(BufferRef(0, 0, nb), BufferRef(2, 0, nb), n, 16, DTYPE_BF16)),
             KernelCall.Silu(UnaryCall(BufferRef(1, 0, nb), BufferRef(3, 0, nb), n, 16, DTYPE_BF16)),
             KernelCall.Add(BinaryCall(BufferRef(2, 0, nb), BufferRef(3, 0, nb), BufferRef(4, 0, nb), n,
                                       16, DTYPE_BF16))]
    return build(calls, [(0, n, DTYPE_BF16), (1, n, DTYPE_BF16)], [(4, n, DTYPE_BF16)])


def test_memo_on_skips_the_steps_whose_operands_did_not_change(torch_cuda, backend):
    arch = two_chain_archive()
    sess = HipSession(backend, arch)
    rng = np.random.default_rng(10)
    x1, y1, y2, x2 = (bf16(rng.standard_normal(4096).astype(np.float32)) for _ in range(4))

    def oracle_out(x, y):
        o = OracleSession(arch)
        o.set_input(0, x.tobytes())
        o.set_input(1, y.tobytes())
        o.run()
        return o.output(0).tobytes()

    assert sess.execute([x1.tobytes(), y1.tobytes()])[0] == oracle_out(x1, y1)
    assert sess.last_walk == (3, 0)
    assert sess.execute([x1.tobytes(), y2.tobytes()])[0] == oracle_out(x1, y2)
    assert sess.last_walk == (2, 1)                   # Gelu(x) still holds its value
    assert sess.execute([x1.tobytes(), y2.tobytes()])[0] == oracle_out(x1, y2)
    assert sess.last_memo_hit and sess.last_walk == (0, 3)
    assert sess.execute([x2.tobytes(), y2.tobytes()])[0] == oracle_out(x2, y2)
    assert sess.last_walk == (2, 1)                   # Silu(y) kept
    sess.set_memo(False)
    assert sess.execute([x2.tobytes(), y2.tobytes()])[0] == oracle_out(x2, y2)
    assert sess.last_walk == (3, 0)
    sess.close()


def test_memo_on_decode_steps_with_in_place_caches(torch_cuda, backend):
    """A decode step (in-place int8 appends, fused groups) executed step after
    step with the memo on gives, at every step, the bytes a memo-off session
    gives for the same inputs: steps that touch the caches always run."""
    from hologram_amd.decoder_graph import build_decode_step, init_weights
    from test_gpu_session import CFG, step_inputs
    cfg = CFG
    archive = build_decode_step(cfg, init_weights(cfg, seed=12))
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    caches = [bytes(P * S * Dh), bytes(P * S * 4), bytes(P * S * Dh), bytes(P * S * 4)] * cfg.layers
    on, off = HipSession(backend, archive), HipSession(backend, archive)
    off.set_memo(False)
    tokens = np.arange(cfg.batch) * 5
    for step in range(3):
        ins = step_inputs(cfg, step, tokens) + caches
        a, b = on.execute(ins), off.execute(ins)
        assert a == b, step
        tokens = np.frombuffer(a[0], np.int32)[:cfg.batch]
        caches = [a[2 + j] for j in range(4 * cfg.layers)]
    on.close()
    off.close()
