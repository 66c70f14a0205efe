"""GPU: a decode step's q/k/v group leaves its split-K epilogue (the sum of the
partials, RoPE of q and k, the int8 appends of k and v: rope_float,
float_kernels.rs:3123-3186; quantize_row_i8, simd.rs:4755-4785, placed as
kernels.rs:455-501) to the int8 decode attention after it, which runs it in
front of the attention in one launch: each workgroup finishes its own plane's
heads, then attends over them. The same device code computes every value, so
the walk must give the bits of the walk with the epilogue as a launch of its
own (NO_ATTN_PROLOGUE) and of the unfused walk (NO_DEVICE_FUSION): tokens,
logits, caches and scales over several steps.

Shapes: head_dim 64 and 128 at 32 planes (eight waves a plane) and 160 planes
(four); a bucket the appends wrap (12 steps over 8 rows); and shapes the fused
launch does not take, where the epilogue runs on its own at dispatch: 8 planes
(the balanced split form) and head_dim 32 (the generic kernel)."""
import numpy as np
import pytest

from hologram_amd import HipSession
from hologram_amd.decoder_graph import DecoderConfig, build_decode_step, init_weights, rope_tables
from hologram_amd.session import NO_ATTN_PROLOGUE, NO_DEVICE_FUSION

pytestmark = pytest.mark.gpu

CFGS = {
    "d64_32planes": DecoderConfig(layers=2, hidden=256, heads=8, kv_heads=4, head_dim=64, ffn=512,
                                  vocab=512, batch=8, bucket=64),
    "d128_32planes": DecoderConfig(layers=1, hidden=512, heads=4, kv_heads=4, head_dim=128, ffn=512,
                                   vocab=256, batch=8, bucket=128),
    "d64_160planes": DecoderConfig(layers=1, hidden=256, heads=8, kv_heads=4, head_dim=64, ffn=512,
                                   vocab=256, batch=40, bucket=64),
    # a bucket of 8 rows walked for 12 steps: the appends wrap the ring (the
    # appended row at pos % bucket, every row visible)
    "d64_ring_wrap": DecoderConfig(layers=1, hidden=256, heads=8, kv_heads=4, head_dim=64, ffn=512,
                                   vocab=256, batch=8, bucket=8),
    "split_form": DecoderConfig(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                                vocab=256, batch=4, bucket=64),
    "d32_generic": DecoderConfig(layers=1, hidden=256, heads=8, kv_heads=4, head_dim=32, ffn=512,
                                 vocab=256, batch=8, bucket=64),
}


def step_inputs(cfg, tokens, step):
    cq, sq = rope_tables(cfg, np.array([step]), cfg.heads)
    ck, sk = rope_tables(cfg, np.array([step]), cfg.kv_heads)
    return [np.asarray(tokens, np.int32).tobytes(), np.uint32(step).tobytes(),
            np.full(cfg.batch, step + 1, np.uint32).tobytes(), cq, sq, ck, sk]


def zero_caches(sess, cfg):
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    for layer in range(cfg.layers):
        for j, z in enumerate([bytes(P * S * Dh), bytes(P * S * 4)] * 2):
            sess.write_input(7 + 4 * layer + j, z)


def decode(backend, cfg, archive, flags, steps, capture=False):
    """Greedy steps from fixed first tokens; every output of every step. With
    `capture`, step 0 is the eager walk inside the capture and the later steps
    are replays with new inputs."""
    sess = HipSession(backend, archive, flags=flags)
    zero_caches(sess, cfg)
    tokens = np.arange(cfg.batch) * 5 + 1
    rec = []
    for step in range(steps):
        for i, b in enumerate(step_inputs(cfg, tokens, step)):
            sess.write_input(i, b)
        if not capture:
            sess.run()
        elif step == 0:
            sess.capture()
        else:
            sess.replay()
        sess.synchronize()
        rec.append([sess.read_output(o) for o in range(len(sess.outputs))])
        tokens = np.frombuffer(rec[-1][0], np.int32)[:cfg.batch]
    n = sess.attn_prologues
    sess.close()
    return rec, n


@pytest.mark.parametrize("name", list(CFGS))
def test_prologue_walk_bit_identical(torch_cuda, backend, name):
    cfg = CFGS[name]
    steps = 12 if cfg.bucket < 12 else 5
    archive = build_decode_step(cfg, init_weights(cfg, seed=11))
    fused, n = decode(backend, cfg, archive, 0, steps)
    assert n == cfg.layers
    for flags in (NO_ATTN_PROLOGUE, NO_DEVICE_FUSION):
        other, m = decode(backend, cfg, archive, flags, steps)
        assert m == 0
        for step, (x, y) in enumerate(zip(fused, other)):
            for o, (u, v) in enumerate(zip(x, y)):
                assert u == v, f"{name}, flags {flags}: step {step}, output {o} differs"


@pytest.mark.parametrize("name", ["d64_32planes", "d128_32planes"])
def test_prologue_graph_replays(torch_cuda, backend, name):
    """The fused launch captured in the session's graph: each replay with new
    inputs gives the eager walk's bits."""
    cfg = CFGS[name]
    archive = build_decode_step(cfg, init_weights(cfg, seed=12))
    eager, _ = decode(backend, cfg, archive, 0, 5)
    replayed, _ = decode(backend, cfg, archive, 0, 5, capture=True)
    for step, (x, y) in enumerate(zip(eager, replayed)):
        for o, (u, v) in enumerate(zip(x, y)):
            assert u == v, f"{name}: step {step}, output {o} differs after replay"
