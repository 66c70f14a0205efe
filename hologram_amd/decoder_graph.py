"""Llama-style decode-step graph, emitted as a `.holo` archive.

The reference compiles such graphs with hologram-graph/hologram-compiler
(crates/hologram-bench/examples/decode_profile.rs:235-365 builds RmsNorm ->
q/k/v/o projections -> Add -> RmsNorm -> gate/up -> Silu -> Mul -> down -> Add;
the attention step graph is crates/hologram-exec/tests/
decode_attention_valid_e2e.rs:110-162). No Rust toolchain exists here, so this
module emits the compiled form directly: the KernelCalls, ports, constants and
a sequential exec plan, through HoloWriter (writer.rs layout).

One step advances every sequence of the batch by one token:

    x      = Gather(embedding, tokens)                    [B, Dm]
    per layer:
      h    = RmsNorm(x) ; q,k,v = h Wq, h Wk, h Wv
      q,k  = RoPE(q, cos_q, sin_q), RoPE(k, cos_k, sin_k)
      K,V  = KvQuantAppend(k / v -> int8 caches at row `pos`)   (in place)
      a    = DecodeAttentionI8(q, K, V, lens)
      x    = x + a Wo
      h    = RmsNorm(x) ; x = x + (Silu(h Wg) * h Wu) Wd
    logits = RmsNorm(x) Wlm ;  next = ArgMax(logits)

Inputs (in port order): tokens i32[B], pos u32[1], lens u32[B], cos_q/sin_q
bf16[B,H,Dh], cos_k/sin_k bf16[B,Hkv,Dh], then per layer the int8 K cache,
its f32 scales, the int8 V cache and its scales ([B*Hkv, bucket, Dh] and
[B*Hkv, bucket]). Outputs: next i32[B], logits bf16[B,V], then the updated
caches (each aliases its input: the in-place move).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from .archive import ConstantEntry, HoloWriter, PortDescriptor
from .kernel_call import (DTYPE_BF16, DTYPE_F32, DTYPE_I8, DTYPE_I32, ArgMaxCall,
                          AttentionI8RowsCall, BinaryCall, BufferRef, DecodeAttentionI8Call,
                          GatherCall, KernelCall, KvQuantAppendCall, MatMulCall, NormCall, RoPECall,
                          TransposeCall, UnaryCall)


@dataclass(frozen=True)
class DecoderConfig:
    layers: int = 16
    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 8192
    vocab: int = 32000
    batch: int = 8
    bucket: int = 1024          # KV rows per sequence (prompt + generated <= bucket)
    eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def planes(self) -> int:
        return self.batch * self.kv_heads


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bf16_bytes(a: np.ndarray) -> bytes:
    """f32 array -> bf16 bytes by truncation (the reference's write_bf16)."""
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()


def init_weights(cfg: DecoderConfig, seed: int, std: float = 0.02) -> dict:
    """Random-init bf16 weights ~ N(0, std) (norm gains 1), as raw bf16 bytes.
    Each matrix draws from its own generator spawned from `seed` (so the
    matrices can be drawn on several threads with the same result)."""
    from concurrent.futures import ThreadPoolExecutor
    Dm, Hd, Kd = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    shapes = [("embedding", (cfg.vocab, Dm)), ("lm_head", (Dm, cfg.vocab))]
    for layer in range(cfg.layers):
        shapes += [((layer, "wq"), (Dm, Hd)), ((layer, "wk"), (Dm, Kd)), ((layer, "wv"), (Dm, Kd)),
                   ((layer, "wo"), (Hd, Dm)), ((layer, "wg"), (Dm, cfg.ffn)),
                   ((layer, "wu"), (Dm, cfg.ffn)), ((layer, "wd"), (cfg.ffn, Dm))]
    seeds = np.random.SeedSequence(seed).spawn(len(shapes))

    def draw(i):
        rng = np.random.default_rng(seeds[i])
        return bf16_bytes(rng.standard_normal(shapes[i][1], dtype=np.float32) * np.float32(std))

    with ThreadPoolExecutor(8) as ex:
        mats = list(ex.map(draw, range(len(shapes))))
    ones = bf16_bytes(np.ones(Dm, np.float32))
    out = {"final_norm": ones}
    for (key, _), m in zip(shapes, mats):
        if isinstance(key, tuple):
            out.setdefault(f"l{key[0]}", {"attn_norm": ones, "ffn_norm": ones})[key[1]] = m
        else:
            out[key] = m
    return out


class _Builder:
    def __init__(self):
        self.next_slot = 0
        self.calls: list[KernelCall] = []
        self.sizes: dict[int, int] = {}

    def slot(self, nbytes: int) -> BufferRef:
        s = self.next_slot
        self.next_slot += 1
        self.sizes[s] = nbytes
        return BufferRef(s, 0, nbytes)

    def add(self, call: KernelCall) -> None:
        self.calls.append(call)


def build_decode_step(cfg: DecoderConfig, weights: dict) -> bytes:
    """The `.holo` archive of one decode step (see the module docstring)."""
    return _build(cfg, weights, 1)


def build_prefill(cfg: DecoderConfig, weights: dict, rows: int) -> bytes:
    """The `.holo` archive of a prompt pass: `rows` tokens of every sequence at
    once, appended to the caches at ring rows pos .. pos + rows - 1.

    Same weights and cache ports as the decode step. Per-row tensors are
    token-major [B * rows, ...]; k and v go through Transpose
    ([B, rows, Hkv, Dh] -> [B, Hkv, rows, Dh], the caches' row order) before the
    append, and attention is AttentionI8Rows (row t sees lens[b] - (rows - 1 - t)
    keys: causal). Only each sequence's last row continues past the layers
    (Gather), so logits and the next token are [B] as in the decode step.
    Inputs: tokens i32[B, rows], pos u32[1], lens u32[B] (= pos + rows),
    cos_q/sin_q bf16[B, rows, H, Dh], cos_k/sin_k bf16[B, rows, Hkv, Dh], caches."""
    if rows < 2:
        raise ValueError("a prompt pass has at least two rows; one row is the decode step")
    return _build(cfg, weights, rows)


def _build(cfg: DecoderConfig, weights: dict, T: int) -> bytes:
    B, Dm, H, Hkv, Dh, F, V, S = (cfg.batch, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim,
                                  cfg.ffn, cfg.vocab, cfg.bucket)
    P = cfg.planes
    R = B * T           # rows through the layers
    g = _Builder()
    w = HoloWriter()
    bf = 2
    eps = f32_bits(cfg.eps)

    def port(name, ref, count, dtype, shape, out=False):
        (w.outputs if out else w.inputs).append(PortDescriptor(name, ref.slot, count, dtype,
                                                               list(shape)))

    def const(body: bytes, dtype=DTYPE_BF16, inline=False) -> BufferRef:
        ref = g.slot(len(body))
        w.constants.append(ConstantEntry(ref.slot, dtype, body, by_reference=not inline))
        return ref

    tokens = g.slot(4 * R)
    pos = g.slot(4)
    lens = g.slot(4 * B)
    cos_q, sin_q = g.slot(R * H * Dh * bf), g.slot(R * H * Dh * bf)
    cos_k, sin_k = g.slot(R * Hkv * Dh * bf), g.slot(R * Hkv * Dh * bf)
    rshape = [B] if T == 1 else [B, T]
    port("tokens", tokens, R, DTYPE_I32, rshape)
    port("pos", pos, 1, DTYPE_I32, [1])
    port("lens", lens, B, DTYPE_I32, [B])
    port("cos_q", cos_q, R * H * Dh, DTYPE_BF16, rshape + [H, Dh])
    port("sin_q", sin_q, R * H * Dh, DTYPE_BF16, rshape + [H, Dh])
    port("cos_k", cos_k, R * Hkv * Dh, DTYPE_BF16, rshape + [Hkv, Dh])
    port("sin_k", sin_k, R * Hkv * Dh, DTYPE_BF16, rshape + [Hkv, Dh])
    caches = []
    for layer in range(cfg.layers):
        kq, ks = g.slot(P * S * Dh), g.slot(P * S * 4)
        vq, vs = g.slot(P * S * Dh), g.slot(P * S * 4)
        for nm, ref, cnt, dt, shp in ((f"k_cache.{layer}", kq, P * S * Dh, DTYPE_I8, [P, S, Dh]),
                                      (f"k_scales.{layer}", ks, P * S, DTYPE_F32, [P, S]),
                                      (f"v_cache.{layer}", vq, P * S * Dh, DTYPE_I8, [P, S, Dh]),
                                      (f"v_scales.{layer}", vs, P * S, DTYPE_F32, [P, S])):
            port(nm, ref, cnt, dt, shp)
        caches.append((kq, ks, vq, vs))

    emb = const(weights["embedding"])
    x = g.slot(R * Dm * bf)
    g.add(KernelCall.Gather(GatherCall(emb, tokens, x, 1, V, Dm, R, DTYPE_I32, DTYPE_BF16)))
    new_caches = []
    for layer in range(cfg.layers):
        lw = weights[f"l{layer}"]
        kq, ks, vq, vs = caches[layer]
        h = g.slot(R * Dm * bf)
        g.add(KernelCall.RmsNorm(NormCall(x, const(lw["attn_norm"]), h, R, Dm, eps, DTYPE_BF16)))
        q, k, v = g.slot(R * H * Dh * bf), g.slot(R * Hkv * Dh * bf), g.slot(R * Hkv * Dh * bf)
        g.add(KernelCall.MatMul(MatMulCall(h, const(lw["wq"]), q, R, Dm, H * Dh, DTYPE_BF16)))
        g.add(KernelCall.MatMul(MatMulCall(h, const(lw["wk"]), k, R, Dm, Hkv * Dh, DTYPE_BF16)))
        g.add(KernelCall.MatMul(MatMulCall(h, const(lw["wv"]), v, R, Dm, Hkv * Dh, DTYPE_BF16)))
        qr, kr = g.slot(R * H * Dh * bf), g.slot(R * Hkv * Dh * bf)
        g.add(KernelCall.RotaryEmbedding(RoPECall(q, cos_q, sin_q, qr, Dh, R * H * Dh, DTYPE_BF16)))
        g.add(KernelCall.RotaryEmbedding(RoPECall(k, cos_k, sin_k, kr, Dh, R * Hkv * Dh,
                                                  DTYPE_BF16)))
        if T > 1:   # token-major rows -> the caches' [plane][row] order
            kt, vt = g.slot(R * Hkv * Dh * bf), g.slot(R * Hkv * Dh * bf)
            for src, dst in ((kr, kt), (v, vt)):
                g.add(KernelCall.Transpose(TransposeCall(src, dst, (B, T, Hkv, Dh), (0, 2, 1, 3),
                                                         DTYPE_BF16)))
            kr, v = kt, vt
        kq2, ks2 = g.slot(P * S * Dh), g.slot(P * S * 4)
        vq2, vs2 = g.slot(P * S * Dh), g.slot(P * S * 4)
        g.add(KernelCall.KvQuantAppend(KvQuantAppendCall(kr, pos, kq, ks, kq2, ks2, P, S, T, Dh,
                                                         DTYPE_BF16)))
        g.add(KernelCall.KvQuantAppend(KvQuantAppendCall(v, pos, vq, vs, vq2, vs2, P, S, T, Dh,
                                                         DTYPE_BF16)))
        new_caches.append((kq2, ks2, vq2, vs2))
        a = g.slot(R * H * Dh * bf)
        attn = DecodeAttentionI8Call(qr, kq2, vq2, ks2, vs2, lens, a, B, H, Hkv, S, Dh, 0,
                                     DTYPE_BF16)
        g.add(KernelCall.DecodeAttentionI8(attn) if T == 1
              else KernelCall.AttentionI8Rows(AttentionI8RowsCall(attn, T)))
        o = g.slot(R * Dm * bf)
        g.add(KernelCall.MatMul(MatMulCall(a, const(lw["wo"]), o, R, H * Dh, Dm, DTYPE_BF16)))
        x2 = g.slot(R * Dm * bf)
        g.add(KernelCall.Add(BinaryCall(x, o, x2, R * Dm, 16, DTYPE_BF16)))
        h2 = g.slot(R * Dm * bf)
        g.add(KernelCall.RmsNorm(NormCall(x2, const(lw["ffn_norm"]), h2, R, Dm, eps, DTYPE_BF16)))
        gt, up = g.slot(R * F * bf), g.slot(R * F * bf)
        g.add(KernelCall.MatMul(MatMulCall(h2, const(lw["wg"]), gt, R, Dm, F, DTYPE_BF16)))
        g.add(KernelCall.MatMul(MatMulCall(h2, const(lw["wu"]), up, R, Dm, F, DTYPE_BF16)))
        sg = g.slot(R * F * bf)
        g.add(KernelCall.Silu(UnaryCall(gt, sg, R * F, 16, DTYPE_BF16)))
        mm = g.slot(R * F * bf)
        g.add(KernelCall.Mul(BinaryCall(sg, up, mm, R * F, 16, DTYPE_BF16)))
        dn = g.slot(R * Dm * bf)
        g.add(KernelCall.MatMul(MatMulCall(mm, const(lw["wd"]), dn, R, F, Dm, DTYPE_BF16)))
        x3 = g.slot(R * Dm * bf)
        g.add(KernelCall.Add(BinaryCall(x2, dn, x3, R * Dm, 16, DTYPE_BF16)))
        x = x3
    if T > 1:       # each sequence's last row
        last = np.arange(1, B + 1, dtype=np.int32) * T - 1
        xl = g.slot(B * Dm * bf)
        g.add(KernelCall.Gather(GatherCall(x, const(last.tobytes(), DTYPE_I32, inline=True), xl, 1,
                                           R, Dm, B, DTYPE_I32, DTYPE_BF16)))
        x = xl
    hf = g.slot(B * Dm * bf)
    g.add(KernelCall.RmsNorm(NormCall(x, const(weights["final_norm"]), hf, B, Dm, eps,
                                      DTYPE_BF16)))
    logits = g.slot(B * V * bf)
    g.add(KernelCall.MatMul(MatMulCall(hf, const(weights["lm_head"]), logits, B, Dm, V,
                                       DTYPE_BF16)))
    nxt = g.slot(4 * B)
    g.add(KernelCall.ArgMax(ArgMaxCall(logits, nxt, B, V, DTYPE_BF16)))
    port("next_tokens", nxt, B, DTYPE_I32, [B], out=True)
    port("logits", logits, B * V, DTYPE_BF16, [B, V], out=True)
    for layer, (kq2, ks2, vq2, vs2) in enumerate(new_caches):
        port(f"k_cache.{layer}", kq2, P * S * Dh, DTYPE_I8, [P, S, Dh], out=True)
        port(f"k_scales.{layer}", ks2, P * S, DTYPE_F32, [P, S], out=True)
        port(f"v_cache.{layer}", vq2, P * S * Dh, DTYPE_I8, [P, S, Dh], out=True)
        port(f"v_scales.{layer}", vs2, P * S, DTYPE_F32, [P, S], out=True)
    w.kernel_calls = g.calls
    w.exec_plan = [[i] for i in range(len(g.calls))]
    return w.finish()


def rope_tables(cfg: DecoderConfig, positions: np.ndarray, heads: int) -> tuple:
    """cos/sin in the rotate-half layout RoPECall expects, bf16 bytes of shape
    [len(positions), B, heads, Dh] (one [B, heads, Dh] block per position)."""
    Dh = cfg.head_dim
    half = Dh // 2
    inv = cfg.rope_theta ** (-np.arange(half, dtype=np.float64) * 2.0 / Dh)
    ang = positions.astype(np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1).astype(np.float32)            # [P, Dh]
    shape = (len(positions), cfg.batch, heads, Dh)
    c = np.broadcast_to(np.cos(ang)[:, None, None, :], shape)
    s = np.broadcast_to(np.sin(ang)[:, None, None, :], shape)
    return bf16_bytes(c), bf16_bytes(s)


def rope_tables_rows(cfg: DecoderConfig, positions: np.ndarray, heads: int) -> tuple:
    """cos/sin for a prompt pass: bf16 bytes of shape [B, len(positions), heads, Dh]
    (every sequence at the same positions), the token-major rows of build_prefill."""
    c, s = rope_tables(cfg, positions, heads)
    shape = (len(positions), cfg.batch, heads, cfg.head_dim)
    tr = lambda b: np.ascontiguousarray(
        np.frombuffer(b, np.uint16).reshape(shape).transpose(1, 0, 2, 3)).tobytes()
    return tr(c), tr(s)
