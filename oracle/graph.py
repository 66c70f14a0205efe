"""CPU restatement of the reference's `.holo` session walk, TEST INFRASTRUCTURE.

Reads an archive on its own (header, section table, BLAKE3 footer with the
pure-Python hash, loader.rs:141-263; ports, exec plan, constants and weights,
writer.rs / constant_codec.rs; kernel calls from the reference wire form,
kernel_codec.rs put_*), then walks the plan level by level over host slot
buffers, each node computed by the C oracle's restatement of the reference
CPU kernel (session.rs compute_and_label :1052-1289 with the CpuBackend;
honest-copy KV writes, no memo). Imported only by tests/ and bench.py's CPU
leg, as the checker of hologram_amd's HipSession.
"""
from __future__ import annotations

import struct

import numpy as np

from . import _p, lib
from .blake3_ref import blake3

DT_BYTES = {0: 1, 1: 1, 2: 1, 3: 8, 4: 4, 5: 8, 6: 2, 7: 2, 8: 4, 9: 8}
BF16, F32 = 7, 8


class _R:
    def __init__(self, b: bytes, at: int = 0):
        self.b, self.at = b, at

    def u(self, fmt: str):
        v = struct.unpack_from("<" + fmt, self.b, self.at)
        self.at += struct.calcsize("<" + fmt)
        return v if len(v) > 1 else v[0]

    def buf(self):
        return self.u("IQQ")

    def take(self, n: int) -> bytes:
        v = self.b[self.at:self.at + n]
        self.at += n
        return v


# per-tag field layout of the reference encoders (kernel_codec.rs put_*)
def _decode_call(r: _R) -> tuple:
    tag = r.u("H")
    if tag in (12, 13, 14, 15, 18):                  # put_unary
        return tag, dict(input=r.buf(), output=r.buf(), n=r.u("Q"), witt=r.u("H"), dtype=r.u("B"))
    if tag in (5, 7):                                # put_binary
        return tag, dict(a=r.buf(), b=r.buf(), output=r.buf(), n=r.u("Q"), witt=r.u("H"),
                         dtype=r.u("B"))
    if tag == 51:                                    # put_norm
        return tag, dict(x=r.buf(), gamma=r.buf(), beta=r.buf(), residual=r.buf(),
                         output=r.buf(), batch=r.u("I"), feature=r.u("I"), channels=r.u("I"),
                         groups=r.u("I"), eps=r.u("Q"), dtype=r.u("B"))
    if tag == 75:                                    # put_rope
        return tag, dict(x=r.buf(), cos=r.buf(), sin=r.buf(), output=r.buf(), head_dim=r.u("I"),
                         n=r.u("Q"), dtype=r.u("B"))
    if tag == 114:                                   # put_gather
        return tag, dict(data=r.buf(), idx=r.buf(), output=r.buf(), outer=r.u("Q"),
                         axis=r.u("Q"), inner=r.u("Q"), num=r.u("Q"), idx_dtype=r.u("B"),
                         dtype=r.u("B"))
    if tag == 119:                                   # put_decattn
        return tag, dict(q=r.buf(), kp=r.buf(), vp=r.buf(), kn=r.buf(), vn=r.buf(),
                         mask=r.buf(), output=r.buf(), batch=r.u("I"), heads=r.u("I"),
                         kv_heads=r.u("I"), q_rows=r.u("I"), past=r.u("I"), new=r.u("I"),
                         head_dim=r.u("I"), scale_bits=r.u("I"), dtype=r.u("B"))
    if tag == 121:                                   # put_davl
        return tag, dict(q=r.buf(), kp=r.buf(), vp=r.buf(), kn=r.buf(), vn=r.buf(),
                         valid=r.buf(), output=r.buf(), batch=r.u("I"), heads=r.u("I"),
                         kv_heads=r.u("I"), q_rows=r.u("I"), past=r.u("I"), new=r.u("I"),
                         head_dim=r.u("I"), scale_bits=r.u("I"), dtype=r.u("B"))
    if tag == 46:                                    # put_matmul
        return tag, dict(a=r.buf(), b=r.buf(), output=r.buf(), m=r.u("I"), k=r.u("I"),
                         n=r.u("I"), dtype=r.u("B"), packed=r.u("B"))
    if tag in (106, 107, 108):                       # put_matmul + epilogue (:509-524)
        c = dict(a=r.buf(), b=r.buf(), output=r.buf(), m=r.u("I"), k=r.u("I"), n=r.u("I"),
                 dtype=r.u("B"), packed=r.u("B"))
        if tag != 106:
            c["residual"] = r.buf()
        if tag != 107:
            c["act"] = r.u("B")
        return tag, c
    if tag == 122:                                   # int8 quantize + append (new)
        return tag, dict(new=r.buf(), pos=r.buf(), cache=r.buf(), scales=r.buf(),
                         output=r.buf(), output_scales=r.buf(), planes=r.u("I"),
                         bucket=r.u("I"), new_rows=r.u("I"), head_dim=r.u("I"), dtype=r.u("B"))
    if tag == 123:                                   # int8 decode attention (new)
        return tag, dict(q=r.buf(), kq=r.buf(), vq=r.buf(), ks=r.buf(), vs=r.buf(),
                         lens=r.buf(), output=r.buf(), batch=r.u("I"), heads=r.u("I"),
                         kv_heads=r.u("I"), bucket=r.u("I"), head_dim=r.u("I"),
                         scale_bits=r.u("I"), dtype=r.u("B"))
    if tag == 125:                                   # multi-row int8 attention (new)
        return tag, dict(q=r.buf(), kq=r.buf(), vq=r.buf(), ks=r.buf(), vs=r.buf(),
                         lens=r.buf(), output=r.buf(), batch=r.u("I"), heads=r.u("I"),
                         kv_heads=r.u("I"), bucket=r.u("I"), head_dim=r.u("I"),
                         scale_bits=r.u("I"), dtype=r.u("B"), q_rows=r.u("I"))
    if tag == 61:                                    # put_transpose
        c = dict(input=r.buf(), output=r.buf(), rank=r.u("B"))
        c["dims"] = [r.u("I") for _ in range(8)][:c["rank"]]
        c["perm"] = [r.u("B") for _ in range(8)][:c["rank"]]
        c["dtype"] = r.u("B")
        return tag, c
    if tag in (60, 63):                              # put_layout (Reshape, Slice)
        return tag, dict(input=r.buf(), output=r.buf(), n=r.u("Q"), dtype=r.u("B"))
    if tag == 124:                                   # argmax (new)
        return tag, dict(input=r.buf(), output=r.buf(), rows=r.u("I"), cols=r.u("I"),
                         dtype=r.u("B"))
    raise ValueError(f"oracle graph: no restatement for discriminant {tag}")


def _ports(b: bytes) -> list:
    r = _R(b)
    out = []
    for _ in range(r.u("I")):
        name = r.take(r.u("H")).decode()
        slot, count, dtype, rank = r.u("IQBB")
        shape = [r.u("Q") for _ in range(rank)]
        out.append(dict(name=name, slot=slot, count=count, dtype=dtype, shape=shape))
    return out


class OracleSession:
    """Load an archive and run it on the CPU oracle, step by step."""

    def __init__(self, archive: bytes, verify_footer: bool = True, products: str = "f64",
                 threads: int = 1):
        """products: "f64" sums every MatMul in f64 (the reference metric's
        exact product, tests/conformance.rs:100-112); "f32" sums in f32
        through numpy's BLAS (as the reference CPU engine accumulates in f32,
        in another order). Two walks that differ only here measure how far
        two correct bf16 walks of the same archive land apart.
        "cpu_baseline" times the reference CPU engines instead (bench.py's
        CPU leg): MatMul through oracle/cpu_baseline.c's restatement of the
        reference kernels (few-row bf16 streamed, simd.rs:3808-3858; else the
        blocked f32 engine), decode attention through its two-pass rows, on
        `threads` host threads, and int8 appends in place as the reference
        executor's KV move does (session.rs:1313-1370)."""
        if products not in ("f64", "f32", "cpu_baseline"):
            raise ValueError(products)
        self.products = products
        self.threads = threads
        if archive[:4] != b"HOLO":
            raise ValueError("bad magic")
        ver, _flags, nsec = struct.unpack_from("<HHH", archive, 4)
        if not 2 <= ver <= 3:
            raise ValueError(f"unsupported version {ver}")
        if verify_footer and blake3(archive[:-32]) != archive[-32:]:
            raise ValueError("footer fingerprint mismatch")
        sec = {}
        for i in range(nsec):
            kind, off, n = struct.unpack_from("<B7xQQ", archive, 10 + 24 * i)
            sec.setdefault(kind, archive[off:off + n])
        r = _R(sec[1])
        self.calls = [_decode_call(r) for _ in range(r.u("I"))]
        self.inputs = _ports(sec.get(9, struct.pack("<I", 0)))
        self.outputs = _ports(sec.get(10, struct.pack("<I", 0)))
        if 12 in sec:
            r = _R(sec[12])
            self.plan = [[r.u("I") for _ in range(r.u("I"))] for _ in range(r.u("I"))]
        else:
            self.plan = [list(range(len(self.calls)))]
        weights = {}
        if 3 in sec:
            r = _R(sec[3])
            for _ in range(r.u("I")):
                fp = r.take(32)
                weights[fp] = r.take(r.u("Q"))
        self.slots: dict[int, np.ndarray] = {}
        if 11 in sec:
            r = _R(sec[11])
            for _ in range(r.u("I")):
                tag, slot, _dt = r.u("BIB")
                body = r.take(r.u("I")) if tag == 0 else weights[r.take(32)]
                self.slots[slot] = np.frombuffer(body, np.uint8).copy()

    # slot access: a BufferRef view as a numpy byte array
    def _view(self, ref, nbytes=None) -> np.ndarray:
        slot, off, length = ref
        buf = self.slots[slot]
        end = len(buf) if length == 0 else min(off + length, len(buf))
        v = buf[min(off, len(buf)):end]
        return v if nbytes is None else v[:nbytes]

    def _out(self, ref, nbytes: int) -> np.ndarray:
        slot, off, _ = ref
        need = off + nbytes
        if slot not in self.slots or len(self.slots[slot]) < need:
            old = self.slots.get(slot)
            self.slots[slot] = np.zeros(max(need, 64), np.uint8)
            if old is not None:
                self.slots[slot][:len(old)] = old
        return self.slots[slot][off:off + nbytes]

    def set_input(self, index: int, data: bytes) -> None:
        self.slots[self.inputs[index]["slot"]] = np.frombuffer(bytes(data), np.uint8).copy()

    def output(self, index: int) -> np.ndarray:
        p = self.outputs[index]
        return self.slots[p["slot"]][:p["count"] * DT_BYTES[p["dtype"]]]

    def run(self) -> None:
        for level in self.plan:
            for i in level:
                self._node(*self.calls[i])

    def _node(self, tag: int, c: dict) -> None:
        L = lib()
        if tag in (12, 13, 14, 15, 18):
            from . import build_table
            act = {12: 0, 13: 1, 14: 2, 15: 3, 18: 4}[tag]
            t = build_table(act, c["dtype"])
            x = np.ascontiguousarray(self._view(c["input"], 2 * c["n"]).view(np.uint16))
            o = self._out(c["output"], 2 * c["n"]).view(np.uint16)
            L.or_unary_lut(_p(t), _p(x), _p(o), c["n"])
        elif tag in (5, 7):
            es = DT_BYTES[c["dtype"]]
            a = np.ascontiguousarray(self._view(c["a"], es * c["n"]))
            b = np.ascontiguousarray(self._view(c["b"], es * c["n"]))
            o = np.zeros(es * c["n"], np.uint8)
            L.or_binary(0 if tag == 5 else 1, _p(a), _p(b), _p(o), c["n"], c["dtype"])
            self._out(c["output"], es * c["n"])[:] = o
        elif tag == 51:
            es = DT_BYTES[c["dtype"]]
            n = c["batch"] * c["feature"] * es
            x = np.ascontiguousarray(self._view(c["x"], n))
            g = None
            if c["gamma"][0] != 0xFFFFFFFF:
                g = np.ascontiguousarray(self._view(c["gamma"], c["feature"] * es))
            o = np.zeros(n, np.uint8)
            rc = L.or_rms_norm(_p(x), _p(g) if g is not None else None, _p(o), c["batch"],
                               c["feature"], c["eps"], c["dtype"])
            if rc != 0:
                raise ValueError("rms_norm refused")
            self._out(c["output"], n)[:] = o
        elif tag == 75:
            es = DT_BYTES[c["dtype"]]
            n = c["n"] * es
            x, cs, sn = (np.ascontiguousarray(self._view(c[k], n)) for k in ("x", "cos", "sin"))
            o = np.zeros(n, np.uint8)
            if L.or_rope(_p(x), _p(cs), _p(sn), _p(o), c["head_dim"], c["n"], c["dtype"]) != 0:
                raise ValueError("rope refused")
            self._out(c["output"], n)[:] = o
        elif tag == 114:
            es = DT_BYTES[c["dtype"]]
            row = c["inner"] * es
            iw = 8 if c["idx_dtype"] == 5 else 4
            d = np.ascontiguousarray(self._view(c["data"], c["outer"] * c["axis"] * row))
            ix = np.ascontiguousarray(self._view(c["idx"], c["num"] * iw))
            o = np.zeros(c["outer"] * c["num"] * row, np.uint8)
            if L.or_gather(_p(d), _p(ix), _p(o), c["outer"], c["axis"], row, c["num"],
                           int(iw == 8)) != 0:
                raise ValueError("gather: index out of range")
            self._out(c["output"], len(o))[:] = o
        elif tag in (46, 106, 107, 108):
            # matmul_float, then the fused epilogues of float_kernels.rs:816-935
            m, k, n = c["m"], c["k"], c["n"]
            dt = c["dtype"]
            es = DT_BYTES[dt]
            def operands():
                a = self._f32(self._view(c["a"], m * k * es), dt)
                if c["packed"]:                      # layout.rs:16-45 (f32 weights only)
                    if dt != F32:
                        raise ValueError("a panel-packed B is an f32 layout")
                    from . import packed_len, unpack_b_panels
                    b = unpack_b_panels(self._f32(self._view(c["b"], packed_len(k, n) * 4), dt),
                                        k, n)
                else:
                    b = self._f32(self._view(c["b"], k * n * es), dt)
                return a, b
            from . import FUSED_TO_LUT, build_table, fused_act_f32, matmul_f64_blas, matmul_ref_f64
            if self.products == "cpu_baseline" and dt == BF16:
                raw_a = np.ascontiguousarray(self._view(c["a"], m * k * es))
                raw_b = np.ascontiguousarray(self._view(c["b"], k * n * es))
                prod = self._baseline_matmul(None, None, raw_a, raw_b, m, k, n, dt)
            elif self.products == "cpu_baseline":
                prod = self._baseline_matmul(*operands(), None, None, m, k, n, dt)
            elif self.products == "f32":
                a, b = operands()
                prod = (a.reshape(m, k) @ b.reshape(k, n)).ravel()
            else:
                a, b = operands()
                ref = matmul_ref_f64 if m * k * n <= (1 << 24) else matmul_f64_blas
                prod = ref(a, b, m, k, n)
            v = self._f32(self._narrow(prod, dt), dt)
            if tag in (107, 108):
                v = v + self._f32(self._view(c["residual"], m * n * es), dt)
            if tag == 106 and dt == BF16 and c["act"] not in FUSED_TO_LUT:
                # Relu/Elu/Selu on a 16-bit product: f on the widened value, narrowed
                v = fused_act_f32(c["act"], v)
            elif tag == 106 and dt == BF16:
                t = build_table(FUSED_TO_LUT[c["act"]], dt)
                v = self._f32(t[self._narrow(v, dt).view(np.uint16)].view(np.uint8), dt)
            elif tag in (106, 108):
                v = fused_act_f32(c["act"], v)
            self._out(c["output"], m * n * es)[:] = self._narrow(v, dt)
        elif tag == 122 and self.products == "cpu_baseline":
            # the executor's in-place move: the cache slots are updated and the
            # output slots alias them (no honest copy of the whole cache)
            P, S, R, Dh = c["planes"], c["bucket"], c["new_rows"], c["head_dim"]
            es = DT_BYTES[c["dtype"]]
            new = np.ascontiguousarray(self._view(c["new"], P * R * Dh * es))
            pos = int(np.ascontiguousarray(self._view(c["pos"], 4)).view(np.uint32)[0])
            cq, cs = self.slots[c["cache"][0]], self.slots[c["scales"][0]]
            if L.or_kv_quant_append(_p(new), c["dtype"], pos, _p(cq), _p(cs), P, S, R, Dh) != 0:
                raise ValueError("kv_quant_append refused")
            self.slots[c["output"][0]] = cq
            self.slots[c["output_scales"][0]] = cs
        elif tag == 122:
            P, S, R, Dh = c["planes"], c["bucket"], c["new_rows"], c["head_dim"]
            es = DT_BYTES[c["dtype"]]
            new = np.ascontiguousarray(self._view(c["new"], P * R * Dh * es))
            pos = int(np.ascontiguousarray(self._view(c["pos"], 4)).view(np.uint32)[0])
            cq = np.ascontiguousarray(self._view(c["cache"], P * S * Dh)).view(np.int8).copy()
            cs = np.ascontiguousarray(self._view(c["scales"], P * S * 4)).view(np.float32).copy()
            if L.or_kv_quant_append(_p(new), c["dtype"], pos, _p(cq), _p(cs), P, S, R, Dh) != 0:
                raise ValueError("kv_quant_append refused")
            self._out(c["output"], P * S * Dh)[:] = cq.view(np.uint8)
            self._out(c["output_scales"], P * S * 4)[:] = cs.view(np.uint8)
        elif tag == 123:
            B, H, Hkv, S, D = c["batch"], c["heads"], c["kv_heads"], c["bucket"], c["head_dim"]
            es = DT_BYTES[c["dtype"]]
            q = self._f32(self._view(c["q"], B * H * D * es), c["dtype"])
            kq = np.ascontiguousarray(self._view(c["kq"], B * Hkv * S * D)).view(np.int8)
            vq = np.ascontiguousarray(self._view(c["vq"], B * Hkv * S * D)).view(np.int8)
            ks = np.ascontiguousarray(self._view(c["ks"], B * Hkv * S * 4)).view(np.float32)
            vs = np.ascontiguousarray(self._view(c["vs"], B * Hkv * S * 4)).view(np.float32)
            lens = np.ascontiguousarray(self._view(c["lens"], B * 4)).view(np.uint32)
            from . import attn_scale, decode_attention_i8
            if self.products == "cpu_baseline":
                o = np.zeros(B * H * D, np.float32)
                q = np.ascontiguousarray(q)
                lens = np.ascontiguousarray(lens)
                L.cb_decode_attention_i8(_p(q), _p(kq), _p(ks), _p(vq), _p(vs), _p(lens), _p(o),
                                         B, H, Hkv, S, D, attn_scale(D, c["scale_bits"]),
                                         self.threads)
            else:
                o = decode_attention_i8(q, kq, ks, vq, vs, lens, B, H, Hkv, S, D,
                                        attn_scale(D, c["scale_bits"]))
            self._out(c["output"], B * H * D * es)[:] = self._narrow(o, c["dtype"])
        elif tag == 121:
            B, H, M, D = c["batch"], c["heads"], c["q_rows"], c["head_dim"]
            hkv = H if c["kv_heads"] == 0 else c["kv_heads"]
            es = DT_BYTES[c["dtype"]]
            pn, nn = B * hkv * c["past"] * D * es, B * hkv * c["new"] * D * es
            ops = [np.ascontiguousarray(self._view(c[k], n)) for k, n in
                   (("q", B * H * M * D * es), ("kp", pn), ("vp", pn), ("kn", nn), ("vn", nn))]
            valid = int(np.ascontiguousarray(self._view(c["valid"], 4)).view(np.uint32)[0])
            from . import decode_attention_valid
            o = decode_attention_valid(*ops, valid, B, H, c["kv_heads"], M, c["past"], c["new"],
                                       D, c["scale_bits"], c["dtype"])
            self._out(c["output"], o.nbytes)[:] = o.view(np.uint8)
        elif tag == 119:
            B, H, M, D = c["batch"], c["heads"], c["q_rows"], c["head_dim"]
            hkv = H if c["kv_heads"] == 0 else c["kv_heads"]
            es = DT_BYTES[c["dtype"]]
            pn, nn = B * hkv * c["past"] * D * es, B * hkv * c["new"] * D * es
            ops = [np.ascontiguousarray(self._view(c[k], n)) for k, n in
                   (("q", B * H * M * D * es), ("kp", pn), ("vp", pn), ("kn", nn), ("vn", nn))]
            mask = np.ascontiguousarray(self._view(c["mask"], M * (c["past"] + c["new"]) * 4))
            from . import decode_attention
            o = decode_attention(*ops, mask.view(np.float32), B, H, c["kv_heads"], M, c["past"],
                                 c["new"], D, c["scale_bits"], c["dtype"])
            self._out(c["output"], o.nbytes)[:] = o.view(np.uint8)
        elif tag == 125:
            B, T, H, Hkv = c["batch"], c["q_rows"], c["heads"], c["kv_heads"]
            S, D = c["bucket"], c["head_dim"]
            es = DT_BYTES[c["dtype"]]
            q = self._f32(self._view(c["q"], B * T * H * D * es), c["dtype"])
            kq = np.ascontiguousarray(self._view(c["kq"], B * Hkv * S * D)).view(np.int8)
            vq = np.ascontiguousarray(self._view(c["vq"], B * Hkv * S * D)).view(np.int8)
            ks = np.ascontiguousarray(self._view(c["ks"], B * Hkv * S * 4)).view(np.float32)
            vs = np.ascontiguousarray(self._view(c["vs"], B * Hkv * S * 4)).view(np.float32)
            lens = np.ascontiguousarray(self._view(c["lens"], B * 4)).view(np.uint32)
            from . import attention_i8_rows, attn_scale
            o = attention_i8_rows(q, kq, ks, vq, vs, lens, B, T, H, Hkv, S, D,
                                  attn_scale(D, c["scale_bits"]))
            self._out(c["output"], B * T * H * D * es)[:] = self._narrow(o, c["dtype"])
        elif tag == 61:
            es = DT_BYTES[c["dtype"]]
            n = int(np.prod(c["dims"]))
            x = np.ascontiguousarray(self._view(c["input"], n * es)).view(f"u{es}")
            from . import transpose
            self._out(c["output"], n * es)[:] = transpose(x, c["dims"], c["perm"]).view(np.uint8)
        elif tag in (60, 63):
            # layout_float / layout_copy (float_kernels.rs:2939-2954, kernels.rs:688-701):
            # element_count elements of a float dtype, element_count bytes otherwise;
            # f64 refused (kernels.rs:1611-1615). The reference walk binds an interior
            # Reshape / Slice as a view of its input: the same bytes.
            if c["dtype"] == 9:
                raise ValueError("f64 is not a supported compute dtype")
            nb = c["n"] * (DT_BYTES[c["dtype"]] if c["dtype"] in (6, 7, 8) else 1)
            x = self._view(c["input"])
            if len(x) < nb:
                raise ValueError("layout: input shorter than element_count")
            self._out(c["output"], nb)[:] = x[:nb]
        elif tag == 124:
            es = DT_BYTES[c["dtype"]]
            x = np.ascontiguousarray(self._view(c["input"], c["rows"] * c["cols"] * es))
            o = np.zeros(c["rows"], np.int32)
            L.or_argmax(_p(x), _p(o), c["rows"], c["cols"], c["dtype"])
            self._out(c["output"], 4 * c["rows"])[:] = o.view(np.uint8)
        else:
            raise ValueError(f"oracle graph: no restatement for discriminant {tag}")

    def _baseline_matmul(self, a, b, raw_a, raw_b, m, k, n, dt) -> np.ndarray:
        """The reference CPU MatMul engines (cpu_baseline.c), f32 result."""
        L = lib()
        th = self.threads
        if dt == BF16 and raw_b is not None:
            out = np.zeros(m * n, np.uint16)
            fn = L.cb_matmul_bf16_gemv if m <= 8 else L.cb_matmul_bf16
            fn(_p(raw_a), _p(raw_b), _p(out), m, k, n, th)
            return (out.astype(np.uint32) << 16).view(np.float32)
        out = np.zeros(m * n, np.float32)
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        L.cb_matmul_f32(_p(a), _p(b), _p(out), m, k, n, th)
        return out

    @staticmethod
    def _f32(b: np.ndarray, dtype: int) -> np.ndarray:
        b = np.ascontiguousarray(b)
        if dtype == BF16:
            return (b.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        return b.view(np.float32).copy()

    @staticmethod
    def _narrow(x: np.ndarray, dtype: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        if dtype == BF16:
            return (x.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        return x.view(np.uint8)
