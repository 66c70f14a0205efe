"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every
function include/holo_hip.h declares; the host-side refusals mirror the
reference CPU kernels' (src/cpu/kernels.rs, float_kernels.rs, buffer.rs); the
wire codec agrees with kernel_codec.rs; the host-built tables equal the
oracle's. No device work."""
import ctypes
import re
import struct

import numpy as np
import pytest

import oracle
from conftest import ROOT
from hologram_amd import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, BufferRef, DecodeAttentionCall,
                          DecodeAttentionI8Call,
                          KernelCall, KvCacheWriteCall, KvQuantAppendCall, MatMulCall,
                          NormCall, SlotOutOfRange, UnaryCall, UnsupportedOp, decode_call, lut_table,
                          validate)
from hologram_amd import _ffi


def declared_functions():
    text = (ROOT / "include" / "holo_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(holo_hip_\w+)\s*\(", text,
                                 re.M)))


def test_library_exports_every_declared_symbol():
    lib = _ffi.lib()
    names = declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert name in _ffi.SIGNATURES, f"{name} has no ctypes signature"


def test_no_device_backend_create_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    from hologram_amd import HipBackend, InitError
    with pytest.raises(InitError):
        HipBackend(0)


@pytest.mark.parametrize("act", range(6))
@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16])
def test_host_tables_equal_oracle(act, dtype):
    assert np.array_equal(lut_table(act, dtype), oracle.build_table(act, dtype))


@pytest.mark.parametrize("table,fused", [(6, 1), (7, 6), (8, 7)])   # Relu, Elu, Selu
@pytest.mark.parametrize("dtype", [DTYPE_BF16, DTYPE_F16])
def test_host_relu_elu_selu_tables_are_widen_f_narrow(table, fused, dtype):
    """16-bit Relu / Elu / Selu run unary_float (float_kernels.rs:170-233):
    widen, the scalar f, narrow (bf16 truncation, f16 the reference's rule);
    a table of that over all 65536 patterns is the same map."""
    bits = np.arange(65536, dtype=np.uint16)
    L = oracle.lib()
    if dtype == DTYPE_BF16:
        x = (bits.astype(np.uint32) << 16).view(np.float32)
        want = (oracle.fused_act_f32(fused, x).view(np.uint32) >> 16).astype(np.uint16)
    else:
        x = np.array([L.or_f16_to_f32(int(b)) for b in bits], np.float32)
        y = oracle.fused_act_f32(fused, x)
        want = np.array([L.or_f32_to_f16(float(v)) for v in y], np.uint16)
    assert np.array_equal(lut_table(table, dtype), want)


def test_unknown_table_not_built():
    with pytest.raises(UnsupportedOp):
        lut_table(9, DTYPE_BF16)


# ---- refusals (validate = dispatch's host checks, no device) -----------------

def unary(n, dtype=DTYPE_BF16, inp=BufferRef(0), out=BufferRef(1)):
    return KernelCall.Gelu(UnaryCall(inp, out, n, 16, dtype))


def test_unary_sizes():
    validate(unary(8), [16, 16])
    with pytest.raises(SlotOutOfRange):
        validate(unary(9), [16, 18])        # input short
    with pytest.raises(SlotOutOfRange):
        validate(unary(8), [16, 15])        # output short
    with pytest.raises(SlotOutOfRange):
        validate(unary(8), [16])            # output slot unbound
    validate(unary(8, DTYPE_F32), [32, 32])  # f32: computed, not tabled
    with pytest.raises(SlotOutOfRange):
        validate(unary(8, DTYPE_F32), [32, 31])
    with pytest.raises(UnsupportedOp):
        validate(unary(8, 2), [64, 64])     # the integer ring form is not served here
    validate(unary(0), [])                  # empty is a no-op before any lookup


def test_split_borrow_overlap_rule():
    # same slot, disjoint ranges: allowed (buffer.rs:974-998)
    validate(unary(4, inp=BufferRef(0, 0, 8), out=BufferRef(0, 8, 8)), [16])
    with pytest.raises(SlotOutOfRange):
        validate(unary(4, inp=BufferRef(0, 0, 8), out=BufferRef(0, 4, 8)), [16])


def test_view_offsets_clamp_like_buf_range():
    # offset past the end resolves to an empty view -> too short
    with pytest.raises(SlotOutOfRange):
        validate(unary(1, inp=BufferRef(0, 100)), [16, 16])


def test_matmul_refusals():
    mm = lambda **kw: KernelCall.MatMul(MatMulCall(BufferRef(0), BufferRef(1), BufferRef(2),
                                                   **kw))
    validate(mm(m=2, k=3, n=4, dtype=DTYPE_F32), [24, 48, 32])
    with pytest.raises(SlotOutOfRange):
        validate(mm(m=2, k=3, n=4, dtype=DTYPE_F32), [24, 47, 32])
    validate(mm(m=2, k=3, n=4, dtype=DTYPE_F16), [12, 24, 16])    # f16 is served
    with pytest.raises(SlotOutOfRange):
        validate(mm(m=2, k=3, n=4, dtype=DTYPE_F16), [12, 23, 16])
    with pytest.raises(UnsupportedOp):                                # i8 is no MatMul dtype
        validate(mm(m=2, k=3, n=4, dtype=2), [24, 48, 32])
    # a packed B spans layout::packed_len(k, n) = ceil(n/16)*k*16 elements
    # (float_kernels.rs:317-324); the compiler packs f32 weights only
    with pytest.raises(SlotOutOfRange):
        validate(mm(m=2, k=3, n=4, dtype=DTYPE_F32, b_packed=True), [24, 48, 32])
    validate(mm(m=2, k=3, n=4, dtype=DTYPE_F32, b_packed=True), [24, 192, 32])
    with pytest.raises(UnsupportedOp):
        validate(mm(m=2, k=3, n=4, dtype=DTYPE_BF16, b_packed=True), [24, 96, 32])
    validate(mm(m=0, k=3, n=4, dtype=DTYPE_F32), [])


def test_kv_write_refusals():
    kw = lambda **k: KernelCall.KvCacheWrite(KvCacheWriteCall(
        BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), **k))
    validate(kw(planes=2, bucket_rows=4, new_rows=1, row_bytes=8), [64, 16, 4, 64])
    with pytest.raises(UnsupportedOp):
        validate(kw(planes=2, bucket_rows=4, new_rows=5, row_bytes=8), [64, 80, 4, 64])
    with pytest.raises(UnsupportedOp):
        validate(kw(planes=2, bucket_rows=0, new_rows=0, row_bytes=8), [64, 16, 4, 64])
    with pytest.raises(SlotOutOfRange):
        validate(kw(planes=2, bucket_rows=4, new_rows=1, row_bytes=8), [64, 16, 3, 64])


def test_kv_quant_append_forms():
    def call(out_q, out_s, **k):
        return KernelCall.KvQuantAppend(KvQuantAppendCall(
            BufferRef(0), BufferRef(1), BufferRef(2), BufferRef(3), out_q, out_s, **k))
    geo = dict(planes=2, bucket_rows=4, new_rows=1, head_dim=8, dtype=DTYPE_BF16)
    sizes = [32, 4, 64, 32, 64, 32]
    validate(call(BufferRef(4), BufferRef(5), **geo), sizes)          # copy form
    validate(call(BufferRef(2), BufferRef(3), **geo), sizes)          # in-place form
    with pytest.raises(SlotOutOfRange):                              # output aliases new rows
        validate(call(BufferRef(0), BufferRef(5), **geo), [64, 4, 64, 32, 64, 32])
    with pytest.raises(UnsupportedOp):
        validate(call(BufferRef(4), BufferRef(5), **{**geo, "dtype": 2}), sizes)


def test_attn_refusals():
    def call(**k):
        return KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
            *[BufferRef(s) for s in range(7)], **k))
    B, H, Hkv, bucket, D = 2, 8, 2, 16, 128
    rows = B * Hkv * bucket
    sizes = [B * H * D * 2, rows * D, rows * D, rows * 4, rows * 4, B * 4, B * H * D * 2]
    validate(call(batch=B, heads=H, kv_heads=Hkv, bucket_rows=bucket, head_dim=D), sizes)
    with pytest.raises(UnsupportedOp):
        validate(call(batch=B, heads=H, kv_heads=3, bucket_rows=bucket, head_dim=D), sizes)
    # any head_dim up to 4096 is served (head_dim 96: the generic kernel)
    d96 = [B * H * 96 * 2, rows * 96, rows * 96, rows * 4, rows * 4, B * 4, B * H * 96 * 2]
    validate(call(batch=B, heads=H, kv_heads=Hkv, bucket_rows=bucket, head_dim=96), d96)
    with pytest.raises(UnsupportedOp):
        validate(call(batch=B, heads=H, kv_heads=Hkv, bucket_rows=bucket, head_dim=8192),
                 [x * 64 for x in sizes])
    with pytest.raises(SlotOutOfRange):
        short = list(sizes)
        short[5] = 4
        validate(call(batch=B, heads=H, kv_heads=Hkv, bucket_rows=bucket, head_dim=D), short)


def test_decode_attention_mask_form_refusals():
    """decode_attention_float's refusals (float_kernels.rs:2489-2580): an empty
    key list, kv_heads not dividing heads, a mask shorter than q_rows * (past +
    new) f32, and a dtype other than f32/f16/bf16 after the buffer checks."""
    def call(**k):
        geo = dict(batch=2, heads=4, kv_heads=2, q_rows=3, past_len=5, new_len=2, head_dim=8,
                   scale_bits=0, dtype=DTYPE_BF16)
        geo.update(k)
        return KernelCall.DecodeAttention(DecodeAttentionCall(
            *[BufferRef(s) for s in range(7)], **geo))
    es, B, H, Hkv, M, P, N, D = 2, 2, 4, 2, 3, 5, 2, 8
    sizes = [B * H * M * D * es, B * Hkv * P * D * es, B * Hkv * P * D * es,
             B * Hkv * N * D * es, B * Hkv * N * D * es, M * (P + N) * 4, B * H * M * D * es]
    validate(call(), sizes)
    validate(call(batch=0), sizes)
    with pytest.raises(UnsupportedOp):
        validate(call(past_len=0, new_len=0), sizes)
    with pytest.raises(UnsupportedOp):
        validate(call(kv_heads=3), sizes)
    short = list(sizes)
    short[5] -= 4
    with pytest.raises(SlotOutOfRange):
        validate(call(), short)
    with pytest.raises(UnsupportedOp):
        validate(call(dtype=2), [s // 2 if i != 5 else s for i, s in enumerate(sizes)])


def test_unknown_tag_is_unsupported():
    kc = _ffi.KernelCallC()
    kc.tag = 64   # Softmax: no device kernel here
    with pytest.raises(UnsupportedOp):
        from hologram_amd.backend import check
        check(_ffi.lib().holo_hip_validate(ctypes.byref(kc), None, 0))


# ---- wire codec ---------------------------------------------------------------

def test_codec_layout_matches_kernel_codec():
    c = KernelCall.MatMul(MatMulCall(BufferRef(1, 2, 3), BufferRef(4), BufferRef(5, 6), 7, 8, 9,
                                     DTYPE_BF16))
    wire = c.encode()
    # u16 discriminant 46, three (u32, u64, u64) refs, three u32, two u8
    assert len(wire) == 2 + 3 * 20 + 12 + 2
    assert struct.unpack_from("<H", wire)[0] == 46
    kc, used = decode_call(wire)
    assert used == len(wire)
    m = kc.u.matmul
    assert (m.a.slot, m.a.offset, m.a.length) == (1, 2, 3)
    assert (m.m, m.k, m.n, m.dtype, m.b_packed) == (7, 8, 9, DTYPE_BF16, 0)


@pytest.mark.parametrize("call", [
    KernelCall.Exp(UnaryCall(BufferRef(3), BufferRef(4, 16, 32), 99, 16, DTYPE_F16)),
    KernelCall.Erf(UnaryCall(BufferRef(1), BufferRef(2), 7, 32, DTYPE_F32)),
    KernelCall.AddRmsNorm(NormCall(BufferRef(0), BufferRef(1), BufferRef(2), 3, 64, 0x3727C5AC,
                                   DTYPE_F32, residual=BufferRef(5, 8, 0))),
    KernelCall.KvCacheWrite(KvCacheWriteCall(BufferRef(0), BufferRef(1), BufferRef(2),
                                             BufferRef(3), 5, 6, 1, 128)),
    KernelCall.KvQuantAppend(KvQuantAppendCall(*[BufferRef(i) for i in range(6)], 128, 4096, 1,
                                               128, DTYPE_BF16)),
    KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(*[BufferRef(i) for i in range(7)], 32, 32,
                                                       8, 32768, 128, 0, DTYPE_BF16)),
    KernelCall.DecodeAttention(DecodeAttentionCall(*[BufferRef(i, i, 2 * i) for i in range(7)], 1,
                                                   32, 8, 4, 4096, 4, 128, 0x3E000000,
                                                   DTYPE_F16)),
])
def test_codec_round_trip(call):
    wire = call.encode()
    kc, used = decode_call(wire + b"\xff\xff")     # trailing bytes belong to the next call
    assert used == len(wire)
    assert bytes(kc) == bytes(call.to_c())


def test_codec_truncated_payload():
    from hologram_amd import DispatchError
    wire = KernelCall.Gelu(UnaryCall(BufferRef(0), BufferRef(1), 5)).encode()
    with pytest.raises(DispatchError):
        decode_call(wire[:-1])


def test_ctypes_layouts_match_the_header(tmp_path):
    """Every call struct the ctypes binding declares has the C header's size and
    field offsets (a drift would hand the library garbage)."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("no C compiler")
    pairs = [(name[:-1], cls) for name, cls in vars(_ffi).items()
             if name.endswith("C") and isinstance(cls, type)
             and issubclass(cls, ctypes.Structure) and name != "KernelCallC"]
    cname = {"BufferRef": "holo_buffer_ref", "KernelCall": "holo_kernel_call"}

    def c_name(py):
        if py in cname:
            return cname[py]
        return "holo_" + re.sub(r"(?<!^)(?=[A-Z])", "_", py).lower()
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "holo_hip.h"', 'int main(void){']
    checks = []
    for py, cls in pairs + [("KernelCall", _ffi.KernelCallC)]:
        c = {"MatMulActCall": "holo_matmul_act_call", "MatMulAddCall": "holo_matmul_add_call",
             "MatMulAddActCall": "holo_matmul_add_act_call", "MatMulCall": "holo_matmul_call",
             "MatMulDequantCall": "holo_matmul_dequant_call",
             "DecodeAttentionI8Call": "holo_decode_attention_i8_call",
             "AttentionI8RowsCall": "holo_attention_i8_rows_call",
             "ArgMaxCall": "holo_argmax_call", "KvCacheWriteCall": "holo_kv_cache_write_call",
             "KvQuantAppendCall": "holo_kv_quant_append_call",
             "DecodeAttentionValidCall": "holo_decode_attention_valid_call",
             "DequantActivationCall": "holo_dequant_activation_call",
             "RopeCall": "holo_rope_call"}.get(py) or c_name(py)
        lines.append(f'printf("%zu\\n", sizeof({c}));')
        checks.append((py, "sizeof", ctypes.sizeof(cls)))
        for f, _ in cls._fields_:
            lines.append(f'printf("%zu\\n", offsetof({c}, {f}));')
            checks.append((py, f, getattr(cls, f).offset))
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    assert len(got) == len(checks)
    for (py, what, want), g in zip(checks, got):
        assert g == want, f"{py}.{what}: C {g}, ctypes {want}"
