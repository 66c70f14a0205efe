"""Python binding of the CPU oracle (oracle/libholo_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and the timed CPU baseline. The
product (hologram_amd/) never imports it. Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libholo_oracle.so"

DTYPE_I8, DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 2, 6, 7, 8
ACT_SIGMOID, ACT_TANH, ACT_GELU, ACT_SILU, ACT_EXP, ACT_ERF = 0, 1, 2, 3, 4, 5

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_U32 = ctypes.c_uint32
_F = ctypes.c_float
_SIGS = {
    "or_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "or_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "or_f16_to_f32": (_F, [ctypes.c_uint16]),
    "or_f32_to_f16": (ctypes.c_uint16, [_F]),
    "or_exp_f32_det": (_F, [_F]),
    "or_libm_expf": (_F, [_F]),
    "or_libm_erff": (_F, [_F]),
    "or_sigmoid_f": (_F, [_F]),
    "or_tanh_f": (_F, [_F]),
    "or_gelu_f": (_F, [_F]),
    "or_silu_f": (_F, [_F]),
    "or_lut_act_ref": (_F, [ctypes.c_int, _F]),
    "or_fused_act_f32": (ctypes.c_int, [ctypes.c_int, _P, _P, _S]),
    "or_build_table": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _P]),
    "or_unary_lut": (None, [_P, _P, _P, _S]),
    "or_quantize_row_i8": (_F, [_P, _P, _S]),
    "or_matmul_q_omajor": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _S, _S, _S]),
    "or_matmul_i8_pc_omajor": (None, [_P, _P, _P, _P, _S, _S, _S]),
    "or_fnv1a_f32": (ctypes.c_uint64, [_P, _S]),
    "or_dequantize": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.c_int, _P, _P, _U32, _U32, _F,
                                     ctypes.c_int32, ctypes.c_int, _P]),
    "or_dequant_activation": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                             _F, ctypes.c_int32, _P]),
    "or_kv_cache_write": (ctypes.c_int, [_P, _P, _U32, _P, _U32, _U32, _U32, _U32]),
    "or_kv_quant_append": (ctypes.c_int, [_P, ctypes.c_int, _U32, _P, _P, _U32, _U32, _U32,
                                          _U32]),
    "or_dequant_i8": (None, [_P, _P, _P, _S, _S]),
    "or_attn_scale": (_F, [_U32, _U32]),
    "or_decode_attention_valid": (ctypes.c_int, [_P, _P, _P, _P, _P, _U32, _P] + [_U32] * 8
                                  + [ctypes.c_int]),
    "or_decode_attention_valid_f32": (None, [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32,
                                             _U32, _U32, _U32, _F, _U32]),
    "or_decode_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P] + [_U32] * 8
                            + [ctypes.c_int]),
    "or_decode_attention_mask_f32": (None, [_P] * 7 + [_U32] * 7 + [_F]),
    "or_decode_attention_i8": (None, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32,
                                      _F]),
    "or_binary": (None, [ctypes.c_int, _P, _P, _P, _S, ctypes.c_int]),
    "or_rms_norm": (ctypes.c_int, [_P, _P, _P, _U32, _U32, ctypes.c_uint64, ctypes.c_int]),
    "or_add_rms_norm": (ctypes.c_int, [_P, _P, _P, _P, _U32, _U32, ctypes.c_uint64, ctypes.c_int]),
    "or_rope": (ctypes.c_int, [_P, _P, _P, _P, _U32, _S, ctypes.c_int]),
    "or_gather": (ctypes.c_int, [_P, _P, _P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                 ctypes.c_uint64, ctypes.c_int]),
    "or_argmax": (None, [_P, _P, _U32, _U32, ctypes.c_int]),
    "or_matmul_ref_f64": (None, [_P, _P, _P, _S, _S, _S]),
    "or_max_rel_err": (ctypes.c_double, [_P, _P, _S]),
    # cpu_baseline.c (timing engines)
    "cb_lut": (None, [_P, _P, _P, _S, ctypes.c_int]),
    "cb_matmul_f32": (None, [_P, _P, _P, _S, _S, _S, ctypes.c_int]),
    "cb_matmul_bf16": (None, [_P, _P, _P, _S, _S, _S, ctypes.c_int]),
    "cb_matmul_bf16_gemv": (None, [_P, _P, _P, _S, _S, _S, ctypes.c_int]),
    "cb_kv_quant_append_copy": (ctypes.c_int, [_P, ctypes.c_int, _U32, _P, _P, _P, _P, _U32,
                                               _U32, _U32, _U32, ctypes.c_int]),
    "cb_decode_attention_i8": (None, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32,
                                      _F, ctypes.c_int]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


_TABLES: dict = {}


def build_table(act: int, dtype: int = DTYPE_BF16) -> np.ndarray:
    """The oracle's (act, dtype) table, built once per process (a copy is
    returned, so callers may modify it)."""
    key = (act, dtype)
    if key not in _TABLES:
        t = np.zeros(65536, np.uint16)
        if lib().or_build_table(act, dtype, _p(t)) != 0:
            raise ValueError("no oracle table for this activation/dtype")
        _TABLES[key] = t
    return _TABLES[key].copy()


def unary_lut(table: np.ndarray, x: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    lib().or_unary_lut(_p(table), _p(x), _p(out), x.size)
    return out


def quantize_row_i8(a: np.ndarray) -> tuple:
    a = np.ascontiguousarray(a, np.float32)
    q = np.zeros(a.size, np.int8)
    s = lib().or_quantize_row_i8(_p(a), _p(q), a.size)
    return q, np.float32(s)


def matmul_i8_pc_omajor(a, bq, scales, m, k, n) -> np.ndarray:
    out = np.zeros(m * n, np.float32)
    lib().or_matmul_i8_pc_omajor(_p(a), _p(bq), _p(scales), _p(out), m, k, n)
    return out


def matmul_q_omajor(tier: int, a, bq, scales, m, k, n, codebook=None) -> np.ndarray:
    """Output-major W8A8 GEMV for the i8 (2), i4 (10) and e8cb (11) tiers."""
    out = np.zeros(m * n, np.float32)
    a = np.ascontiguousarray(a, np.float32)
    bq = np.ascontiguousarray(bq).view(np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    cb = None if codebook is None else np.ascontiguousarray(codebook).view(np.int8)
    if lib().or_matmul_q_omajor(tier, _p(a), _p(bq), _p(cb) if cb is not None else None,
                                _p(scales), _p(out), m, k, n) != 0:
        raise ValueError("matmul_q_omajor refused")
    return out


def dequantize(q, n: int, quant: int, dtype: int = DTYPE_F32, scale: float = 1.0, zp: int = 0,
               scales=None, zps=None, channels: int = 0, inner: int = 1) -> np.ndarray:
    """Dequantize (kernels.rs:185-296): f32 array, or the bf16/f16 bits as
    uint16. Per-channel when `scales` is given and channels > 0."""
    q = np.ascontiguousarray(q).view(np.uint8)
    out = np.zeros(n, np.float32 if dtype == DTYPE_F32 else np.uint16)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    zp_arr = None if zps is None else np.ascontiguousarray(zps, np.int32)
    if lib().or_dequantize(_p(q), n, quant, _p(sc) if sc is not None else None,
                           _p(zp_arr) if zp_arr is not None else None, channels, inner,
                           float(np.float32(scale)), int(zp), dtype, _p(out)) != 0:
        raise ValueError("dequantize refused")
    return out


def dequant_activation(q, n: int, quant: int, act: int, scale: float, zp: int) -> np.ndarray:
    """DequantActivation (kernels.rs:311-388): the f32 table of the <= 256
    levels through lut_act_ref(act), one lookup per element."""
    q = np.ascontiguousarray(q).view(np.uint8)
    out = np.zeros(n, np.float32)
    if lib().or_dequant_activation(_p(q), n, quant, act, float(np.float32(scale)), int(zp),
                                   _p(out)) != 0:
        raise ValueError("dequant_activation refused")
    return out


def fnv1a_f32(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return lib().or_fnv1a_f32(_p(v), v.size)


def kv_cache_write(cache: np.ndarray, new: np.ndarray, pos: int, planes: int, bucket: int,
                   new_rows: int, row_bytes: int) -> np.ndarray:
    out = np.empty_like(cache)
    rc = lib().or_kv_cache_write(_p(cache), _p(new), pos, _p(out), planes, bucket, new_rows,
                                 row_bytes)
    if rc != 0:
        raise ValueError(f"kv_cache_write refused ({rc})")
    return out


def kv_quant_append(new: np.ndarray, dtype: int, pos: int, cache_q: np.ndarray,
                    cache_s: np.ndarray, planes: int, bucket: int, new_rows: int,
                    head_dim: int) -> tuple:
    """Copy-form quantize+append: returns (new int8 cache, new scale cache)."""
    oq, os_ = cache_q.copy(), cache_s.copy()
    rc = lib().or_kv_quant_append(_p(new), dtype, pos, _p(oq), _p(os_), planes, bucket,
                                  new_rows, head_dim)
    if rc != 0:
        raise ValueError(f"kv_quant_append refused ({rc})")
    return oq, os_


def dequant_i8(q: np.ndarray, scales: np.ndarray, row_len: int) -> np.ndarray:
    rows = q.size // row_len
    out = np.empty(rows * row_len, np.float32)
    lib().or_dequant_i8(_p(q), _p(scales), _p(out), rows, row_len)
    return out


def attn_scale(head_dim: int, scale_bits: int = 0) -> float:
    return lib().or_attn_scale(head_dim, scale_bits)


def decode_attention_valid_f32(q, kp, vp, kn, vn, b, h, hkv, m, past, new, d, scale,
                               vis_past) -> np.ndarray:
    out = np.zeros(b * h * m * d, np.float32)
    lib().or_decode_attention_valid_f32(_p(q), _p(kp), _p(vp), _p(kn), _p(vn), _p(out), b, h,
                                        hkv, m, past, new, d, scale, vis_past)
    return out


def decode_attention_valid(q, kp, vp, kn, vn, valid_len, b, h, hkv, m, past, new, d,
                           scale_bits, dtype) -> np.ndarray:
    """DecodeAttentionValid (float_kernels.rs:4192-4307) on raw operand arrays
    of `dtype` (bf16/f16 as u16 bits, f32); returns the output array of the
    same element type. Raises ValueError where the reference refuses."""
    es = 4 if dtype == DTYPE_F32 else 2
    out = np.zeros(b * h * m * d, np.float32 if es == 4 else np.uint16)
    args = [np.ascontiguousarray(x) for x in (q, kp, vp, kn, vn)]
    rc = lib().or_decode_attention_valid(*[_p(x) for x in args], valid_len, _p(out), b, h, hkv,
                                         m, past, new, d, scale_bits, dtype)
    if rc != 0:
        raise ValueError(f"decode_attention_valid refused ({rc})")
    return out


def decode_attention(q, kp, vp, kn, vn, mask, b, h, hkv, m, past, new, d, scale_bits,
                     dtype) -> np.ndarray:
    """DecodeAttention, the mask form (float_kernels.rs:2482-2660), on raw
    operand arrays of `dtype` (bf16/f16 as u16 bits, f32) and an f32 mask
    [m, past + new]; returns the output array of the same element type.
    Raises ValueError where the reference refuses."""
    es = 4 if dtype == DTYPE_F32 else 2
    out = np.zeros(b * h * m * d, np.float32 if es == 4 else np.uint16)
    args = [np.ascontiguousarray(x) for x in (q, kp, vp, kn, vn)]
    mk = np.ascontiguousarray(mask, dtype=np.float32)
    rc = lib().or_decode_attention(*[_p(x) for x in args], _p(mk), _p(out), b, h, hkv, m, past,
                                   new, d, scale_bits, dtype)
    if rc != 0:
        raise ValueError(f"decode_attention refused ({rc})")
    return out


def decode_attention_i8(q, kq, ks, vq, vs, lens, B, H, Hkv, bucket, D, scale) -> np.ndarray:
    out = np.zeros(B * H * D, np.float32)
    lib().or_decode_attention_i8(_p(q), _p(kq), _p(ks), _p(vq), _p(vs), _p(lens), _p(out), B,
                                 H, Hkv, bucket, D, scale)
    return out


def attention_i8_rows(q, kq, ks, vq, vs, lens, B, T, H, Hkv, bucket, D, scale) -> np.ndarray:
    """The multi-row (prefill) form over an int8 cache: q [B, T, H, D] (f32), row t
    of sequence b a one-query decode over the first clamp(lens[b] - (T - 1 - t),
    0, bucket) rows of its planes. With lens[b] >= T this is
    DecodeAttentionValid{m = new = T, past = lens[b] - T} (float_kernels.rs:3926:
    row qi sees the past prefix and min(qi + 1, new) new rows). With T > 1 every
    lens[b] must be at most bucket: past a ring wrap the earlier rows' keys are
    overwritten, and no causal result exists."""
    if T > 1 and np.any(np.asarray(lens, np.int64)[:B] > bucket):
        raise ValueError("attention_i8_rows: a length exceeds the bucket (ring wrapped)")
    q = np.ascontiguousarray(q, np.float32).reshape(B, T, H, D)
    out = np.zeros((B, T, H, D), np.float32)
    pl, ps = Hkv * bucket * D, Hkv * bucket
    for b in range(B):
        planes = [np.ascontiguousarray(a) for a in (kq[b * pl:(b + 1) * pl], ks[b * ps:(b + 1) * ps],
                                                   vq[b * pl:(b + 1) * pl], vs[b * ps:(b + 1) * ps])]
        for t in range(T):
            L = max(int(lens[b]) - (T - 1 - t), 0)
            out[b, t] = decode_attention_i8(np.ascontiguousarray(q[b, t]).ravel(), *planes,
                                            np.array([L], np.uint32), 1, H, Hkv, bucket, D,
                                            scale).reshape(H, D)
    return out.ravel()


def transpose(x: np.ndarray, dims, perm) -> np.ndarray:
    """transpose_float (float_kernels.rs:2980-3028): output axis i is input axis
    perm[i] of the row-major input of shape dims."""
    return np.ascontiguousarray(np.transpose(np.asarray(x).reshape(tuple(dims)), tuple(perm))).ravel()


def fused_act_f32(act: int, x: np.ndarray) -> np.ndarray:
    """fused_act_fn (float_kernels.rs:768-780) over f32 values; act is a
    fused_activation id (kernel_call.rs:861-870)."""
    x = np.ascontiguousarray(x, np.float32)
    o = np.empty_like(x)
    if lib().or_fused_act_f32(act, _p(x), _p(o), x.size) != 0:
        raise ValueError(f"fused activation {act} is not restated")
    return o


FUSED_TO_LUT = {2: ACT_GELU, 3: ACT_SILU, 4: ACT_SIGMOID, 5: ACT_TANH, 8: ACT_EXP}


def matmul_ref_f64(a, b, m, k, n) -> np.ndarray:
    out = np.zeros(m * n, np.float32)
    lib().or_matmul_ref_f64(_p(a), _p(b), _p(out), m, k, n)
    return out


PANEL = 16   # layout.rs: the panel width of a packed B


def packed_len(k: int, n: int) -> int:
    """layout::packed_len: ceil(n / 16) * k * 16 elements."""
    return -(-n // PANEL) * k * PANEL


def pack_b_panels(b: np.ndarray, k: int, n: int) -> np.ndarray:
    """pack_b_panels (layout.rs:16-45): packed[(p*k + kk)*16 + c] = b[kk*n + p*16 + c],
    zero where p*16 + c >= n."""
    npan = -(-n // PANEL)
    padded = np.zeros((k, npan * PANEL), np.asarray(b).dtype)
    padded[:, :n] = np.asarray(b).reshape(k, n)
    return np.ascontiguousarray(padded.reshape(k, npan, PANEL).transpose(1, 0, 2)).ravel()


def unpack_b_panels(packed: np.ndarray, k: int, n: int) -> np.ndarray:
    """The inverse of pack_b_panels: the row-major k x n weight."""
    npan = -(-n // PANEL)
    p = np.asarray(packed)[:npan * k * PANEL].reshape(npan, k, PANEL).transpose(1, 0, 2)
    return np.ascontiguousarray(p.reshape(k, npan * PANEL)[:, :n]).ravel()


def matmul_f64_blas(a, b, m, k, n) -> np.ndarray:
    """The same f64 reference as matmul_ref_f64 (products and sums in f64,
    one rounding to f32 at the end) through numpy's f64 BLAS, for graph-sized
    products the scalar loop would take minutes on; only the order of the f64
    sums differs."""
    a64 = np.ascontiguousarray(a, np.float32).reshape(m, k).astype(np.float64)
    b64 = np.ascontiguousarray(b, np.float32).reshape(k, n).astype(np.float64)
    return (a64 @ b64).astype(np.float32).ravel()


def max_rel_err(got, want) -> float:
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    return lib().or_max_rel_err(_p(got), _p(want), got.size)


def host_threads() -> int:
    """Threads for the CPU baseline: this process's CPU share, at most 16 (the
    GPU box allots 16 host cores to each GPU, whatever nproc shows there)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_info() -> dict:
    """The host the CPU baseline runs on: nproc, this process's affinity, the
    CPU model, and the thread count the multi-threaded legs use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "affinity": aff, "cpu_model": model,
            "threads_used": host_threads(),
            "thread_cap": "16: the box's host-core share per GPU"}
