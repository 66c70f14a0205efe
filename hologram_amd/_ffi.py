"""ctypes view of include/holo_hip.h and the loader for libholo_hip.so.

The library is the product: nothing here computes. If the shared library is
missing, every entry point raises; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libholo_hip.so"

# holo_status (crates/hologram-compute/src/error.rs:6-20)
OK = 0
ERR_SLOT_OUT_OF_RANGE = 1
ERR_SHAPE_MISMATCH = 2
ERR_UNSUPPORTED_OP = 3
ERR_INIT = 4
ERR_DISPATCH = 5


class BufferRefC(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("length", ctypes.c_uint64)]


class UnaryCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("output", BufferRefC), ("element_count", ctypes.c_uint64),
                ("witt_bits", ctypes.c_uint16), ("dtype", ctypes.c_uint8)]


class BinaryCallC(ctypes.Structure):
    _fields_ = [("a", BufferRefC), ("b", BufferRefC), ("output", BufferRefC),
                ("element_count", ctypes.c_uint64), ("witt_bits", ctypes.c_uint16),
                ("dtype", ctypes.c_uint8)]


class NormCallC(ctypes.Structure):
    _fields_ = [("x", BufferRefC), ("gamma", BufferRefC), ("beta", BufferRefC),
                ("residual", BufferRefC), ("output", BufferRefC), ("batch", ctypes.c_uint32),
                ("feature", ctypes.c_uint32), ("channels", ctypes.c_uint32),
                ("num_groups", ctypes.c_uint32), ("epsilon_bits", ctypes.c_uint64),
                ("dtype", ctypes.c_uint8)]


class RopeCallC(ctypes.Structure):
    _fields_ = [("x", BufferRefC), ("cos", BufferRefC), ("sin", BufferRefC),
                ("output", BufferRefC), ("head_dim", ctypes.c_uint32),
                ("element_count", ctypes.c_uint64), ("dtype", ctypes.c_uint8)]


class GatherCallC(ctypes.Structure):
    _fields_ = [("data", BufferRefC), ("indices", BufferRefC), ("output", BufferRefC),
                ("outer", ctypes.c_uint64), ("axis_dim", ctypes.c_uint64),
                ("inner", ctypes.c_uint64), ("num_indices", ctypes.c_uint64),
                ("idx_dtype", ctypes.c_uint8), ("dtype", ctypes.c_uint8)]


class ArgMaxCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("output", BufferRefC), ("rows", ctypes.c_uint32),
                ("cols", ctypes.c_uint32), ("dtype", ctypes.c_uint8)]


class MatMulCallC(ctypes.Structure):
    _fields_ = [("a", BufferRefC), ("b", BufferRefC), ("output", BufferRefC),
                ("m", ctypes.c_uint32), ("k", ctypes.c_uint32), ("n", ctypes.c_uint32),
                ("dtype", ctypes.c_uint8), ("b_packed", ctypes.c_uint8)]


class MatMulActCallC(ctypes.Structure):
    _fields_ = [("mm", MatMulCallC), ("act", ctypes.c_uint8)]


class MatMulAddCallC(ctypes.Structure):
    _fields_ = [("mm", MatMulCallC), ("residual", BufferRefC)]


class MatMulAddActCallC(ctypes.Structure):
    _fields_ = [("mm", MatMulCallC), ("residual", BufferRefC), ("act", ctypes.c_uint8)]


class KvCacheWriteCallC(ctypes.Structure):
    _fields_ = [("cache", BufferRefC), ("new_rows_buf", BufferRefC), ("pos", BufferRefC),
                ("output", BufferRefC), ("planes", ctypes.c_uint32),
                ("bucket_rows", ctypes.c_uint32), ("new_rows", ctypes.c_uint32),
                ("row_bytes", ctypes.c_uint32)]


class KvQuantAppendCallC(ctypes.Structure):
    _fields_ = [("new_rows_buf", BufferRefC), ("pos", BufferRefC), ("cache", BufferRefC),
                ("cache_scales", BufferRefC), ("output", BufferRefC),
                ("output_scales", BufferRefC), ("planes", ctypes.c_uint32),
                ("bucket_rows", ctypes.c_uint32), ("new_rows", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("dtype", ctypes.c_uint8)]


class DecodeAttentionValidCallC(ctypes.Structure):
    _fields_ = [("q", BufferRefC), ("k_past", BufferRefC), ("v_past", BufferRefC),
                ("k_new", BufferRefC), ("v_new", BufferRefC), ("valid_len", BufferRefC),
                ("output", BufferRefC), ("batch", ctypes.c_uint32), ("heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("q_rows", ctypes.c_uint32),
                ("past_len", ctypes.c_uint32), ("new_len", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("scale_bits", ctypes.c_uint32),
                ("dtype", ctypes.c_uint8)]


class DecodeAttentionCallC(ctypes.Structure):
    _fields_ = [("q", BufferRefC), ("k_past", BufferRefC), ("v_past", BufferRefC),
                ("k_new", BufferRefC), ("v_new", BufferRefC), ("mask", BufferRefC),
                ("output", BufferRefC), ("batch", ctypes.c_uint32), ("heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("q_rows", ctypes.c_uint32),
                ("past_len", ctypes.c_uint32), ("new_len", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("scale_bits", ctypes.c_uint32),
                ("dtype", ctypes.c_uint8)]


class DecodeAttentionI8CallC(ctypes.Structure):
    _fields_ = [("q", BufferRefC), ("k_cache", BufferRefC), ("v_cache", BufferRefC),
                ("k_scales", BufferRefC), ("v_scales", BufferRefC), ("lens", BufferRefC),
                ("output", BufferRefC), ("batch", ctypes.c_uint32), ("heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("bucket_rows", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("scale_bits", ctypes.c_uint32),
                ("dtype", ctypes.c_uint8)]


class AttentionI8RowsCallC(ctypes.Structure):
    _fields_ = [("attn", DecodeAttentionI8CallC), ("q_rows", ctypes.c_uint32)]


class TransposeCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("output", BufferRefC), ("rank", ctypes.c_uint8),
                ("dims", ctypes.c_uint32 * 8), ("perm", ctypes.c_uint8 * 8),
                ("dtype", ctypes.c_uint8)]


class LayoutCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("output", BufferRefC), ("element_count", ctypes.c_uint64),
                ("dtype", ctypes.c_uint8)]


class DequantizeCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("scales", BufferRefC), ("zero_points", BufferRefC),
                ("output", BufferRefC), ("element_count", ctypes.c_uint64),
                ("channels", ctypes.c_uint32), ("inner", ctypes.c_uint32),
                ("quant_dtype", ctypes.c_uint8), ("dtype", ctypes.c_uint8),
                ("scale_bits", ctypes.c_uint32), ("zero_point", ctypes.c_int32),
                ("codebook", BufferRefC), ("weight_layout", ctypes.c_uint8),
                ("act_quant", ctypes.c_uint8)]


class MatMulDequantCallC(ctypes.Structure):
    _fields_ = [("a", BufferRefC), ("bq", BufferRefC), ("scales", BufferRefC),
                ("zero_points", BufferRefC), ("output", BufferRefC),
                ("m", ctypes.c_uint32), ("k", ctypes.c_uint32), ("n", ctypes.c_uint32),
                ("channels", ctypes.c_uint32), ("inner", ctypes.c_uint32),
                ("quant_dtype", ctypes.c_uint8), ("dtype", ctypes.c_uint8),
                ("scale_bits", ctypes.c_uint32), ("zero_point", ctypes.c_int32),
                ("bq_omajor", ctypes.c_uint8), ("act_quant", ctypes.c_uint8),
                ("act", ctypes.c_uint8), ("residual", BufferRefC), ("codebook", BufferRefC)]


class DequantActivationCallC(ctypes.Structure):
    _fields_ = [("input", BufferRefC), ("output", BufferRefC), ("element_count", ctypes.c_uint64),
                ("quant_dtype", ctypes.c_uint8), ("act", ctypes.c_uint8), ("dtype", ctypes.c_uint8),
                ("scale_bits", ctypes.c_uint32), ("zero_point", ctypes.c_int32)]


class CallUnion(ctypes.Union):
    _fields_ = [("unary", UnaryCallC), ("binary", BinaryCallC), ("norm", NormCallC),
                ("rope", RopeCallC), ("gather", GatherCallC), ("argmax", ArgMaxCallC),
                ("matmul", MatMulCallC), ("matmul_act", MatMulActCallC),
                ("matmul_add", MatMulAddCallC), ("matmul_add_act", MatMulAddActCallC),
                ("kv_write", KvCacheWriteCallC),
                ("kv_quant_append", KvQuantAppendCallC), ("attn_valid", DecodeAttentionValidCallC),
                ("attn_mask", DecodeAttentionCallC),
                ("dequantize", DequantizeCallC), ("matmul_dequant", MatMulDequantCallC),
                ("dequant_act", DequantActivationCallC), ("attn_i8", DecodeAttentionI8CallC),
                ("attn_i8_rows", AttentionI8RowsCallC), ("transpose", TransposeCallC),
                ("layout", LayoutCallC)]


class KernelCallC(ctypes.Structure):
    _fields_ = [("tag", ctypes.c_uint32), ("u", CallUnion)]


# Every function include/holo_hip.h declares, with its ctypes signature.
_P = ctypes.c_void_p
SIGNATURES = {
    "holo_hip_backend_create": (ctypes.c_int, [ctypes.c_int, _P, ctypes.POINTER(_P)]),
    "holo_hip_backend_destroy": (ctypes.c_int, [_P]),
    "holo_hip_set_stream": (ctypes.c_int, [_P, _P]),
    "holo_hip_slot_bind": (ctypes.c_int, [_P, ctypes.c_uint32, _P, ctypes.c_uint64]),
    "holo_hip_slot_unbind": (ctypes.c_int, [_P, ctypes.c_uint32]),
    "holo_hip_dispatch": (ctypes.c_int, [_P, ctypes.POINTER(KernelCallC)]),
    "holo_hip_dispatch_noalloc": (ctypes.c_int, [_P, ctypes.POINTER(KernelCallC)]),
    "holo_hip_dispatch_encoded": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_size_t,
                                                 ctypes.POINTER(ctypes.c_size_t)]),
    "holo_hip_synchronize": (ctypes.c_int, [_P]),
    "holo_hip_validate": (ctypes.c_int, [ctypes.POINTER(KernelCallC),
                                         ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint32]),
    "holo_hip_decode_call": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t,
                                            ctypes.POINTER(KernelCallC),
                                            ctypes.POINTER(ctypes.c_size_t)]),
    "holo_hip_lut_table": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _P]),
    "holo_hip_session_load": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_size_t,
                                             ctypes.POINTER(_P)]),
    "holo_hip_session_load_ex": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_size_t,
                                                ctypes.c_uint32, ctypes.POINTER(_P)]),
    "holo_hip_session_nodes": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint32),
                                              ctypes.POINTER(ctypes.c_uint32)]),
    "holo_hip_session_call": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.POINTER(KernelCallC)]),
    "holo_hip_session_output_labels": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_char_p]),
    "holo_hip_session_execute_bytes": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_void_p),
                                                      ctypes.POINTER(ctypes.c_uint64),
                                                      ctypes.c_uint32,
                                                      ctypes.POINTER(ctypes.c_int)]),
    "holo_hip_session_set_memo": (ctypes.c_int, [_P, ctypes.c_int]),
    "holo_hip_session_close": (ctypes.c_int, [_P]),
    "holo_hip_session_info": (ctypes.c_int, [_P] + [ctypes.POINTER(ctypes.c_uint32)] * 4),
    "holo_hip_session_port": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_uint32,
                                             ctypes.POINTER(ctypes.c_uint32),
                                             ctypes.POINTER(ctypes.c_uint64),
                                             ctypes.POINTER(ctypes.c_uint8),
                                             ctypes.POINTER(ctypes.c_uint64)]),
    "holo_hip_session_fingerprint": (ctypes.c_int, [_P, ctypes.c_char_p]),
    "holo_hip_session_bind_input": (ctypes.c_int, [_P, ctypes.c_uint32, _P, ctypes.c_uint64]),
    "holo_hip_session_write_input": (ctypes.c_int, [_P, ctypes.c_uint32, _P, ctypes.c_uint64]),
    "holo_hip_session_execute": (ctypes.c_int, [_P]),
    "holo_hip_session_capture": (ctypes.c_int, [_P]),
    "holo_hip_session_replay": (ctypes.c_int, [_P]),
    "holo_hip_session_synchronize": (ctypes.c_int, [_P]),
    "holo_hip_session_stream": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "holo_hip_session_output": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.POINTER(_P),
                                               ctypes.POINTER(ctypes.c_uint64)]),
    "holo_hip_session_read_output": (ctypes.c_int, [_P, ctypes.c_uint32, _P, ctypes.c_uint64]),
    "holo_hip_blake3": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p]),
    "holo_hip_address_bytes": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p]),
    "holo_hip_derive_label": (ctypes.c_int, [ctypes.c_uint16, ctypes.c_char_p, ctypes.c_uint64,
                                             ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p]),
    "holo_hip_derive_label_boundary": (ctypes.c_int, [ctypes.c_uint16, ctypes.c_char_p,
                                                      ctypes.c_uint64, ctypes.c_char_p,
                                                      ctypes.c_uint64, ctypes.c_char_p]),
    "holo_hip_session_last_walk": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint32),
                                                  ctypes.POINTER(ctypes.c_uint32)]),
    "holo_hip_session_packed": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint32),
                                               ctypes.POINTER(ctypes.c_uint64)]),
    "holo_hip_session_attn_prologues": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint32)]),
    "holo_hip_op_signature": (ctypes.c_int, [ctypes.POINTER(KernelCallC),
                                             ctypes.POINTER(ctypes.c_uint16), ctypes.c_char_p,
                                             ctypes.POINTER(ctypes.c_uint32)]),
    "holo_hip_last_error_message": (ctypes.c_char_p, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libholo_hip.so once; raise loudly if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP backend first "
                "(python -m hologram_amd.build). There is no CPU fallback.")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().holo_hip_last_error_message()
    return msg.decode() if msg else ""
