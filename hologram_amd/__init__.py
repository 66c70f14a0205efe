"""hologram_amd — MI355X (gfx950) compute backend for Hologram's hot path.

The reference operator API (Backend::dispatch over KernelCall and a slot
workspace, crates/hologram-compute/src/backend.rs:8-15) over hand-written HIP
kernels: bf16/f16 LUT activations, f32/bf16 MatMul on MFMA, int8 KV-cache
quantize+append and int8-KV GQA decode attention. The compute lives in
libholo_hip.so (C ABI: include/holo_hip.h); this package is its host mirror.
"""
from .backend import (BackendError, DeviceWorkspace, DispatchError, HipBackend, InitError,
                      ShapeMismatch, SlotOutOfRange, UnsupportedOp, decode_call, lut_table,
                      validate)
from .kernel_call import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_I8, SLOT_ABSENT, BufferRef,
                          DecodeAttentionI8Call, KernelCall, KvCacheWriteCall,
                          KvQuantAppendCall, MatMulCall, UnaryCall, encode_calls, lut_act)

__all__ = [
    "BackendError", "DeviceWorkspace", "DispatchError", "HipBackend", "InitError",
    "ShapeMismatch", "SlotOutOfRange", "UnsupportedOp", "decode_call", "lut_table", "validate",
    "DTYPE_BF16", "DTYPE_F16", "DTYPE_F32", "DTYPE_I8", "SLOT_ABSENT", "BufferRef",
    "DecodeAttentionI8Call", "KernelCall", "KvCacheWriteCall", "KvQuantAppendCall",
    "MatMulCall", "UnaryCall", "encode_calls", "lut_act",
]
