"""hologram_amd — MI355X (gfx950) compute backend for Hologram's hot path.

The reference operator API (Backend::dispatch over KernelCall and a slot
workspace, crates/hologram-compute/src/backend.rs:8-15) over hand-written HIP
kernels: bf16/f16 LUT activations, f32/bf16 MatMul on MFMA, int8 KV-cache
quantize+append, int8-KV GQA decode attention, the rest of a decode step
(RmsNorm, RoPE, Gather, Add, Mul, ArgMax) and the `.holo` session walk that
runs a compiled graph over device-resident slots. The compute lives in
libholo_hip.so (C ABI: include/holo_hip.h); this package is its host mirror.
"""
from .backend import (BackendError, DeviceWorkspace, DispatchError, HipBackend, InitError,
                      ShapeMismatch, SlotOutOfRange, UnsupportedOp, decode_call, lut_table,
                      validate)
from .kernel_call import (DTYPE_BF16, DTYPE_E8CB, DTYPE_F16, DTYPE_F32, DTYPE_I4, DTYPE_I8,
                          DTYPE_I32, DTYPE_I64, DTYPE_U8, NO_BUFFER, SLOT_ABSENT, ArgMaxCall,
                          AttentionI8RowsCall, BinaryCall, BufferRef, DecodeAttentionCall,
                          DecodeAttentionI8Call, DecodeAttentionValidCall, DequantActivationCall,
                          DequantizeCall, GatherCall, KernelCall, KvCacheWriteCall, KvQuantAppendCall,
                          MatMulActivationCall, MatMulAddActivationCall, MatMulAddCall,
                          MatMulCall, MatMulDequantCall, NormCall, RoPECall, TransposeCall, LayoutCall,
                          UnaryCall, encode_calls, fused_activation, lut_act, mm_act_quant,
                          weight_layout)
from .archive import ConstantEntry, HoloWriter, PortDescriptor, blake3
from .session import HipSession

__all__ = [
    "BackendError", "DeviceWorkspace", "DispatchError", "HipBackend", "InitError",
    "ShapeMismatch", "SlotOutOfRange", "UnsupportedOp", "decode_call", "lut_table", "validate",
    "DTYPE_BF16", "DTYPE_E8CB", "DTYPE_F16", "DTYPE_F32", "DTYPE_I4", "DTYPE_I8", "DTYPE_I32",
    "DTYPE_I64", "DTYPE_U8", "NO_BUFFER", "SLOT_ABSENT", "ArgMaxCall", "AttentionI8RowsCall",
    "BinaryCall", "BufferRef", "DecodeAttentionCall", "DecodeAttentionI8Call",
    "DecodeAttentionValidCall", "DequantActivationCall", "DequantizeCall", "GatherCall", "KernelCall", "KvCacheWriteCall",
    "KvQuantAppendCall", "MatMulActivationCall", "MatMulAddActivationCall", "MatMulAddCall",
    "MatMulCall", "MatMulDequantCall", "NormCall", "RoPECall", "TransposeCall", "LayoutCall", "UnaryCall",
    "encode_calls", "fused_activation", "lut_act", "mm_act_quant", "weight_layout",
    "ConstantEntry", "HoloWriter", "PortDescriptor", "blake3", "HipSession",
]
