"""KernelCall: the reference's closed kernel-call surface, for the hot ops.

Mirrors crates/hologram-compute/src/kernel_call.rs (field names, order and
widths) for the variants this backend executes, plus the two new int8-KV
capabilities, which take new archive discriminants (122, 123) as the
reference's codec rule requires (crates/hologram-archive/src/kernel_codec.rs:124-128).
`KernelCall.encode()` writes the archive wire form (u16 LE discriminant + LE
payload, kernel_codec.rs:557-813).
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass, field

from . import _ffi

# dtype tags, crates/hologram-types/src/dtype_id.rs:52-61
DTYPE_U8 = 1
DTYPE_I8 = 2
DTYPE_I32 = 4
DTYPE_I64 = 5
DTYPE_F16 = 6
DTYPE_BF16 = 7
DTYPE_F32 = 8
DTYPE_I4 = 10     # two per byte, low nibble first (dtype_id.rs:150-161)
DTYPE_E8CB = 11   # one codebook index per 8-element group


class lut_act:  # noqa: N801 - the reference's module name (kernel_call.rs:877-885)
    SIGMOID = 0
    TANH = 1
    GELU = 2
    SILU = 3
    EXP = 4
    ERF = 5
    COUNT = 6


# archive discriminants, kernel_codec.rs:18-128
D_ADD = 5
D_MUL = 7
D_RELU = 11
D_SIGMOID = 12
D_TANH = 13
D_GELU = 14
D_SILU = 15
D_ELU = 16
D_SELU = 17
D_EXP = 18
D_ERF = 32      # decoded; not served on the device
D_DEQ = 105     # Dequantize (118 on the wire when it declares anything)
D_DEQ2 = 118
D_MMDQ = 111    # MatMulDequant (116 with the extended fields, 117 with a codebook)
D_MMDQ2 = 116
D_MMDQ3 = 117
D_DQACT = 113   # DequantActivation
D_MATMUL = 46
D_MMA = 106     # MatMulActivation (the loader's epilogue fusion)
D_MMADD = 107   # MatMulAdd
D_MMAA = 108    # MatMulAddActivation
D_RN = 51
D_ADDRMS = 54   # AddRmsNorm: rms_norm(x + residual)
D_ROTARY = 75
D_GATHER = 114
D_DECATTN = 119   # DecodeAttention, the mask form
D_KVWR = 120
D_DAVL = 121
D_KVQA = 122   # new: int8 quantize + append
D_DAI8 = 123   # new: decode attention over an int8 cache
D_ARGMAX = 124  # new: per-row argmax (the greedy pick of a decode step)
D_AI8R = 125    # new: multi-row (prefill) form of D_DAI8
D_TRANSPOSE = 61
D_RESHAPE = 60
D_SLICE = 63

SLOT_ABSENT = 0xFFFFFFFF


class fused_activation:  # noqa: N801 - the reference's module (kernel_call.rs:861-870)
    RELU = 1
    GELU = 2
    SILU = 3
    SIGMOID = 4
    TANH = 5
    ELU = 6
    SELU = 7
    EXP = 8


@dataclass(frozen=True)
class BufferRef:
    """crates/hologram-compute/src/workspace.rs:16-24 (length 0 = whole slot)."""
    slot: int
    offset: int = 0
    length: int = 0

    def c(self) -> _ffi.BufferRefC:
        return _ffi.BufferRefC(self.slot, self.offset, self.length)

    def wire(self) -> bytes:
        return struct.pack("<IQQ", self.slot, self.offset, self.length)


@dataclass(frozen=True)
class UnaryCall:
    """kernel_call.rs:28-36."""
    input: BufferRef
    output: BufferRef
    element_count: int
    witt_bits: int = 16
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_unary, kernel_codec.rs:575-581
        return (self.input.wire() + self.output.wire()
                + struct.pack("<QHB", self.element_count, self.witt_bits, self.dtype))


@dataclass(frozen=True)
class BinaryCall:
    """kernel_call.rs:38-46."""
    a: BufferRef
    b: BufferRef
    output: BufferRef
    element_count: int
    witt_bits: int = 16
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_binary, kernel_codec.rs:582-589
        return (self.a.wire() + self.b.wire() + self.output.wire()
                + struct.pack("<QHB", self.element_count, self.witt_bits, self.dtype))


NO_BUFFER = BufferRef(SLOT_ABSENT)


class mm_act_quant:  # noqa: N801 - the reference's module (kernel_call.rs:66-104)
    W8A32 = 0
    W8A8_TOKEN_SYM = 1
    K_MAX = 133144   # i32::MAX // (127 * 127): the exact-i32 dot bound


class weight_layout:  # noqa: N801 - hologram-types dtype_id.rs:18-28
    ROW_MAJOR = 0
    OUTPUT_MAJOR = 1


@dataclass(frozen=True)
class DequantizeCall:
    """kernel_call.rs:790-840: out[i] = ((q[i] - zp) as f32 * scale) as dtype;
    per-channel when channels > 0 and scales is present (channel (i / inner) %
    channels). The extended wire form (118) declares the weight slot's layout,
    its activation treatment and a codebook."""
    input: BufferRef
    scales: BufferRef
    zero_points: BufferRef
    output: BufferRef
    element_count: int
    channels: int = 0
    inner: int = 1
    quant_dtype: int = DTYPE_I8
    dtype: int = DTYPE_F32
    scale_bits: int = 0
    zero_point: int = 0
    codebook: BufferRef = NO_BUFFER
    weight_layout: int = 0
    act_quant: int = 0

    def per_channel(self) -> bool:
        return self.channels > 0 and self.scales.slot != SLOT_ABSENT

    def extended(self) -> bool:  # kernel_call.rs:837-839
        return self.weight_layout != 0 or self.act_quant != 0 or self.codebook.slot != SLOT_ABSENT

    def wire_tag(self) -> int:
        return D_DEQ2 if self.extended() else D_DEQ

    def wire(self) -> bytes:  # put_dequantize, kernel_codec.rs:861-872 (+ :497-506)
        body = (self.input.wire() + self.scales.wire() + self.zero_points.wire()
                + self.output.wire()
                + struct.pack("<QIIBBIi", self.element_count, self.channels, self.inner,
                              self.quant_dtype, self.dtype, self.scale_bits, self.zero_point))
        if self.extended():
            body += struct.pack("<BB", self.weight_layout, self.act_quant) + self.codebook.wire()
        return body


@dataclass(frozen=True)
class MatMulDequantCall:
    """kernel_call.rs:162-273: out = act(A . dequant(Bq) [+ residual]), f32.
    bq_omajor with act_quant W8A8_TOKEN_SYM is the output-major W8A8 GEMV
    (i8 / i4 / e8cb + codebook); otherwise the [k, n] weight is dequantized
    (W8A32)."""
    a: BufferRef
    bq: BufferRef
    scales: BufferRef
    zero_points: BufferRef
    output: BufferRef
    m: int
    k: int
    n: int
    channels: int = 0
    inner: int = 1
    quant_dtype: int = DTYPE_I8
    dtype: int = DTYPE_F32
    scale_bits: int = 0
    zero_point: int = 0
    bq_omajor: bool = False
    act_quant: int = 0
    act: int = 0
    residual: BufferRef = NO_BUFFER
    codebook: BufferRef = NO_BUFFER

    def per_channel(self) -> bool:
        return self.channels > 0 and self.scales.slot != SLOT_ABSENT

    def extended(self) -> bool:  # kernel_call.rs:250-256
        return (self.bq_omajor or self.act_quant != 0 or self.act != 0
                or self.residual.slot != SLOT_ABSENT or self.codebook.slot != SLOT_ABSENT)

    def wire_tag(self) -> int:
        if self.codebook.slot != SLOT_ABSENT:
            return D_MMDQ3
        return D_MMDQ2 if self.extended() else D_MMDQ

    def wire(self) -> bytes:  # put_matmul_dequant, kernel_codec.rs:835-850 (+ :525-546)
        body = (self.a.wire() + self.bq.wire() + self.scales.wire() + self.zero_points.wire()
                + self.output.wire()
                + struct.pack("<IIIIIBBIi", self.m, self.k, self.n, self.channels, self.inner,
                              self.quant_dtype, self.dtype, self.scale_bits, self.zero_point))
        tag = self.wire_tag()
        if tag != D_MMDQ:
            body += (struct.pack("<BBB", int(self.bq_omajor), self.act_quant, self.act)
                     + self.residual.wire())
        if tag == D_MMDQ3:
            body += self.codebook.wire()
        return body


@dataclass(frozen=True)
class DequantActivationCall:
    """kernel_call.rs:275-290: out[i] = f((q[i] - zp) as f32 * scale), f32,
    f the lut_act function `act`; per-tensor."""
    input: BufferRef
    output: BufferRef
    element_count: int
    quant_dtype: int = DTYPE_I8
    act: int = lut_act.GELU
    dtype: int = DTYPE_F32
    scale_bits: int = 0
    zero_point: int = 0

    def wire(self) -> bytes:  # put_dequant_activation, kernel_codec.rs:851-860
        return (self.input.wire() + self.output.wire()
                + struct.pack("<QBBBIi", self.element_count, self.quant_dtype, self.act,
                              self.dtype, self.scale_bits, self.zero_point))


@dataclass(frozen=True)
class NormCall:
    """kernel_call.rs:422-446 (RmsNorm uses x, gamma, output; beta and
    residual absent)."""
    x: BufferRef
    gamma: BufferRef
    output: BufferRef
    batch: int
    feature: int
    epsilon_bits: int = 0
    dtype: int = DTYPE_BF16
    beta: BufferRef = NO_BUFFER
    residual: BufferRef = NO_BUFFER
    channels: int = 0
    num_groups: int = 0

    def wire(self) -> bytes:  # put_norm, kernel_codec.rs:656-668
        return (self.x.wire() + self.gamma.wire() + self.beta.wire() + self.residual.wire()
                + self.output.wire()
                + struct.pack("<IIIIQB", self.batch, self.feature, self.channels,
                              self.num_groups, self.epsilon_bits, self.dtype))


@dataclass(frozen=True)
class RoPECall:
    """kernel_call.rs:500-515."""
    x: BufferRef
    cos: BufferRef
    sin: BufferRef
    output: BufferRef
    head_dim: int
    element_count: int
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_rope, kernel_codec.rs:711-719
        return (self.x.wire() + self.cos.wire() + self.sin.wire() + self.output.wire()
                + struct.pack("<IQB", self.head_dim, self.element_count, self.dtype))


@dataclass(frozen=True)
class GatherCall:
    """kernel_call.rs:380-404."""
    data: BufferRef
    indices: BufferRef
    output: BufferRef
    outer: int
    axis_dim: int
    inner: int
    num_indices: int
    idx_dtype: int = DTYPE_I32
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_gather, kernel_codec.rs:626-636
        return (self.data.wire() + self.indices.wire() + self.output.wire()
                + struct.pack("<QQQQBB", self.outer, self.axis_dim, self.inner,
                              self.num_indices, self.idx_dtype, self.dtype))


@dataclass(frozen=True)
class ArgMaxCall:
    """New (discriminant 124): per-row argmax into i32 (include/holo_hip.h)."""
    input: BufferRef
    output: BufferRef
    rows: int
    cols: int
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:
        return self.input.wire() + self.output.wire() + struct.pack("<IIB", self.rows, self.cols,
                                                                    self.dtype)


@dataclass(frozen=True)
class MatMulCall:
    """kernel_call.rs:49-65."""
    a: BufferRef
    b: BufferRef
    output: BufferRef
    m: int
    k: int
    n: int
    dtype: int = DTYPE_F32
    b_packed: bool = False

    def wire(self) -> bytes:  # put_matmul, kernel_codec.rs:590-599
        return (self.a.wire() + self.b.wire() + self.output.wire()
                + struct.pack("<IIIBB", self.m, self.k, self.n, self.dtype, int(self.b_packed)))


@dataclass(frozen=True)
class MatMulActivationCall:
    """kernel_call.rs:892-896: out = act(A*B)."""
    mm: MatMulCall
    act: int

    def wire(self) -> bytes:  # kernel_codec.rs:509-513
        return self.mm.wire() + struct.pack("<B", self.act)


@dataclass(frozen=True)
class MatMulAddCall:
    """kernel_call.rs:906-911: out = A*B + residual."""
    mm: MatMulCall
    residual: BufferRef

    def wire(self) -> bytes:  # kernel_codec.rs:514-518
        return self.mm.wire() + self.residual.wire()


@dataclass(frozen=True)
class MatMulAddActivationCall:
    """kernel_call.rs:923-929: out = act(A*B + residual)."""
    mm: MatMulCall
    residual: BufferRef
    act: int

    def wire(self) -> bytes:  # kernel_codec.rs:519-524
        return self.mm.wire() + self.residual.wire() + struct.pack("<B", self.act)


@dataclass(frozen=True)
class KvCacheWriteCall:
    """kernel_call.rs:742-759."""
    cache: BufferRef
    new: BufferRef
    pos: BufferRef
    output: BufferRef
    planes: int
    bucket_rows: int
    new_rows: int
    row_bytes: int

    def wire(self) -> bytes:  # put_kvwr, kernel_codec.rs:804-813
        return (self.cache.wire() + self.new.wire() + self.pos.wire() + self.output.wire()
                + struct.pack("<IIII", self.planes, self.bucket_rows, self.new_rows,
                              self.row_bytes))


@dataclass(frozen=True)
class KvQuantAppendCall:
    """New (discriminant 122): int8 quantize + ring append (include/holo_hip.h)."""
    new: BufferRef
    pos: BufferRef
    cache: BufferRef
    cache_scales: BufferRef
    output: BufferRef
    output_scales: BufferRef
    planes: int
    bucket_rows: int
    new_rows: int
    head_dim: int
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:
        return (self.new.wire() + self.pos.wire() + self.cache.wire() + self.cache_scales.wire()
                + self.output.wire() + self.output_scales.wire()
                + struct.pack("<IIIIB", self.planes, self.bucket_rows, self.new_rows,
                              self.head_dim, self.dtype))


@dataclass(frozen=True)
class DecodeAttentionCall:
    """kernel_call.rs:632-656: decode attention with an additive f32 mask
    [q_rows, past_len + new_len] (every past row, then every new row, is a
    key; -inf erases one)."""
    q: BufferRef
    k_past: BufferRef
    v_past: BufferRef
    k_new: BufferRef
    v_new: BufferRef
    mask: BufferRef
    output: BufferRef
    batch: int
    heads: int
    kv_heads: int
    q_rows: int
    past_len: int
    new_len: int
    head_dim: int
    scale_bits: int = 0
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_decattn, kernel_codec.rs:768-785
        return (self.q.wire() + self.k_past.wire() + self.v_past.wire() + self.k_new.wire()
                + self.v_new.wire() + self.mask.wire() + self.output.wire()
                + struct.pack("<IIIIIIIIB", self.batch, self.heads, self.kv_heads, self.q_rows,
                              self.past_len, self.new_len, self.head_dim, self.scale_bits,
                              self.dtype))


@dataclass(frozen=True)
class DecodeAttentionValidCall:
    """kernel_call.rs:691-716: the reference's decode attention over 16-bit or
    f32 K/V (past prefix of valid_len realized rows, then new rows causally)."""
    q: BufferRef
    k_past: BufferRef
    v_past: BufferRef
    k_new: BufferRef
    v_new: BufferRef
    valid_len: BufferRef
    output: BufferRef
    batch: int
    heads: int
    kv_heads: int
    q_rows: int
    past_len: int
    new_len: int
    head_dim: int
    scale_bits: int = 0
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_davl, kernel_codec.rs:786-803
        return (self.q.wire() + self.k_past.wire() + self.v_past.wire() + self.k_new.wire()
                + self.v_new.wire() + self.valid_len.wire() + self.output.wire()
                + struct.pack("<IIIIIIIIB", self.batch, self.heads, self.kv_heads, self.q_rows,
                              self.past_len, self.new_len, self.head_dim, self.scale_bits,
                              self.dtype))


@dataclass(frozen=True)
class DecodeAttentionI8Call:
    """New (discriminant 123): GQA decode over an int8 cache (include/holo_hip.h)."""
    q: BufferRef
    k_cache: BufferRef
    v_cache: BufferRef
    k_scales: BufferRef
    v_scales: BufferRef
    lens: BufferRef
    output: BufferRef
    batch: int
    heads: int
    kv_heads: int
    bucket_rows: int
    head_dim: int
    scale_bits: int = 0
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:
        return (self.q.wire() + self.k_cache.wire() + self.v_cache.wire() + self.k_scales.wire()
                + self.v_scales.wire() + self.lens.wire() + self.output.wire()
                + struct.pack("<IIIIIIB", self.batch, self.heads, self.kv_heads,
                              self.bucket_rows, self.head_dim, self.scale_bits, self.dtype))


@dataclass(frozen=True)
class AttentionI8RowsCall:
    """New (discriminant 125): DecodeAttentionI8 over q_rows query rows per
    sequence, row t seeing lens[b] - (q_rows - 1 - t) keys (include/holo_hip.h)."""
    attn: DecodeAttentionI8Call
    q_rows: int

    def wire(self) -> bytes:
        return self.attn.wire() + struct.pack("<I", self.q_rows)


@dataclass(frozen=True)
class TransposeCall:
    """kernel_call.rs:487-499: output axis i is input axis perm[i]."""
    input: BufferRef
    output: BufferRef
    dims: tuple
    perm: tuple
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_transpose, kernel_codec.rs:687-697
        rank = len(self.dims)
        dims = list(self.dims) + [0] * (8 - rank)
        perm = list(self.perm) + [0] * (8 - rank)
        return (self.input.wire() + self.output.wire() + struct.pack("<B", rank)
                + struct.pack("<8I", *dims) + struct.pack("<8B", *perm)
                + struct.pack("<B", self.dtype))


@dataclass(frozen=True)
class LayoutCall:
    """kernel_call.rs:479-485 (Reshape, Slice): the first element_count
    elements of the input view, copied; a session binds an interior one as a
    view of its input instead (session.rs:1106-1150)."""
    input: BufferRef
    output: BufferRef
    element_count: int
    dtype: int = DTYPE_BF16

    def wire(self) -> bytes:  # put_layout, kernel_codec.rs:681-686
        return (self.input.wire() + self.output.wire()
                + struct.pack("<QB", self.element_count, self.dtype))


_NAMES = {D_RESHAPE: "Reshape", D_SLICE: "Slice", D_ADD: "Add", D_MUL: "Mul", D_RN: "RmsNorm", D_ADDRMS: "AddRmsNorm", D_ROTARY: "RotaryEmbedding",
          D_RELU: "Relu", D_ELU: "Elu", D_SELU: "Selu", D_ERF: "Erf", D_DEQ: "Dequantize",
          D_MMDQ: "MatMulDequant", D_DQACT: "DequantActivation",
          D_GATHER: "Gather", D_ARGMAX: "ArgMax", D_SIGMOID: "Sigmoid", D_TANH: "Tanh", D_GELU: "Gelu", D_SILU: "Silu", D_EXP: "Exp",
          D_MATMUL: "MatMul", D_MMA: "MatMulActivation", D_MMADD: "MatMulAdd",
          D_MMAA: "MatMulAddActivation", D_KVWR: "KvCacheWrite", D_KVQA: "KvQuantAppend",
          D_DECATTN: "DecodeAttention", D_DAVL: "DecodeAttentionValid", D_DAI8: "DecodeAttentionI8", D_AI8R: "AttentionI8Rows", D_TRANSPOSE: "Transpose"}


@dataclass(frozen=True)
class KernelCall:
    """One variant of the closed KernelCall enum: discriminant + payload."""
    tag: int
    payload: object = field(repr=True)

    # constructors named after the Rust variants (kernel_call.rs:1146-1276)
    @classmethod
    def Sigmoid(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_SIGMOID, c)

    @classmethod
    def Tanh(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_TANH, c)

    @classmethod
    def Gelu(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_GELU, c)

    @classmethod
    def Silu(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_SILU, c)

    @classmethod
    def Exp(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_EXP, c)

    @classmethod
    def Relu(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_RELU, c)

    @classmethod
    def Elu(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_ELU, c)

    @classmethod
    def Selu(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_SELU, c)

    @classmethod
    def Erf(cls, c: UnaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_ERF, c)

    @classmethod
    def Dequantize(cls, c: DequantizeCall) -> "KernelCall":  # noqa: N802
        return cls(D_DEQ, c)

    @classmethod
    def MatMulDequant(cls, c: MatMulDequantCall) -> "KernelCall":  # noqa: N802
        return cls(D_MMDQ, c)

    @classmethod
    def DequantActivation(cls, c: DequantActivationCall) -> "KernelCall":  # noqa: N802
        return cls(D_DQACT, c)

    @classmethod
    def MatMul(cls, c: MatMulCall) -> "KernelCall":  # noqa: N802
        return cls(D_MATMUL, c)

    @classmethod
    def MatMulActivation(cls, c: MatMulActivationCall) -> "KernelCall":  # noqa: N802
        return cls(D_MMA, c)

    @classmethod
    def MatMulAdd(cls, c: MatMulAddCall) -> "KernelCall":  # noqa: N802
        return cls(D_MMADD, c)

    @classmethod
    def MatMulAddActivation(cls, c: MatMulAddActivationCall) -> "KernelCall":  # noqa: N802
        return cls(D_MMAA, c)

    @classmethod
    def Add(cls, c: BinaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_ADD, c)

    @classmethod
    def Mul(cls, c: BinaryCall) -> "KernelCall":  # noqa: N802
        return cls(D_MUL, c)

    @classmethod
    def RmsNorm(cls, c: NormCall) -> "KernelCall":  # noqa: N802
        return cls(D_RN, c)

    @classmethod
    def AddRmsNorm(cls, c: NormCall) -> "KernelCall":  # noqa: N802
        return cls(D_ADDRMS, c)

    @classmethod
    def RotaryEmbedding(cls, c: RoPECall) -> "KernelCall":  # noqa: N802
        return cls(D_ROTARY, c)

    @classmethod
    def Gather(cls, c: GatherCall) -> "KernelCall":  # noqa: N802
        return cls(D_GATHER, c)

    @classmethod
    def ArgMax(cls, c: ArgMaxCall) -> "KernelCall":  # noqa: N802
        return cls(D_ARGMAX, c)

    @classmethod
    def KvCacheWrite(cls, c: KvCacheWriteCall) -> "KernelCall":  # noqa: N802
        return cls(D_KVWR, c)

    @classmethod
    def KvQuantAppend(cls, c: KvQuantAppendCall) -> "KernelCall":  # noqa: N802
        return cls(D_KVQA, c)

    @classmethod
    def DecodeAttention(cls, c: DecodeAttentionCall) -> "KernelCall":  # noqa: N802
        return cls(D_DECATTN, c)

    @classmethod
    def DecodeAttentionValid(cls, c: DecodeAttentionValidCall) -> "KernelCall":  # noqa: N802
        return cls(D_DAVL, c)

    @classmethod
    def DecodeAttentionI8(cls, c: DecodeAttentionI8Call) -> "KernelCall":  # noqa: N802
        return cls(D_DAI8, c)

    @classmethod
    def AttentionI8Rows(cls, c: AttentionI8RowsCall) -> "KernelCall":  # noqa: N802
        return cls(D_AI8R, c)

    @classmethod
    def Transpose(cls, c: TransposeCall) -> "KernelCall":  # noqa: N802
        return cls(D_TRANSPOSE, c)

    @classmethod
    def Reshape(cls, c: LayoutCall) -> "KernelCall":  # noqa: N802
        return cls(D_RESHAPE, c)

    @classmethod
    def Slice(cls, c: LayoutCall) -> "KernelCall":  # noqa: N802
        return cls(D_SLICE, c)

    @property
    def name(self) -> str:
        return _NAMES.get(self.tag, f"op{self.tag}")

    def encode(self) -> bytes:
        """Archive wire form of this one call (kernel_codec.rs encode_one); a
        variant with several wire forms picks its own discriminant."""
        wire_tag = getattr(self.payload, "wire_tag", None)
        tag = wire_tag() if wire_tag else self.tag
        return struct.pack("<H", tag) + self.payload.wire()

    def to_c(self) -> _ffi.KernelCallC:
        kc = _ffi.KernelCallC()
        kc.tag = self.tag
        p = self.payload
        if isinstance(p, UnaryCall):
            kc.u.unary = _ffi.UnaryCallC(p.input.c(), p.output.c(), p.element_count,
                                         p.witt_bits, p.dtype)
        elif isinstance(p, BinaryCall):
            kc.u.binary = _ffi.BinaryCallC(p.a.c(), p.b.c(), p.output.c(), p.element_count,
                                           p.witt_bits, p.dtype)
        elif isinstance(p, NormCall):
            kc.u.norm = _ffi.NormCallC(p.x.c(), p.gamma.c(), p.beta.c(), p.residual.c(),
                                       p.output.c(), p.batch, p.feature, p.channels,
                                       p.num_groups, p.epsilon_bits, p.dtype)
        elif isinstance(p, RoPECall):
            kc.u.rope = _ffi.RopeCallC(p.x.c(), p.cos.c(), p.sin.c(), p.output.c(), p.head_dim,
                                       p.element_count, p.dtype)
        elif isinstance(p, GatherCall):
            kc.u.gather = _ffi.GatherCallC(p.data.c(), p.indices.c(), p.output.c(), p.outer,
                                           p.axis_dim, p.inner, p.num_indices, p.idx_dtype,
                                           p.dtype)
        elif isinstance(p, ArgMaxCall):
            kc.u.argmax = _ffi.ArgMaxCallC(p.input.c(), p.output.c(), p.rows, p.cols, p.dtype)
        elif isinstance(p, MatMulCall):
            kc.u.matmul = _ffi.MatMulCallC(p.a.c(), p.b.c(), p.output.c(), p.m, p.k, p.n,
                                           p.dtype, int(p.b_packed))
        elif isinstance(p, MatMulActivationCall):
            kc.u.matmul_act = _ffi.MatMulActCallC(_mm_c(p.mm), p.act)
        elif isinstance(p, MatMulAddCall):
            kc.u.matmul_add = _ffi.MatMulAddCallC(_mm_c(p.mm), p.residual.c())
        elif isinstance(p, MatMulAddActivationCall):
            kc.u.matmul_add_act = _ffi.MatMulAddActCallC(_mm_c(p.mm), p.residual.c(), p.act)
        elif isinstance(p, KvCacheWriteCall):
            kc.u.kv_write = _ffi.KvCacheWriteCallC(p.cache.c(), p.new.c(), p.pos.c(),
                                                   p.output.c(), p.planes, p.bucket_rows,
                                                   p.new_rows, p.row_bytes)
        elif isinstance(p, KvQuantAppendCall):
            kc.u.kv_quant_append = _ffi.KvQuantAppendCallC(
                p.new.c(), p.pos.c(), p.cache.c(), p.cache_scales.c(), p.output.c(),
                p.output_scales.c(), p.planes, p.bucket_rows, p.new_rows, p.head_dim, p.dtype)
        elif isinstance(p, AttentionI8RowsCall):
            kc.u.attn_i8_rows = _ffi.AttentionI8RowsCallC(_attn_c(p.attn), p.q_rows)
        elif isinstance(p, TransposeCall):
            rank = len(p.dims)
            kc.u.transpose = _ffi.TransposeCallC(
                p.input.c(), p.output.c(), rank,
                (ctypes.c_uint32 * 8)(*(list(p.dims) + [0] * (8 - rank))),
                (ctypes.c_uint8 * 8)(*(list(p.perm) + [0] * (8 - rank))), p.dtype)
        elif isinstance(p, LayoutCall):
            kc.u.layout = _ffi.LayoutCallC(p.input.c(), p.output.c(), p.element_count, p.dtype)
        elif isinstance(p, DecodeAttentionCall):
            kc.u.attn_mask = _ffi.DecodeAttentionCallC(
                p.q.c(), p.k_past.c(), p.v_past.c(), p.k_new.c(), p.v_new.c(), p.mask.c(),
                p.output.c(), p.batch, p.heads, p.kv_heads, p.q_rows, p.past_len, p.new_len,
                p.head_dim, p.scale_bits, p.dtype)
        elif isinstance(p, DecodeAttentionValidCall):
            kc.u.attn_valid = _ffi.DecodeAttentionValidCallC(
                p.q.c(), p.k_past.c(), p.v_past.c(), p.k_new.c(), p.v_new.c(), p.valid_len.c(),
                p.output.c(), p.batch, p.heads, p.kv_heads, p.q_rows, p.past_len, p.new_len,
                p.head_dim, p.scale_bits, p.dtype)
        elif isinstance(p, DecodeAttentionI8Call):
            kc.u.attn_i8 = _ffi.DecodeAttentionI8CallC(
                p.q.c(), p.k_cache.c(), p.v_cache.c(), p.k_scales.c(), p.v_scales.c(),
                p.lens.c(), p.output.c(), p.batch, p.heads, p.kv_heads, p.bucket_rows,
                p.head_dim, p.scale_bits, p.dtype)
        elif isinstance(p, DequantizeCall):
            kc.u.dequantize = _ffi.DequantizeCallC(
                p.input.c(), p.scales.c(), p.zero_points.c(), p.output.c(), p.element_count,
                p.channels, p.inner, p.quant_dtype, p.dtype, p.scale_bits, p.zero_point,
                p.codebook.c(), p.weight_layout, p.act_quant)
        elif isinstance(p, MatMulDequantCall):
            kc.u.matmul_dequant = _ffi.MatMulDequantCallC(
                p.a.c(), p.bq.c(), p.scales.c(), p.zero_points.c(), p.output.c(), p.m, p.k, p.n,
                p.channels, p.inner, p.quant_dtype, p.dtype, p.scale_bits, p.zero_point,
                int(p.bq_omajor), p.act_quant, p.act, p.residual.c(), p.codebook.c())
        elif isinstance(p, DequantActivationCall):
            kc.u.dequant_act = _ffi.DequantActivationCallC(
                p.input.c(), p.output.c(), p.element_count, p.quant_dtype, p.act, p.dtype,
                p.scale_bits, p.zero_point)
        else:
            raise TypeError(f"no C form for payload {type(p).__name__}")
        return kc


def _attn_c(p: DecodeAttentionI8Call) -> _ffi.DecodeAttentionI8CallC:
    return _ffi.DecodeAttentionI8CallC(p.q.c(), p.k_cache.c(), p.v_cache.c(), p.k_scales.c(),
                                       p.v_scales.c(), p.lens.c(), p.output.c(), p.batch,
                                       p.heads, p.kv_heads, p.bucket_rows, p.head_dim,
                                       p.scale_bits, p.dtype)


def _mm_c(p: MatMulCall) -> _ffi.MatMulCallC:
    return _ffi.MatMulCallC(p.a.c(), p.b.c(), p.output.c(), p.m, p.k, p.n, p.dtype,
                            int(p.b_packed))


def encode_calls(calls: list[KernelCall]) -> bytes:
    """kernel_codec.rs:130-137: u32 LE count, then each call."""
    return struct.pack("<I", len(calls)) + b"".join(c.encode() for c in calls)
