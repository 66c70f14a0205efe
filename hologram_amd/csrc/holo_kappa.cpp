// holo_kappa.cpp — κ-labels, the reference's content addresses
// (crates/hologram-archive/src/address.rs): a label is "blake3:" followed by
// the 64 lowercase hex digits of a BLAKE3 digest, 71 ASCII bytes.
//   address_bytes(bytes)                  the digest of the bytes (:96-99)
//   derive_label(opcode, params, labels)  the digest of opcode (u16 LE) ||
//                                         params || each operand label, in
//                                         order (:108-116)
// A computed value's label is derived from its call's op signature
// (KernelCall::op_signature, crates/hologram-compute/src/kernel_call.rs:
// 1321-1500: an opcode plus the call's scalar fields in LE order) and the
// labels of its operands (buffers(), :1526-1660, output last; absent slots
// dropped; the operands of Add and Mul sorted, session.rs:1096-1103).
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "holo_internal.h"

namespace holo {
namespace {

// Fixed-capacity LE parameter bytes of a signature (the reference's Pb).
struct Sig {
    uint8_t b[64];
    uint32_t n = 0;
    Sig &raw(const void *p, uint32_t len) {
        if (n + len <= sizeof b) memcpy(b + n, p, len);
        n += len;
        return *this;
    }
    Sig &u8(uint8_t v) { return raw(&v, 1); }
    Sig &u16(uint16_t v) { return raw(&v, 2); }
    Sig &u32(uint32_t v) { return raw(&v, 4); }
    Sig &u64(uint64_t v) { return raw(&v, 8); }
};

Sig p_unary(const holo_unary_call &c) {
    Sig s;
    return s.u64(c.element_count).u16(c.witt_bits).u8(c.dtype);
}
Sig p_binary(const holo_binary_call &c) {
    Sig s;
    return s.u64(c.element_count).u16(c.witt_bits).u8(c.dtype);
}
Sig p_matmul(const holo_matmul_call &c) {   // b_packed is layout, not identity
    Sig s;
    return s.u32(c.m).u32(c.k).u32(c.n).u8(c.dtype);
}
Sig p_norm(const holo_norm_call &c) {
    Sig s;
    return s.u32(c.batch).u32(c.feature).u32(c.channels).u32(c.num_groups).u64(c.epsilon_bits)
        .u8(c.dtype).u8(c.residual.slot != HOLO_SLOT_ABSENT ? 1 : 0);
}
Sig p_attn_i8(const holo_decode_attention_i8_call &c) {
    Sig s;
    return s.u32(c.batch).u32(c.heads).u32(c.kv_heads).u32(c.bucket_rows).u32(c.head_dim)
        .u32(c.scale_bits).u8(c.dtype);
}

bool per_channel(uint32_t channels, const holo_buffer_ref &scales) {
    return channels > 0 && scales.slot != HOLO_SLOT_ABSENT;
}

}  // namespace

std::string kappa_of_digest(const uint8_t d[32]) {
    static const char hex[] = "0123456789abcdef";
    std::string s = "blake3:";
    for (int i = 0; i < 32; ++i) {
        s.push_back(hex[d[i] >> 4]);
        s.push_back(hex[d[i] & 15]);
    }
    return s;
}

std::string address_bytes(const void *bytes, size_t len) {
    uint8_t d[32];
    blake3_hash(bytes, len, d);
    return kappa_of_digest(d);
}

std::string derive_label(uint16_t opcode, const uint8_t *params, size_t n_params,
                         const std::vector<std::string> &inputs) {
    std::vector<uint8_t> msg(2 + n_params);
    memcpy(msg.data(), &opcode, 2);
    if (n_params) memcpy(msg.data() + 2, params, n_params);
    for (const auto &l : inputs) msg.insert(msg.end(), l.begin(), l.end());
    return address_bytes(msg.data(), msg.size());
}

// The 32-byte digest a "blake3:<64 hex>" label names (compose.rs:108-128);
// false for any other form.
bool digest_of_label(const std::string &l, uint8_t d[32]) {
    if (l.size() != 71 || l.compare(0, 7, "blake3:") != 0) return false;
    auto nib = [](char c) -> int {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    };
    for (int i = 0; i < 32; ++i) {
        const int hi = nib(l[7 + 2 * i]), lo = nib(l[8 + 2 * i]);
        if (hi < 0 || lo < 0) return false;
        d[i] = uint8_t(hi << 4 | lo);
    }
    return true;
}

// compose_ordered_blake3_address (compose.rs:154-164): address_bytes of the
// two digests, left then right.
bool compose_ordered(const std::string &left, const std::string &right, std::string *out) {
    uint8_t canon[64];
    if (!digest_of_label(left, canon) || !digest_of_label(right, canon + 32)) return false;
    *out = address_bytes(canon, 64);
    return true;
}

bool derive_label_boundary(uint16_t opcode, const uint8_t *params, size_t n_params,
                           const std::vector<std::string> &inputs, std::string *out) {
    std::vector<uint8_t> pre(2 + n_params);
    memcpy(pre.data(), &opcode, 2);
    if (n_params) memcpy(pre.data() + 2, params, n_params);
    const std::string op_label = address_bytes(pre.data(), pre.size());
    std::string acc = op_label;
    for (const auto &in : inputs)
        if (!compose_ordered(acc, in, &acc)) return false;
    if (inputs.empty()) return compose_ordered(op_label, op_label, out);
    *out = acc;
    return true;
}

bool op_signature(const holo_kernel_call &c, uint16_t *opcode, uint8_t params[64], uint32_t *len) {
    Sig s;
    uint16_t op = 0;
    switch (c.tag) {
        case HOLO_OP_RELU: s = p_unary(c.u.unary), op = 10; break;
        case HOLO_OP_SIGMOID: s = p_unary(c.u.unary), op = 11; break;
        case HOLO_OP_TANH: s = p_unary(c.u.unary), op = 12; break;
        case HOLO_OP_GELU: s = p_unary(c.u.unary), op = 13; break;
        case HOLO_OP_SILU: s = p_unary(c.u.unary), op = 14; break;
        case HOLO_OP_ELU: s = p_unary(c.u.unary), op = 15; break;
        case HOLO_OP_SELU: s = p_unary(c.u.unary), op = 16; break;
        case HOLO_OP_EXP: s = p_unary(c.u.unary), op = 17; break;
        case HOLO_OP_ERF: s = p_unary(c.u.unary), op = 31; break;
        case HOLO_OP_ADD: s = p_binary(c.u.binary), op = 4; break;
        case HOLO_OP_MUL: s = p_binary(c.u.binary), op = 6; break;
        case HOLO_OP_MATMUL: s = p_matmul(c.u.matmul), op = 45; break;
        case HOLO_OP_RMS_NORM: s = p_norm(c.u.norm), op = 50; break;
        case HOLO_OP_ADD_RMS_NORM: s = p_norm(c.u.norm), op = 53; break;
        case HOLO_OP_TRANSPOSE: {
            const auto &t = c.u.transpose;
            s.u8(t.rank).u8(t.dtype);
            for (uint32_t i = 0; i < t.rank && i < 8; ++i) s.u32(t.dims[i]).u8(t.perm[i]);
            op = 60;
            break;
        }
        case HOLO_OP_RESHAPE: s.u64(c.u.layout.element_count).u8(c.u.layout.dtype), op = 59; break;
        case HOLO_OP_SLICE: s.u64(c.u.layout.element_count).u8(c.u.layout.dtype), op = 62; break;
        case HOLO_OP_ROTARY: {
            const auto &r = c.u.rope;
            s.u64(r.element_count).u32(r.head_dim).u8(r.dtype);
            op = 74;
            break;
        }
        case HOLO_OP_DEQUANTIZE: {
            const auto &d = c.u.dequantize;
            s.u64(d.element_count).u32(d.channels).u32(d.inner).u8(d.quant_dtype).u8(d.dtype)
                .u32(d.scale_bits).u32(uint32_t(d.zero_point)).u8(per_channel(d.channels, d.scales));
            op = 104;
            break;
        }
        case HOLO_OP_MATMUL_ACT: s = p_matmul(c.u.matmul_act.mm), s.u8(c.u.matmul_act.act), op = 105; break;
        case HOLO_OP_MATMUL_ADD: s = p_matmul(c.u.matmul_add.mm), op = 106; break;
        case HOLO_OP_MATMUL_ADD_ACT:
            s = p_matmul(c.u.matmul_add_act.mm), s.u8(c.u.matmul_add_act.act), op = 107;
            break;
        case HOLO_OP_MATMUL_DEQUANT: {   // bq_omajor is layout and excluded
            const auto &d = c.u.matmul_dequant;
            s.u32(d.m).u32(d.k).u32(d.n).u32(d.channels).u32(d.inner).u8(d.quant_dtype).u8(d.dtype)
                .u32(d.scale_bits).u32(uint32_t(d.zero_point));
            const bool res = d.residual.slot != HOLO_SLOT_ABSENT;
            if (d.codebook.slot != HOLO_SLOT_ABSENT)
                s.u8(d.act_quant).u8(d.act).u8(res).u8(1), op = 117;
            else if (d.act_quant != 0 || d.act != 0 || res)
                s.u8(d.act_quant).u8(d.act).u8(res), op = 116;
            else
                op = 108;
            break;
        }
        case HOLO_OP_DEQUANT_ACT: {
            const auto &d = c.u.dequant_act;
            s.u64(d.element_count).u8(d.quant_dtype).u8(d.act).u8(d.dtype).u32(d.scale_bits)
                .u32(uint32_t(d.zero_point));
            op = 113;
            break;
        }
        case HOLO_OP_GATHER: {
            const auto &g = c.u.gather;
            s.u64(g.outer).u64(g.axis_dim).u64(g.inner).u64(g.num_indices).u8(g.idx_dtype).u8(g.dtype);
            op = 114;
            break;
        }
        case HOLO_OP_KV_CACHE_WRITE: {
            const auto &k = c.u.kv_write;
            s.u32(k.planes).u32(k.bucket_rows).u32(k.new_rows).u32(k.row_bytes);
            op = 120;
            break;
        }
        case HOLO_OP_DECODE_ATTN: {
            const auto &a = c.u.attn_mask;
            s.u32(a.batch).u32(a.heads).u32(a.kv_heads).u32(a.q_rows).u32(a.past_len).u32(a.new_len)
                .u32(a.head_dim).u32(a.scale_bits).u8(a.dtype);
            op = 119;
            break;
        }
        case HOLO_OP_DECODE_ATTN_VALID: {
            const auto &a = c.u.attn_valid;
            s.u32(a.batch).u32(a.heads).u32(a.kv_heads).u32(a.q_rows).u32(a.past_len).u32(a.new_len)
                .u32(a.head_dim).u32(a.scale_bits).u8(a.dtype);
            op = 121;
            break;
        }
        // the new capabilities take the opcode of their new discriminant
        case HOLO_OP_KV_QUANT_APPEND: {
            const auto &k = c.u.kv_quant_append;
            s.u32(k.planes).u32(k.bucket_rows).u32(k.new_rows).u32(k.head_dim).u8(k.dtype);
            op = 122;
            break;
        }
        case HOLO_OP_DECODE_ATTN_I8: s = p_attn_i8(c.u.attn_i8), op = 123; break;
        case HOLO_OP_ARGMAX: {
            const auto &a = c.u.argmax;
            s.u32(a.rows).u32(a.cols).u8(a.dtype);
            op = 124;
            break;
        }
        case HOLO_OP_ATTN_I8_ROWS:
            s = p_attn_i8(c.u.attn_i8_rows.attn), s.u32(c.u.attn_i8_rows.q_rows), op = 125;
            break;
        default: return false;
    }
    if (s.n > 64) return false;
    *opcode = op;
    memcpy(params, s.b, s.n);
    *len = s.n;
    return true;
}

bool label_operands(const holo_kernel_call &c, std::vector<uint32_t> *ins,
                    std::vector<uint32_t> *outs, bool *commutative) {
    ins->clear();
    outs->clear();
    *commutative = c.tag == HOLO_OP_ADD || c.tag == HOLO_OP_MUL;
    auto r = [&](const holo_buffer_ref &b) {
        if (b.slot != HOLO_SLOT_ABSENT) ins->push_back(b.slot);
    };
    auto w = [&](const holo_buffer_ref &b) { outs->push_back(b.slot); };
    switch (c.tag) {
        case HOLO_OP_RELU: case HOLO_OP_SIGMOID: case HOLO_OP_TANH: case HOLO_OP_GELU:
        case HOLO_OP_SILU: case HOLO_OP_ELU: case HOLO_OP_SELU: case HOLO_OP_EXP: case HOLO_OP_ERF:
            r(c.u.unary.input), w(c.u.unary.output); break;
        case HOLO_OP_ADD: case HOLO_OP_MUL:
            r(c.u.binary.a), r(c.u.binary.b), w(c.u.binary.output); break;
        case HOLO_OP_MATMUL: r(c.u.matmul.a), r(c.u.matmul.b), w(c.u.matmul.output); break;
        case HOLO_OP_MATMUL_ACT:
            r(c.u.matmul_act.mm.a), r(c.u.matmul_act.mm.b), w(c.u.matmul_act.mm.output); break;
        case HOLO_OP_MATMUL_ADD:
            r(c.u.matmul_add.mm.a), r(c.u.matmul_add.mm.b), r(c.u.matmul_add.residual);
            w(c.u.matmul_add.mm.output); break;
        case HOLO_OP_MATMUL_ADD_ACT:
            r(c.u.matmul_add_act.mm.a), r(c.u.matmul_add_act.mm.b), r(c.u.matmul_add_act.residual);
            w(c.u.matmul_add_act.mm.output); break;
        case HOLO_OP_RMS_NORM: case HOLO_OP_ADD_RMS_NORM:   // the residual is not an operand here
            r(c.u.norm.x), r(c.u.norm.gamma), r(c.u.norm.beta), w(c.u.norm.output); break;
        case HOLO_OP_TRANSPOSE: r(c.u.transpose.input), w(c.u.transpose.output); break;
        case HOLO_OP_RESHAPE: case HOLO_OP_SLICE: r(c.u.layout.input), w(c.u.layout.output); break;
        case HOLO_OP_ROTARY:
            r(c.u.rope.x), r(c.u.rope.cos), r(c.u.rope.sin), w(c.u.rope.output); break;
        case HOLO_OP_GATHER:
            r(c.u.gather.data), r(c.u.gather.indices), w(c.u.gather.output); break;
        case HOLO_OP_DEQUANTIZE: {
            const auto &d = c.u.dequantize;
            r(d.input);
            if (per_channel(d.channels, d.scales)) r(d.scales), r(d.zero_points);
            w(d.output);
            break;
        }
        case HOLO_OP_DEQUANT_ACT: r(c.u.dequant_act.input), w(c.u.dequant_act.output); break;
        case HOLO_OP_MATMUL_DEQUANT: {
            const auto &d = c.u.matmul_dequant;
            r(d.a), r(d.bq);
            if (per_channel(d.channels, d.scales)) r(d.scales), r(d.zero_points);
            r(d.codebook), r(d.residual), w(d.output);
            break;
        }
        case HOLO_OP_KV_CACHE_WRITE: {
            const auto &k = c.u.kv_write;
            r(k.cache), r(k.new_rows_buf), r(k.pos), w(k.output);
            break;
        }
        case HOLO_OP_DECODE_ATTN: {
            const auto &a = c.u.attn_mask;
            r(a.q), r(a.k_past), r(a.v_past), r(a.k_new), r(a.v_new), r(a.mask), w(a.output);
            break;
        }
        case HOLO_OP_DECODE_ATTN_VALID: {
            const auto &a = c.u.attn_valid;
            r(a.q), r(a.k_past), r(a.v_past), r(a.k_new), r(a.v_new), r(a.valid_len), w(a.output);
            break;
        }
        case HOLO_OP_KV_QUANT_APPEND: {
            const auto &k = c.u.kv_quant_append;
            r(k.new_rows_buf), r(k.pos), r(k.cache), r(k.cache_scales);
            w(k.output), w(k.output_scales);
            break;
        }
        case HOLO_OP_DECODE_ATTN_I8: case HOLO_OP_ATTN_I8_ROWS: {
            const auto &a = c.tag == HOLO_OP_ATTN_I8_ROWS ? c.u.attn_i8_rows.attn : c.u.attn_i8;
            r(a.q), r(a.k_cache), r(a.v_cache), r(a.k_scales), r(a.v_scales), r(a.lens), w(a.output);
            break;
        }
        case HOLO_OP_ARGMAX: r(c.u.argmax.input), w(c.u.argmax.output); break;
        default: return false;
    }
    return true;
}

}  // namespace holo

// ------------------------------------------------------------------ C ABI --
int holo_hip_address_bytes(const void *bytes, uint64_t len, char out[72]) {
    if ((!bytes && len) || !out) return holo::set_error(HOLO_ERR_INIT, "address_bytes: null argument");
    const std::string l = holo::address_bytes(bytes, size_t(len));
    memcpy(out, l.c_str(), l.size() + 1);
    return HOLO_OK;
}

int holo_hip_derive_label(uint16_t opcode, const uint8_t *params, uint64_t n_params,
                          const char *labels, uint64_t n_labels, char out[72]) {
    if ((!params && n_params) || (!labels && n_labels) || !out)
        return holo::set_error(HOLO_ERR_INIT, "derive_label: null argument");
    std::vector<std::string> in;
    for (uint64_t i = 0; i < n_labels; ++i)
        in.emplace_back(labels + i * HOLO_LABEL_LEN, HOLO_LABEL_LEN);
    const std::string l = holo::derive_label(opcode, params, size_t(n_params), in);
    memcpy(out, l.c_str(), l.size() + 1);
    return HOLO_OK;
}

int holo_hip_derive_label_boundary(uint16_t opcode, const uint8_t *params, uint64_t n_params,
                                   const char *labels, uint64_t n_labels, char out[72]) {
    if ((!params && n_params) || (!labels && n_labels) || !out)
        return holo::set_error(HOLO_ERR_INIT, "derive_label_boundary: null argument");
    std::vector<std::string> in;
    for (uint64_t i = 0; i < n_labels; ++i)
        in.emplace_back(labels + i * HOLO_LABEL_LEN, HOLO_LABEL_LEN);
    std::string l;
    if (!holo::derive_label_boundary(opcode, params, size_t(n_params), in, &l))
        return holo::set_error(HOLO_ERR_DISPATCH,
                               "derive_label_boundary: an operand label is not a blake3 label");
    memcpy(out, l.c_str(), l.size() + 1);
    return HOLO_OK;
}

int holo_hip_op_signature(const holo_kernel_call *call, uint16_t *opcode, uint8_t params[64],
                          uint32_t *n_params) {
    if (!call || !opcode || !params || !n_params)
        return holo::set_error(HOLO_ERR_INIT, "op_signature: null argument");
    if (!holo::op_signature(*call, opcode, params, n_params))
        return holo::set_error(HOLO_ERR_UNSUPPORTED_OP,
                               "op_signature: kernel call tag " + std::to_string(call->tag) +
                                   " is not served by this backend");
    return HOLO_OK;
}
