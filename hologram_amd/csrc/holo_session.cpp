// holo_session.cpp — a `.holo` archive executed over device-resident slots:
// the InferenceSession of crates/hologram-exec/src/session.rs with the
// MI355X backend behind every node.
//
// Load (session.rs:428-797): header, version 2..=3 and the BLAKE3 footer over
// every preceding byte (crates/hologram-archive/src/loader.rs:141-185); the
// section table (loader.rs:220-263); KernelCalls (kernel_codec.rs wire form),
// Inputs/Outputs ports (writer.rs decode_ports), ExecPlan levels (writer.rs
// decode_exec_plan; absent = one level holding every call in order),
// Constants (constant_codec.rs; a by-reference body resolves through the
// Weights section, whose fingerprints are re-verified, writer.rs
// decode_weights). Per-slot sizes follow session.rs:544-623: the largest
// referencing BufferRef length, port byte count or constant body, at least 64
// bytes, rounded up to 64. Constants are uploaded to the device once; every
// other slot gets one device buffer for the life of the session (the
// reference binds a fresh pool buffer per node per walk; with the graph memo
// off, a slot's previous value is never read again, so the buffer is reused).
//
// Execute (session.rs:846-932 and compute_and_label :1052-1289): the levels
// in order, each node dispatched on the backend with operands resolved
// through the session's slot table. A KvCacheWrite / KvQuantAppend whose
// cache operand no other node reads and that is no output port is run as the
// in-place move (session.rs:1163-1190, 1313-1370): the call is rewritten at
// load to write its cache operand, and its output slot aliases that buffer.
// The whole walk can be captured once into a HIP graph and replayed, which
// removes the per-node host cost from a decode step (the reference's ~191 ns
// per node is per-execute host work that a GPU walk must not serialize on).
//
// Also here: the loader's fusion passes (fuse_dequant_matmul,
// fuse_matmul_epilogue, fuse_dequant_activation, session.rs:493-509, 1853-2373)
// and a device fusion of this backend's own; κ-labels derived for every node
// (holo_kappa.cpp) and the whole-graph memo with its off switch.
// Not carried over: paged weight providers, leases and warm-start sections
// (WarmStart is ignored).
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <map>
#include <memory>
#include <string>
#include <tuple>
#include <vector>

#include "holo_hip.h"
#include "holo_internal.h"
#include "holo_kernels.h"

namespace {

using holo::set_error;
using holo::SlotRange;

constexpr uint16_t kFormatVersion = 3, kMinReadVersion = 2;   // format.rs:16-21
enum : uint8_t {
    kSecKernelCalls = 1, kSecWeights = 3, kSecInputs = 9, kSecOutputs = 10, kSecConstants = 11,
    kSecExecPlan = 12,
};

struct Port {
    std::string name;
    uint32_t slot = 0;
    uint64_t count = 0;
    uint8_t dtype = 0;
    std::vector<uint64_t> shape;
};

struct Cursor {
    const uint8_t *p;
    size_t len, at = 0;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (at + sizeof(T) > len) {
            ok = false;
            at = len;
            return v;
        }
        memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    const uint8_t *take(size_t n) {
        if (at + n > len || at + n < at) {
            ok = false;
            at = len;
            return nullptr;
        }
        const uint8_t *r = p + at;
        at += n;
        return r;
    }
};

// port_bytes_per_element (session.rs): the element width of a port's dtype.
uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t sat_mul(uint64_t a, uint64_t b) { return b && a > UINT64_MAX / b ? UINT64_MAX : a * b; }

uint64_t port_bytes(uint8_t dt) {
    switch (dt) {
        case 0: case 1: case HOLO_DTYPE_I8: return 1;   // bool, u8, i8
        case HOLO_DTYPE_F16: case HOLO_DTYPE_BF16: return 2;
        case HOLO_DTYPE_I32: case HOLO_DTYPE_F32: return 4;
        case 3: case HOLO_DTYPE_I64: case 9: return 8;  // u64, i64, f64
        default: return 1;
    }
}

// DequantizeCall::per_channel (kernel_call.rs:850-854).
bool dequant_per_channel(const holo_dequantize_call &d) {
    return d.channels > 0 && d.scales.slot != HOLO_SLOT_ABSENT;
}

// The BufferRefs a call reads and writes. Writes are the call's outputs
// (two for KvQuantAppend: the int8 cache and its scales).
void call_operands(const holo_kernel_call &c, std::vector<holo_buffer_ref> *reads,
                   std::vector<holo_buffer_ref> *writes) {
    reads->clear();
    writes->clear();
    auto r = [&](const holo_buffer_ref &b) {
        if (b.slot != HOLO_SLOT_ABSENT) reads->push_back(b);
    };
    auto w = [&](const holo_buffer_ref &b) { writes->push_back(b); };
    switch (c.tag) {
        case HOLO_OP_SIGMOID: case HOLO_OP_TANH: case HOLO_OP_GELU: case HOLO_OP_SILU:
        case HOLO_OP_EXP: case HOLO_OP_RELU: case HOLO_OP_ELU: case HOLO_OP_SELU: case HOLO_OP_ERF:
            r(c.u.unary.input); w(c.u.unary.output); break;
        case HOLO_OP_DEQUANTIZE: {   // buffers(), kernel_call.rs:1656-1657
            const auto &d = c.u.dequantize;
            r(d.input);
            if (dequant_per_channel(d)) { r(d.scales); r(d.zero_points); }
            w(d.output); break;
        }
        case HOLO_OP_DEQUANT_ACT:
            r(c.u.dequant_act.input); w(c.u.dequant_act.output); break;
        case HOLO_OP_MATMUL_DEQUANT: {   // buffers(), kernel_call.rs:1583-1601
            const auto &d = c.u.matmul_dequant;
            r(d.a); r(d.bq);
            if (d.channels > 0 && d.scales.slot != HOLO_SLOT_ABSENT) { r(d.scales); r(d.zero_points); }
            r(d.codebook); r(d.residual);
            w(d.output); break;
        }
        case HOLO_OP_ADD: case HOLO_OP_MUL:
            r(c.u.binary.a); r(c.u.binary.b); w(c.u.binary.output); break;
        case HOLO_OP_RMS_NORM: case HOLO_OP_ADD_RMS_NORM:
            r(c.u.norm.x); r(c.u.norm.gamma); r(c.u.norm.beta); r(c.u.norm.residual);
            w(c.u.norm.output); break;
        case HOLO_OP_ROTARY:
            r(c.u.rope.x); r(c.u.rope.cos); r(c.u.rope.sin); w(c.u.rope.output); break;
        case HOLO_OP_GATHER:
            r(c.u.gather.data); r(c.u.gather.indices); w(c.u.gather.output); break;
        case HOLO_OP_ARGMAX:
            r(c.u.argmax.input); w(c.u.argmax.output); break;
        case HOLO_OP_MATMUL:
            r(c.u.matmul.a); r(c.u.matmul.b); w(c.u.matmul.output); break;
        case HOLO_OP_MATMUL_ACT:
            r(c.u.matmul_act.mm.a); r(c.u.matmul_act.mm.b); w(c.u.matmul_act.mm.output); break;
        case HOLO_OP_MATMUL_ADD:
            r(c.u.matmul_add.mm.a); r(c.u.matmul_add.mm.b); r(c.u.matmul_add.residual);
            w(c.u.matmul_add.mm.output); break;
        case HOLO_OP_MATMUL_ADD_ACT:
            r(c.u.matmul_add_act.mm.a); r(c.u.matmul_add_act.mm.b); r(c.u.matmul_add_act.residual);
            w(c.u.matmul_add_act.mm.output); break;
        case HOLO_OP_KV_CACHE_WRITE:
            r(c.u.kv_write.cache); r(c.u.kv_write.new_rows_buf); r(c.u.kv_write.pos);
            w(c.u.kv_write.output); break;
        case HOLO_OP_KV_QUANT_APPEND: {
            const auto &k = c.u.kv_quant_append;
            r(k.new_rows_buf); r(k.pos); r(k.cache); r(k.cache_scales);
            w(k.output); w(k.output_scales); break;
        }
        case HOLO_OP_TRANSPOSE:
            r(c.u.transpose.input); w(c.u.transpose.output); break;
        case HOLO_OP_RESHAPE: case HOLO_OP_SLICE:
            r(c.u.layout.input); w(c.u.layout.output); break;
        case HOLO_OP_DECODE_ATTN_VALID: {
            const auto &a = c.u.attn_valid;
            r(a.q); r(a.k_past); r(a.v_past); r(a.k_new); r(a.v_new); r(a.valid_len);
            w(a.output); break;
        }
        case HOLO_OP_DECODE_ATTN: {
            const auto &a = c.u.attn_mask;
            r(a.q); r(a.k_past); r(a.v_past); r(a.k_new); r(a.v_new); r(a.mask);
            w(a.output); break;
        }
        case HOLO_OP_DECODE_ATTN_I8:
        case HOLO_OP_ATTN_I8_ROWS: {
            const auto &a = c.tag == HOLO_OP_ATTN_I8_ROWS ? c.u.attn_i8_rows.attn : c.u.attn_i8;
            r(a.q); r(a.k_cache); r(a.v_cache); r(a.k_scales); r(a.v_scales); r(a.lens);
            w(a.output); break;
        }
        default: break;
    }
}

int parse_ports(const uint8_t *p, size_t n, std::vector<Port> *out) {
    Cursor c{p, n};
    const uint32_t count = c.get<uint32_t>();
    for (uint32_t i = 0; i < count && c.ok; ++i) {
        Port port;
        const uint16_t nl = c.get<uint16_t>();
        const uint8_t *nm = c.take(nl);
        if (nm) port.name.assign(reinterpret_cast<const char *>(nm), nl);
        port.slot = c.get<uint32_t>();
        port.count = c.get<uint64_t>();
        port.dtype = c.get<uint8_t>();
        const uint8_t rank = c.get<uint8_t>();
        for (uint8_t d = 0; d < rank; ++d) port.shape.push_back(c.get<uint64_t>());
        out->push_back(port);
    }
    if (!c.ok) return set_error(HOLO_ERR_DISPATCH, "session_load: truncated port section");
    return HOLO_OK;
}

// fused_activation id of a standalone activation call (KernelCall::
// fused_activation, crates/hologram-compute/src/kernel_call.rs:1282-1296), or 0.
uint32_t fused_activation(const holo_kernel_call &c) {
    switch (c.tag) {
        case HOLO_OP_GELU: return HOLO_FUSED_GELU;
        case HOLO_OP_SILU: return HOLO_FUSED_SILU;
        case HOLO_OP_SIGMOID: return HOLO_FUSED_SIGMOID;
        case HOLO_OP_TANH: return HOLO_FUSED_TANH;
        case HOLO_OP_EXP: return HOLO_FUSED_EXP;
        case HOLO_OP_RELU: return HOLO_FUSED_RELU;
        case HOLO_OP_ELU: return HOLO_FUSED_ELU;
        case HOLO_OP_SELU: return HOLO_FUSED_SELU;
        default: return 0;
    }
}

// The per-slot census the loader's fusion passes share (session.rs:1861-1876):
// how many calls write and read each slot, the last reader, the output ports.
struct Census {
    std::map<uint32_t, uint32_t> prod, read;
    std::map<uint32_t, size_t> read_idx;
    std::vector<uint32_t> out_slots;

    Census(const std::vector<holo_kernel_call> &calls, const std::vector<Port> &outputs) {
        std::vector<holo_buffer_ref> rd, wr;
        for (size_t i = 0; i < calls.size(); ++i) {
            call_operands(calls[i], &rd, &wr);
            for (auto &r : rd) {
                read[r.slot]++;
                read_idx[r.slot] = i;
            }
            for (auto &w : wr)
                if (w.slot != HOLO_SLOT_ABSENT) prod[w.slot]++;
        }
        for (auto &p : outputs) out_slots.push_back(p.slot);
    }
    static uint32_t count(const std::map<uint32_t, uint32_t> &m, uint32_t s) {
        auto it = m.find(s);
        return it == m.end() ? 0u : it->second;
    }
    bool is_out(uint32_t s) const {
        return std::find(out_slots.begin(), out_slots.end(), s) != out_slots.end();
    }
    // Slot s, written by call i, is a private intermediate (one producer, one
    // reader, no output port) whose reader is a call not yet absorbed: *j.
    bool sole_reader(uint32_t s, size_t i, const std::vector<bool> &absorbed, size_t *j) const {
        if (s == HOLO_SLOT_ABSENT || is_out(s)) return false;
        if (count(prod, s) != 1 || count(read, s) != 1) return false;
        *j = read_idx.at(s);
        return *j != i && !absorbed[*j];
    }
};

// Drop the absorbed calls, put each fused call in its producer's place, and
// renumber the plan (empty levels vanish), as every reference pass does.
void compact(std::vector<holo_kernel_call> &calls, std::vector<std::vector<uint32_t>> &plan,
             const std::vector<bool> &absorbed, const std::vector<holo_kernel_call> &fused,
             const std::vector<bool> &is_fused) {
    const size_t n = calls.size();
    if (std::find(absorbed.begin(), absorbed.end(), true) == absorbed.end()) {
        for (size_t i = 0; i < n; ++i)
            if (is_fused[i]) calls[i] = fused[i];
        return;
    }
    std::vector<holo_kernel_call> nc;
    std::vector<uint32_t> remap(n, HOLO_SLOT_ABSENT);
    for (size_t i = 0; i < n; ++i) {
        if (absorbed[i]) continue;
        remap[i] = uint32_t(nc.size());
        nc.push_back(is_fused[i] ? fused[i] : calls[i]);
    }
    std::vector<std::vector<uint32_t>> np;
    for (auto &level : plan) {
        std::vector<uint32_t> lv;
        for (uint32_t ci : level)
            if (ci < n && !absorbed[ci]) lv.push_back(remap[ci]);
        if (!lv.empty()) np.push_back(std::move(lv));
    }
    calls = std::move(nc);
    plan = std::move(np);
}

// fuse_dequant_matmul (crates/hologram-exec/src/session.rs:1853-2044): a
// Dequantize whose output is a private intermediate read only as the B operand
// of an unpacked f32 MatMul becomes one MatMulDequant in the MatMul's place.
// A weight slot that declares the output-major W8A8 form (weight_layout 1 with
// act_quant 1) is fused as the W8A8 GEMV when the tier and shape allow it; an
// output-major declaration nothing can read ([n, k] bytes) refuses the load.
int fuse_dequant_matmul(std::vector<holo_kernel_call> &calls, std::vector<std::vector<uint32_t>> &plan,
                        const std::vector<Port> &outputs) {
    const size_t n = calls.size();
    const Census cs(calls, outputs);
    std::vector<bool> absorbed(n, false), is_fused(n, false);
    std::vector<holo_kernel_call> fused(calls);
    for (size_t i = 0; i < n; ++i) {
        if (calls[i].tag != HOLO_OP_DEQUANTIZE) continue;
        const holo_dequantize_call dq = calls[i].u.dequantize;
        size_t j;
        if (!cs.sole_reader(dq.output.slot, i, absorbed, &j)) continue;
        if (calls[j].tag != HOLO_OP_MATMUL) continue;
        const holo_matmul_call mm = calls[j].u.matmul;
        if (mm.dtype != HOLO_DTYPE_F32 || mm.b_packed || mm.b.slot != dq.output.slot) continue;
        // the quant_tier registry (quant_tier.rs:137-178)
        const uint8_t q = dq.quant_dtype;
        if (q != HOLO_DTYPE_I8 && q != HOLO_DTYPE_U8 && q != HOLO_DTYPE_I4 && q != HOLO_DTYPE_E8CB) continue;
        const bool needs_cb = q == HOLO_DTYPE_E8CB, has_cb = dq.codebook.slot != HOLO_SLOT_ABSENT;
        const bool k_ok = q == HOLO_DTYPE_I8 || (q == HOLO_DTYPE_I4 && mm.k % 2 == 0) ||
                          (q == HOLO_DTYPE_E8CB && mm.k % 8 == 0);
        const bool declares = dq.weight_layout == 1 && dq.act_quant == 1;
        const bool omajor_ok = declares && q != HOLO_DTYPE_U8 && k_ok && dequant_per_channel(dq) &&
                               dq.inner == 1 && dq.channels == mm.n && mm.k <= holo::kI8DotKMax &&
                               needs_cb == has_cb;
        if (dq.weight_layout == 1 && !omajor_ok)
            return set_error(HOLO_ERR_DISPATCH,
                             "session_load: kernel call " + std::to_string(i) +
                                 " declares an output-major weight that no kernel can read");
        if (!omajor_ok && q == HOLO_DTYPE_E8CB) continue;   // not scalar-decodable: left unfused
        holo_kernel_call f{};
        f.tag = HOLO_OP_MATMUL_DEQUANT;
        auto &md = f.u.matmul_dequant;
        md.a = mm.a;
        md.bq = dq.input;
        md.scales = dq.scales;
        md.zero_points = dq.zero_points;
        md.output = mm.output;
        md.m = mm.m;
        md.k = mm.k;
        md.n = mm.n;
        md.channels = dq.channels;
        md.inner = dq.inner;
        md.quant_dtype = q;
        md.dtype = mm.dtype;
        md.scale_bits = dq.scale_bits;
        md.zero_point = dq.zero_point;
        md.bq_omajor = omajor_ok;
        md.act_quant = omajor_ok ? 1 : 0;
        md.act = 0;
        md.residual = holo_buffer_ref{HOLO_SLOT_ABSENT, 0, 0};
        md.codebook = omajor_ok ? dq.codebook : holo_buffer_ref{HOLO_SLOT_ABSENT, 0, 0};
        fused[j] = f;
        is_fused[j] = true;
        absorbed[i] = true;
    }
    for (size_t i = 0; i < n; ++i)
        if (!absorbed[i] && calls[i].tag == HOLO_OP_DEQUANTIZE && calls[i].u.dequantize.weight_layout == 1)
            return set_error(HOLO_ERR_DISPATCH,
                             "session_load: kernel call " + std::to_string(i) +
                                 " declares an output-major weight that no kernel can read");
    compact(calls, plan, absorbed, fused, is_fused);
    return HOLO_OK;
}

// fuse_dequant_activation (crates/hologram-exec/src/session.rs:2061-2148): a
// per-tensor f32 Dequantize read only by an f32 Sigmoid / Tanh / Gelu / Silu /
// Exp / Erf becomes one DequantActivation (lut_act id) in the activation's place.
void fuse_dequant_activation(std::vector<holo_kernel_call> &calls,
                             std::vector<std::vector<uint32_t>> &plan, const std::vector<Port> &outputs) {
    const size_t n = calls.size();
    const Census cs(calls, outputs);
    std::vector<bool> absorbed(n, false), is_fused(n, false);
    std::vector<holo_kernel_call> fused(calls);
    for (size_t i = 0; i < n; ++i) {
        if (calls[i].tag != HOLO_OP_DEQUANTIZE) continue;
        const holo_dequantize_call dq = calls[i].u.dequantize;
        if (dequant_per_channel(dq) || dq.dtype != HOLO_DTYPE_F32) continue;
        size_t j;
        if (!cs.sole_reader(dq.output.slot, i, absorbed, &j)) continue;
        int act = -1;   // dequant_act_id: the lut_act ids
        switch (calls[j].tag) {
            case HOLO_OP_SIGMOID: act = 0; break;
            case HOLO_OP_TANH: act = 1; break;
            case HOLO_OP_GELU: act = 2; break;
            case HOLO_OP_SILU: act = 3; break;
            case HOLO_OP_EXP: act = 4; break;
            case HOLO_OP_ERF: act = 5; break;
            default: break;
        }
        if (act < 0) continue;
        const holo_unary_call ac = calls[j].u.unary;
        if (ac.dtype != HOLO_DTYPE_F32 || ac.input.slot != dq.output.slot) continue;
        holo_kernel_call f{};
        f.tag = HOLO_OP_DEQUANT_ACT;
        auto &da = f.u.dequant_act;
        da.input = dq.input;
        da.output = ac.output;
        da.element_count = dq.element_count;
        da.quant_dtype = dq.quant_dtype;
        da.act = uint8_t(act);
        da.dtype = HOLO_DTYPE_F32;
        da.scale_bits = dq.scale_bits;
        da.zero_point = dq.zero_point;
        fused[j] = f;
        is_fused[j] = true;
        absorbed[i] = true;
    }
    compact(calls, plan, absorbed, fused, is_fused);
}

// fuse_matmul_epilogue (crates/hologram-exec/src/session.rs:2150-2373): a
// MatMul (f32, bf16, f16) or an epilogue-free f32 MatMulDequant whose output
// has one producer and one reader, and is no output port, absorbs that reader
// when it is an activation (-> MatMulActivation) or a residual Add whose other
// operand is ready no later than the producer's level (-> MatMulAdd; for an
// f32 producer a single activation reader of the sum is absorbed too,
// -> MatMulAddActivation); a MatMulDequant takes the same epilogue in its own
// act / residual fields. Absorbed calls leave the call list and the plan. One
// difference: a fusion whose activation this device does not serve is skipped
// (the unfused calls give the same result).
void fuse_matmul_epilogue(std::vector<holo_kernel_call> &calls,
                          std::vector<std::vector<uint32_t>> &plan, const std::vector<Port> &outputs) {
    const size_t n = calls.size();
    const Census cs(calls, outputs);
    std::vector<holo_buffer_ref> rd, wr;
    std::map<uint32_t, size_t> slot_level;
    for (size_t li = 0; li < plan.size(); ++li)
        for (uint32_t ci : plan[li]) {
            call_operands(calls[ci], &rd, &wr);
            if (!wr.empty() && wr.back().slot != HOLO_SLOT_ABSENT) slot_level[wr.back().slot] = li;
        }
    std::vector<bool> absorbed(n, false), is_fused(n, false);
    std::vector<holo_kernel_call> fused(calls);
    for (size_t i = 0; i < n; ++i) {
        const bool is_mmd = calls[i].tag == HOLO_OP_MATMUL_DEQUANT;
        uint8_t dtype;
        uint32_t s;
        if (calls[i].tag == HOLO_OP_MATMUL) {
            const holo_matmul_call &mm = calls[i].u.matmul;
            if (mm.dtype != HOLO_DTYPE_F32 && mm.dtype != HOLO_DTYPE_BF16 && mm.dtype != HOLO_DTYPE_F16) continue;
            dtype = mm.dtype;
            s = mm.output.slot;
        } else if (is_mmd) {
            const holo_matmul_dequant_call &md = calls[i].u.matmul_dequant;
            if (md.dtype != HOLO_DTYPE_F32 || md.act != 0 || md.residual.slot != HOLO_SLOT_ABSENT) continue;
            dtype = HOLO_DTYPE_F32;
            s = md.output.slot;
        } else {
            continue;
        }
        // the producer with its output moved to `out` and the epilogue set
        auto make = [&](const holo_buffer_ref &out, const holo_buffer_ref *residual, uint32_t act) {
            holo_kernel_call f{};
            if (is_mmd) {
                f.tag = HOLO_OP_MATMUL_DEQUANT;
                f.u.matmul_dequant = calls[i].u.matmul_dequant;
                f.u.matmul_dequant.output = out;
                f.u.matmul_dequant.act = uint8_t(act);
                if (residual) f.u.matmul_dequant.residual = *residual;
                return f;
            }
            holo_matmul_call mm = calls[i].u.matmul;
            mm.output = out;
            if (!residual) {
                f.tag = HOLO_OP_MATMUL_ACT;
                f.u.matmul_act.mm = mm;
                f.u.matmul_act.act = uint8_t(act);
            } else if (!act) {
                f.tag = HOLO_OP_MATMUL_ADD;
                f.u.matmul_add.mm = mm;
                f.u.matmul_add.residual = *residual;
            } else {
                f.tag = HOLO_OP_MATMUL_ADD_ACT;
                f.u.matmul_add_act.mm = mm;
                f.u.matmul_add_act.residual = *residual;
                f.u.matmul_add_act.act = uint8_t(act);
            }
            return f;
        };
        size_t j;
        if (!cs.sole_reader(s, i, absorbed, &j)) continue;
        std::vector<holo_buffer_ref> jins, jw;
        call_operands(calls[j], &jins, &jw);
        if (jw.size() != 1) continue;
        const holo_buffer_ref jout = jw[0];
        if (const uint32_t act = fused_activation(calls[j])) {
            if (jins.size() != 1 || jins[0].slot != s) continue;
            if (!holo::fused_act_supported(act, dtype, false)) continue;
            fused[i] = make(jout, nullptr, act);
            is_fused[i] = true;
            absorbed[j] = true;
        } else if (calls[j].tag == HOLO_OP_ADD) {
            if (jins.size() != 2) continue;
            holo_buffer_ref residual;
            if (jins[0].slot == s) residual = jins[1];
            else if (jins[1].slot == s) residual = jins[0];
            else continue;
            const auto rl = slot_level.find(residual.slot), ml = slot_level.find(s);
            const bool ready = rl == slot_level.end() || ml == slot_level.end() || rl->second < ml->second;
            if (!ready) continue;
            // three-op chain producer -> add -> activation, f32 only
            const uint32_t add_out = jout.slot;
            size_t k;
            if (dtype == HOLO_DTYPE_F32 && cs.sole_reader(add_out, j, absorbed, &k)) {
                const uint32_t act = fused_activation(calls[k]);
                std::vector<holo_buffer_ref> kins, kw;
                call_operands(calls[k], &kins, &kw);
                if (act && kins.size() == 1 && kins[0].slot == add_out && kw.size() == 1 &&
                    holo::fused_act_supported(act, dtype, true)) {
                    fused[i] = make(kw[0], &residual, act);
                    is_fused[i] = true;
                    absorbed[j] = true;
                    absorbed[k] = true;
                    continue;
                }
            }
            fused[i] = make(jout, &residual, 0);
            is_fused[i] = true;
            absorbed[j] = true;
        }
    }
    compact(calls, plan, absorbed, fused, is_fused);
}

// A step of the walk: one call, or a fused group (index into groups).
struct Node {
    int group = -1;
    uint32_t call = 0;
    // a group whose split-K epilogue the next node runs (attn_prologue_fusion)
    bool epi_next = false;
};

}  // namespace

struct holo_session {
    holo_backend *be = nullptr;
    hipStream_t stream = nullptr;                 // session-owned, default priority
    std::vector<holo_kernel_call> calls;
    std::vector<std::vector<uint32_t>> plan;
    std::vector<Port> inputs, outputs;
    std::vector<uint64_t> slot_bytes;             // padded size per slot
    std::vector<SlotRange> slots;                 // current bindings
    std::vector<SlotRange> owned;                 // the session's own buffer per slot
    std::vector<std::pair<uint32_t, uint32_t>> aliases;   // (output slot, cache slot) moves
    // slots bound to (a sub-range of) another slot's memory instead of being
    // computed: interior Reshape / Slice (session.rs:1106-1150) and duplicates
    // of an earlier call's value (resident reuse, :1121-1131); applied after
    // the moves, in walk order
    struct ViewAlias {
        uint32_t out, in;
        uint64_t off, len;   // len 0: to the end of the source
    };
    std::vector<ViewAlias> views;
    uint32_t n_elided = 0;                        // calls bound instead of dispatched
    // per walk step: the root slots it reads and writes (through moves and
    // views), and whether it runs on every walk (in-place moves, output ports)
    std::vector<std::vector<uint32_t>> node_rd, node_wr;
    std::vector<uint8_t> node_always;
    std::vector<uint32_t> root;
    uint32_t last_dispatched = 0, last_skipped = 0;
    void *const_arena = nullptr, *work_arena = nullptr;
    uint8_t fingerprint[32] = {};
    hipGraphExec_t graph = nullptr;
    std::vector<SlotRange> graph_slots;           // bindings the graph was captured with
    uint32_t flags = 0;                           // HOLO_SESSION_* load options
    std::vector<Node> nodes;                      // the walk, in order
    std::vector<holo::GroupDesc> groups;          // fused few-row MatMul groups
    float *norm_arena = nullptr;                  // RmsNorm statistics of fused norms
    // each fused norm split between groups: (producer group, its segment,
    // consumer group)
    struct NormLink {
        size_t p, seg, c;
    };
    std::vector<NormLink> norm_links;
    void *packed_arena = nullptr;                 // weights of packed groups, fragment order
    uint64_t packed_bytes = 0;
    // split-K partials of this session's walks (few-row MatMuls, attention):
    // its own, so no other session or direct dispatch on the same backend
    // frees or shares what a captured graph of this walk reads and writes
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    void *graph_scratch = nullptr;                // the scratch the graph was captured with
    // κ-labels (address.rs): the calls and plan as the reference's loader
    // passes leave them (before this backend's in-place moves and device
    // fusion), and each constant's BLAKE3 digest
    std::vector<holo_kernel_call> label_calls;
    std::vector<std::vector<uint32_t>> label_plan;
    std::vector<std::pair<uint32_t, std::array<uint8_t, 32>>> const_digests;
    // the whole-graph memo of session.rs:841-905 over the byte boundary: the
    // input labels of the last walk, valid while nothing else has touched the
    // session's memory; per port, the last bytes hashed and their label
    bool memo_enabled = true, memo_valid = false;
    std::vector<std::string> memo_key;
    std::vector<std::vector<uint8_t>> input_seen;
    std::vector<std::string> input_seen_label;
};

namespace {

// ------------------------------------------------------------ device fusion --
// After the reference's passes, few-row MatMul-family calls that share their
// A operand are gathered into one group (one launch for every product, one
// for every epilogue), and each product's sole consumer is pulled into the
// group's epilogue when it is a rotary embedding, an in-place int8
// quantize+append, or an element-wise Mul with another member's product. A call
// joins a group only if no call still in place between the group and it
// touches what it reads or writes, and members and epilogues of one group
// share no written slot with each other's reads; every epilogue step is the
// standalone kernel's arithmetic, so the result is bit-identical.
struct MmView {
    holo_matmul_call mm{};
    uint8_t base = holo::kEpiStore;
    uint32_t act = 0;
    holo_buffer_ref residual{HOLO_SLOT_ABSENT, 0, 0};
};

// The MatMul payload of a MatMul-family call (46, 106-108), or null.
holo_matmul_call *matmul_of(holo_kernel_call &c) {
    switch (c.tag) {
        case HOLO_OP_MATMUL: return &c.u.matmul;
        case HOLO_OP_MATMUL_ACT: return &c.u.matmul_act.mm;
        case HOLO_OP_MATMUL_ADD: return &c.u.matmul_add.mm;
        case HOLO_OP_MATMUL_ADD_ACT: return &c.u.matmul_add_act.mm;
        default: return nullptr;
    }
}

bool matmul_family(const holo_kernel_call &c, MmView *v) {
    switch (c.tag) {
        case HOLO_OP_MATMUL: v->mm = c.u.matmul; v->base = holo::kEpiStore; return true;
        case HOLO_OP_MATMUL_ACT:
            v->mm = c.u.matmul_act.mm; v->base = holo::kEpiAct; v->act = c.u.matmul_act.act; return true;
        case HOLO_OP_MATMUL_ADD:
            v->mm = c.u.matmul_add.mm; v->base = holo::kEpiAdd; v->residual = c.u.matmul_add.residual;
            return true;
        case HOLO_OP_MATMUL_ADD_ACT:
            v->mm = c.u.matmul_add_act.mm; v->base = holo::kEpiAddAct;
            v->residual = c.u.matmul_add_act.residual; v->act = c.u.matmul_add_act.act; return true;
        default: return false;
    }
}

bool same_ref(const holo_buffer_ref &a, const holo_buffer_ref &b) {
    return a.slot == b.slot && a.offset == b.offset;
}

bool pow2_head(uint32_t d) { return d >= 2 && d <= 128 && (d & (d - 1)) == 0; }

// Slots a segment's epilogue reads and writes (for the cross-segment check).
void seg_slots(const holo::GroupSegDesc &s, std::vector<uint32_t> *rd, std::vector<uint32_t> *wr) {
    rd->clear();
    wr->clear();
    if (s.base == holo::kEpiAdd || s.base == holo::kEpiAddAct) rd->push_back(s.residual.slot);
    if (s.write_out) wr->push_back(s.out.slot);
    if (s.rope) {
        rd->push_back(s.cos.slot);
        rd->push_back(s.sin.slot);
        if (s.write_rope) wr->push_back(s.rope_out.slot);
    }
    if (s.quant) {
        rd->push_back(s.pos.slot);
        wr->push_back(s.cq.slot);
        wr->push_back(s.cs.slot);
    }
    if (s.pair >= 0) wr->push_back(s.mul_out.slot);
}

bool segments_disjoint(const std::vector<holo::GroupSegDesc> &segs, const holo_buffer_ref &a) {
    std::vector<std::vector<uint32_t>> rd(segs.size()), wr(segs.size());
    for (size_t i = 0; i < segs.size(); ++i) {
        seg_slots(segs[i], &rd[i], &wr[i]);
        rd[i].push_back(a.slot);
        rd[i].push_back(segs[i].b.slot);
    }
    for (size_t i = 0; i < segs.size(); ++i)
        for (size_t j = 0; j < segs.size(); ++j)
            for (uint32_t w : wr[i]) {
                if (std::find(rd[j].begin(), rd[j].end(), w) != rd[j].end()) return false;
                if (j != i && std::find(wr[j].begin(), wr[j].end(), w) != wr[j].end()) return false;
            }
    return true;
}

void device_fusion(holo_session *s, const std::vector<uint8_t> &is_output,
                   const std::vector<uint8_t> &is_input) {
    const auto &calls = s->calls;
    std::vector<uint32_t> order;
    for (auto &lv : s->plan)
        for (uint32_t ci : lv) order.push_back(ci);
    const size_t n = order.size(), npos = size_t(-1);
    std::vector<std::vector<holo_buffer_ref>> R(calls.size()), W(calls.size());
    std::vector<uint32_t> readers(is_output.size(), 0);
    for (size_t i = 0; i < calls.size(); ++i) {
        call_operands(calls[i], &R[i], &W[i]);
        for (auto &r : R[i])
            if (r.slot < readers.size()) readers[r.slot]++;
    }
    std::vector<bool> taken(calls.size(), false);
    auto conflicts = [&](uint32_t x, uint32_t c) {
        for (auto &w : W[x]) {
            for (auto &r : R[c])
                if (w.slot == r.slot) return true;
            for (auto &w2 : W[c])
                if (w.slot == w2.slot) return true;
        }
        for (auto &r : R[x])
            for (auto &w2 : W[c])
                if (r.slot == w2.slot) return true;
        return false;
    };
    auto movable = [&](size_t qc, size_t p) {
        const uint32_t c = order[qc];
        for (size_t q = p + 1; q < qc; ++q)
            if (!taken[order[q]] && conflicts(order[q], c)) return false;
        return true;
    };
    auto sole_reader = [&](uint32_t v, size_t p) -> size_t {
        if (v >= readers.size() || readers[v] != 1 || is_output[v]) return npos;
        for (size_t q = p + 1; q < n; ++q) {
            if (taken[order[q]]) continue;
            for (auto &r : R[order[q]])
                if (r.slot == v) return q;
        }
        return npos;
    };
    // few-row products (the split-K kernel), or large-M bf16 products the
    // tiled DMA kernel takes on their own (grouped, each result keeps the
    // single call's bits)
    auto tiled = [&](const MmView &m) {
        const uint32_t n = m.mm.n;
        return m.mm.dtype == HOLO_DTYPE_BF16 && m.mm.output.offset % 16 == 0 &&
               m.mm.output.slot < is_input.size() && !is_input[m.mm.output.slot] &&
               holo::matmul_group_tiled_applies(m.mm.m, m.mm.k, &n, 1);
    };
    auto groupable = [&](const MmView &m) {
        if (m.mm.dtype != HOLO_DTYPE_BF16 && m.mm.dtype != HOLO_DTYPE_F32) return false;
        if (m.mm.b_packed) return false;
        if (holo::matmul_skinny_plan(m.mm.m, m.mm.k, m.mm.n, m.mm.dtype).mt == 0 && !tiled(m))
            return false;
        if ((m.mm.a.offset | m.mm.b.offset) % 16 != 0) return false;
        if (m.mm.a.slot >= is_input.size() || m.mm.b.slot >= is_input.size()) return false;
        // input ports can be rebound to caller memory of any alignment
        return !is_input[m.mm.a.slot] && !is_input[m.mm.b.slot];
    };
    for (size_t p = 0; p < n; ++p) {
        const uint32_t i = order[p];
        if (taken[i]) continue;
        MmView mi;
        if (!matmul_family(calls[i], &mi) || !groupable(mi)) {
            s->nodes.push_back(Node{-1, i});
            continue;
        }
        const holo::SkinnyPlan pl = holo::matmul_skinny_plan(mi.mm.m, mi.mm.k, mi.mm.n, mi.mm.dtype);
        holo::GroupDesc g;
        g.a = mi.mm.a;
        g.m = mi.mm.m;
        g.k = mi.mm.k;
        g.dtype = mi.mm.dtype;
        auto seg_of = [](const MmView &m) {
            holo::GroupSegDesc d;
            d.b = m.mm.b;
            d.out = m.mm.output;
            d.n = m.mm.n;
            d.base = m.base;
            d.act = m.act;
            d.residual = m.residual;
            return d;
        };
        g.segs.push_back(seg_of(mi));
        std::vector<uint32_t> members{i};
        std::vector<uint32_t> absorbed;
        for (size_t q = p + 1; q < n && q <= p + 32 && g.segs.size() < size_t(holo::kSkinnyMaxSeg); ++q) {
            const uint32_t j = order[q];
            MmView mj;
            if (taken[j] || !matmul_family(calls[j], &mj) || !groupable(mj)) continue;
            if (!same_ref(mj.mm.a, mi.mm.a) || mj.mm.m != mi.mm.m || mj.mm.k != mi.mm.k ||
                mj.mm.dtype != mi.mm.dtype)
                continue;
            const holo::SkinnyPlan pj = holo::matmul_skinny_plan(mj.mm.m, mj.mm.k, mj.mm.n, mj.mm.dtype);
            if (pj.mt != pl.mt || pj.steps != pl.steps || pj.ks != pl.ks || !movable(q, p)) continue;
            if (pl.mt == 0 && !tiled(mj)) continue;
            g.segs.push_back(seg_of(mj));
            if (!segments_disjoint(g.segs, g.a)) {
                g.segs.pop_back();
                continue;
            }
            members.push_back(j);
            taken[j] = true;
        }
        // pull each product's sole consumer into the epilogue (tiled groups:
        // only the SwiGLU product of a group of exactly two)
        const bool tiled_group = pl.mt == 0;
        std::vector<holo_buffer_ref> value(g.segs.size());
        std::vector<bool> done(g.segs.size(), tiled_group && g.segs.size() != 2);
        for (size_t t = 0; t < g.segs.size(); ++t) value[t] = g.segs[t].out;
        for (size_t t = 0; t < g.segs.size(); ++t) {
            while (!done[t]) {
                const size_t qc = sole_reader(value[t].slot, p);
                if (qc == npos || !movable(qc, p)) break;
                const uint32_t c = order[qc];
                const holo_kernel_call &cc = calls[c];
                holo::GroupSegDesc trial = g.segs[t];
                const uint64_t mn = uint64_t(g.m) * trial.n;
                const bool free_seg = !trial.quant && trial.pair < 0 && !trial.skip;
                std::vector<holo::GroupSegDesc> segs2 = g.segs;
                bool ok = false, last = false;
                int partner = -1;
                if (tiled_group && cc.tag != HOLO_OP_MUL) break;
                if (cc.tag == HOLO_OP_ROTARY && free_seg && !trial.rope) {
                    const auto &r = cc.u.rope;
                    if (same_ref(r.x, value[t]) && r.dtype == g.dtype && pow2_head(r.head_dim) &&
                        trial.n % r.head_dim == 0 && r.element_count == mn &&
                        (trial.head_dim == 0 || trial.head_dim == r.head_dim)) {
                        trial.rope = true;
                        trial.cos = r.cos;
                        trial.sin = r.sin;
                        trial.rope_out = r.output;
                        trial.head_dim = r.head_dim;
                        trial.write_out = false;
                        ok = true;
                    }
                } else if (cc.tag == HOLO_OP_KV_QUANT_APPEND && free_seg) {
                    const auto &k = cc.u.kv_quant_append;
                    if (same_ref(k.new_rows_buf, value[t]) && same_ref(k.output, k.cache) &&
                        same_ref(k.output_scales, k.cache_scales) && k.dtype == g.dtype &&
                        pow2_head(k.head_dim) && trial.n % k.head_dim == 0 &&
                        (trial.head_dim == 0 || trial.head_dim == k.head_dim) && k.new_rows >= 1 &&
                        k.bucket_rows >= 1 && uint64_t(k.planes) * k.new_rows * k.head_dim == mn) {
                        trial.quant = true;
                        trial.pos = k.pos;
                        trial.cq = k.cache;
                        trial.cs = k.cache_scales;
                        trial.bucket = k.bucket_rows;
                        trial.new_rows = k.new_rows;
                        trial.head_dim = k.head_dim;
                        if (trial.rope) trial.write_rope = false;
                        else trial.write_out = false;
                        ok = last = true;
                    }
                } else if (cc.tag == HOLO_OP_MUL && free_seg && !trial.rope && trial.head_dim == 0) {
                    const auto &b = cc.u.binary;
                    const holo_buffer_ref other = same_ref(b.a, value[t]) ? b.b
                                                : same_ref(b.b, value[t]) ? b.a : holo_buffer_ref{HOLO_SLOT_ABSENT, 0, 0};
                    for (size_t u = 0; u < g.segs.size() && other.slot != HOLO_SLOT_ABSENT; ++u) {
                        const auto &su = g.segs[u];
                        if (u == t || !same_ref(value[u], other) || su.rope || su.quant ||
                            su.pair >= 0 || su.skip || su.head_dim || su.n != trial.n || done[u])
                            continue;
                        if (sole_reader(value[u].slot, p) != qc) continue;
                        partner = int(u);
                        break;
                    }
                    // tiled pair: a plain or table-activated gate, a plain up
                    if (tiled_group && partner >= 0 &&
                        !((trial.base == holo::kEpiStore || trial.base == holo::kEpiAct) &&
                          g.segs[size_t(partner)].base == holo::kEpiStore &&
                          b.output.offset % 16 == 0))
                        partner = -1;
                    if (partner >= 0 && b.dtype == g.dtype && b.element_count == mn) {
                        trial.pair = partner;
                        trial.mul_out = b.output;
                        trial.write_out = false;
                        segs2[partner].skip = true;
                        segs2[partner].write_out = false;
                        ok = last = true;
                    }
                }
                if (!ok) break;
                segs2[t] = trial;
                if (!segments_disjoint(segs2, g.a)) break;
                g.segs = segs2;
                taken[c] = true;
                absorbed.push_back(c);
                if (cc.tag == HOLO_OP_ROTARY) value[t] = cc.u.rope.output;
                if (last) {
                    done[t] = true;
                    if (partner >= 0) done[partner] = true;
                }
            }
        }
        if (g.segs.size() == 1 && absorbed.empty()) {
            s->nodes.push_back(Node{-1, i});
            continue;
        }
        taken[i] = true;
        s->groups.push_back(std::move(g));
        s->nodes.push_back(Node{int(s->groups.size() - 1), i});
    }
}

// ------------------------------------------------------------- norm fusion --
// A bf16 RmsNorm between two few-row MatMuls (the decode step's norms: the
// residual sum of Wo or Wd, normalized, read only by the next q/k/v, gate/up
// or LM-head group) leaves the walk. The group that produces its input also
// writes each row's sums of squares (the four wave sums of the standalone
// kernel), and the group that reads its output reads the input instead and
// normalizes A as it loads it. The normalized rows are never stored; every
// value keeps the standalone kernel's bits.
//
// Conditions: the norm's input is the whole output of the nearest earlier
// writer of its slot, an element-wise product of batch x feature; its output
// is read by exactly one node, as that group's A, before its slot is written
// again, and is no graph output; the producer is a group of one product; no node between the norm and that reader
// writes the input or gamma; operands 16-byte aligned and not caller-bound.
void node_slots(const holo_session *s, const Node &nd, std::vector<uint32_t> *rd,
                std::vector<uint32_t> *wr) {
    rd->clear();
    wr->clear();
    if (nd.group < 0) {
        std::vector<holo_buffer_ref> r, w;
        call_operands(s->calls[nd.call], &r, &w);
        for (auto &x : r) rd->push_back(x.slot);
        for (auto &x : w) wr->push_back(x.slot);
        return;
    }
    const holo::GroupDesc &g = s->groups[size_t(nd.group)];
    rd->push_back(g.a.slot);
    if (g.a_gamma.slot != HOLO_SLOT_ABSENT) rd->push_back(g.a_gamma.slot);
    std::vector<uint32_t> r, w;
    for (const auto &sg : g.segs) {
        seg_slots(sg, &r, &w);
        rd->push_back(sg.b.slot);
        rd->insert(rd->end(), r.begin(), r.end());
        wr->insert(wr->end(), w.begin(), w.end());
    }
}

bool has_slot(const std::vector<uint32_t> &v, uint32_t slot) {
    return std::find(v.begin(), v.end(), slot) != v.end();
}

// Whether a group can run as one launch over packed weights
// (gemv_packed.hip): bf16, at most 16 rows of a 16-byte aligned A in session
// memory, every weight a constant, the segments' tiles and heads in reach of
// the kernel.
bool packable_group(const holo_session *s, const holo::GroupDesc &g, const std::vector<uint8_t> &is_input,
                    const std::vector<uint8_t> &is_const) {
    const size_t nslots = is_const.size();
    auto caller_bound = [&](uint32_t slot) { return slot >= is_input.size() || is_input[slot]; };
    auto aligned16 = [&](const holo_buffer_ref &r) { return r.offset % 16 == 0 && !caller_bound(r.slot); };
    if (g.dtype != HOLO_DTYPE_BF16 || g.m == 0 || g.m > 16 || !aligned16(g.a) ||
        (g.a_gamma.slot != HOLO_SLOT_ABSENT && !aligned16(g.a_gamma)) || g.segs.empty() ||
        g.segs.size() > size_t(holo::kSkinnyMaxSeg))
        return false;
    holo::EpiSeg es[holo::kSkinnyMaxSeg];
    for (size_t i = 0; i < g.segs.size(); ++i) {
        const auto &d = g.segs[i];
        if (d.b.slot >= nslots || !is_const[d.b.slot] || d.b.offset % 16 ||
            s->slot_bytes[d.b.slot] < d.b.offset + uint64_t(g.k) * d.n * 2)
            return false;
        if ((d.base == holo::kEpiAct || d.base == holo::kEpiAddAct) &&
            !holo::fused_act_supported(d.act, g.dtype, d.base == holo::kEpiAddAct))
            return false;
        holo::EpiSeg &e = es[i];
        e.n = d.n;
        e.base = d.base;
        e.head_dim = d.head_dim;
        e.rope = d.rope;
        e.quant = d.quant;
        e.bucket = d.bucket;
        e.new_rows = d.new_rows;
        e.pair = d.pair;
        e.skip = d.skip;
    }
    return holo::packed_group_applies(g.m, g.k, es, int(g.segs.size()), g.a_norm);
}

int norm_fusion(holo_session *s, const std::vector<uint8_t> &is_output,
                const std::vector<uint8_t> &is_input, const std::vector<uint8_t> &is_const,
                bool packing) {
    auto &nodes = s->nodes;
    const size_t nn = nodes.size();
    std::vector<std::vector<uint32_t>> R(nn), W(nn);
    for (size_t i = 0; i < nn; ++i) node_slots(s, nodes[i], &R[i], &W[i]);
    auto caller_bound = [&](uint32_t slot) { return slot >= is_input.size() || is_input[slot]; };
    auto aligned16 = [&](const holo_buffer_ref &r) { return r.offset % 16 == 0 && !caller_bound(r.slot); };
    // a plain MatMul-family call node as a group of one segment
    auto as_group = [&](size_t i) -> holo::GroupDesc * {
        Node &nd = nodes[i];
        if (nd.group >= 0) return &s->groups[size_t(nd.group)];
        MmView mv;
        if (!matmul_family(s->calls[nd.call], &mv)) return nullptr;
        holo::GroupDesc g;
        g.a = mv.mm.a;
        g.m = mv.mm.m;
        g.k = mv.mm.k;
        g.dtype = mv.mm.dtype;
        holo::GroupSegDesc d;
        d.b = mv.mm.b;
        d.out = mv.mm.output;
        d.n = mv.mm.n;
        d.base = mv.base;
        d.act = mv.act;
        d.residual = mv.residual;
        g.segs.push_back(d);
        s->groups.push_back(std::move(g));
        nd.group = int(s->groups.size() - 1);
        return &s->groups.back();
    };
    // would-be group view of node i without converting it
    auto view = [&](size_t i, holo::GroupDesc *tmp) -> const holo::GroupDesc * {
        const Node &nd = nodes[i];
        if (nd.group >= 0) return &s->groups[size_t(nd.group)];
        MmView mv;
        const holo_kernel_call &c = s->calls[nd.call];
        if (!matmul_family(c, &mv) || mv.mm.b_packed) return nullptr;
        tmp->a = mv.mm.a;
        tmp->m = mv.mm.m;
        tmp->k = mv.mm.k;
        tmp->dtype = mv.mm.dtype;
        tmp->segs.assign(1, holo::GroupSegDesc{});
        tmp->segs[0].b = mv.mm.b;
        tmp->segs[0].out = mv.mm.output;
        tmp->segs[0].n = mv.mm.n;
        tmp->segs[0].base = mv.base;
        tmp->segs[0].residual = mv.residual;
        return tmp;
    };
    auto few_row = [&](const holo::GroupDesc &g) {
        if (g.dtype != HOLO_DTYPE_BF16 || (g.a.offset % 16) || caller_bound(g.a.slot)) return false;
        const holo::SkinnyPlan pl = holo::matmul_skinny_plan(g.m, g.k, g.segs[0].n, g.dtype);
        if (pl.mt == 0) return false;
        for (const auto &sg : g.segs) {
            const holo::SkinnyPlan p = holo::matmul_skinny_plan(g.m, g.k, sg.n, g.dtype);
            if (p.mt != pl.mt || p.steps != pl.steps || p.ks != pl.ks || sg.b.offset % 16 ||
                caller_bound(sg.b.slot))
                return false;
        }
        return true;
    };
    std::vector<bool> drop(nn, false);
    std::vector<std::pair<int, int>> links;   // (producer group, segment), consumer group
    std::vector<int> link_cons;
    auto linked_seg = [&](int grp, int seg) {
        return grp >= 0 && std::find(links.begin(), links.end(), std::make_pair(grp, seg)) != links.end();
    };
    auto linked_cons = [&](int grp) {
        return grp >= 0 && std::find(link_cons.begin(), link_cons.end(), grp) != link_cons.end();
    };
    for (size_t k = 0; k < nn; ++k) {
        if (nodes[k].group >= 0 || s->calls[nodes[k].call].tag != HOLO_OP_RMS_NORM) continue;
        const holo_norm_call &nc = s->calls[nodes[k].call].u.norm;
        if (nc.dtype != HOLO_DTYPE_BF16 || nc.residual.slot != HOLO_SLOT_ABSENT || nc.channels ||
            nc.num_groups || nc.batch == 0 || nc.feature % 8 || nc.feature > 8192 || nc.feature == 0)
            continue;
        float eps = 1e-9f;
        if (nc.epsilon_bits != 0) {
            const uint32_t eb = uint32_t(nc.epsilon_bits);
            memcpy(&eps, &eb, 4);
            if (!(std::isfinite(eps) && eps > 0.0f)) continue;
        }
        const holo_buffer_ref x = nc.x, y = nc.output;
        const bool has_g = nc.gamma.slot != HOLO_SLOT_ABSENT;
        if (x.slot == y.slot || !aligned16(x) || (has_g && !aligned16(nc.gamma)) ||
            y.slot >= is_output.size() || is_output[y.slot])
            continue;
        // producer: the nearest earlier writer of x, when it is a few-row
        // product that can leave the statistics
        size_t j = k;
        while (j > 0 && !has_slot(W[j - 1], x.slot)) --j;
        int pseg = -1;
        if (j > 0) {
            --j;
            holo::GroupDesc tp;
            const holo::GroupDesc *pg = view(j, &tp);
            if (pg && pg->segs.size() == 1 && few_row(*pg) && pg->m == nc.batch) {
                for (size_t t = 0; t < pg->segs.size(); ++t) {
                    const auto &sg = pg->segs[t];
                    if (same_ref(sg.out, x) && sg.write_out && sg.n == nc.feature && !sg.head_dim &&
                        !sg.rope && !sg.quant && sg.pair < 0 && !sg.skip && !sg.ssq && aligned16(sg.out) &&
                        (!(sg.base == holo::kEpiAdd || sg.base == holo::kEpiAddAct) || aligned16(sg.residual)))
                        pseg = int(t);
                }
                if (pseg >= 0 && linked_seg(nodes[j].group, pseg)) pseg = -1;
            }
        }
        // consumer: the one reader of y before y's slot is written again
        size_t q = nn, readers = 0;
        for (size_t t = k + 1; t < nn; ++t) {
            if (has_slot(R[t], y.slot)) {
                ++readers;
                q = t;
            }
            if (has_slot(W[t], y.slot)) break;
        }
        if (readers != 1) continue;
        holo::GroupDesc tc;
        const holo::GroupDesc *cg = view(q, &tc);
        if (!cg || linked_cons(nodes[q].group) || !same_ref(cg->a, y) || cg->m != nc.batch ||
            cg->k != nc.feature || cg->a_norm)
            continue;
        // with no producer to leave the statistics, a reader that runs packed
        // takes them itself
        bool self_stats = false;
        if (pseg < 0) {
            if (!packing) continue;
            holo::GroupDesc probe = *cg;
            probe.a = x;
            probe.a_gamma = has_g ? nc.gamma : holo_buffer_ref{HOLO_SLOT_ABSENT, 0, 0};
            probe.a_norm = true;
            if (!packable_group(s, probe, is_input, is_const)) continue;
            self_stats = true;
        } else if (!few_row(*cg)) {
            continue;
        }
        {   // y read only as A
            std::vector<uint32_t> r, w;
            bool other = false;
            for (const auto &sg : cg->segs) {
                seg_slots(sg, &r, &w);
                other = other || sg.b.slot == y.slot || has_slot(r, y.slot);
            }
            if (other) continue;
        }
        bool clobbered = false;
        for (size_t t = k + 1; t < q && !clobbered; ++t)
            clobbered = has_slot(W[t], x.slot) || (has_g && has_slot(W[t], nc.gamma.slot));
        if (clobbered) continue;
        // commit
        if (!self_stats) as_group(j);
        holo::GroupDesc *C = as_group(q);
        C->a = x;
        C->a_gamma = has_g ? nc.gamma : holo_buffer_ref{HOLO_SLOT_ABSENT, 0, 0};
        C->a_eps = eps;
        C->a_norm = true;
        if (!self_stats) {
            links.push_back({nodes[j].group, pseg});
            link_cons.push_back(nodes[q].group);
            node_slots(s, nodes[j], &R[j], &W[j]);
        }
        drop[k] = true;
        node_slots(s, nodes[q], &R[q], &W[q]);
        R[k].clear();
        W[k].clear();
    }
    std::vector<Node> kept;
    for (size_t i = 0; i < nn; ++i)
        if (!drop[i]) kept.push_back(nodes[i]);
    nodes.swap(kept);
    if (links.empty()) return HOLO_OK;
    // the statistics: [64 rows][4] floats per fused norm, in session memory
    // (a dry load has no device: the groups are only counted)
    float *arena = nullptr;
    if (s->be) {
        if (hipMalloc(&arena, links.size() * 64 * 4 * sizeof(float)) != hipSuccess) {
            (void)hipGetLastError();
            return set_error(HOLO_ERR_INIT, "session_load: device allocation failed (norm statistics)");
        }
        s->norm_arena = arena;
    }
    for (size_t f = 0; f < links.size(); ++f) {
        s->norm_links.push_back({size_t(links[f].first), size_t(links[f].second), size_t(link_cons[f])});
        float *st = arena ? arena + f * 64 * 4 : nullptr;
        holo::GroupDesc &pgd = s->groups[size_t(links[f].first)];
        holo::GroupDesc &cgd = s->groups[size_t(link_cons[f])];
        pgd.segs[size_t(links[f].second)].ssq = st;
        cgd.a_ssq = st;
    }
    return HOLO_OK;
}

// Every slot's label walked through the plan as compute_and_label derives it
// (session.rs:1052-1289): constants by content, input ports by `in`, each
// call by derive_label over its op signature and operand labels (Add and Mul
// sort theirs), a Reshape by its input's label; a call whose operand has no
// label leaves its outputs unlabelled. A call with two outputs (the int8
// append's cache and scales) labels output j with its params followed by the
// byte j. With `boundary`, a call writing an output port also gives that port
// the boundary form (derive_label_boundary), which later calls do not see.
int label_walk(const holo_session *s, const std::vector<std::string> &in, bool boundary,
               std::vector<std::string> *lab_out, std::vector<std::string> *witnessed) {
    std::vector<std::string> &lab = *lab_out;
    lab.assign(s->slot_bytes.size(), std::string());
    for (const auto &cd : s->const_digests)
        if (cd.first < lab.size()) lab[cd.first] = holo::kappa_of_digest(cd.second.data());
    for (size_t i = 0; i < s->inputs.size(); ++i)
        if (s->inputs[i].slot < lab.size()) lab[s->inputs[i].slot] = in[i];
    std::vector<uint8_t> is_out(lab.size(), 0);
    for (const auto &p : s->outputs)
        if (p.slot < is_out.size()) is_out[p.slot] = 1;
    if (witnessed) witnessed->assign(lab.size(), std::string());
    std::vector<uint32_t> ins, outs;
    std::vector<std::string> il;
    for (const auto &level : s->label_plan)
        for (uint32_t ci : level) {
            const holo_kernel_call &c = s->label_calls[ci];
            bool comm = false;
            uint16_t op = 0;
            uint8_t params[65];
            uint32_t np = 0;
            if (!holo::label_operands(c, &ins, &outs, &comm) || !holo::op_signature(c, &op, params, &np))
                return set_error(HOLO_ERR_UNSUPPORTED_OP,
                                 "session_output_labels: kernel call " + std::to_string(ci) + " has no signature");
            bool ok = true;
            il.clear();
            for (uint32_t sl : ins) {
                if (sl >= lab.size() || lab[sl].empty()) {
                    ok = false;
                    break;
                }
                il.push_back(lab[sl]);
            }
            if (comm) std::sort(il.begin(), il.end());
            for (size_t j = 0; j < outs.size(); ++j) {
                if (outs[j] >= lab.size()) continue;
                if (!ok) {
                    lab[outs[j]].clear();
                    if (witnessed) (*witnessed)[outs[j]].clear();
                    continue;
                }
                uint32_t n = np;
                if (outs.size() > 1) params[n++] = uint8_t(j);
                if (boundary && witnessed && is_out[outs[j]]) {
                    std::string w;
                    if (!holo::derive_label_boundary(op, params, n, il, &w))
                        return set_error(HOLO_ERR_DISPATCH, "session_output_labels: an operand label "
                                                            "is not a blake3 label");
                    (*witnessed)[outs[j]] = w;
                }
                // Reshape re-addresses: its value's label is its input's
                lab[outs[j]] = c.tag == HOLO_OP_RESHAPE && !il.empty()
                                   ? il[0] : holo::derive_label(op, params, n, il);
            }
        }
    return HOLO_OK;
}

// ------------------------------------------------------- bound, not run --
// After fusion, two kinds of walk step are bound instead of dispatched, as
// compute_and_label binds them (session.rs:1106-1150):
//  - an interior Reshape (its value's label is its input's, resident) or
//    Slice (a view of the field its input operand names): the output slot is
//    bound to the input's memory, nothing moves;
//  - a step whose value some earlier step of the same walk already holds
//    (equal κ-label, derived here with a token per input port so that the
//    equality holds for every input): its output slot is bound to that
//    step's memory (the resident reuse of :1121-1131).
// A step writing an output port always runs (the reference dispatches it to
// mint the port's boundary label), as does any step that touches a KV cache
// (the in-place move mutates memory a binding would share). Then each kept
// step's root slots (through moves and bindings), which memo-on reuse tracks.
void elide_steps(holo_session *s, const std::vector<uint8_t> &is_output,
                 const std::vector<uint8_t> &is_input, const std::vector<uint8_t> &is_const) {
    const size_t nslots = is_output.size();
    std::vector<std::string> tok, sym;
    for (size_t i = 0; i < s->inputs.size(); ++i) tok.push_back("input port " + std::to_string(i));
    if (label_walk(s, tok, false, &sym, nullptr) != HOLO_OK) sym.assign(nslots, std::string());
    sym.resize(nslots);
    auto &nodes = s->nodes;
    const size_t nn = nodes.size();
    std::vector<std::vector<uint32_t>> R(nn), W(nn);
    for (size_t i = 0; i < nn; ++i) node_slots(s, nodes[i], &R[i], &W[i]);
    std::vector<uint32_t> writers(nslots, 0);
    std::vector<size_t> last_writer(nslots, 0);
    for (size_t i = 0; i < nn; ++i)
        for (uint32_t w : W[i])
            if (w < nslots) writers[w]++, last_writer[w] = i;
    std::vector<uint8_t> kv(nslots, 0);   // a KV op's cache operand, or a moved slot
    auto mark = [&](const holo_buffer_ref &b) {
        if (b.slot < nslots) kv[b.slot] = 1;
    };
    for (const auto &c : s->calls) {
        if (c.tag == HOLO_OP_KV_CACHE_WRITE) mark(c.u.kv_write.cache), mark(c.u.kv_write.output);
        if (c.tag == HOLO_OP_KV_QUANT_APPEND) {
            const auto &k = c.u.kv_quant_append;
            mark(k.cache), mark(k.cache_scales), mark(k.output), mark(k.output_scales);
        }
    }
    for (const auto &a : s->aliases) {
        if (a.first < nslots) kv[a.first] = 1;
        if (a.second < nslots) kv[a.second] = 1;
    }
    auto is_kv_op = [](uint32_t tag) {
        return tag == HOLO_OP_KV_CACHE_WRITE || tag == HOLO_OP_KV_QUANT_APPEND;
    };
    // a slot only this step writes, that no port, constant or KV op touches
    auto plain = [&](uint32_t sl) {
        return sl < nslots && !is_output[sl] && !is_input[sl] && !is_const[sl] && writers[sl] == 1 &&
               !kv[sl];
    };
    // the slot holds its final value before step i (nothing at or after i writes it)
    auto settled = [&](uint32_t sl, size_t i) {
        return sl < nslots && (writers[sl] == 0 || last_writer[sl] < i);
    };
    auto bound = [&](uint32_t sl) { return sl < nslots && (is_input[sl] || is_const[sl] || writers[sl] > 0); };
    std::vector<uint8_t> is_view(nslots, 0), drop(nn, 0);
    std::map<std::string, uint32_t> held;   // label -> the slot holding that value
    for (size_t i = 0; i < nn; ++i) {
        const Node &nd = nodes[i];
        if (nd.group < 0) {
            const holo_kernel_call &c = s->calls[nd.call];
            if (c.tag == HOLO_OP_RESHAPE || c.tag == HOLO_OP_SLICE) {
                const holo_layout_call &l = c.u.layout;
                const uint32_t o = l.output.slot, in = l.input.slot;
                const bool reshape = c.tag == HOLO_OP_RESHAPE;
                // a Reshape binds its input's resident value (not a view's)
                const bool ok = plain(o) && !kv[in] && settled(in, i) && bound(in) &&
                                (!reshape || !is_view[in]);
                if (ok) {
                    if (reshape) {
                        s->views.push_back({o, in, 0, 0});
                    } else {
                        s->views.push_back({o, in, l.input.offset, l.input.length});
                        is_view[o] = 1;
                    }
                    drop[i] = 1;
                    if (reshape && !sym[o].empty()) held.emplace(sym[o], o);
                    continue;
                }
            } else if (!is_kv_op(c.tag) && W[i].size() == 1 && plain(W[i][0]) && !sym[W[i][0]].empty()) {
                const auto it = held.find(sym[W[i][0]]);
                if (it != held.end() && it->second != W[i][0]) {
                    s->views.push_back({W[i][0], it->second, 0, 0});
                    drop[i] = 1;
                    continue;
                }
            }
        }
        for (uint32_t w : W[i])
            if (plain(w) && !sym[w].empty()) held.emplace(sym[w], w);
    }
    std::vector<Node> kept;
    std::vector<std::vector<uint32_t>> kr, kw;
    for (size_t i = 0; i < nn; ++i) {
        if (drop[i]) {
            s->n_elided++;
            continue;
        }
        kept.push_back(nodes[i]);
        kr.push_back(std::move(R[i]));
        kw.push_back(std::move(W[i]));
    }
    nodes = std::move(kept);
    // root slots: a moved output is its cache, a bound slot its source
    s->root.resize(nslots);
    for (size_t i = 0; i < nslots; ++i) s->root[i] = uint32_t(i);
    auto find = [&](uint32_t x) {
        while (x < nslots && s->root[x] != x) x = s->root[x];
        return x;
    };
    for (const auto &a : s->aliases)
        if (a.first < nslots && a.second < nslots) s->root[a.first] = find(a.second);
    for (const auto &v : s->views) s->root[v.out] = find(v.in);
    s->node_rd.assign(nodes.size(), {});
    s->node_wr.assign(nodes.size(), {});
    s->node_always.assign(nodes.size(), 0);
    for (size_t i = 0; i < nodes.size(); ++i) {
        for (uint32_t r : kr[i])
            if (r < nslots) s->node_rd[i].push_back(find(r));
        for (uint32_t w : kw[i]) {
            if (w >= nslots) continue;
            s->node_wr[i].push_back(find(w));
            if (is_output[w] || kv[w]) s->node_always[i] = 1;
        }
    }
}

// Few-row bf16 groups over constant weights run as one launch
// (gemv_packed.hip): each weight is copied once, at load, into the matrix
// cores' operand order. A plain few-row MatMul-family call over a constant
// weight becomes a group of one for this. A packed group that reads A through
// a fused RmsNorm takes the row statistics itself, so its producer stops
// writing them; a producer whose reader stays split-K keeps writing them and
// stays split-K too (a packed launch leaves no statistics).
// The q/k/v group of a decode step hands its split-K epilogue to the decode
// attention that follows it, which runs it in front of the attention in one
// launch (attn_pro_kernel: each workgroup finishes the heads of its own plane,
// then attends over them). Conditions: the group is bf16 and not packed; its
// segments are all head-wise at the attention's head_dim, each with a multiple
// of kv_heads heads a row and at most one appended row, with no SwiGLU pair and
// no statistics; the next node is a DecodeAttentionI8 over batch = the group's
// rows, whose q is a segment's stored output of heads x head_dim columns (the
// rotated one for a rotary segment), whose k and v caches and scales are two
// different quant segments' (through the in-place moves), and whose lengths and
// output are no slot the group writes. A workgroup of the fused launch then
// reads back only what its own prologue stored. Whether the launch applies
// (the grid form, one chunk a plane) is decided at dispatch; where it does
// not, the epilogue runs on its own before the attention.
void attn_prologue_fusion(holo_session *s) {
    auto root = [&](uint32_t slot) {
        for (const auto &a : s->aliases)
            if (a.first == slot) return a.second;
        return slot;
    };
    auto same = [&](const holo_buffer_ref &a, const holo_buffer_ref &b) {
        return root(a.slot) == root(b.slot) && a.offset == b.offset;
    };
    std::vector<uint32_t> rd, wr;
    for (size_t i = 0; i + 1 < s->nodes.size(); ++i) {
        Node &nd = s->nodes[i];
        const Node &nx = s->nodes[i + 1];
        if (nd.group < 0 || nx.group >= 0) continue;
        const holo_kernel_call &c = s->calls[nx.call];
        if (c.tag != HOLO_OP_DECODE_ATTN_I8) continue;
        const holo_decode_attention_i8_call &at = c.u.attn_i8;
        const holo::GroupDesc &g = s->groups[size_t(nd.group)];
        const uint32_t hkv = at.kv_heads == 0 ? at.heads : at.kv_heads;
        if (g.packed || g.dtype != HOLO_DTYPE_BF16 || at.dtype != HOLO_DTYPE_BF16 || g.m != at.batch ||
            hkv == 0 || at.head_dim == 0 || g.segs.empty())
            continue;
        bool ok = true;
        int qs = -1, ks = -1, vs = -1;
        for (size_t j = 0; j < g.segs.size() && ok; ++j) {
            const holo::GroupSegDesc &sg = g.segs[j];
            ok = sg.head_dim == at.head_dim && sg.pair < 0 && !sg.skip && !sg.ssq &&
                 sg.n % (uint64_t(at.head_dim) * hkv) == 0 && (!sg.quant || sg.new_rows == 1);
            if (!ok) break;
            const bool stored = sg.rope ? sg.write_rope : sg.write_out;
            if (stored && uint64_t(sg.n) == uint64_t(at.heads) * at.head_dim &&
                same(sg.rope ? sg.rope_out : sg.out, at.q))
                qs = int(j);
            if (sg.quant && uint64_t(sg.n) == uint64_t(hkv) * at.head_dim) {
                if (same(sg.cq, at.k_cache) && same(sg.cs, at.k_scales)) ks = int(j);
                if (same(sg.cq, at.v_cache) && same(sg.cs, at.v_scales)) vs = int(j);
            }
        }
        if (!ok || qs < 0 || ks < 0 || vs < 0 || ks == vs) continue;
        node_slots(s, nd, &rd, &wr);
        bool clash = false;
        for (uint32_t w : wr) clash = clash || root(w) == root(at.lens.slot) || root(w) == root(at.output.slot);
        if (clash) continue;
        nd.epi_next = true;
    }
}

int pack_weights(holo_session *s, const std::vector<uint8_t> &is_input,
                 const std::vector<uint8_t> &is_const) {
    auto packable = [&](const holo::GroupDesc &g) { return packable_group(s, g, is_input, is_const); };
    // plain few-row calls over a constant weight: groups of one
    for (auto &nd : s->nodes) {
        if (nd.group >= 0) continue;
        MmView mv;
        if (!matmul_family(s->calls[nd.call], &mv) || mv.mm.b_packed) continue;
        holo::GroupDesc g;
        g.a = mv.mm.a;
        g.m = mv.mm.m;
        g.k = mv.mm.k;
        g.dtype = mv.mm.dtype;
        holo::GroupSegDesc d;
        d.b = mv.mm.b;
        d.out = mv.mm.output;
        d.n = mv.mm.n;
        d.base = mv.base;
        d.act = mv.act;
        d.residual = mv.residual;
        g.segs.push_back(d);
        if (!packable(g)) continue;
        s->groups.push_back(std::move(g));
        nd.group = int(s->groups.size() - 1);
    }
    std::vector<uint8_t> live(s->groups.size(), 0);
    for (const auto &nd : s->nodes)
        if (nd.group >= 0) live[size_t(nd.group)] = 1;
    for (size_t i = 0; i < s->groups.size(); ++i) s->groups[i].packed = live[i] && packable(s->groups[i]);
    // fused norms split between a producer group and its reader
    const auto &links = s->norm_links;
    for (bool changed = true; changed;) {
        changed = false;
        for (const auto &l : links)
            if (!s->groups[l.c].packed && s->groups[l.p].packed) {
                s->groups[l.p].packed = false;
                changed = true;
            }
    }
    for (const auto &l : links)
        if (s->groups[l.c].packed) s->groups[l.p].segs[l.seg].ssq = nullptr;
    for (size_t i = 0; i < s->groups.size(); ++i)
        if (live[i] && s->groups[i].a_norm && !s->groups[i].a_ssq && s->be && !s->groups[i].packed)
            return set_error(HOLO_ERR_INIT, "session_load: a fused RmsNorm's reader cannot run packed");
    // the tile width each packed group's weights take
    for (auto &g : s->groups) {
        if (!g.packed) continue;
        holo::EpiSeg es[holo::kSkinnyMaxSeg];
        for (size_t i = 0; i < g.segs.size(); ++i) {
            es[i].n = g.segs[i].n;
            es[i].head_dim = g.segs[i].head_dim;
            es[i].skip = g.segs[i].skip;
        }
        g.packed_tw = holo::packed_tile_width(g.m, g.k, es, int(g.segs.size()));
    }
    if (!s->be) return HOLO_OK;   // a dry load: decided, nothing to copy
    // one fragment-order copy per distinct weight and tile width
    auto seg_tw = [](const holo::GroupDesc &g, const holo::GroupSegDesc &d) {
        return d.head_dim ? 16u : g.packed_tw;
    };
    // a rotary-only head-wise segment is packed in rope tiles
    auto seg_rope = [](const holo::GroupSegDesc &d) { return d.head_dim && d.rope && !d.quant ? d.head_dim : 0u; };
    std::map<std::tuple<uint32_t, uint64_t, uint32_t, uint32_t, uint32_t, uint32_t>, uint64_t> at;
    uint64_t total = 0;
    for (const auto &g : s->groups) {
        if (!g.packed) continue;
        for (const auto &d : g.segs) {
            const auto key = std::make_tuple(d.b.slot, d.b.offset, g.k, d.n, seg_tw(g, d), seg_rope(d));
            if (at.count(key)) continue;
            at[key] = total;
            total += (holo::packed_b_bytes(g.k, d.n, seg_tw(g, d)) + 255) / 256 * 256;
        }
    }
    if (total == 0) return HOLO_OK;
    if (hipMalloc(&s->packed_arena, total) != hipSuccess) {
        (void)hipGetLastError();
        s->packed_arena = nullptr;
        return set_error(HOLO_ERR_INIT, "session_load: device allocation failed (packed weights, " +
                                            std::to_string(total) + " bytes)");
    }
    s->packed_bytes = total;
    uint8_t *base = static_cast<uint8_t *>(s->packed_arena);
    for (const auto &kv : at) {
        const uint32_t slot = std::get<0>(kv.first);
        const uint64_t off = std::get<1>(kv.first);
        if (holo::launch_pack_b(s->owned[slot].ptr + off, base + kv.second, std::get<2>(kv.first),
                                std::get<3>(kv.first), std::get<4>(kv.first), std::get<5>(kv.first),
                                s->stream) != hipSuccess) {
            (void)hipGetLastError();
            return set_error(HOLO_ERR_INIT, "session_load: weight packing launch failed");
        }
    }
    if (hipStreamSynchronize(s->stream) != hipSuccess)
        return set_error(HOLO_ERR_INIT, "session_load: weight packing failed");
    for (auto &g : s->groups) {
        if (!g.packed) continue;
        for (auto &d : g.segs)
            d.bp = base + at[std::make_tuple(d.b.slot, d.b.offset, g.k, d.n, seg_tw(g, d), seg_rope(d))];
    }
    return HOLO_OK;
}

void release(holo_session *s) {
    if (!s) return;
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->graph) (void)hipGraphExecDestroy(s->graph);
    if (s->norm_arena) (void)hipFree(s->norm_arena);
    if (s->packed_arena) (void)hipFree(s->packed_arena);
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->const_arena) (void)hipFree(s->const_arena);
    if (s->work_arena) (void)hipFree(s->work_arena);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

int load_impl(holo_backend *be, const uint8_t *bytes, size_t len, uint32_t flags, holo_session **out) {
    const char *op = "session_load";
    // --- header + footer (loader.rs:141-185)
    if (len < 4 + 2 + 2 + 2 + 32)
        return set_error(HOLO_ERR_DISPATCH, "session_load: archive truncated (< 42 bytes)");
    if (memcmp(bytes, "HOLO", 4) != 0) return set_error(HOLO_ERR_DISPATCH, "session_load: bad magic");
    uint16_t ver;
    memcpy(&ver, bytes + 4, 2);
    if (ver < kMinReadVersion || ver > kFormatVersion)
        return set_error(HOLO_ERR_DISPATCH, "session_load: unsupported .holo version " + std::to_string(ver));
    auto s = std::unique_ptr<holo_session, void (*)(holo_session *)>(new holo_session(), release);
    s->be = be;
    s->flags = flags;
    holo::blake3_hash(bytes, len - 32, s->fingerprint);
    if (memcmp(s->fingerprint, bytes + len - 32, 32) != 0)
        return set_error(HOLO_ERR_DISPATCH, "session_load: footer fingerprint mismatch (BLAKE3)");
    // --- section table (loader.rs:220-263)
    uint16_t nsec;
    memcpy(&nsec, bytes + 8, 2);
    std::map<uint8_t, std::pair<const uint8_t *, size_t>> sec;
    const size_t body_end = len - 32;
    size_t cur = 10;
    for (uint16_t i = 0; i < nsec; ++i) {
        if (cur + 24 > body_end) return set_error(HOLO_ERR_DISPATCH, "session_load: section table truncated");
        const uint8_t kind = bytes[cur];
        if (kind < 1 || kind > 16) return set_error(HOLO_ERR_DISPATCH, "session_load: unknown section kind");
        uint64_t off, n;
        memcpy(&off, bytes + cur + 8, 8);
        memcpy(&n, bytes + cur + 16, 8);
        cur += 24;
        if (off > body_end || n > body_end - off)
            return set_error(HOLO_ERR_DISPATCH, "session_load: section out of range");
        if (!sec.count(kind)) sec[kind] = {bytes + off, size_t(n)};   // first of a kind wins
    }
    // --- kernel calls
    auto it = sec.find(kSecKernelCalls);
    if (it == sec.end()) return set_error(HOLO_ERR_DISPATCH, "session_load: no KernelCalls section");
    {
        Cursor c{it->second.first, it->second.second};
        const uint32_t n = c.get<uint32_t>();
        if (!c.ok) return set_error(HOLO_ERR_DISPATCH, "session_load: truncated KernelCalls");
        for (uint32_t i = 0; i < n; ++i) {
            holo_kernel_call call;
            size_t used = 0;
            const int rc = holo::decode_call(c.p + c.at, c.len - c.at, &call, &used);
            if (rc != HOLO_OK) return rc;
            c.at += used;
            s->calls.push_back(call);
        }
    }
    // --- ports, plan
    if ((it = sec.find(kSecInputs)) != sec.end()) {
        const int rc = parse_ports(it->second.first, it->second.second, &s->inputs);
        if (rc != HOLO_OK) return rc;
    }
    if ((it = sec.find(kSecOutputs)) != sec.end()) {
        const int rc = parse_ports(it->second.first, it->second.second, &s->outputs);
        if (rc != HOLO_OK) return rc;
    }
    if ((it = sec.find(kSecExecPlan)) != sec.end()) {
        Cursor c{it->second.first, it->second.second};
        const uint32_t nl = c.get<uint32_t>();
        for (uint32_t l = 0; l < nl && c.ok; ++l) {
            const uint32_t n = c.get<uint32_t>();
            std::vector<uint32_t> lv;
            for (uint32_t i = 0; i < n && c.ok; ++i) lv.push_back(c.get<uint32_t>());
            s->plan.push_back(std::move(lv));
        }
        if (!c.ok) return set_error(HOLO_ERR_DISPATCH, "session_load: truncated ExecPlan");
        for (auto &lv : s->plan)
            for (uint32_t i : lv)
                if (i >= s->calls.size())
                    return set_error(HOLO_ERR_DISPATCH, "session_load: ExecPlan index out of range");
    } else {
        std::vector<uint32_t> all(s->calls.size());
        for (size_t i = 0; i < all.size(); ++i) all[i] = uint32_t(i);
        s->plan.push_back(std::move(all));
    }
    // --- slot ids are host-side indices from here on: every call's write
    // operands and every port must name a real slot (an absent write, or a
    // port on the absent sentinel, is a malformed archive, not an operand to skip)
    {
        std::vector<holo_buffer_ref> rd0, wr0;
        for (size_t i = 0; i < s->calls.size(); ++i) {
            call_operands(s->calls[i], &rd0, &wr0);
            for (auto &b : wr0)
                if (b.slot == HOLO_SLOT_ABSENT)
                    return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE,
                                     "session_load: kernel call " + std::to_string(i) +
                                         " writes the absent slot");
        }
        for (auto *ports : {&s->inputs, &s->outputs})
            for (auto &p : *ports)
                if (p.slot == HOLO_SLOT_ABSENT)
                    return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE,
                                     "session_load: port '" + p.name + "' names the absent slot");
    }
    // --- the loader's fusion passes, in the reference's order (session.rs:
    // 493-504): dequant -> MatMul first, so the quantized weight is read in
    // place rather than traded for an epilogue fusion
    if (!(flags & HOLO_SESSION_NO_DEQUANT_FUSION)) {
        const int rc = fuse_dequant_matmul(s->calls, s->plan, s->outputs);
        if (rc != HOLO_OK) return rc;
    } else {
        for (size_t i = 0; i < s->calls.size(); ++i)
            if (s->calls[i].tag == HOLO_OP_DEQUANTIZE && s->calls[i].u.dequantize.weight_layout == 1)
                return set_error(HOLO_ERR_DISPATCH,
                                 "session_load: kernel call " + std::to_string(i) +
                                     " declares an output-major weight that no kernel can read");
    }
    if (!(flags & HOLO_SESSION_NO_EPILOGUE_FUSION)) fuse_matmul_epilogue(s->calls, s->plan, s->outputs);
    if (!(flags & HOLO_SESSION_NO_DEQUANT_FUSION)) fuse_dequant_activation(s->calls, s->plan, s->outputs);
    s->label_calls = s->calls;
    s->label_plan = s->plan;
    // --- weights (fingerprint -> body), constants
    std::map<std::string, std::pair<const uint8_t *, uint64_t>> weights;
    if ((it = sec.find(kSecWeights)) != sec.end()) {
        Cursor c{it->second.first, it->second.second};
        const uint32_t n = c.get<uint32_t>();
        for (uint32_t i = 0; i < n && c.ok; ++i) {
            const uint8_t *fp = c.take(32);
            const uint64_t bl = c.get<uint64_t>();
            const uint8_t *body = c.take(size_t(bl));
            if (!c.ok) break;
            uint8_t h[32];
            holo::blake3_hash(body, bl, h);
            if (memcmp(h, fp, 32) != 0)
                return set_error(HOLO_ERR_DISPATCH, "session_load: weight body does not match its fingerprint");
            weights[std::string(reinterpret_cast<const char *>(fp), 32)] = {body, bl};
        }
        if (!c.ok) return set_error(HOLO_ERR_DISPATCH, "session_load: truncated Weights section");
    }
    struct Const {
        uint32_t slot;
        const uint8_t *body;
        uint64_t len;
    };
    std::vector<Const> consts;
    if ((it = sec.find(kSecConstants)) != sec.end()) {
        Cursor c{it->second.first, it->second.second};
        const uint32_t n = c.get<uint32_t>();
        for (uint32_t i = 0; i < n && c.ok; ++i) {
            const uint8_t tag = c.get<uint8_t>();
            const uint32_t slot = c.get<uint32_t>();
            (void)c.get<uint8_t>();   // dtype
            if (c.ok && slot == HOLO_SLOT_ABSENT)
                return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE,
                                 "session_load: constant " + std::to_string(i) + " names the absent slot");
            if (tag == 0) {
                const uint32_t bl = c.get<uint32_t>();
                const uint8_t *body = c.take(bl);
                if (c.ok) {
                    consts.push_back({slot, body, bl});
                    std::array<uint8_t, 32> d;
                    holo::blake3_hash(body, bl, d.data());   // address_bytes of the body
                    s->const_digests.push_back({slot, d});
                }
            } else if (tag == 1) {
                const uint8_t *fp = c.take(32);
                if (!c.ok) break;
                auto w = weights.find(std::string(reinterpret_cast<const char *>(fp), 32));
                if (w == weights.end())
                    return set_error(HOLO_ERR_DISPATCH,
                                     "session_load: constant references a weight the archive does not carry");
                consts.push_back({slot, w->second.first, w->second.second});
                std::array<uint8_t, 32> d;   // label_from_fingerprint: the verified digest
                memcpy(d.data(), fp, 32);
                s->const_digests.push_back({slot, d});
            } else {
                return set_error(HOLO_ERR_DISPATCH, "session_load: unknown ConstantEntry tag");
            }
        }
        if (!c.ok) return set_error(HOLO_ERR_DISPATCH, "session_load: truncated Constants section");
    }
    // --- panel-packed f32 weights (compiler.rs:590-613 packs every constant
    // f32 MatMul weight for the CPU engine, layout.rs:16-45): a constant read
    // only as the packed B of f32 MatMuls of one (k, n) is laid back out
    // row-major here, once, so those calls take the device's own MatMul
    // kernels (few-row, grouped). Any other packed B runs the packed kernel.
    std::vector<std::vector<uint8_t>> unpacked;
    {
        std::map<uint32_t, std::vector<holo_matmul_call *>> users;   // const slot -> packed uses
        std::map<uint32_t, bool> other;                              // read any other way
        std::vector<holo_buffer_ref> rd0, wr0;
        std::map<uint32_t, size_t> const_of;
        for (size_t i = 0; i < consts.size(); ++i) const_of[consts[i].slot] = i;
        for (auto &call : s->calls) {
            holo_matmul_call *mm = matmul_of(call);
            if (mm && mm->b_packed && mm->dtype == HOLO_DTYPE_F32 && mm->b.offset == 0 &&
                const_of.count(mm->b.slot)) {
                users[mm->b.slot].push_back(mm);
                call_operands(call, &rd0, &wr0);
                int n_b = 0;
                for (auto &r : rd0) n_b += r.slot == mm->b.slot;
                if (n_b != 1) other[mm->b.slot] = true;          // also read as A or residual
                continue;
            }
            call_operands(call, &rd0, &wr0);
            for (auto &r : rd0) other[r.slot] = true;
            for (auto &w : wr0) other[w.slot] = true;
        }
        unpacked.reserve(users.size());   // bodies below point into these buffers
        for (auto &u : users) {
            if (other.count(u.first)) continue;
            const uint32_t k = u.second[0]->k, n = u.second[0]->n;
            bool same = true;
            for (auto *mm : u.second) same = same && mm->k == k && mm->n == n;
            Const &cst = consts[const_of[u.first]];
            if (!same || cst.len < holo::packed_len(k, n) * 4) continue;
            std::vector<uint8_t> rm(uint64_t(k) * n * 4);
            const uint32_t np = (n + 15) / 16;
            for (uint32_t pnl = 0; pnl < np; ++pnl) {
                const uint32_t cols = n - pnl * 16 < 16 ? n - pnl * 16 : 16;
                for (uint32_t kk = 0; kk < k; ++kk)
                    memcpy(rm.data() + (uint64_t(kk) * n + pnl * 16) * 4,
                           cst.body + ((uint64_t(pnl) * k + kk) * 16) * 4, cols * 4);
            }
            unpacked.push_back(std::move(rm));
            cst.body = unpacked.back().data();
            cst.len = unpacked.back().size();
            for (auto *mm : u.second) {
                mm->b_packed = 0;
                mm->b.length = uint64_t(k) * n * 4;
            }
        }
    }
    // --- per-slot sizes (session.rs:544-623)
    size_t nslots = 0;
    std::vector<holo_buffer_ref> rd, wr;
    auto bump = [&](uint32_t slot) {
        if (slot != HOLO_SLOT_ABSENT && size_t(slot) + 1 > nslots) nslots = size_t(slot) + 1;
    };
    for (const auto &call : s->calls) {
        call_operands(call, &rd, &wr);
        for (auto &b : rd) bump(b.slot);
        for (auto &b : wr) bump(b.slot);
    }
    for (auto &p : s->inputs) bump(p.slot);
    for (auto &p : s->outputs) bump(p.slot);
    for (auto &k : consts) bump(k.slot);
    if (nslots > (1u << 24)) return set_error(HOLO_ERR_DISPATCH, "session_load: slot ids above 2^24");
    std::vector<uint64_t> sz(nslots, 0);
    std::vector<uint8_t> is_const(nslots, 0), is_input(nslots, 0), is_output(nslots, 0);
    for (const auto &call : s->calls) {
        call_operands(call, &rd, &wr);
        for (auto *v : {&rd, &wr})
            for (auto &b : *v) sz[b.slot] = std::max(sz[b.slot], sat_add(b.offset, b.length));
    }
    for (auto *ports : {&s->inputs, &s->outputs})
        for (auto &p : *ports) sz[p.slot] = std::max(sz[p.slot], sat_mul(p.count, port_bytes(p.dtype)));
    for (auto &k : consts) {
        sz[k.slot] = std::max(sz[k.slot], k.len);
        is_const[k.slot] = 1;
    }
    for (auto &p : s->inputs) is_input[p.slot] = 1;
    for (auto &p : s->outputs) is_output[p.slot] = 1;
    for (auto &v : sz) {
        // a slot no device could hold is refused here, before any rounding wraps
        if (v > (uint64_t(1) << 46))
            return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_load: a slot is referenced beyond 2^46 bytes");
        v = std::max<uint64_t>(v, 64), v = (v + 63) / 64 * 64;
    }
    // --- device memory: one arena for constants, one for every other slot,
    // each slot 256-byte aligned
    uint64_t cbytes = 0, wbytes = 0;
    std::vector<uint64_t> off(nslots, 0);
    for (size_t i = 0; i < nslots; ++i) {
        uint64_t &total = is_const[i] ? cbytes : wbytes;
        off[i] = total;
        total += (sz[i] + 255) / 256 * 256;
    }
    s->slot_bytes = sz;
    if (!be) {   // a dry load: parse and validate only (no device)
        s->slots.assign(nslots, SlotRange{});
        s->owned = s->slots;
        goto plan_moves;
    }
    if (hipSetDevice(holo::backend_device(be)) != hipSuccess)
        return set_error(HOLO_ERR_INIT, "session_load: hipSetDevice failed");
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess)
        return set_error(HOLO_ERR_INIT, "session_load: stream creation failed");
    if (cbytes && hipMalloc(&s->const_arena, cbytes) != hipSuccess)
        return set_error(HOLO_ERR_INIT, "session_load: constant arena allocation failed (" +
                                            std::to_string(cbytes) + " bytes)");
    if (wbytes && hipMalloc(&s->work_arena, wbytes) != hipSuccess)
        return set_error(HOLO_ERR_INIT, "session_load: slot arena allocation failed (" +
                                            std::to_string(wbytes) + " bytes)");
    s->owned.resize(nslots);
    for (size_t i = 0; i < nslots; ++i) {
        uint8_t *base = static_cast<uint8_t *>(is_const[i] ? s->const_arena : s->work_arena);
        s->owned[i] = SlotRange{base + off[i], sz[i]};
    }
    for (auto &k : consts)
        if (k.len && hipMemcpy(s->owned[k.slot].ptr, k.body, k.len, hipMemcpyHostToDevice) != hipSuccess)
            return set_error(HOLO_ERR_INIT, "session_load: constant upload failed");
    s->slots = s->owned;
plan_moves:
    // --- in-place KV moves (compute_stealable, session.rs:281): the cache
    // operand has no other reader, is no output port and no constant
    std::vector<uint32_t> readers(nslots, 0);
    for (const auto &call : s->calls) {
        call_operands(call, &rd, &wr);
        for (auto &b : rd) readers[b.slot]++;
    }
    for (auto &call : s->calls) {
        if (call.tag == HOLO_OP_KV_CACHE_WRITE) {
            auto &k = call.u.kv_write;
            const uint32_t cs = k.cache.slot, os = k.output.slot;
            if (cs == HOLO_SLOT_ABSENT || cs == os || readers[cs] != 1 || is_output[cs] || is_const[cs] || k.cache.offset != 0 ||
                k.output.offset != 0)
                continue;
            if (k.new_rows_buf.slot == cs || k.pos.slot == cs) continue;
            s->aliases.push_back({os, cs});
            k.output = k.cache;
        } else if (call.tag == HOLO_OP_KV_QUANT_APPEND) {
            auto &k = call.u.kv_quant_append;
            const uint32_t cq = k.cache.slot, cs = k.cache_scales.slot;
            const uint32_t oq = k.output.slot, os = k.output_scales.slot;
            if (cq == HOLO_SLOT_ABSENT || cs == HOLO_SLOT_ABSENT || cq == oq || cs == os || cq == cs || readers[cq] != 1 || readers[cs] != 1 ||
                is_output[cq] || is_output[cs] || is_const[cq] || is_const[cs] ||
                k.cache.offset != 0 || k.cache_scales.offset != 0 || k.output.offset != 0 ||
                k.output_scales.offset != 0)
                continue;
            if (k.new_rows_buf.slot == cq || k.new_rows_buf.slot == cs || k.pos.slot == cq || k.pos.slot == cs)
                continue;
            s->aliases.push_back({oq, cq});
            s->aliases.push_back({os, cs});
            k.output = k.cache;
            k.output_scales = k.cache_scales;
        }
    }
    // every call must be one this backend runs (validated on the slot sizes)
    for (size_t i = 0; i < s->calls.size(); ++i) {
        const int rc = holo_hip_validate(&s->calls[i], s->slot_bytes.data(), uint32_t(nslots));
        if (rc != HOLO_OK) {
            std::string m = holo_hip_last_error_message();
            return set_error(rc, std::string(op) + ": kernel call " + std::to_string(i) + " (tag " +
                                     std::to_string(s->calls[i].tag) + "): " + m);
        }
    }
    // --- the walk: fused groups, or every call in plan order
    if (flags & HOLO_SESSION_NO_DEVICE_FUSION) {
        for (auto &lv : s->plan)
            for (uint32_t ci : lv) s->nodes.push_back(Node{-1, ci});
    } else {
        device_fusion(s.get(), is_output, is_input);
        if (!(flags & HOLO_SESSION_NO_NORM_FUSION)) {
            const int rc = norm_fusion(s.get(), is_output, is_input, is_const,
                                       !(flags & HOLO_SESSION_NO_WEIGHT_PACKING));
            if (rc != HOLO_OK) return rc;
        }
    }
    elide_steps(s.get(), is_output, is_input, is_const);
    if (!(flags & (HOLO_SESSION_NO_DEVICE_FUSION | HOLO_SESSION_NO_WEIGHT_PACKING))) {
        const int rc = pack_weights(s.get(), is_input, is_const);
        if (rc != HOLO_OK) return rc;
    }
    if (!(flags & (HOLO_SESSION_NO_DEVICE_FUSION | HOLO_SESSION_NO_ATTN_PROLOGUE)))
        attn_prologue_fusion(s.get());
    *out = s.release();
    return HOLO_OK;
}

// The slot bindings a walk uses: each moved output is its cache's memory,
// each bound slot (a view or a reused value) the range of its source.
void apply_bindings(const holo_session *s, std::vector<SlotRange> &slots) {
    for (const auto &a : s->aliases) slots[a.first] = slots[a.second];
    for (const auto &v : s->views) {
        const SlotRange src = slots[v.in];
        const uint64_t start = std::min<uint64_t>(v.off, src.bytes);
        const uint64_t len = v.len == 0 ? src.bytes - start : std::min<uint64_t>(v.len, src.bytes - start);
        slots[v.out] = SlotRange{src.ptr ? src.ptr + start : nullptr, len};
    }
}

// One walk: each level's nodes in order on the session stream; a step whose
// `skip` entry is set is left out (its outputs already hold its value).
int walk(holo_session *s, const std::vector<uint8_t> *skip = nullptr) {
    if (!s->be) return set_error(HOLO_ERR_INIT, "session_execute: loaded without a backend (dry load)");
    apply_bindings(s, s->slots);
    const hipStream_t saved = holo::backend_stream(s->be);
    holo::set_backend_stream(s->be, s->stream);
    holo::swap_scratch(s->be, &s->scratch, &s->scratch_bytes);   // the session's scratch in
    int rc = HOLO_OK;
    s->last_dispatched = 0;
    s->last_skipped = s->n_elided;
    // a group's deferred split-K epilogue, run by the next node dispatched
    holo::EpiArgs pend;
    bool pending = false;
    for (size_t i = 0; i < s->nodes.size(); ++i) {
        const Node &nd = s->nodes[i];
        const bool skipped = skip && (*skip)[i];
        if (pending && (skipped || nd.group >= 0)) {
            pending = false;
            rc = holo::launch_deferred_epilogue(s->be, pend);
            if (rc != HOLO_OK) break;
        }
        if (skipped) {
            s->last_skipped++;
            continue;
        }
        s->last_dispatched++;
        if (nd.group >= 0) {
            rc = holo::dispatch_group(s->be, s->slots, s->groups[size_t(nd.group)],
                                      nd.epi_next ? &pend : nullptr);
            pending = rc == HOLO_OK && nd.epi_next && pend.ks != 0;
        } else if (pending) {
            pending = false;
            rc = holo::dispatch_with_epilogue(s->be, s->slots, &s->calls[nd.call], pend);
        } else {
            rc = holo::dispatch_with_slots(s->be, s->slots, &s->calls[nd.call]);
        }
        if (rc != HOLO_OK) {
            std::string m = holo_hip_last_error_message();
            set_error(rc, "session_execute: kernel call " + std::to_string(nd.call) +
                              (nd.group >= 0 ? " (fused group)" : "") + ": " + m);
            break;
        }
    }
    if (rc == HOLO_OK && pending) rc = holo::launch_deferred_epilogue(s->be, pend);
    holo::swap_scratch(s->be, &s->scratch, &s->scratch_bytes);   // and out again
    holo::set_backend_stream(s->be, saved);
    return rc;
}

bool same_bindings(const std::vector<SlotRange> &a, const std::vector<SlotRange> &b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (a[i].ptr != b[i].ptr || a[i].bytes != b[i].bytes) return false;
    return true;
}

}  // namespace

extern "C" {

int holo_hip_session_load(holo_backend *be, const uint8_t *bytes, size_t len, holo_session **out) {
    if (!bytes || !out) return set_error(HOLO_ERR_INIT, "session_load: null argument");
    *out = nullptr;
    return load_impl(be, bytes, len, 0, out);
}

int holo_hip_session_load_ex(holo_backend *be, const uint8_t *bytes, size_t len, uint32_t flags,
                             holo_session **out) {
    if (!bytes || !out) return set_error(HOLO_ERR_INIT, "session_load: null argument");
    *out = nullptr;
    return load_impl(be, bytes, len, flags, out);
}

int holo_hip_session_nodes(const holo_session *s, uint32_t *n_nodes, uint32_t *n_groups) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_nodes: null session");
    if (n_nodes) *n_nodes = uint32_t(s->nodes.size());
    if (n_groups) *n_groups = uint32_t(s->groups.size());
    return HOLO_OK;
}

int holo_hip_session_call(const holo_session *s, uint32_t index, holo_kernel_call *out) {
    if (!s || !out) return set_error(HOLO_ERR_INIT, "session_call: null argument");
    if (index >= s->calls.size())
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_call: index past the loaded calls");
    *out = s->calls[index];
    return HOLO_OK;
}

int holo_hip_session_packed(const holo_session *s, uint32_t *groups, uint64_t *bytes) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_packed: null session");
    uint32_t n = 0;
    std::vector<uint8_t> live(s->groups.size(), 0);
    for (const auto &nd : s->nodes)
        if (nd.group >= 0) live[size_t(nd.group)] = 1;
    for (size_t i = 0; i < s->groups.size(); ++i) n += live[i] && s->groups[i].packed;
    if (groups) *groups = n;
    if (bytes) *bytes = s->packed_bytes;
    return HOLO_OK;
}

int holo_hip_session_attn_prologues(const holo_session *s, uint32_t *n) {
    if (!s || !n) return set_error(HOLO_ERR_INIT, "session_attn_prologues: null argument");
    uint32_t c = 0;
    for (const auto &nd : s->nodes) c += nd.group >= 0 && nd.epi_next;
    *n = c;
    return HOLO_OK;
}

int holo_hip_session_close(holo_session *s) {
    release(s);
    return HOLO_OK;
}

int holo_hip_session_info(const holo_session *s, uint32_t *n_inputs, uint32_t *n_outputs,
                          uint32_t *n_calls, uint32_t *n_slots) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_info: null session");
    if (n_inputs) *n_inputs = uint32_t(s->inputs.size());
    if (n_outputs) *n_outputs = uint32_t(s->outputs.size());
    if (n_calls) *n_calls = uint32_t(s->calls.size());
    if (n_slots) *n_slots = uint32_t(s->slots.size());
    return HOLO_OK;
}

int holo_hip_session_port(const holo_session *s, int is_output, uint32_t index, uint32_t *slot,
                          uint64_t *element_count, uint8_t *dtype, uint64_t *bytes) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_port: null session");
    const auto &ports = is_output ? s->outputs : s->inputs;
    if (index >= ports.size()) return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_port: index out of range");
    const Port &p = ports[index];
    if (slot) *slot = p.slot;
    if (element_count) *element_count = p.count;
    if (dtype) *dtype = p.dtype;
    if (bytes) *bytes = p.count * port_bytes(p.dtype);
    return HOLO_OK;
}

int holo_hip_session_fingerprint(const holo_session *s, uint8_t out32[32]) {
    if (!s || !out32) return set_error(HOLO_ERR_INIT, "session_fingerprint: null argument");
    memcpy(out32, s->fingerprint, 32);
    return HOLO_OK;
}

int holo_hip_session_bind_input(holo_session *s, uint32_t index, void *dev_ptr, uint64_t bytes) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_bind_input: null session");
    s->memo_valid = false;
    if (index >= s->inputs.size())
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_bind_input: index out of range");
    const Port &p = s->inputs[index];
    if (!dev_ptr) {
        s->slots[p.slot] = s->owned[p.slot];
        return HOLO_OK;
    }
    const uint64_t need = p.count * port_bytes(p.dtype);
    if (bytes < need)
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_bind_input: port '" + p.name + "' needs " +
                                                         std::to_string(need) + " bytes, got " +
                                                         std::to_string(bytes));
    s->slots[p.slot] = SlotRange{static_cast<uint8_t *>(dev_ptr), bytes};
    return HOLO_OK;
}

int holo_hip_session_write_input(holo_session *s, uint32_t index, const void *host, uint64_t bytes) {
    if (!s || !host) return set_error(HOLO_ERR_INIT, "session_write_input: null argument");
    s->memo_valid = false;
    if (index >= s->inputs.size())
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_write_input: index out of range");
    const Port &p = s->inputs[index];
    const SlotRange &dst = s->slots[p.slot];
    const uint64_t n = std::min<uint64_t>(bytes, p.count * port_bytes(p.dtype));
    if (n > dst.bytes) return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_write_input: too many bytes");
    if (hipMemcpyAsync(dst.ptr, host, n, hipMemcpyHostToDevice, s->stream) != hipSuccess ||
        hipStreamSynchronize(s->stream) != hipSuccess)
        return set_error(HOLO_ERR_DISPATCH, "session_write_input: copy failed");
    return HOLO_OK;
}

int holo_hip_session_execute(holo_session *s) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_execute: null session");
    s->memo_valid = false;
    return walk(s);
}

namespace {

// The output ports' κ-labels for the given input-port labels: the boundary
// label a writing call gave the port, else (a port no call writes) the
// label of the input or constant it holds.
int derive_outputs(const holo_session *s, const std::vector<std::string> &in,
                   std::vector<std::string> *out) {
    std::vector<std::string> lab, wit;
    const int rc = label_walk(s, in, true, &lab, &wit);
    if (rc != HOLO_OK) return rc;
    out->clear();
    for (const auto &p : s->outputs) {
        const std::string *l = p.slot < wit.size() && !wit[p.slot].empty() ? &wit[p.slot]
                               : p.slot < lab.size() && !lab[p.slot].empty() ? &lab[p.slot]
                                                                              : nullptr;
        if (!l)
            return set_error(HOLO_ERR_UNSUPPORTED_OP,
                             "session_output_labels: output '" + p.name + "' is not addressable");
        out->push_back(*l);
    }
    return HOLO_OK;
}

}  // namespace

int holo_hip_session_output_labels(const holo_session *s, const char *input_labels, char *out) {
    if (!s || (!input_labels && !s->inputs.empty()) || (!out && !s->outputs.empty()))
        return set_error(HOLO_ERR_INIT, "session_output_labels: null argument");
    std::vector<std::string> in;
    for (size_t i = 0; i < s->inputs.size(); ++i)
        in.emplace_back(input_labels + i * HOLO_LABEL_LEN, HOLO_LABEL_LEN);
    std::vector<std::string> labels;
    const int rc = derive_outputs(s, in, &labels);
    if (rc != HOLO_OK) return rc;
    for (size_t i = 0; i < labels.size(); ++i) memcpy(out + i * HOLO_LABEL_LEN, labels[i].data(), HOLO_LABEL_LEN);
    return HOLO_OK;
}

int holo_hip_session_set_memo(holo_session *s, int enabled) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_set_memo: null session");
    s->memo_enabled = enabled != 0;
    if (!s->memo_enabled) s->memo_valid = false;
    return HOLO_OK;
}

int holo_hip_session_execute_bytes(holo_session *s, const void *const *inputs, const uint64_t *sizes,
                                   uint32_t n, int *memo_hit) {
    if (!s || (n && (!inputs || !sizes))) return set_error(HOLO_ERR_INIT, "session_execute_bytes: null argument");
    if (memo_hit) *memo_hit = 0;
    if (n != s->inputs.size())
        return set_error(HOLO_ERR_SHAPE_MISMATCH,
                         "session_execute_bytes: expected " + std::to_string(s->inputs.size()) + " inputs");
    if (!s->be) return set_error(HOLO_ERR_INIT, "session_execute_bytes: a dry-loaded session cannot execute");
    std::vector<std::string> key;
    if (s->memo_enabled) {
        s->input_seen.resize(n);
        s->input_seen_label.resize(n);
        for (uint32_t i = 0; i < n; ++i) {
            const Port &p = s->inputs[i];
            const uint64_t len = std::min<uint64_t>(sizes[i], sat_mul(p.count, port_bytes(p.dtype)));
            const uint8_t *b = static_cast<const uint8_t *>(inputs[i]);
            auto &seen = s->input_seen[i];
            if (seen.size() != len || (len && memcmp(seen.data(), b, len) != 0) || s->input_seen_label[i].empty()) {
                seen.assign(b, b + len);   // a repeated input is not hashed again
                s->input_seen_label[i] = holo::address_bytes(b, len);
            }
            key.push_back(s->input_seen_label[i]);
        }
        // hit: the outputs of these inputs are still in the output slots
        if (s->memo_valid && key == s->memo_key) {
            if (memo_hit) *memo_hit = 1;
            s->last_dispatched = 0;
            s->last_skipped = uint32_t(s->nodes.size()) + s->n_elided;
            return HOLO_OK;
        }
    }
    // resident reuse across walks (session.rs:1121-1131): a step none of
    // whose operands changed since the last walk (labels derive from the
    // inputs' labels, so equal inputs give equal labels) still holds its
    // value and is skipped; steps on an in-place KV move or an output port
    // always run
    std::vector<uint8_t> skip;
    if (s->memo_enabled && s->memo_valid && s->memo_key.size() == n && !s->root.empty()) {
        std::vector<uint8_t> dirty(s->root.size(), 0);
        for (uint32_t i = 0; i < n; ++i)
            if (key[i] != s->memo_key[i] && s->inputs[i].slot < dirty.size())
                dirty[s->root[s->inputs[i].slot]] = 1;
        skip.assign(s->nodes.size(), 0);
        for (size_t j = 0; j < s->nodes.size(); ++j) {
            bool d = s->node_always[j] != 0;
            for (uint32_t r : s->node_rd[j]) d = d || dirty[r];
            if (d)
                for (uint32_t w : s->node_wr[j]) dirty[w] = 1;
            else
                skip[j] = 1;
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        const int rc = holo_hip_session_write_input(s, i, inputs[i], sizes[i]);
        if (rc != HOLO_OK) return rc;
    }
    s->memo_valid = false;
    const int rc = walk(s, skip.empty() ? nullptr : &skip);
    if (rc != HOLO_OK) return rc;
    s->memo_key = std::move(key);
    s->memo_valid = s->memo_enabled;
    return HOLO_OK;
}

int holo_hip_session_output(const holo_session *s, uint32_t index, void **dev_ptr, uint64_t *bytes) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_output: null session");
    if (index >= s->outputs.size())
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_output: index out of range");
    const Port &p = s->outputs[index];
    if (dev_ptr) *dev_ptr = s->slots[p.slot].ptr;
    if (bytes) *bytes = p.count * port_bytes(p.dtype);
    return HOLO_OK;
}

int holo_hip_session_read_output(holo_session *s, uint32_t index, void *host, uint64_t bytes) {
    if (!s || !host) return set_error(HOLO_ERR_INIT, "session_read_output: null argument");
    if (index >= s->outputs.size())
        return set_error(HOLO_ERR_SLOT_OUT_OF_RANGE, "session_read_output: index out of range");
    const Port &p = s->outputs[index];
    const uint64_t n = std::min<uint64_t>(bytes, p.count * port_bytes(p.dtype));
    if (hipStreamSynchronize(s->stream) != hipSuccess ||
        hipMemcpy(host, s->slots[p.slot].ptr, n, hipMemcpyDeviceToHost) != hipSuccess)
        return set_error(HOLO_ERR_DISPATCH, "session_read_output: copy failed");
    return HOLO_OK;
}

int holo_hip_session_synchronize(holo_session *s) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_synchronize: null session");
    const hipStream_t saved = holo::backend_stream(s->be);
    holo::set_backend_stream(s->be, s->stream);
    const int rc = holo_hip_synchronize(s->be);
    holo::set_backend_stream(s->be, saved);
    return rc;
}

int holo_hip_session_stream(const holo_session *s, void **stream) {
    if (!s || !stream) return set_error(HOLO_ERR_INIT, "session_stream: null argument");
    *stream = s->stream;
    return HOLO_OK;
}

int holo_hip_session_capture(holo_session *s) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_capture: null session");
    s->memo_valid = false;
    // An eager walk first: it sizes the backend's scratch (no allocation may
    // happen under capture) and surfaces any refusal with a message.
    int rc = walk(s);
    if (rc != HOLO_OK) return rc;
    if (hipStreamSynchronize(s->stream) != hipSuccess)
        return set_error(HOLO_ERR_DISPATCH, "session_capture: eager walk failed");
    if (s->graph) {
        (void)hipGraphExecDestroy(s->graph);
        s->graph = nullptr;
    }
    if (hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return set_error(HOLO_ERR_DISPATCH, "session_capture: begin capture failed");
    rc = walk(s);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s->stream, &g);
    if (rc != HOLO_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess || !g) return set_error(HOLO_ERR_DISPATCH, "session_capture: end capture failed");
    const hipError_t ie = hipGraphInstantiate(&s->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) {
        s->graph = nullptr;
        return set_error(HOLO_ERR_DISPATCH, "session_capture: graph instantiation failed");
    }
    s->graph_slots = s->slots;
    s->graph_scratch = s->scratch;
    return HOLO_OK;
}

int holo_hip_session_replay(holo_session *s) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_replay: null session");
    s->memo_valid = false;
    if (!s->graph) return set_error(HOLO_ERR_DISPATCH, "session_replay: no captured walk");
    std::vector<SlotRange> now = s->slots;
    apply_bindings(s, now);
    if (!same_bindings(now, s->graph_slots))
        return set_error(HOLO_ERR_DISPATCH,
                         "session_replay: an input was rebound since the capture; capture again");
    if (s->scratch != s->graph_scratch)
        return set_error(HOLO_ERR_DISPATCH,
                         "session_replay: the session's scratch was reallocated since the capture; capture again");
    if (hipGraphLaunch(s->graph, s->stream) != hipSuccess)
        return set_error(HOLO_ERR_DISPATCH, "session_replay: graph launch failed");
    s->last_dispatched = uint32_t(s->nodes.size());
    s->last_skipped = s->n_elided;
    return HOLO_OK;
}

int holo_hip_session_last_walk(const holo_session *s, uint32_t *dispatched, uint32_t *skipped) {
    if (!s) return set_error(HOLO_ERR_INIT, "session_last_walk: null session");
    if (dispatched) *dispatched = s->last_dispatched;
    if (skipped) *skipped = s->last_skipped;
    return HOLO_OK;
}

int holo_hip_blake3(const void *data, size_t len, uint8_t out32[32]) {
    if ((!data && len) || !out32) return set_error(HOLO_ERR_DISPATCH, "blake3: null argument");
    holo::blake3_hash(data, len, out32);
    return HOLO_OK;
}

}  // extern "C"
