// holo_backend.cpp — the C ABI of include/holo_hip.h: the Backend::dispatch
// boundary (crates/hologram-compute/src/backend.rs:8-15) over device-resident
// slots, with the reference CPU kernels' refusals reproduced before any
// device work.
#include "holo_hip.h"

#include <hip/hip_runtime.h>
#include <string.h>

#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "holo_internal.h"
#include "holo_kernels.h"

namespace holo {
bool build_lut_table(int act, bool f16, uint16_t *t);
bool lut_act_value(int act, float x, float *y);
}

namespace {

thread_local std::string g_last_error;
const int kZero = 0;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

struct Range {
    uint8_t *ptr = nullptr;
    uint64_t bytes = 0;
};

// A resolved operand: [base, base + bytes) in device memory.
struct View {
    uint8_t *base = nullptr;
    uint64_t bytes = 0;
    uint64_t key = 0;  // 0: compare device addresses; else the slot a size-only check saw
};

}  // namespace

struct holo_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    std::map<uint32_t, Range> slots;
    uint16_t *lut_dev[9][2] = {};       // [table id][0 = f16, 1 = bf16], uploaded once
    void *scratch = nullptr;            // split-K partials (decode attention, few-row MatMul)
    size_t scratch_bytes = 0;
    int *dev_err = nullptr;             // device-side refusals (Gather's index range), read at sync
};

namespace {

// Slot-size source for validation: a live backend's slot table, or the plain
// slot_bytes array of holo_hip_validate (no device memory behind it).
struct SlotTable {
    const holo_backend *be = nullptr;
    const uint64_t *sizes = nullptr;
    uint32_t nsizes = 0;
    const std::vector<holo::SlotRange> *vec = nullptr;   // a session's slot table

    bool lookup(uint32_t slot, uint8_t **ptr, uint64_t *bytes, uint64_t *key) const {
        if (vec) {
            if (slot >= vec->size() || !(*vec)[slot].ptr) return false;
            *ptr = (*vec)[slot].ptr;
            *bytes = (*vec)[slot].bytes;
            *key = 0;
            return true;
        }
        if (be) {
            auto it = be->slots.find(slot);
            if (it == be->slots.end()) return false;
            *ptr = it->second.ptr;
            *bytes = it->second.bytes;
            *key = 0;
            return true;
        }
        if (slot >= nsizes) return false;
        // Size-only check: slots are distinct buffers, ranges are offsets.
        *ptr = nullptr;
        *bytes = sizes[slot];
        *key = uint64_t(slot) + 1;
        return true;
    }
};

// BufferArena::buf_range (crates/hologram-exec/src/buffer.rs:312-335):
// start = min(offset, len); end = length == 0 ? len : min(start + length, len).
bool resolve(const SlotTable &st, const holo_buffer_ref &r, View *v) {
    uint8_t *p;
    uint64_t len, key;
    if (!st.lookup(r.slot, &p, &len, &key)) return false;
    const uint64_t start = r.offset < len ? r.offset : len;
    // (saturating: a length past the slot's end, however large, ends at len)
    const uint64_t end = (r.length == 0 || r.length > len - start) ? len : start + r.length;
    v->base = p + start;
    v->bytes = end - start;
    v->key = key;
    return true;
}

bool overlaps(const View &a, const View &b) {
    if (a.key != b.key) return false;
    return a.base < b.base + b.bytes && b.base < a.base + a.bytes;
}

// split_borrow (buffer.rs:974-998): every read resolves and no read range
// overlaps the write range; a refusal is SlotOutOfRange(write slot).
int split_borrow(const SlotTable &st, const holo_buffer_ref *reads, View *rv, int nreads,
                 const holo_buffer_ref &write, View *wv, const char *op) {
    if (!resolve(st, write, wv))
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    std::string(op) + ": output slot " + std::to_string(write.slot) + " unbound");
    for (int i = 0; i < nreads; ++i) {
        if (!resolve(st, reads[i], &rv[i]))
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, std::string(op) + ": input slot " +
                                                        std::to_string(reads[i].slot) + " unbound");
        if (overlaps(rv[i], *wv))
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                        std::string(op) + ": input overlaps output slot " +
                            std::to_string(write.slot));
    }
    return HOLO_OK;
}

// Device address alignment of a resolved view (offsets included). A size-only
// validation has no addresses; its views are checked by offset alone.
bool aligned(const View &v, uint64_t a) {
    return (reinterpret_cast<uintptr_t>(v.base) % a) == 0;
}

int need(const View &v, uint64_t bytes, uint32_t slot, const char *op, const char *what) {
    if (v.bytes < bytes)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    std::string(op) + ": " + what + " (slot " + std::to_string(slot) + ") holds " +
                        std::to_string(v.bytes) + " bytes, needs " + std::to_string(bytes));
    return HOLO_OK;
}

#define HOLO_TRY(expr)                    \
    do {                                  \
        int _rc = (expr);                 \
        if (_rc != HOLO_OK) return _rc;   \
    } while (0)

int launched(hipError_t e, const char *op) {
    if (e != hipSuccess)
        return fail(HOLO_ERR_DISPATCH, std::string(op) + ": launch failed: " + hipGetErrorString(e));
    return HOLO_OK;
}

// The fused_activation id (kernel_call.rs:861-870) of a unary activation tag.
uint32_t fused_of_unary(uint32_t tag) {
    switch (tag) {
        case HOLO_OP_RELU: return 1;
        case HOLO_OP_GELU: return 2;
        case HOLO_OP_SILU: return 3;
        case HOLO_OP_SIGMOID: return 4;
        case HOLO_OP_TANH: return 5;
        case HOLO_OP_ELU: return 6;
        case HOLO_OP_SELU: return 7;
        case HOLO_OP_EXP: return 8;
        case HOLO_OP_ERF: return holo::kActErf;
        default: return 0;
    }
}

size_t dtype_size(uint8_t dt) {
    switch (dt) {
        case HOLO_DTYPE_I8: return 1;
        case HOLO_DTYPE_F16:
        case HOLO_DTYPE_BF16: return 2;
        case HOLO_DTYPE_F32: return 4;
        default: return 0;
    }
}

// The device copy of the (act, dtype) table, built and uploaded on first use
// (once per backend; a session's eager walk does this before any capture).
int lut_table(holo_backend *be, int act, bool f16, const uint16_t **out, const char *op) {
    uint16_t *&tab = be->lut_dev[act][f16 ? 0 : 1];
    if (!tab) {
        std::vector<uint16_t> host(65536);
        holo::build_lut_table(act, f16, host.data());
        void *d = nullptr;
        hipError_t e = hipMalloc(&d, 65536 * 2);
        if (e != hipSuccess) return fail(HOLO_ERR_INIT, std::string(op) + ": table allocation failed");
        e = hipMemcpy(d, host.data(), 65536 * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return fail(HOLO_ERR_INIT, std::string(op) + ": table upload failed");
        }
        tab = static_cast<uint16_t *>(d);
    }
    *out = tab;
    return HOLO_OK;
}

// ---------------------------------------------------------------- LUT ----
// unary_act -> unary_lut (src/cpu/kernels.rs:1586-1598, src/cpu/lut.rs:76-98).
// 16-bit: the table of narrow(f(widen(x))); f32: f per element.
int do_unary(holo_backend *be, const SlotTable &st, uint32_t tag, const holo_unary_call &c) {
    const char *op = "unary_lut";
    const uint32_t fa = fused_of_unary(tag);
    const int act = holo::lut_act_of_fused(fa);
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "unary: the device path serves bf16/f16 (tables) and f32 (computed)");
    if (c.element_count == 0) return HOLO_OK;
    View in, out;
    HOLO_TRY(split_borrow(st, &c.input, &in, 1, c.output, &out, op));
    const uint64_t es = c.dtype == HOLO_DTYPE_F32 ? 4 : 2;
    const uint64_t bytes = c.element_count * es;
    HOLO_TRY(need(in, bytes, c.input.slot, op, "input"));
    HOLO_TRY(need(out, bytes, c.output.slot, op, "output"));
    if (!aligned(in, es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "unary: operands must be element-aligned");
    if (!be) return HOLO_OK;
    if (c.dtype == HOLO_DTYPE_F32)
        return launched(holo::launch_act_f32(reinterpret_cast<const float *>(in.base),
                                             reinterpret_cast<float *>(out.base), c.element_count,
                                             fa, be->stream),
                        op);
    const uint16_t *tab = nullptr;
    HOLO_TRY(lut_table(be, act, c.dtype == HOLO_DTYPE_F16, &tab, op));
    return launched(holo::launch_lut_u16(tab, reinterpret_cast<const uint16_t *>(in.base),
                                         reinterpret_cast<uint16_t *>(out.base), c.element_count,
                                         be->stream),
                    op);
}

// The backend's split-K scratch grows to the largest request; the old buffer
// is released only after the stream has drained (kernels may still read it).
// Never under stream capture: a captured graph would hold the freed buffer
// (a session's capture is preceded by an eager walk that sizes it).
int ensure_scratch(holo_backend *be, size_t bytes, const char *op) {
    if (bytes <= be->scratch_bytes) return HOLO_OK;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(be->stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(HOLO_ERR_DISPATCH,
                    std::string(op) + ": scratch would grow under stream capture; walk once eagerly first");
    if (be->scratch) {
        (void)hipStreamSynchronize(be->stream);
        (void)hipFree(be->scratch);
        be->scratch = nullptr;
        be->scratch_bytes = 0;
    }
    if (hipMalloc(&be->scratch, bytes) != hipSuccess)
        return fail(HOLO_ERR_INIT, std::string(op) + ": scratch allocation failed");
    be->scratch_bytes = bytes;
    return HOLO_OK;
}

// ------------------------------------------------------------- MatMul ----
// matmul_float (src/cpu/float_kernels.rs:298-399).
int do_matmul(holo_backend *be, const SlotTable &st, const holo_matmul_call &c) {
    const char *op = "matmul";
    if (c.m == 0 || c.k == 0 || c.n == 0) return HOLO_OK;
    if (c.dtype != HOLO_DTYPE_F32 && c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul: the device path serves f32, bf16 and f16");
    // the compiler panel-packs constant f32 weights only (compiler.rs:590-613)
    if (c.b_packed && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul: a panel-packed B is served for f32 only");
    const uint64_t es = dtype_size(c.dtype);
    holo_buffer_ref reads[2] = {c.a, c.b};
    View rv[2], out;
    HOLO_TRY(split_borrow(st, reads, rv, 2, c.output, &out, op));
    HOLO_TRY(need(rv[0], uint64_t(c.m) * c.k * es, c.a.slot, op, "a"));
    // a packed weight spans layout::packed_len(k, n) elements (float_kernels.rs:317-324)
    HOLO_TRY(need(rv[1], (c.b_packed ? holo::packed_len(c.k, c.n) : uint64_t(c.k) * c.n) * es,
                  c.b.slot, op, "b"));
    HOLO_TRY(need(out, uint64_t(c.m) * c.n * es, c.output.slot, op, "output"));
    if (!aligned(rv[0], es) || !aligned(rv[1], es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul: operands must be element-aligned");
    if ((uint64_t(c.m) + 127) / 128 > 65535)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul: m above 8388480");
    if (!be) return HOLO_OK;
    if (c.b_packed)
        return launched(holo::launch_matmul_f32_packed(
                            reinterpret_cast<const float *>(rv[0].base),
                            reinterpret_cast<const float *>(rv[1].base),
                            reinterpret_cast<float *>(out.base), c.m, c.k, c.n, be->stream),
                        op);
    HOLO_TRY(ensure_scratch(be, holo::matmul_scratch_bytes(c.m, c.k, c.n, c.dtype), op));
    return launched(holo::launch_matmul(rv[0].base, rv[1].base, out.base, c.m, c.k, c.n, c.dtype,
                                        be->scratch, be->stream),
                    op);
}

// ------------------------------------------------------- fused groups ----
// Every member's product in one few-row launch (fp32 partials), then one
// epilogue launch that finishes each segment. A one-segment group with an
// element-wise epilogue that the few-row kernels do not serve runs the tiled
// MatMul into its output and the epilogue over it in place.
int dispatch_group_impl(holo_backend *be, const SlotTable &st, const holo::GroupDesc &g,
                        const char *op, holo::EpiArgs *defer = nullptr) {
    const size_t nseg = g.segs.size();
    if (nseg == 0 || nseg > size_t(holo::kSkinnyMaxSeg))
        return fail(HOLO_ERR_DISPATCH, std::string(op) + ": fused group of " + std::to_string(nseg) +
                                           " products");
    const bool bf16 = g.dtype == HOLO_DTYPE_BF16;
    const uint64_t es = dtype_size(g.dtype), mk = uint64_t(g.m) * g.k;
    auto get = [&](const holo_buffer_ref &r, uint64_t bytes, const char *what, View *v) {
        if (!resolve(st, r, v))
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, std::string(op) + ": " + what + " slot " +
                                                        std::to_string(r.slot) + " unbound");
        return need(*v, bytes, r.slot, op, what);
    };
    View a;
    HOLO_TRY(get(g.a, mk * es, "a", &a));
    bool fast = aligned(a, 16);
    holo::SkinnyPlan plan = holo::matmul_skinny_plan(g.m, g.k, g.segs[0].n, g.dtype);
    holo::SkinnySegment ss[holo::kSkinnyMaxSeg];
    holo::EpiArgs e;
    e.m = g.m;
    e.bf16 = bf16;
    e.nseg = uint32_t(nseg);
    uint32_t ntot = 0;
    for (size_t i = 0; i < nseg; ++i) {
        const holo::GroupSegDesc &s = g.segs[i];
        holo::EpiSeg &d = e.seg[i];
        const uint64_t mn = uint64_t(g.m) * s.n;
        View v;
        HOLO_TRY(get(s.b, uint64_t(g.k) * s.n * es, "b", &v));
        fast = fast && aligned(v, 16);
        ss[i] = holo::SkinnySegment{v.base, s.n};
        const holo::SkinnyPlan p = holo::matmul_skinny_plan(g.m, g.k, s.n, g.dtype);
        if (p.mt != plan.mt || p.steps != plan.steps || p.ks != plan.ks) fast = false;
        // the few-row epilogue reads side operands through 32-bit offsets
        if (mn * es > 0x7fffffffull) fast = false;
        d.n = s.n;
        d.col0 = ntot;
        ntot += s.n;
        d.base = s.base;
        d.act = s.act;
        if ((s.base == holo::kEpiAct || s.base == holo::kEpiAddAct) &&
            !holo::fused_act_supported(s.act, g.dtype, s.base == holo::kEpiAddAct))
            return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": activation " +
                                                     std::to_string(s.act) + " is not served");
        if (s.base == holo::kEpiAct && bf16)
            HOLO_TRY(lut_table(be, holo::lut_act_of_fused(s.act), false, &d.lut, op));
        if (s.base == holo::kEpiAdd || s.base == holo::kEpiAddAct) {
            HOLO_TRY(get(s.residual, mn * es, "residual", &v));
            d.residual = v.base;
        }
        if (s.write_out) {
            HOLO_TRY(get(s.out, mn * es, "output", &v));
            d.out = v.base;
        }
        d.head_dim = s.head_dim;
        d.rope = s.rope;
        if (s.rope) {
            HOLO_TRY(get(s.cos, mn * es, "cos", &v));
            d.cos = v.base;
            HOLO_TRY(get(s.sin, mn * es, "sin", &v));
            d.sin = v.base;
            if (s.write_rope) {
                HOLO_TRY(get(s.rope_out, mn * es, "rope output", &v));
                d.rope_out = v.base;
            }
        }
        d.quant = s.quant;
        if (s.quant) {
            const uint64_t planes = mn / s.head_dim / s.new_rows;
            HOLO_TRY(get(s.pos, 4, "pos", &v));
            if (!aligned(v, 4)) return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": pos must be aligned");
            d.pos = reinterpret_cast<const uint32_t *>(v.base);
            HOLO_TRY(get(s.cq, planes * s.bucket * s.head_dim, "int8 cache", &v));
            d.cq = reinterpret_cast<int8_t *>(v.base);
            HOLO_TRY(get(s.cs, planes * s.bucket * 4, "scale cache", &v));
            if (!aligned(v, 4)) return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": scales must be aligned");
            d.cs = reinterpret_cast<float *>(v.base);
            d.bucket = s.bucket;
            d.new_rows = s.new_rows;
        }
        d.pair = s.pair;
        if (s.pair >= 0) {
            HOLO_TRY(get(s.mul_out, mn * es, "product output", &v));
            d.mul_out = v.base;
        }
        d.skip = s.skip;
        d.ssq = s.ssq;
        if (s.ssq && (!bf16 || s.head_dim || s.pair >= 0 || s.skip || s.n % 8 != 0 || s.n > 8192 ||
                      ((reinterpret_cast<uintptr_t>(d.out) | reinterpret_cast<uintptr_t>(d.residual)) & 15)))
            return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a norm-statistics epilogue needs a "
                                                             "bf16 element-wise product of <= 8192 "
                                                             "16-byte aligned columns");
    }
    holo::SkinnyNormA na;
    const bool a_norm = g.a_norm;
    if (a_norm && !g.packed && !g.a_ssq)
        return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a normalized A without row statistics");
    if (a_norm) {
        if (!bf16) return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a normalized A must be bf16");
        na.ssq = g.a_ssq;
        na.eps = g.a_eps;
        if (g.a_gamma.slot != HOLO_SLOT_ABSENT) {
            View gv;
            if (!resolve(st, g.a_gamma, &gv))
                return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, std::string(op) + ": gamma slot unbound");
            // affine_operand (float_kernels.rs:39-44): an empty gamma is the identity
            if (gv.bytes > 0) {
                HOLO_TRY(need(gv, uint64_t(g.k) * es, g.a_gamma.slot, op, "gamma"));
                if (!aligned(gv, 16))
                    return fail(HOLO_ERR_DISPATCH, std::string(op) + ": gamma must be 16-byte aligned");
                na.gamma = reinterpret_cast<const uint16_t *>(gv.base);
            }
        }
    }
    if (g.packed && (aligned(a, 16) || (a_norm && !g.a_ssq))) {
        // one launch over the fragment-order weights; a normalized A's
        // statistics are taken in it (an A the launch's 16-byte loads cannot
        // take, bound by the caller, goes the split-K way: same bits)
        holo::PackedGroup pg;
        pg.a = a.base;
        pg.m = g.m;
        pg.k = g.k;
        pg.nseg = int(nseg);
        pg.norm = a_norm;
        pg.gamma = na.gamma;
        pg.eps = na.eps;
        pg.tw = g.packed_tw;
        for (size_t i = 0; i < nseg; ++i) {
            pg.bp[i] = g.segs[i].bp;
            pg.seg[i] = e.seg[i];
            pg.seg[i].ssq = nullptr;
            if (!pg.bp[i])
                return fail(HOLO_ERR_DISPATCH, std::string(op) + ": packed group without packed weights");
        }
        if (!bf16 || !aligned(a, 16) || !holo::packed_group_applies(g.m, g.k, pg.seg, int(nseg), a_norm))
            return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a packed group needs bf16, <= 16 rows of "
                                                             "16-byte aligned A and 16-column tiles");
        return launched(holo::launch_packed_group(pg, be->stream), op);
    }
    bool stats = false;
    for (size_t i = 0; i < nseg; ++i) stats = stats || g.segs[i].ssq;
    fast = fast && plan.mt != 0;
    if (!fast && (a_norm || stats))
        return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a fused RmsNorm needs the few-row path "
                                                         "(16-byte aligned operands)");
    if (!fast && nseg == 2 && bf16 && (g.segs[0].pair == 1 || g.segs[1].pair == 0)) {
        // large M, SwiGLU pair: both products and f(gate) * g(up) in one
        // launch of the tiled kernel
        const size_t gi = g.segs[0].pair == 1 ? 0 : 1, ui = 1 - gi;
        const holo::GroupSegDesc &sg = g.segs[gi], &su = g.segs[ui];
        if (!(sg.base == holo::kEpiStore || sg.base == holo::kEpiAct) || su.base != holo::kEpiStore ||
            sg.write_out || su.write_out || sg.head_dim || su.head_dim || sg.ssq || su.ssq || !su.skip)
            return fail(HOLO_ERR_DISPATCH, std::string(op) + ": a tiled pair needs a plain or "
                                                             "table-activated gate and a plain up");
        return launched(holo::launch_matmul_pair_tiled(
                            a.base, g.m, g.k, ss[gi].b, ss[ui].b, sg.n, e.seg[gi].mul_out,
                            sg.base == holo::kEpiAct ? e.seg[gi].lut : nullptr, be->stream),
                        op);
    }
    if (!fast && nseg > 1 && bf16) {
        // large M: one launch of the tiled kernel for every product, then
        // each segment's element-wise epilogue in place
        bool plain = true;
        uint32_t ns[holo::kSkinnyMaxSeg];
        void *cs[holo::kSkinnyMaxSeg];
        for (size_t i = 0; i < nseg; ++i) {
            const holo::GroupSegDesc &s = g.segs[i];
            plain = plain && s.write_out && !s.head_dim && !s.rope && !s.quant && s.pair < 0 &&
                    !s.skip && !s.ssq;
            ns[i] = s.n;
            cs[i] = e.seg[i].out;
        }
        uintptr_t al = reinterpret_cast<uintptr_t>(a.base);
        for (size_t i = 0; i < nseg; ++i)
            al |= reinterpret_cast<uintptr_t>(ss[i].b) | reinterpret_cast<uintptr_t>(cs[i]);
        if (plain && (al & 15) != 0) {
            // operands the grouped kernel's 16-byte loads cannot take: each
            // product on its own through the general MatMul, epilogue in place
            for (size_t i = 0; i < nseg; ++i) {
                HOLO_TRY(ensure_scratch(be, holo::matmul_scratch_bytes(g.m, g.k, ns[i], g.dtype), op));
                HOLO_TRY(launched(holo::launch_matmul(a.base, ss[i].b, cs[i], g.m, g.k, ns[i], g.dtype,
                                                      be->scratch, be->stream),
                                  op));
                if (g.segs[i].base == holo::kEpiStore) continue;
                holo::TileEpi te;
                te.kind = g.segs[i].base;
                te.act = g.segs[i].act;
                te.lut = e.seg[i].lut;
                te.residual = e.seg[i].residual;
                HOLO_TRY(launched(holo::launch_tile_epilogue(cs[i], uint64_t(g.m) * ns[i], bf16, te,
                                                             be->stream),
                                  op));
            }
            return HOLO_OK;
        }
        if (plain && holo::matmul_group_tiled_applies(g.m, g.k, ns, int(nseg))) {
            // residual adds ride in the tiled kernel's store where the
            // residual suits its 16-byte loads; otherwise they run in place after
            const void *rs[holo::kSkinnyMaxSeg] = {};
            for (size_t i = 0; i < nseg; ++i)
                if (g.segs[i].base == holo::kEpiAdd && ns[i] < (1u << 21) &&
                    (reinterpret_cast<uintptr_t>(e.seg[i].residual) & 15) == 0)
                    rs[i] = e.seg[i].residual;
            HOLO_TRY(launched(holo::launch_matmul_group_tiled(a.base, g.m, g.k, ss, cs, int(nseg),
                                                              be->stream, rs),
                              op));
            for (size_t i = 0; i < nseg; ++i) {
                if (g.segs[i].base == holo::kEpiStore || rs[i]) continue;
                holo::TileEpi te;
                te.kind = g.segs[i].base;
                te.act = g.segs[i].act;
                te.lut = e.seg[i].lut;
                te.residual = e.seg[i].residual;
                HOLO_TRY(launched(holo::launch_tile_epilogue(cs[i], uint64_t(g.m) * ns[i], bf16, te,
                                                             be->stream),
                                  op));
            }
            return HOLO_OK;
        }
    }
    if (!fast) {
        const holo::GroupSegDesc &s = g.segs[0];
        const bool elementwise = nseg == 1 && s.write_out && !s.head_dim && s.pair < 0;
        if (!elementwise)
            return fail(HOLO_ERR_DISPATCH,
                        std::string(op) + ": a fused group needs the few-row path (16-byte aligned "
                                          "operands, one common split)");
        if (bf16 && s.base == holo::kEpiAdd && s.n < (1u << 21) &&
            holo::matmul_group_tiled_applies(g.m, g.k, &s.n, 1) &&
            ((reinterpret_cast<uintptr_t>(a.base) | reinterpret_cast<uintptr_t>(ss[0].b) |
              reinterpret_cast<uintptr_t>(e.seg[0].out) |
              reinterpret_cast<uintptr_t>(e.seg[0].residual)) & 15) == 0) {
            // MatMulAdd at large M: the residual is added in the tiled kernel's store
            void *cs[1] = {e.seg[0].out};
            const void *rs[1] = {e.seg[0].residual};
            return launched(holo::launch_matmul_group_tiled(a.base, g.m, g.k, ss, cs, 1, be->stream, rs),
                            op);
        }
        // the tiled product into the output, then the epilogue over it in place
        HOLO_TRY(ensure_scratch(be, holo::matmul_scratch_bytes(g.m, g.k, s.n, g.dtype), op));
        HOLO_TRY(launched(holo::launch_matmul(a.base, ss[0].b, e.seg[0].out, g.m, g.k, s.n, g.dtype,
                                              be->scratch, be->stream),
                          op));
        if (s.base == holo::kEpiStore) return HOLO_OK;
        holo::TileEpi te;
        te.kind = s.base;
        te.act = s.act;
        te.lut = e.seg[0].lut;
        te.residual = e.seg[0].residual;
        return launched(holo::launch_tile_epilogue(e.seg[0].out, uint64_t(g.m) * s.n, bf16, te,
                                                   be->stream),
                        op);
    }
    HOLO_TRY(ensure_scratch(be, size_t(plan.ks) * g.m * ntot * 4, op));
    e.P = static_cast<const float *>(be->scratch);
    e.ks = plan.ks;
    e.ntot = ntot;
    HOLO_TRY(launched(holo::launch_skinny_partials(a.base, g.m, g.k, g.dtype, ss, int(nseg), plan,
                                                   static_cast<float *>(be->scratch), be->stream,
                                                   a_norm ? &na : nullptr),
                      op));
    if (defer) {
        // the caller runs the epilogue with the next call (its partials stay
        // in the scratch, which nothing may grow before then)
        *defer = e;
        return HOLO_OK;
    }
    return launched(holo::launch_epilogue(e, be->stream), op);
}

// ------------------------------------------------ fused MatMul epilogues ----
// matmul_activation_float / matmul_add_float / matmul_add_activation_float
// (src/cpu/float_kernels.rs:816-935): the product, then the epilogue over the
// m*n results. Few-row shapes finish the product in the epilogue launch (one
// group of one segment); the tiled path applies it in place afterwards.
int do_matmul_fused(holo_backend *be, const SlotTable &st, uint32_t tag, const holo_matmul_call &c,
                    const holo_buffer_ref &residual, uint32_t act) {
    const char *op = tag == HOLO_OP_MATMUL_ACT ? "matmul_activation"
                     : tag == HOLO_OP_MATMUL_ADD ? "matmul_add" : "matmul_add_activation";
    const bool has_res = tag != HOLO_OP_MATMUL_ACT, has_act = tag != HOLO_OP_MATMUL_ADD;
    if (has_act && !holo::fused_act_supported(act, c.dtype, tag == HOLO_OP_MATMUL_ADD_ACT))
        return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": activation " + std::to_string(act) +
                                                 " is not served on the device for this dtype");
    HOLO_TRY(do_matmul(nullptr, st, c));   // the product's own refusals, no device work
    if (c.m == 0 || c.k == 0 || c.n == 0) return HOLO_OK;
    const uint64_t es = dtype_size(c.dtype), count = uint64_t(c.m) * c.n;
    View rv[3], out;
    if (has_res) {
        HOLO_TRY(split_borrow(st, &residual, rv, 1, c.output, &out, op));
        HOLO_TRY(need(rv[0], count * es, residual.slot, op, "residual"));
        if (!aligned(rv[0], es))
            return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": residual must be element-aligned");
    }
    if (!be) return HOLO_OK;
    if (c.dtype == HOLO_DTYPE_F16) {
        // the f16 product into the output, then its epilogue in place
        HOLO_TRY(do_matmul(be, st, c));
        View o;
        HOLO_TRY(split_borrow(st, nullptr, nullptr, 0, c.output, &o, op));
        const uint32_t kind = tag == HOLO_OP_MATMUL_ACT ? 1u : tag == HOLO_OP_MATMUL_ADD ? 2u : 3u;
        return launched(holo::launch_epilogue_f16(reinterpret_cast<uint16_t *>(o.base),
                                                  has_res ? reinterpret_cast<const uint16_t *>(rv[0].base)
                                                          : nullptr,
                                                  count, kind, act, be->stream),
                        op);
    }
    if (c.b_packed) {
        // the packed product into the output, then the epilogue over it in place
        HOLO_TRY(do_matmul(be, st, c));
        View o;
        HOLO_TRY(split_borrow(st, nullptr, nullptr, 0, c.output, &o, op));
        holo::TileEpi te;
        te.kind = tag == HOLO_OP_MATMUL_ACT ? holo::kEpiAct
                  : tag == HOLO_OP_MATMUL_ADD ? holo::kEpiAdd : holo::kEpiAddAct;
        te.act = act;
        te.residual = has_res ? rv[0].base : nullptr;
        return launched(holo::launch_tile_epilogue(o.base, count, false, te, be->stream), op);
    }
    holo::GroupDesc g;
    g.a = c.a;
    g.m = c.m;
    g.k = c.k;
    g.dtype = c.dtype;
    holo::GroupSegDesc s;
    s.b = c.b;
    s.out = c.output;
    s.n = c.n;
    s.base = tag == HOLO_OP_MATMUL_ACT ? holo::kEpiAct
             : tag == HOLO_OP_MATMUL_ADD ? holo::kEpiAdd : holo::kEpiAddAct;
    s.act = act;
    if (has_res) s.residual = residual;
    g.segs.push_back(s);
    return dispatch_group_impl(be, st, g, op);
}

// ------------------------------------------------------- KvCacheWrite ----
// kv_cache_write (src/cpu/kernels.rs:455-501): honest copy + ring rows.
int do_kv_write(holo_backend *be, const SlotTable &st, const holo_kv_cache_write_call &c) {
    const char *op = "kv_cache_write";
    if (c.bucket_rows == 0 || c.row_bytes == 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_cache_write: bucket_rows and row_bytes must be >= 1");
    if (c.new_rows > c.bucket_rows)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_cache_write: new_rows exceeds bucket_rows");
    // output == cache (same slot and offset): the executor's in-place move
    // (session.rs:1313-1370) — only the new rows are written.
    const bool in_place = c.output.slot == c.cache.slot && c.output.offset == c.cache.offset;
    holo_buffer_ref reads[3] = {c.new_rows_buf, c.pos, c.cache};
    View rv3[3], out;
    HOLO_TRY(split_borrow(st, reads, rv3, in_place ? 2 : 3, c.output, &out, op));
    View rv[3] = {in_place ? out : rv3[2], rv3[0], rv3[1]};
    const uint64_t plane = uint64_t(c.bucket_rows) * c.row_bytes;
    const uint64_t total = plane * c.planes;
    if (rv[0].bytes < total || rv[1].bytes < uint64_t(c.planes) * c.new_rows * c.row_bytes ||
        rv[2].bytes < 4 || out.bytes < total)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "kv_cache_write: an operand is shorter than the declared geometry (slot " +
                        std::to_string(c.output.slot) + ")");
    if (!be) return HOLO_OK;
    if (!in_place) HOLO_TRY(launched(holo::launch_copy_bytes(rv[0].base, out.base, total, be->stream), op));
    if (c.planes == 0 || c.new_rows == 0) return HOLO_OK;
    return launched(holo::launch_kv_place_rows(rv[1].base,
                                               reinterpret_cast<const uint32_t *>(rv[2].base),
                                               out.base, c.planes, c.bucket_rows, c.new_rows,
                                               c.row_bytes, be->stream),
                    op);
}

// ------------------------------------------------------ KvQuantAppend ----
int do_kv_quant(holo_backend *be, const SlotTable &st, const holo_kv_quant_append_call &c) {
    const char *op = "kv_quant_append";
    if (c.bucket_rows == 0 || c.head_dim == 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_quant_append: bucket_rows and head_dim must be >= 1");
    if (c.new_rows > c.bucket_rows)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_quant_append: new_rows exceeds bucket_rows");
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_quant_append: new rows must be bf16, f16 or f32");
    if (c.head_dim > 8192)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_quant_append: head_dim above 8192");
    const bool in_place = c.output.slot == c.cache.slot && c.output.offset == c.cache.offset &&
                          c.output_scales.slot == c.cache_scales.slot &&
                          c.output_scales.offset == c.cache_scales.offset;
    const uint64_t qbytes = uint64_t(c.planes) * c.bucket_rows * c.head_dim;
    const uint64_t sbytes = uint64_t(c.planes) * c.bucket_rows * 4;
    const uint64_t nbytes = uint64_t(c.planes) * c.new_rows * c.head_dim * dtype_size(c.dtype);
    View nw, pos, cq, cs, oq, os;
    if (in_place) {
        // The move form: the new rows and pos must not alias the cache.
        holo_buffer_ref reads[2] = {c.new_rows_buf, c.pos};
        View rv[2];
        HOLO_TRY(split_borrow(st, reads, rv, 2, c.output, &oq, op));
        HOLO_TRY(split_borrow(st, reads, rv, 2, c.output_scales, &os, op));
        nw = rv[0];
        pos = rv[1];
        if (overlaps(oq, os))
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, "kv_quant_append: int8 cache overlaps scales");
    } else {
        holo_buffer_ref reads[4] = {c.new_rows_buf, c.pos, c.cache, c.cache_scales};
        View rv[4];
        HOLO_TRY(split_borrow(st, reads, rv, 4, c.output, &oq, op));
        HOLO_TRY(split_borrow(st, reads, rv, 4, c.output_scales, &os, op));
        if (overlaps(oq, os))
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, "kv_quant_append: outputs overlap");
        nw = rv[0];
        pos = rv[1];
        cq = rv[2];
        cs = rv[3];
        HOLO_TRY(need(cq, qbytes, c.cache.slot, op, "cache"));
        HOLO_TRY(need(cs, sbytes, c.cache_scales.slot, op, "cache_scales"));
    }
    HOLO_TRY(need(nw, nbytes, c.new_rows_buf.slot, op, "new rows"));
    HOLO_TRY(need(pos, 4, c.pos.slot, op, "pos"));
    HOLO_TRY(need(oq, qbytes, c.output.slot, op, "output"));
    HOLO_TRY(need(os, sbytes, c.output_scales.slot, op, "output_scales"));
    if (!aligned(os, 4) || !aligned(nw, dtype_size(c.dtype)) || !aligned(pos, 4) ||
        (!in_place && !aligned(cs, 4)))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "kv_quant_append: scales and pos must be 4-byte aligned, new rows "
                    "element-aligned");
    if (uint64_t(c.planes) * c.new_rows > 0xffffffffull / 64)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "kv_quant_append: planes * new_rows too large");
    if (!be) return HOLO_OK;
    if (!in_place && c.planes != 0 &&
        holo::kv_quant_copy_fusable(cq.base, cs.base, oq.base, os.base, c.planes, c.bucket_rows,
                                    c.head_dim))
        return launched(holo::launch_kv_quant_copy_append(
                            nw.base, c.dtype, reinterpret_cast<const uint32_t *>(pos.base),
                            reinterpret_cast<const int8_t *>(cq.base),
                            reinterpret_cast<const float *>(cs.base),
                            reinterpret_cast<int8_t *>(oq.base), reinterpret_cast<float *>(os.base),
                            c.planes, c.bucket_rows, c.new_rows, c.head_dim, be->stream),
                        op);
    if (!in_place) {
        HOLO_TRY(launched(holo::launch_copy_bytes(cq.base, oq.base, qbytes, be->stream), op));
        HOLO_TRY(launched(holo::launch_copy_bytes(cs.base, os.base, sbytes, be->stream), op));
    }
    if (c.planes == 0 || c.new_rows == 0) return HOLO_OK;
    return launched(holo::launch_kv_quant_append(nw.base, c.dtype,
                                                 reinterpret_cast<const uint32_t *>(pos.base),
                                                 reinterpret_cast<int8_t *>(oq.base),
                                                 reinterpret_cast<float *>(os.base), c.planes,
                                                 c.bucket_rows, c.new_rows, c.head_dim, be->stream),
                    op);
}

// ---------------------------------------------------- DecodeAttnI8 -------
// Refusals follow decode_attention_valid_float (src/cpu/float_kernels.rs:4192-4220).
int do_attn_i8(holo_backend *be, const SlotTable &st, const holo_decode_attention_i8_call &c,
               uint32_t q_rows = 1, bool static_scratch = false, const holo::EpiArgs *pro = nullptr,
               bool *pro_done = nullptr) {
    const char *op = "decode_attention_i8";
    if (c.batch == 0 || c.heads == 0 || c.head_dim == 0) return HOLO_OK;
    const uint32_t hkv = c.kv_heads == 0 ? c.heads : c.kv_heads;
    if (c.heads % hkv != 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_i8: heads must be a multiple of kv_heads (grouped-query)");
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "decode_attention_i8: q/output must be bf16 or f32");
    // the MFMA kernels take head_dim 64 / 128 with at most 16 query heads per
    // kv head; every other shape takes the generic blocked kernel
    const bool mfma = holo::attn_i8_supported(c.heads, hkv, c.head_dim, c.bucket_rows);
    if (!mfma && !holo::attn_i8_any_supported(c.batch, c.heads, hkv, q_rows, c.head_dim))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_i8: head_dim must be at most 4096 (within the LDS plan) "
                    "and bucket_rows * head_dim at most 2^30");
    if (uint64_t(c.bucket_rows) * c.head_dim > (uint64_t(1) << 30))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_i8: bucket_rows * head_dim must be at most 2^30");
    const uint64_t es = dtype_size(c.dtype);
    if (q_rows == 0) return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": q_rows must be >= 1");
    const uint64_t qn = uint64_t(c.batch) * q_rows * c.heads * c.head_dim;
    const uint64_t rows = uint64_t(c.batch) * hkv * c.bucket_rows;
    holo_buffer_ref reads[6] = {c.q, c.k_cache, c.v_cache, c.k_scales, c.v_scales, c.lens};
    View rv[6], out;
    HOLO_TRY(split_borrow(st, reads, rv, 6, c.output, &out, op));
    HOLO_TRY(need(rv[0], qn * es, c.q.slot, op, "q"));
    HOLO_TRY(need(rv[1], rows * c.head_dim, c.k_cache.slot, op, "k_cache"));
    HOLO_TRY(need(rv[2], rows * c.head_dim, c.v_cache.slot, op, "v_cache"));
    HOLO_TRY(need(rv[3], rows * 4, c.k_scales.slot, op, "k_scales"));
    HOLO_TRY(need(rv[4], rows * 4, c.v_scales.slot, op, "v_scales"));
    HOLO_TRY(need(rv[5], uint64_t(c.batch) * 4, c.lens.slot, op, "lens"));
    HOLO_TRY(need(out, qn * es, c.output.slot, op, "output"));
    // launch-shape limits of the kernels: grid (chunks, kv_heads, batch)
    if (uint64_t(c.batch) * q_rows > 65535 || hkv > 65535)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    std::string(op) + ": batch * q_rows and kv_heads must be <= 65535");
    // vector loads: 16-byte K/V rows, 4-byte scales/lens, element-aligned q/out
    if (!aligned(rv[1], 16) || !aligned(rv[2], 16) || !aligned(rv[3], 4) || !aligned(rv[4], 4) ||
        !aligned(rv[5], 4) || !aligned(rv[0], es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_i8: caches must be 16-byte aligned, scales/lens 4-byte, "
                    "q/output element-aligned");
    if (!be) return HOLO_OK;
    // score divisor (float_kernels.rs:4256-4266)
    float dflt = std::sqrt(static_cast<float>(c.head_dim));
    if (dflt < 1.0f) dflt = 1.0f;
    float scale = dflt;
    if (c.scale_bits != 0) {
        float sm;
        memcpy(&sm, &c.scale_bits, 4);
        scale = sm > 0.0f ? 1.0f / sm : dflt;
    }
    holo::AttnI8Args a;
    a.q = rv[0].base;
    a.kq = reinterpret_cast<const int8_t *>(rv[1].base);
    a.vq = reinterpret_cast<const int8_t *>(rv[2].base);
    a.ks = reinterpret_cast<const float *>(rv[3].base);
    a.vs = reinterpret_cast<const float *>(rv[4].base);
    a.lens = reinterpret_cast<const uint32_t *>(rv[5].base);
    a.out = out.base;
    a.B = c.batch;
    a.H = c.heads;
    a.Hkv = hkv;
    a.bucket = c.bucket_rows;
    a.D = c.head_dim;
    a.score_scale = scale;
    a.dtype = c.dtype;
    a.q_rows = q_rows;
    if (pro) {
        // the few-row group before this call left its split-K epilogue here:
        // run it in front of the attention in one launch, or on its own first
        *pro_done = true;
        if (mfma && c.bucket_rows != 0 && holo::attn_i8_pro_applies(a, *pro))
            return launched(holo::launch_attn_i8_pro(a, *pro, be->stream), op);
        HOLO_TRY(launched(holo::launch_epilogue(*pro, be->stream), op));
    }
    const size_t scratch_bytes =
        mfma ? holo::attn_i8_scratch_bytes(c.batch, c.heads, hkv, c.bucket_rows, c.head_dim, q_rows)
             : holo::attn_i8_any_scratch_bytes(c.batch, c.heads, hkv, q_rows, c.bucket_rows,
                                               c.head_dim);
    void *scratch = nullptr;
    if (static_scratch) {
        // the allocation-free form: the fixed per-device array, never grown
        if (scratch_bytes > holo::kStaticScratchBytes)
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        std::string(op) + " (no-allocation form): needs " +
                            std::to_string(scratch_bytes) + " bytes of scratch, above the fixed " +
                            std::to_string(holo::kStaticScratchBytes) + "; use holo_hip_dispatch");
        scratch = holo::static_scratch(be->device);
        if (!scratch)
            return fail(HOLO_ERR_INIT, std::string(op) + ": the static scratch has no device address");
    } else {
        HOLO_TRY(ensure_scratch(be, scratch_bytes, op));
        scratch = be->scratch;
    }
    if (c.bucket_rows == 0) {
        // No key can be visible: the pinned zero vector (pinned_semantics.rs).
        return launched(holo::launch_fill_zero(out.base, qn * es, be->stream), op);
    }
    if (q_rows > 1)
        HOLO_TRY(launched(holo::launch_lens_within(a.lens, c.batch, c.bucket_rows, be->dev_err,
                                                   be->stream),
                          op));
    return launched(mfma ? holo::launch_attn_i8(a, scratch, be->stream)
                         : holo::launch_attn_i8_any(a, scratch, be->stream),
                    op);
}

// -------------------------------------------------- DecodeAttentionValid --
// decode_attention_valid_float (src/cpu/float_kernels.rs:4192-4307): refusals
// in the reference's order, then the split-K kernel of attn_valid.hip.
int do_attn_valid(holo_backend *be, const SlotTable &st, const holo_decode_attention_valid_call &c) {
    const char *op = "decode_attention_valid";
    if (c.batch == 0 || c.heads == 0 || c.head_dim == 0) return HOLO_OK;
    if (c.q_rows == 0 || c.q_rows != c.new_len)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_valid: q_rows must equal new_len and be at least 1 "
                    "(the causal law pairs query row i with chunk key row i)");
    const uint32_t hkv = c.kv_heads == 0 ? c.heads : c.kv_heads;
    if (c.heads % hkv != 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_valid: heads must be a multiple of kv_heads (grouped-query)");
    const uint64_t es = dtype_size(c.dtype);
    if (es == 0 || c.dtype == HOLO_DTYPE_I8)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention_valid: only f32/f16/bf16 are supported compute dtypes");
    const uint64_t qn = uint64_t(c.batch) * c.heads * c.q_rows * c.head_dim;
    const uint64_t pn = uint64_t(c.batch) * hkv * c.past_len * c.head_dim;
    const uint64_t nn = uint64_t(c.batch) * hkv * c.new_len * c.head_dim;
    holo_buffer_ref reads[6] = {c.q, c.k_past, c.v_past, c.k_new, c.v_new, c.valid_len};
    View rv[6], out;
    HOLO_TRY(split_borrow(st, reads, rv, 6, c.output, &out, op));
    HOLO_TRY(need(rv[0], qn * es, c.q.slot, op, "q"));
    HOLO_TRY(need(rv[1], pn * es, c.k_past.slot, op, "k_past"));
    HOLO_TRY(need(rv[2], pn * es, c.v_past.slot, op, "v_past"));
    HOLO_TRY(need(rv[3], nn * es, c.k_new.slot, op, "k_new"));
    HOLO_TRY(need(rv[4], nn * es, c.v_new.slot, op, "v_new"));
    HOLO_TRY(need(rv[5], 4, c.valid_len.slot, op, "valid_len"));
    HOLO_TRY(need(out, qn * es, c.output.slot, op, "output"));
    for (int i = 0; i < 5; ++i)
        if (!aligned(rv[i], es))
            return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": operands must be element-aligned");
    if (!aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": operands must be element-aligned");
    if (!holo::attn_valid_supported(c.batch, c.heads, hkv, c.q_rows, c.head_dim))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    std::string(op) + ": head_dim above 4096 or a grid beyond the launch limits");
    if (!be) return HOLO_OK;
    // score divisor (float_kernels.rs:4256-4266)
    float scale = std::sqrt(static_cast<float>(c.head_dim));
    if (scale < 1.0f) scale = 1.0f;
    if (c.scale_bits != 0) {
        float sm;
        memcpy(&sm, &c.scale_bits, 4);
        if (sm > 0.0f) scale = 1.0f / sm;
    }
    HOLO_TRY(ensure_scratch(be, holo::attn_valid_scratch_bytes(c.batch, c.heads, hkv, c.q_rows,
                                                               c.past_len, c.new_len, c.head_dim),
                            op));
    holo::AttnValidArgs a;
    a.q = rv[0].base;
    a.kp = rv[1].base;
    a.vp = rv[2].base;
    a.kn = rv[3].base;
    a.vn = rv[4].base;
    a.valid_len = rv[5].base;
    a.out = out.base;
    a.B = c.batch;
    a.H = c.heads;
    a.Hkv = hkv;
    a.M = c.q_rows;
    a.past = c.past_len;
    a.nnew = c.new_len;
    a.D = c.head_dim;
    a.scale = scale;
    a.dtype = c.dtype;
    return launched(holo::launch_attn_valid(a, be->scratch, be->stream), op);
}

// ----------------------------------------------------- DecodeAttention --
// decode_attention_float (src/cpu/float_kernels.rs:2482-2600), the mask form:
// refusals in the reference's order, then the kernels of attn_valid.hip with
// the mask in place of valid_len.
int do_attn_mask(holo_backend *be, const SlotTable &st, const holo_decode_attention_call &c) {
    const char *op = "decode_attention";
    if (c.batch == 0 || c.heads == 0 || c.q_rows == 0 || c.head_dim == 0) return HOLO_OK;
    const uint64_t L = uint64_t(c.past_len) + c.new_len;
    if (L == 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "decode_attention: past_len + new_len must be at least 1");
    const uint32_t hkv = c.kv_heads == 0 ? c.heads : c.kv_heads;
    if (c.heads % hkv != 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention: heads must be a multiple of kv_heads (grouped-query)");
    const uint64_t es = dtype_size(c.dtype);
    if (es == 0) return fail(HOLO_ERR_UNSUPPORTED_OP, "decode_attention: unknown dtype");
    const uint64_t qn = uint64_t(c.batch) * c.heads * c.q_rows * c.head_dim;
    const uint64_t pn = uint64_t(c.batch) * hkv * c.past_len * c.head_dim;
    const uint64_t nn = uint64_t(c.batch) * hkv * c.new_len * c.head_dim;
    holo_buffer_ref reads[6] = {c.q, c.k_past, c.v_past, c.k_new, c.v_new, c.mask};
    View rv[6], out;
    HOLO_TRY(split_borrow(st, reads, rv, 6, c.output, &out, op));
    HOLO_TRY(need(rv[0], qn * es, c.q.slot, op, "q"));
    HOLO_TRY(need(rv[1], pn * es, c.k_past.slot, op, "k_past"));
    HOLO_TRY(need(rv[2], pn * es, c.v_past.slot, op, "v_past"));
    HOLO_TRY(need(rv[3], nn * es, c.k_new.slot, op, "k_new"));
    HOLO_TRY(need(rv[4], nn * es, c.v_new.slot, op, "v_new"));
    HOLO_TRY(need(rv[5], uint64_t(c.q_rows) * L * 4, c.mask.slot, op, "mask"));   // always f32
    HOLO_TRY(need(out, qn * es, c.output.slot, op, "output"));
    if (c.dtype != HOLO_DTYPE_F32 && c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "decode_attention: only f32/f16/bf16 are supported compute dtypes");
    for (int i = 0; i < 5; ++i)
        if (!aligned(rv[i], es))
            return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": operands must be element-aligned");
    if (!aligned(out, es) || !aligned(rv[5], 4))
        return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": operands must be element-aligned");
    if (L > 0xffffffffull || !holo::attn_valid_supported(c.batch, c.heads, hkv, c.q_rows, c.head_dim))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    std::string(op) + ": head_dim above 4096 or a grid beyond the launch limits");
    if (!be) return HOLO_OK;
    // score divisor (float_kernels.rs:2545-2555)
    float scale = std::sqrt(static_cast<float>(c.head_dim));
    if (scale < 1.0f) scale = 1.0f;
    if (c.scale_bits != 0) {
        float sm;
        memcpy(&sm, &c.scale_bits, 4);
        if (sm > 0.0f) scale = 1.0f / sm;
    }
    HOLO_TRY(ensure_scratch(be, holo::attn_valid_scratch_bytes(c.batch, c.heads, hkv, c.q_rows,
                                                               c.past_len, c.new_len, c.head_dim),
                            op));
    holo::AttnValidArgs a;
    a.q = rv[0].base;
    a.kp = rv[1].base;
    a.vp = rv[2].base;
    a.kn = rv[3].base;
    a.vn = rv[4].base;
    a.valid_len = nullptr;
    a.mask = reinterpret_cast<const float *>(rv[5].base);
    a.out = out.base;
    a.B = c.batch;
    a.H = c.heads;
    a.Hkv = hkv;
    a.M = c.q_rows;
    a.past = c.past_len;
    a.nnew = c.new_len;
    a.D = c.head_dim;
    a.scale = scale;
    a.dtype = c.dtype;
    return launched(holo::launch_attn_valid(a, be->scratch, be->stream), op);
}

// ------------------------------------------------ quantized weights ----
// The level width of a quantized tier (quant_tier.rs:137-178): stored bytes
// of `count` elements, or 0 for a tier this op cannot read.
uint64_t quant_bytes(uint8_t q, uint64_t count) {
    switch (q) {
        case HOLO_DTYPE_I8:
        case HOLO_DTYPE_U8: return count;
        case HOLO_DTYPE_I4: return (count + 1) / 2;
        case HOLO_DTYPE_E8CB: return (count + 7) / 8;
        default: return 0;
    }
}

float f32_of_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// dequantize (src/cpu/kernels.rs:185-296).
int do_dequantize(holo_backend *be, const SlotTable &st, const holo_dequantize_call &c) {
    const char *op = "dequantize";
    const uint64_t n = c.element_count;
    if (c.quant_dtype != HOLO_DTYPE_I8 && c.quant_dtype != HOLO_DTYPE_U8 && c.quant_dtype != HOLO_DTYPE_I4)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "dequantize: quant_dtype must be i8, u8 or i4 (slot " + std::to_string(c.input.slot) + ")");
    const bool per_ch = c.channels > 0 && c.scales.slot != HOLO_SLOT_ABSENT;
    holo_buffer_ref reads[3] = {c.input, c.scales, c.zero_points};
    View rv[3], out;
    HOLO_TRY(split_borrow(st, reads, rv, per_ch ? 3 : 1, c.output, &out, op));
    HOLO_TRY(need(rv[0], quant_bytes(c.quant_dtype, n), c.input.slot, op, "input"));
    uint64_t es = 0;
    if (c.dtype == HOLO_DTYPE_F32) es = 4;
    else if (c.dtype == HOLO_DTYPE_BF16 || c.dtype == HOLO_DTYPE_F16) es = 2;
    else if (c.dtype == 9)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "dequantize: f64 output is not served on the device");
    else
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "dequantize: unknown output dtype (slot " + std::to_string(c.output.slot) + ")");
    HOLO_TRY(need(out, n * es, c.output.slot, op, "output"));
    if (per_ch) {
        HOLO_TRY(need(rv[1], uint64_t(c.channels) * 4, c.scales.slot, op, "scales"));
        HOLO_TRY(need(rv[2], uint64_t(c.channels) * 4, c.zero_points.slot, op, "zero points"));
        if (!aligned(rv[1], 4) || !aligned(rv[2], 4))
            return fail(HOLO_ERR_UNSUPPORTED_OP, "dequantize: scales / zero points must be 4-byte aligned");
    }
    if (!aligned(out, es)) return fail(HOLO_ERR_UNSUPPORTED_OP, "dequantize: output must be element-aligned");
    if (!be || n == 0) return HOLO_OK;
    holo::DequantArgs d;
    d.in = rv[0].base;
    d.scales = per_ch ? reinterpret_cast<const float *>(rv[1].base) : nullptr;
    d.zps = per_ch ? reinterpret_cast<const int32_t *>(rv[2].base) : nullptr;
    d.out = out.base;
    d.n = n;
    d.channels = c.channels;
    d.inner = c.inner ? c.inner : 1;
    d.quant = c.quant_dtype;
    d.dtype = c.dtype;
    d.scale = f32_of_bits(c.scale_bits);
    d.zp = c.zero_point;
    return launched(holo::launch_dequantize(d, be->stream), op);
}

// dequant_activation (src/cpu/kernels.rs:311-388): the table of f((q - zp) as
// f32 * scale) over the quantized domain, built here on the host with the
// reference's scalar f, then one lookup per element; the output is f32.
int do_dequant_act(holo_backend *be, const SlotTable &st, const holo_dequant_activation_call &c) {
    const char *op = "dequant_activation";
    const uint64_t n = c.element_count;
    if (c.quant_dtype != HOLO_DTYPE_I8 && c.quant_dtype != HOLO_DTYPE_U8 && c.quant_dtype != HOLO_DTYPE_I4)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "dequant_activation: quant_dtype must be i8, u8 or i4 (slot " +
                        std::to_string(c.input.slot) + ")");
    View in, out;
    HOLO_TRY(split_borrow(st, &c.input, &in, 1, c.output, &out, op));
    HOLO_TRY(need(in, quant_bytes(c.quant_dtype, n), c.input.slot, op, "input"));
    HOLO_TRY(need(out, n * 4, c.output.slot, op, "output"));
    if (!aligned(out, 4)) return fail(HOLO_ERR_UNSUPPORTED_OP, "dequant_activation: output must be 4-byte aligned");
    float probe;
    if (!holo::lut_act_value(c.act, 0.0f, &probe))
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "dequant_activation: activation " + std::to_string(c.act) + " has no table");
    if (!be || n == 0) return HOLO_OK;
    const float scale = f32_of_bits(c.scale_bits);
    float table[256] = {};
    const bool i4 = c.quant_dtype == HOLO_DTYPE_I4;
    for (int raw = 0; raw < (i4 ? 16 : 256); ++raw) {
        int32_t q = raw;
        if (c.quant_dtype == HOLO_DTYPE_I8) q = int32_t(int8_t(uint8_t(raw)));
        if (i4) q = raw >= 8 ? raw - 16 : raw;
        const int32_t qz = int32_t(uint32_t(q) - uint32_t(c.zero_point));
        holo::lut_act_value(c.act, float(qz) * scale, &table[raw]);
    }
    return launched(holo::launch_dequant_act(in.base, reinterpret_cast<float *>(out.base), n, i4,
                                             table, be->stream),
                    op);
}

// matmul_dequant_float + matmul_dequant_epilogue (src/cpu/float_kernels.rs:459-760).
int do_matmul_dequant(holo_backend *be, const SlotTable &st, const holo_matmul_dequant_call &c) {
    const char *op = "matmul_dequant";
    if (c.m == 0 || c.k == 0 || c.n == 0) return HOLO_OK;
    if (c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: only f32 output is supported");
    const uint64_t kn = uint64_t(c.k) * c.n;
    const uint64_t in_bytes = quant_bytes(c.quant_dtype, kn);
    if (!in_bytes) return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: unknown quantized weight tier");
    const bool needs_cb = c.quant_dtype == HOLO_DTYPE_E8CB;
    const bool has_cb = c.codebook.slot != HOLO_SLOT_ABSENT;
    if (needs_cb != has_cb)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "matmul_dequant: codebook operand missing for a VQ tier (or present without one)");
    const bool per_ch = c.channels > 0 && c.scales.slot != HOLO_SLOT_ABSENT;
    const bool has_res = c.residual.slot != HOLO_SLOT_ABSENT;
    // operands in buffers() order: a, bq[, scales, zero points][, codebook]; the
    // epilogue's residual is its own borrow (float_kernels.rs:727-760)
    holo_buffer_ref reads[5];
    int nr = 0;
    reads[nr++] = c.a;
    reads[nr++] = c.bq;
    if (per_ch) {
        reads[nr++] = c.scales;
        reads[nr++] = c.zero_points;
    }
    const int cb_idx = nr;
    if (has_cb) reads[nr++] = c.codebook;
    View rv[5], out;
    HOLO_TRY(split_borrow(st, reads, rv, nr, c.output, &out, op));
    HOLO_TRY(need(rv[0], uint64_t(c.m) * c.k * 4, c.a.slot, op, "a"));
    HOLO_TRY(need(rv[1], in_bytes, c.bq.slot, op, "bq"));
    HOLO_TRY(need(out, uint64_t(c.m) * c.n * 4, c.output.slot, op, "output"));
    View res;
    if (has_res) {
        HOLO_TRY(split_borrow(st, &c.residual, &res, 1, c.output, &out, op));
        HOLO_TRY(need(res, uint64_t(c.m) * c.n * 4, c.residual.slot, op, "residual"));
    }
    // an id past the table is the identity (float_kernels.rs:767-781)
    const uint32_t act = c.act <= holo::kFusedExp ? c.act : 0;
    if (!aligned(rv[0], 4) || !aligned(out, 4) || (has_res && !aligned(res, 4)))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: f32 operands must be 4-byte aligned");
    const bool omajor = c.bq_omajor != 0, w8a8 = c.act_quant == 1;
    if (omajor || w8a8) {
        if (!(omajor && w8a8))
            return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: bq_omajor and W8A8 must be paired");
        // symmetric per-channel i8 / i4 / e8cb within the exact-i32 k bound;
        // the zero points' values are checked on the device
        const bool tier_ok = c.quant_dtype == HOLO_DTYPE_I8 ||
                             (c.quant_dtype == HOLO_DTYPE_I4 && c.k % 2 == 0) ||
                             (c.quant_dtype == HOLO_DTYPE_E8CB && c.k % 8 == 0);
        if (!(per_ch && tier_ok && c.channels == c.n && c.inner == 1) || c.k > holo::kI8DotKMax)
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "matmul_dequant: W8A8 requires symmetric per-channel i8/i4/e8cb within the k bound");
        // every whole i32 of the zero-point view must be zero (the symmetry
        // test reads the view, not n entries of it)
        HOLO_TRY(need(rv[2], uint64_t(c.n) * 4, c.scales.slot, op, "scales"));
        if (has_cb) HOLO_TRY(need(rv[cb_idx], 256 * 8, c.codebook.slot, op, "codebook"));
        if (!aligned(rv[2], 4))
            return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: scales must be 4-byte aligned");
        if ((uint64_t(c.n) + 15) / 16 > 0x7fffffffull || (uint64_t(c.m) + 63) / 64 > 65535)
            return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: grid beyond the launch limits");
        if (!be) return HOLO_OK;
        HOLO_TRY(launched(holo::launch_zero_points_check(rv[3].base, rv[3].bytes / 4, be->dev_err,
                                                         be->stream),
                          op));
        HOLO_TRY(ensure_scratch(be, holo::q_omajor_scratch_bytes(c.m, c.k), op));
        holo::QOmajorArgs a;
        a.a = reinterpret_cast<const float *>(rv[0].base);
        a.bq = rv[1].base;
        a.codebook = has_cb ? reinterpret_cast<const int8_t *>(rv[cb_idx].base) : nullptr;
        a.scales = reinterpret_cast<const float *>(rv[2].base);
        a.residual = has_res ? reinterpret_cast<const float *>(res.base) : nullptr;
        a.out = reinterpret_cast<float *>(out.base);
        a.m = c.m;
        a.k = c.k;
        a.n = c.n;
        a.tier = c.quant_dtype;
        a.act = act;
        return launched(holo::launch_matmul_q_omajor(a, be->scratch, be->stream), op);
    }
    // W8A32: the [k, n] weight dequantized to an f32 panel, the f32 product,
    // then the epilogue in place
    if (c.quant_dtype == HOLO_DTYPE_E8CB)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "matmul_dequant: quant_dtype is not scalar-decodable (e8cb needs the fused omajor path)");
    if (per_ch) {
        HOLO_TRY(need(rv[2], uint64_t(c.channels) * 4, c.scales.slot, op, "scales"));
        HOLO_TRY(need(rv[3], uint64_t(c.channels) * 4, c.zero_points.slot, op, "zero points"));
        if (!aligned(rv[2], 4) || !aligned(rv[3], 4))
            return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: scales / zero points must be 4-byte aligned");
    }
    if ((uint64_t(c.m) + 127) / 128 > 65535)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "matmul_dequant: m above 8388480");
    if (!be) return HOLO_OK;
    const uint64_t panel = (kn * 4 + 255) / 256 * 256;
    HOLO_TRY(ensure_scratch(be, panel + holo::matmul_scratch_bytes(c.m, c.k, c.n, HOLO_DTYPE_F32), op));
    holo::DequantArgs d;
    d.in = rv[1].base;
    d.scales = per_ch ? reinterpret_cast<const float *>(rv[2].base) : nullptr;
    d.zps = per_ch ? reinterpret_cast<const int32_t *>(rv[3].base) : nullptr;
    d.out = be->scratch;
    d.n = kn;
    d.channels = c.channels;
    d.inner = c.inner ? c.inner : 1;
    d.quant = c.quant_dtype;
    d.dtype = HOLO_DTYPE_F32;
    d.scale = f32_of_bits(c.scale_bits);
    d.zp = c.zero_point;
    HOLO_TRY(launched(holo::launch_dequantize(d, be->stream), op));
    HOLO_TRY(launched(holo::launch_matmul(rv[0].base, be->scratch, out.base, c.m, c.k, c.n,
                                          HOLO_DTYPE_F32, static_cast<uint8_t *>(be->scratch) + panel,
                                          be->stream),
                      op));
    if (act == 0 && !has_res) return HOLO_OK;
    holo::TileEpi te;
    te.kind = has_res ? (act ? holo::kEpiAddAct : holo::kEpiAdd) : holo::kEpiAct;
    te.act = act;
    te.residual = has_res ? res.base : nullptr;
    return launched(holo::launch_tile_epilogue(out.base, uint64_t(c.m) * c.n, false, te, be->stream), op);
}

// ------------------------------------------------------- Add / Mul -----
// binary_float (src/cpu/float_kernels.rs:238-300).
int do_binary(holo_backend *be, const SlotTable &st, uint32_t tag, const holo_binary_call &c) {
    const char *op = tag == HOLO_OP_ADD ? "add" : "mul";
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    std::string(op) + ": the device path serves f16, bf16 and f32");
    if (c.element_count == 0) return HOLO_OK;
    const uint64_t es = dtype_size(c.dtype), bytes = c.element_count * es;
    holo_buffer_ref reads[2] = {c.a, c.b};
    View rv[2], out;
    HOLO_TRY(split_borrow(st, reads, rv, 2, c.output, &out, op));
    HOLO_TRY(need(rv[0], bytes, c.a.slot, op, "a"));
    HOLO_TRY(need(rv[1], bytes, c.b.slot, op, "b"));
    HOLO_TRY(need(out, bytes, c.output.slot, op, "output"));
    if (!aligned(rv[0], es) || !aligned(rv[1], es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, std::string(op) + ": operands must be element-aligned");
    if (!be) return HOLO_OK;
    return launched(holo::launch_binary(tag == HOLO_OP_ADD ? 0 : 1, rv[0].base, rv[1].base, out.base,
                                        c.element_count, c.dtype, be->stream),
                    op);
}

// ------------------------------------------------------------ RmsNorm ----
// rms_norm_float (src/cpu/float_kernels.rs:1683-1755); epsilon rule :1324-1336.
int do_rmsnorm(holo_backend *be, const SlotTable &st, const holo_norm_call &c) {
    const char *op = "rms_norm";
    if (c.batch == 0 || c.feature == 0) return HOLO_OK;
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "rms_norm: the device path serves f16, bf16 and f32");
    if (c.residual.slot != HOLO_SLOT_ABSENT || c.channels != 0 || c.num_groups != 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "rms_norm: residual / grouped forms are not served by the device path");
    float eps = 1e-9f;
    if (c.epsilon_bits != 0) {
        const uint32_t eb = uint32_t(c.epsilon_bits);
        memcpy(&eps, &eb, 4);
        if (!(std::isfinite(eps) && eps > 0.0f))
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "norm epsilon must be a positive finite f32 (0 selects the default)");
    }
    const uint64_t es = dtype_size(c.dtype), total = uint64_t(c.batch) * c.feature * es;
    const bool has_g = c.gamma.slot != HOLO_SLOT_ABSENT;
    holo_buffer_ref reads[2] = {c.x, c.gamma};
    View rv[2], out;
    HOLO_TRY(split_borrow(st, reads, rv, has_g ? 2 : 1, c.output, &out, op));
    HOLO_TRY(need(rv[0], total, c.x.slot, op, "x"));
    HOLO_TRY(need(out, total, c.output.slot, op, "output"));
    // affine_operand (float_kernels.rs:39-44): an empty gamma is the identity
    const bool use_g = has_g && rv[1].bytes > 0;
    if (use_g) HOLO_TRY(need(rv[1], uint64_t(c.feature) * es, c.gamma.slot, op, "gamma"));
    if (!aligned(rv[0], es) || !aligned(out, es) || (use_g && !aligned(rv[1], es)))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "rms_norm: operands must be element-aligned");
    if (c.batch > 0x7fffffffu) return fail(HOLO_ERR_UNSUPPORTED_OP, "rms_norm: batch too large");
    if (!be) return HOLO_OK;
    return launched(holo::launch_rmsnorm(rv[0].base, use_g ? rv[1].base : nullptr, out.base, c.batch,
                                         c.feature, eps, c.dtype, be->stream),
                    op);
}

// add_rms_norm_float (src/cpu/float_kernels.rs:1566-1672): reads x, the
// residual when present, gamma; channels / groups / beta are not used.
int do_add_rmsnorm(holo_backend *be, const SlotTable &st, const holo_norm_call &c) {
    const char *op = "add_rms_norm";
    if (c.batch == 0 || c.feature == 0) return HOLO_OK;
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "add_rms_norm: the device path serves f16, bf16 and f32");
    float eps = 1e-9f;
    if (c.epsilon_bits != 0) {
        const uint32_t eb = uint32_t(c.epsilon_bits);
        memcpy(&eps, &eb, 4);
        if (!(std::isfinite(eps) && eps > 0.0f))
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "norm epsilon must be a positive finite f32 (0 selects the default)");
    }
    const uint64_t es = dtype_size(c.dtype), total = uint64_t(c.batch) * c.feature * es;
    const bool has_r = c.residual.slot != HOLO_SLOT_ABSENT, has_g = c.gamma.slot != HOLO_SLOT_ABSENT;
    holo_buffer_ref reads[3];
    int nr = 0;
    reads[nr++] = c.x;
    if (has_r) reads[nr++] = c.residual;
    const int gi = nr;
    if (has_g) reads[nr++] = c.gamma;
    View rv[3], out;
    HOLO_TRY(split_borrow(st, reads, rv, nr, c.output, &out, op));
    HOLO_TRY(need(rv[0], total, c.x.slot, op, "x"));
    if (has_r) HOLO_TRY(need(rv[1], total, c.residual.slot, op, "residual"));
    HOLO_TRY(need(out, total, c.output.slot, op, "output"));
    // affine_operand (float_kernels.rs:39-44): an empty gamma is the identity
    const bool use_g = has_g && rv[gi].bytes > 0;
    if (use_g) HOLO_TRY(need(rv[gi], uint64_t(c.feature) * es, c.gamma.slot, op, "gamma"));
    if (!aligned(rv[0], es) || !aligned(out, es) || (has_r && !aligned(rv[1], es)) ||
        (use_g && !aligned(rv[gi], es)))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "add_rms_norm: operands must be element-aligned");
    if (c.batch > 0x7fffffffu) return fail(HOLO_ERR_UNSUPPORTED_OP, "add_rms_norm: batch too large");
    if (!be) return HOLO_OK;
    return launched(holo::launch_add_rmsnorm(rv[0].base, has_r ? rv[1].base : nullptr,
                                             use_g ? rv[gi].base : nullptr, out.base, c.batch,
                                             c.feature, eps, c.dtype, be->stream),
                    op);
}

// -------------------------------------------------------------- RoPE -----
// rope_float (src/cpu/float_kernels.rs:3123-3186).
int do_rope(holo_backend *be, const SlotTable &st, const holo_rope_call &c) {
    const char *op = "rope";
    if (c.head_dim == 0 || c.head_dim % 2 != 0 || c.element_count % c.head_dim != 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "rope: head_dim must be even and divide the element count");
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "rope: the device path serves f16, bf16 and f32");
    if (c.element_count == 0) return HOLO_OK;
    const uint64_t es = dtype_size(c.dtype), bytes = c.element_count * es;
    holo_buffer_ref reads[3] = {c.x, c.cos, c.sin};
    View rv[3], out;
    HOLO_TRY(split_borrow(st, reads, rv, 3, c.output, &out, op));
    HOLO_TRY(need(rv[0], bytes, c.x.slot, op, "x"));
    HOLO_TRY(need(rv[1], bytes, c.cos.slot, op, "cos"));
    HOLO_TRY(need(rv[2], bytes, c.sin.slot, op, "sin"));
    HOLO_TRY(need(out, bytes, c.output.slot, op, "output"));
    if (!aligned(rv[0], es) || !aligned(rv[1], es) || !aligned(rv[2], es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "rope: operands must be element-aligned");
    if (!be) return HOLO_OK;
    return launched(holo::launch_rope(rv[0].base, rv[1].base, rv[2].base, out.base, c.head_dim,
                                      c.element_count, c.dtype, be->stream),
                    op);
}

// ------------------------------------------------------------ Gather -----
// gather (src/cpu/kernels.rs:389-447): rows copied byte for byte.
int do_gather(holo_backend *be, const SlotTable &st, const holo_gather_call &c) {
    const char *op = "gather";
    const uint64_t elem = c.dtype == HOLO_DTYPE_I32 ? 4 : c.dtype == HOLO_DTYPE_I64 ? 8
                        : c.dtype == 1 || c.dtype == HOLO_DTYPE_I8 ? 1 : dtype_size(c.dtype);
    if (elem == 0)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "gather: sub-byte or unknown element dtype not supported");
    uint64_t idx_w;
    if (c.idx_dtype == HOLO_DTYPE_I32)
        idx_w = 4;
    else if (c.idx_dtype == HOLO_DTYPE_I64)
        idx_w = 8;
    else
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "gather: index dtype must be i32 or i64 (slot " + std::to_string(c.indices.slot) + ")");
    const uint64_t row = c.inner * elem;
    holo_buffer_ref reads[2] = {c.data, c.indices};
    View rv[2], out;
    HOLO_TRY(split_borrow(st, reads, rv, 2, c.output, &out, op));
    if (rv[0].bytes < c.outer * c.axis_dim * row || rv[1].bytes < c.num_indices * idx_w ||
        out.bytes < c.outer * c.num_indices * row)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "gather: an operand is shorter than the declared geometry (slot " +
                        std::to_string(c.output.slot) + ")");
    if (!aligned(rv[1], idx_w)) return fail(HOLO_ERR_UNSUPPORTED_OP, "gather: indices must be aligned");
    if (c.outer == 0 || c.num_indices == 0 || row == 0) return HOLO_OK;
    if (c.outer > 65535 || c.num_indices > 0x7fffffffull)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "gather: outer above 65535 or too many indices");
    if (!be) return HOLO_OK;
    return launched(holo::launch_gather(rv[0].base, rv[1].base, out.base, c.outer, c.axis_dim,
                                        c.num_indices, row, c.idx_dtype == HOLO_DTYPE_I64,
                                        be->dev_err, be->stream),
                    op);
}

// --------------------------------------------------------- Transpose -----
// transpose_float (src/cpu/float_kernels.rs:2980-3028).
int do_transpose(holo_backend *be, const SlotTable &st, const holo_transpose_call &c) {
    const char *op = "transpose";
    if (c.rank == 0 || c.rank > 8)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "transpose: rank must be 1..=8");
    if (c.dtype != HOLO_DTYPE_F16 && c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "transpose: the device path serves f16, bf16 and f32");
    uint32_t seen = 0;
    for (uint32_t i = 0; i < c.rank; ++i) {
        if (c.perm[i] >= c.rank || (seen >> c.perm[i]) & 1u)
            return fail(HOLO_ERR_UNSUPPORTED_OP, "transpose: perm must be a permutation of 0..rank");
        seen |= 1u << c.perm[i];
    }
    const uint64_t es = dtype_size(c.dtype);
    uint64_t total = 1;
    for (uint32_t i = 0; i < c.rank; ++i) total *= c.dims[i];
    View in, out;
    HOLO_TRY(split_borrow(st, &c.input, &in, 1, c.output, &out, op));
    if (in.bytes < total * es || out.bytes < total * es)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                    "transpose: an operand is shorter than the tensor (slot " +
                        std::to_string(c.output.slot) + ")");
    if (!aligned(in, es) || !aligned(out, es))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "transpose: operands must be element-aligned");
    if (!be || total == 0) return HOLO_OK;
    return launched(holo::launch_transpose(in.base, out.base, c.rank, c.dims, c.perm, uint32_t(es),
                                           be->stream),
                    op);
}

// ---------------------------------------------------- Reshape / Slice ----
// layout_float (src/cpu/float_kernels.rs:2939-2954) for f16/bf16/f32: the
// first element_count elements; layout_copy (src/cpu/kernels.rs:688-701) for
// every other dtype: the first element_count bytes (the byte domain). f64 is
// refused as try_dispatch_float refuses it (kernels.rs:1611-1615). A session
// runs this only for a Reshape or Slice that writes an output port; an
// interior one is bound as a view of its input.
int do_layout(holo_backend *be, const SlotTable &st, uint32_t tag, const holo_layout_call &c) {
    const char *op = tag == HOLO_OP_RESHAPE ? "reshape" : "slice";
    if (c.dtype == HOLO_DTYPE_F64)
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "f64 is not a supported compute dtype (hologram computes in f16/bf16/f32)");
    const bool flt = c.dtype == HOLO_DTYPE_F16 || c.dtype == HOLO_DTYPE_BF16 ||
                     c.dtype == HOLO_DTYPE_F32;
    const uint64_t es = flt ? dtype_size(c.dtype) : 1;
    if (c.element_count > UINT64_MAX / es)
        return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, std::string(op) + ": element_count overflows");
    const uint64_t bytes = c.element_count * es;
    View in, out;
    HOLO_TRY(split_borrow(st, &c.input, &in, 1, c.output, &out, op));
    HOLO_TRY(need(in, bytes, c.input.slot, op, "input"));
    HOLO_TRY(need(out, bytes, c.output.slot, op, "output"));
    if (!be || bytes == 0) return HOLO_OK;
    return launched(holo::launch_copy_bytes(in.base, out.base, bytes, be->stream), op);
}

// ------------------------------------------------------------ ArgMax -----
int do_argmax(holo_backend *be, const SlotTable &st, const holo_argmax_call &c) {
    const char *op = "argmax";
    if (c.dtype != HOLO_DTYPE_BF16 && c.dtype != HOLO_DTYPE_F32)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "argmax: input must be bf16 or f32");
    if (c.rows == 0) return HOLO_OK;
    const uint64_t es = dtype_size(c.dtype);
    View in, out;
    HOLO_TRY(split_borrow(st, &c.input, &in, 1, c.output, &out, op));
    HOLO_TRY(need(in, uint64_t(c.rows) * c.cols * es, c.input.slot, op, "input"));
    HOLO_TRY(need(out, uint64_t(c.rows) * 4, c.output.slot, op, "output"));
    if (!aligned(in, es) || !aligned(out, 4))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "argmax: operands must be element-aligned");
    if (c.rows > 0x7fffffffu) return fail(HOLO_ERR_UNSUPPORTED_OP, "argmax: too many rows");
    if (!be) return HOLO_OK;
    return launched(holo::launch_argmax(in.base, reinterpret_cast<int32_t *>(out.base), c.rows,
                                        c.cols, c.dtype == HOLO_DTYPE_BF16, be->stream),
                    op);
}

int dispatch_impl(holo_backend *be, const SlotTable &st, const holo_kernel_call *call) {
    if (!call) return fail(HOLO_ERR_DISPATCH, "dispatch: null call");
    switch (call->tag) {
        case HOLO_OP_SIGMOID:
        case HOLO_OP_TANH:
        case HOLO_OP_GELU:
        case HOLO_OP_SILU:
        case HOLO_OP_EXP:
        case HOLO_OP_RELU:
        case HOLO_OP_ELU:
        case HOLO_OP_SELU:
        case HOLO_OP_ERF: return do_unary(be, st, call->tag, call->u.unary);
        case HOLO_OP_DEQUANTIZE: return do_dequantize(be, st, call->u.dequantize);
        case HOLO_OP_DEQUANT_ACT: return do_dequant_act(be, st, call->u.dequant_act);
        case HOLO_OP_MATMUL_DEQUANT: return do_matmul_dequant(be, st, call->u.matmul_dequant);
        case HOLO_OP_ADD:
        case HOLO_OP_MUL: return do_binary(be, st, call->tag, call->u.binary);
        case HOLO_OP_RMS_NORM: return do_rmsnorm(be, st, call->u.norm);
        case HOLO_OP_ADD_RMS_NORM: return do_add_rmsnorm(be, st, call->u.norm);
        case HOLO_OP_ROTARY: return do_rope(be, st, call->u.rope);
        case HOLO_OP_GATHER: return do_gather(be, st, call->u.gather);
        case HOLO_OP_ARGMAX: return do_argmax(be, st, call->u.argmax);
        case HOLO_OP_MATMUL: return do_matmul(be, st, call->u.matmul);
        case HOLO_OP_MATMUL_ACT:
            return do_matmul_fused(be, st, call->tag, call->u.matmul_act.mm, holo_buffer_ref{},
                                   call->u.matmul_act.act);
        case HOLO_OP_MATMUL_ADD:
            return do_matmul_fused(be, st, call->tag, call->u.matmul_add.mm,
                                   call->u.matmul_add.residual, 0);
        case HOLO_OP_MATMUL_ADD_ACT:
            return do_matmul_fused(be, st, call->tag, call->u.matmul_add_act.mm,
                                   call->u.matmul_add_act.residual, call->u.matmul_add_act.act);
        case HOLO_OP_KV_CACHE_WRITE: return do_kv_write(be, st, call->u.kv_write);
        case HOLO_OP_KV_QUANT_APPEND: return do_kv_quant(be, st, call->u.kv_quant_append);
        case HOLO_OP_DECODE_ATTN_VALID: return do_attn_valid(be, st, call->u.attn_valid);
        case HOLO_OP_DECODE_ATTN: return do_attn_mask(be, st, call->u.attn_mask);
        case HOLO_OP_DECODE_ATTN_I8: return do_attn_i8(be, st, call->u.attn_i8);
        case HOLO_OP_ATTN_I8_ROWS:
            return do_attn_i8(be, st, call->u.attn_i8_rows.attn, call->u.attn_i8_rows.q_rows);
        case HOLO_OP_TRANSPOSE: return do_transpose(be, st, call->u.transpose);
        case HOLO_OP_RESHAPE:
        case HOLO_OP_SLICE: return do_layout(be, st, call->tag, call->u.layout);
        default:
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "dispatch: kernel call tag " + std::to_string(call->tag) +
                            " has no device kernel in this backend");
    }
}

// -------------------------------------------------------- wire codec ----
// crates/hologram-archive/src/kernel_codec.rs:557-813 (LE fields).
struct Reader {
    const uint8_t *p;
    size_t len, at = 0;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (at + sizeof(T) > len) {
            ok = false;
            return v;
        }
        memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    holo_buffer_ref buf() {
        holo_buffer_ref b;
        memset(&b, 0, sizeof b);   // padding too: decoded calls compare byte for byte
        b.slot = get<uint32_t>();
        b.offset = get<uint64_t>();
        b.length = get<uint64_t>();
        return b;
    }
};

int decode_impl(const uint8_t *wire, size_t len, holo_kernel_call *out, size_t *consumed) {
    if (!wire || !out) return fail(HOLO_ERR_DISPATCH, "decode_call: null argument");
    Reader r{wire, len};
    memset(out, 0, sizeof(*out));
    out->tag = r.get<uint16_t>();
    switch (out->tag) {
        case HOLO_OP_SIGMOID:
        case HOLO_OP_TANH:
        case HOLO_OP_GELU:
        case HOLO_OP_SILU:
        case HOLO_OP_EXP:
        case HOLO_OP_RELU:
        case HOLO_OP_ELU:
        case HOLO_OP_SELU:
        case HOLO_OP_ERF: {  // put_unary :575-581
            auto &c = out->u.unary;
            c.input = r.buf();
            c.output = r.buf();
            c.element_count = r.get<uint64_t>();
            c.witt_bits = r.get<uint16_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_DEQUANTIZE:
        case 118: {  // put_dequantize :861-872; 118 adds layout, act quant, codebook (decoder.rs:166-176)
            auto &c = out->u.dequantize;
            c.input = r.buf();
            c.scales = r.buf();
            c.zero_points = r.buf();
            c.output = r.buf();
            c.element_count = r.get<uint64_t>();
            c.channels = r.get<uint32_t>();
            c.inner = r.get<uint32_t>();
            c.quant_dtype = r.get<uint8_t>();
            c.dtype = r.get<uint8_t>();
            c.scale_bits = r.get<uint32_t>();
            c.zero_point = int32_t(r.get<uint32_t>());
            c.codebook.slot = HOLO_SLOT_ABSENT;
            if (out->tag == 118) {
                c.weight_layout = r.get<uint8_t>();
                c.act_quant = r.get<uint8_t>();
                c.codebook = r.buf();
            }
            out->tag = HOLO_OP_DEQUANTIZE;
            break;
        }
        case HOLO_OP_MATMUL_DEQUANT:
        case 116:
        case 117: {  // put_matmul_dequant :835-850, then the 116 / 117 tails (decoder.rs:190-212)
            auto &c = out->u.matmul_dequant;
            c.a = r.buf();
            c.bq = r.buf();
            c.scales = r.buf();
            c.zero_points = r.buf();
            c.output = r.buf();
            c.m = r.get<uint32_t>();
            c.k = r.get<uint32_t>();
            c.n = r.get<uint32_t>();
            c.channels = r.get<uint32_t>();
            c.inner = r.get<uint32_t>();
            c.quant_dtype = r.get<uint8_t>();
            c.dtype = r.get<uint8_t>();
            c.scale_bits = r.get<uint32_t>();
            c.zero_point = int32_t(r.get<uint32_t>());
            c.residual.slot = HOLO_SLOT_ABSENT;
            c.codebook.slot = HOLO_SLOT_ABSENT;
            if (out->tag != HOLO_OP_MATMUL_DEQUANT) {
                c.bq_omajor = r.get<uint8_t>() != 0;
                c.act_quant = r.get<uint8_t>();
                c.act = r.get<uint8_t>();
                c.residual = r.buf();
                if (out->tag == 117) c.codebook = r.buf();
            }
            out->tag = HOLO_OP_MATMUL_DEQUANT;
            break;
        }
        case HOLO_OP_DEQUANT_ACT: {  // put_dequant_activation :851-860
            auto &c = out->u.dequant_act;
            c.input = r.buf();
            c.output = r.buf();
            c.element_count = r.get<uint64_t>();
            c.quant_dtype = r.get<uint8_t>();
            c.act = r.get<uint8_t>();
            c.dtype = r.get<uint8_t>();
            c.scale_bits = r.get<uint32_t>();
            c.zero_point = int32_t(r.get<uint32_t>());
            break;
        }
        case HOLO_OP_ADD:
        case HOLO_OP_MUL: {  // put_binary :582-589
            auto &c = out->u.binary;
            c.a = r.buf();
            c.b = r.buf();
            c.output = r.buf();
            c.element_count = r.get<uint64_t>();
            c.witt_bits = r.get<uint16_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_RMS_NORM:
        case HOLO_OP_ADD_RMS_NORM: {  // put_norm :656-668
            auto &c = out->u.norm;
            c.x = r.buf();
            c.gamma = r.buf();
            c.beta = r.buf();
            c.residual = r.buf();
            c.output = r.buf();
            c.batch = r.get<uint32_t>();
            c.feature = r.get<uint32_t>();
            c.channels = r.get<uint32_t>();
            c.num_groups = r.get<uint32_t>();
            c.epsilon_bits = r.get<uint64_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_ROTARY: {  // put_rope :711-719
            auto &c = out->u.rope;
            c.x = r.buf();
            c.cos = r.buf();
            c.sin = r.buf();
            c.output = r.buf();
            c.head_dim = r.get<uint32_t>();
            c.element_count = r.get<uint64_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_GATHER: {  // put_gather :626-636
            auto &c = out->u.gather;
            c.data = r.buf();
            c.indices = r.buf();
            c.output = r.buf();
            c.outer = r.get<uint64_t>();
            c.axis_dim = r.get<uint64_t>();
            c.inner = r.get<uint64_t>();
            c.num_indices = r.get<uint64_t>();
            c.idx_dtype = r.get<uint8_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_ARGMAX: {  // field order of holo_argmax_call
            auto &c = out->u.argmax;
            c.input = r.buf();
            c.output = r.buf();
            c.rows = r.get<uint32_t>();
            c.cols = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_MATMUL: {  // put_matmul :590-599
            auto &c = out->u.matmul;
            c.a = r.buf();
            c.b = r.buf();
            c.output = r.buf();
            c.m = r.get<uint32_t>();
            c.k = r.get<uint32_t>();
            c.n = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            c.b_packed = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_MATMUL_ACT:
        case HOLO_OP_MATMUL_ADD:
        case HOLO_OP_MATMUL_ADD_ACT: {  // :509-524: put_matmul, then residual and/or act
            holo_matmul_call mm;
            mm.a = r.buf();
            mm.b = r.buf();
            mm.output = r.buf();
            mm.m = r.get<uint32_t>();
            mm.k = r.get<uint32_t>();
            mm.n = r.get<uint32_t>();
            mm.dtype = r.get<uint8_t>();
            mm.b_packed = r.get<uint8_t>();
            if (out->tag == HOLO_OP_MATMUL_ACT) {
                out->u.matmul_act.mm = mm;
                out->u.matmul_act.act = r.get<uint8_t>();
            } else if (out->tag == HOLO_OP_MATMUL_ADD) {
                out->u.matmul_add.mm = mm;
                out->u.matmul_add.residual = r.buf();
            } else {
                out->u.matmul_add_act.mm = mm;
                out->u.matmul_add_act.residual = r.buf();
                out->u.matmul_add_act.act = r.get<uint8_t>();
            }
            break;
        }
        case HOLO_OP_KV_CACHE_WRITE: {  // put_kvwr :804-813
            auto &c = out->u.kv_write;
            c.cache = r.buf();
            c.new_rows_buf = r.buf();
            c.pos = r.buf();
            c.output = r.buf();
            c.planes = r.get<uint32_t>();
            c.bucket_rows = r.get<uint32_t>();
            c.new_rows = r.get<uint32_t>();
            c.row_bytes = r.get<uint32_t>();
            break;
        }
        case HOLO_OP_KV_QUANT_APPEND: {  // field order of holo_kv_quant_append_call
            auto &c = out->u.kv_quant_append;
            c.new_rows_buf = r.buf();
            c.pos = r.buf();
            c.cache = r.buf();
            c.cache_scales = r.buf();
            c.output = r.buf();
            c.output_scales = r.buf();
            c.planes = r.get<uint32_t>();
            c.bucket_rows = r.get<uint32_t>();
            c.new_rows = r.get<uint32_t>();
            c.head_dim = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_DECODE_ATTN: {  // put_decattn :768-785 (put_davl's order, mask for valid_len)
            auto &c = out->u.attn_mask;
            c.q = r.buf();
            c.k_past = r.buf();
            c.v_past = r.buf();
            c.k_new = r.buf();
            c.v_new = r.buf();
            c.mask = r.buf();
            c.output = r.buf();
            c.batch = r.get<uint32_t>();
            c.heads = r.get<uint32_t>();
            c.kv_heads = r.get<uint32_t>();
            c.q_rows = r.get<uint32_t>();
            c.past_len = r.get<uint32_t>();
            c.new_len = r.get<uint32_t>();
            c.head_dim = r.get<uint32_t>();
            c.scale_bits = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_DECODE_ATTN_VALID: {  // put_davl :786-803
            auto &c = out->u.attn_valid;
            c.q = r.buf();
            c.k_past = r.buf();
            c.v_past = r.buf();
            c.k_new = r.buf();
            c.v_new = r.buf();
            c.valid_len = r.buf();
            c.output = r.buf();
            c.batch = r.get<uint32_t>();
            c.heads = r.get<uint32_t>();
            c.kv_heads = r.get<uint32_t>();
            c.q_rows = r.get<uint32_t>();
            c.past_len = r.get<uint32_t>();
            c.new_len = r.get<uint32_t>();
            c.head_dim = r.get<uint32_t>();
            c.scale_bits = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_DECODE_ATTN_I8:
        case HOLO_OP_ATTN_I8_ROWS: {  // field order of holo_decode_attention_i8_call (+ q_rows)
            auto &c = out->tag == HOLO_OP_ATTN_I8_ROWS ? out->u.attn_i8_rows.attn : out->u.attn_i8;
            c.q = r.buf();
            c.k_cache = r.buf();
            c.v_cache = r.buf();
            c.k_scales = r.buf();
            c.v_scales = r.buf();
            c.lens = r.buf();
            c.output = r.buf();
            c.batch = r.get<uint32_t>();
            c.heads = r.get<uint32_t>();
            c.kv_heads = r.get<uint32_t>();
            c.bucket_rows = r.get<uint32_t>();
            c.head_dim = r.get<uint32_t>();
            c.scale_bits = r.get<uint32_t>();
            c.dtype = r.get<uint8_t>();
            if (out->tag == HOLO_OP_ATTN_I8_ROWS) out->u.attn_i8_rows.q_rows = r.get<uint32_t>();
            break;
        }
        case HOLO_OP_RESHAPE:
        case HOLO_OP_SLICE: {  // put_layout :681-686
            auto &c = out->u.layout;
            c.input = r.buf();
            c.output = r.buf();
            c.element_count = r.get<uint64_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        case HOLO_OP_TRANSPOSE: {  // put_transpose :687-697
            auto &c = out->u.transpose;
            c.input = r.buf();
            c.output = r.buf();
            c.rank = r.get<uint8_t>();
            for (auto &d : c.dims) d = r.get<uint32_t>();
            for (auto &p : c.perm) p = r.get<uint8_t>();
            c.dtype = r.get<uint8_t>();
            break;
        }
        default:
            if (!r.ok) return fail(HOLO_ERR_DISPATCH, "decode_call: truncated discriminant");
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "decode_call: discriminant " + std::to_string(out->tag) +
                            " has no device kernel in this backend");
    }
    if (!r.ok) return fail(HOLO_ERR_DISPATCH, "decode_call: truncated payload");
    if (consumed) *consumed = r.at;
    return HOLO_OK;
}

}  // namespace

namespace holo {

int set_error(int code, const std::string &msg) { return fail(code, msg); }

int dispatch_with_slots(holo_backend *be, const std::vector<SlotRange> &slots,
                        const holo_kernel_call *call) {
    SlotTable st;
    st.vec = &slots;
    return dispatch_impl(be, st, call);
}

int decode_call(const uint8_t *wire, size_t len, holo_kernel_call *out, size_t *consumed) {
    return decode_impl(wire, len, out, consumed);
}

int dispatch_group(holo_backend *be, const std::vector<SlotRange> &slots, const GroupDesc &g,
                   EpiArgs *defer) {
    SlotTable st;
    st.vec = &slots;
    if (defer) defer->ks = 0;
    return dispatch_group_impl(be, st, g, "fused_group", defer);
}

int launch_deferred_epilogue(holo_backend *be, const EpiArgs &e) {
    return launched(launch_epilogue(e, be->stream), "fused_group");
}

int dispatch_with_epilogue(holo_backend *be, const std::vector<SlotRange> &slots,
                           const holo_kernel_call *call, const EpiArgs &pro) {
    SlotTable st;
    st.vec = &slots;
    if (call->tag == HOLO_OP_DECODE_ATTN_I8) {
        bool done = false;
        const int rc = do_attn_i8(be, st, call->u.attn_i8, 1, false, &pro, &done);
        if (done || rc != HOLO_OK) return rc;
    }
    HOLO_TRY(launch_deferred_epilogue(be, pro));
    return dispatch_impl(be, st, call);
}

int lut_act_of_fused(uint32_t act) {
    switch (act) {
        case kFusedGelu: return HOLO_ACT_GELU;
        case kFusedSilu: return HOLO_ACT_SILU;
        case kFusedSigmoid: return HOLO_ACT_SIGMOID;
        case kFusedTanh: return HOLO_ACT_TANH;
        case kFusedExp: return HOLO_ACT_EXP;
        case kFusedRelu: return kTableRelu;
        case kFusedElu: return kTableElu;
        case kFusedSelu: return kTableSelu;
        case kActErf: return HOLO_ACT_ERF;
        default: return -1;
    }
}

// Every fused_activation (kernel_call.rs:861-870) is served: 16-bit products
// through the table of narrow(f(widen(x))), f32 products and every sum after a
// residual add computed in f32 (act_f32).
bool fused_act_supported(uint32_t act, uint8_t dtype, bool after_add) {
    const bool known = act >= 1 && act <= 8;
    if (dtype == HOLO_DTYPE_BF16) return after_add ? known : lut_act_of_fused(act) >= 0;
    if (dtype == HOLO_DTYPE_F32 || dtype == HOLO_DTYPE_F16) return known;
    return false;
}

hipStream_t backend_stream(const holo_backend *be) { return be->stream; }
void set_backend_stream(holo_backend *be, hipStream_t s) { be->stream = s; }
int backend_device(const holo_backend *be) { return be->device; }
void swap_scratch(holo_backend *be, void **ptr, size_t *bytes) {
    std::swap(be->scratch, *ptr);
    std::swap(be->scratch_bytes, *bytes);
}

}  // namespace holo

extern "C" {

int holo_hip_backend_create(int device, void *stream, holo_backend **out) {
    if (!out) return fail(HOLO_ERR_INIT, "backend_create: null out");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(HOLO_ERR_INIT, "backend_create: no HIP device visible");
    if (device < 0 || device >= count)
        return fail(HOLO_ERR_INIT, "backend_create: device index out of range");
    if (hipSetDevice(device) != hipSuccess) return fail(HOLO_ERR_INIT, "backend_create: hipSetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(HOLO_ERR_INIT, "backend_create: device query failed");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(HOLO_ERR_INIT, std::string("backend_create: built for gfx950, device is ") +
                                       prop.gcnArchName);
    // this device's address of the static scratch (holo_hip_dispatch_noalloc),
    // taken once per device while it is current
    const hipError_t se = holo::static_scratch_init(device);
    if (se != hipSuccess)
        return fail(HOLO_ERR_INIT, std::string("backend_create: static scratch address: ") +
                                       hipGetErrorString(se));
    auto *be = new holo_backend();
    be->device = device;
    be->stream = static_cast<hipStream_t>(stream);
    if (hipMalloc(&be->dev_err, sizeof(int)) != hipSuccess ||
        hipMemcpy(be->dev_err, &kZero, sizeof(int), hipMemcpyHostToDevice) != hipSuccess) {
        if (be->dev_err) (void)hipFree(be->dev_err);
        delete be;
        return fail(HOLO_ERR_INIT, "backend_create: device error flag allocation failed");
    }
    *out = be;
    return HOLO_OK;
}

int holo_hip_backend_destroy(holo_backend *be) {
    if (!be) return HOLO_OK;
    (void)hipSetDevice(be->device);
    (void)hipStreamSynchronize(be->stream);
    for (auto &row : be->lut_dev)
        for (auto *t : row)
            if (t) (void)hipFree(t);
    if (be->scratch) (void)hipFree(be->scratch);
    if (be->dev_err) (void)hipFree(be->dev_err);
    delete be;
    return HOLO_OK;
}

int holo_hip_set_stream(holo_backend *be, void *stream) {
    if (!be) return fail(HOLO_ERR_INIT, "set_stream: null backend");
    be->stream = static_cast<hipStream_t>(stream);
    return HOLO_OK;
}

int holo_hip_slot_bind(holo_backend *be, uint32_t slot, void *ptr, uint64_t bytes) {
    if (!be) return fail(HOLO_ERR_INIT, "slot_bind: null backend");
    if (slot == HOLO_SLOT_ABSENT) return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, "slot_bind: reserved slot id");
    if (!ptr && bytes) return fail(HOLO_ERR_SLOT_OUT_OF_RANGE, "slot_bind: null pointer");
    be->slots[slot] = Range{static_cast<uint8_t *>(ptr), bytes};
    return HOLO_OK;
}

int holo_hip_slot_unbind(holo_backend *be, uint32_t slot) {
    if (!be) return fail(HOLO_ERR_INIT, "slot_unbind: null backend");
    be->slots.erase(slot);
    return HOLO_OK;
}

int holo_hip_dispatch(holo_backend *be, const holo_kernel_call *call) {
    if (!be) return fail(HOLO_ERR_INIT, "dispatch: null backend");
    SlotTable st;
    st.be = be;
    return dispatch_impl(be, st, call);
}

int holo_hip_dispatch_noalloc(holo_backend *be, const holo_kernel_call *call) {
    if (!be || !call) return fail(HOLO_ERR_INIT, "dispatch_noalloc: null argument");
    SlotTable st;
    st.be = be;
    switch (call->tag) {
        case HOLO_OP_DECODE_ATTN_I8: return do_attn_i8(be, st, call->u.attn_i8, 1, true);
        case HOLO_OP_ATTN_I8_ROWS:
            return do_attn_i8(be, st, call->u.attn_i8_rows.attn, call->u.attn_i8_rows.q_rows, true);
        default:
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "dispatch_noalloc: serves DecodeAttentionI8 (123) and AttentionI8Rows (125); "
                        "use holo_hip_dispatch");
    }
}

int holo_hip_dispatch_encoded(holo_backend *be, const uint8_t *wire, size_t len, size_t *consumed) {
    holo_kernel_call c;
    HOLO_TRY(decode_impl(wire, len, &c, consumed));
    return holo_hip_dispatch(be, &c);
}

int holo_hip_synchronize(holo_backend *be) {
    if (!be) return fail(HOLO_ERR_INIT, "synchronize: null backend");
    hipError_t e = hipStreamSynchronize(be->stream);
    if (e != hipSuccess) return fail(HOLO_ERR_DISPATCH, std::string("synchronize: ") + hipGetErrorString(e));
    // refusals the kernels could only see on the device: bit 1 a Gather index out
    // of range, bit 2 a multi-row attention length past the ring, bit 4 a nonzero
    // W8A8 zero point
    int flag = 0;
    e = hipMemcpy(&flag, be->dev_err, sizeof(int), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail(HOLO_ERR_DISPATCH, std::string("synchronize: ") + hipGetErrorString(e));
    if (flag) {
        (void)hipMemcpy(be->dev_err, &kZero, sizeof(int), hipMemcpyHostToDevice);
        if (flag & 1)
            return fail(HOLO_ERR_SLOT_OUT_OF_RANGE,
                        "gather: an index is outside [-axis_dim, axis_dim) (reported by the device; "
                        "its output row was zeroed)");
        if (flag & 4)
            return fail(HOLO_ERR_UNSUPPORTED_OP,
                        "matmul_dequant: W8A8 requires symmetric per-channel i8/i4/e8cb within the k "
                        "bound (a nonzero zero point, reported by the device; the output holds the "
                        "symmetric product and must be discarded)");
        return fail(HOLO_ERR_UNSUPPORTED_OP,
                    "attention_i8_rows: a length exceeds bucket_rows (reported by the device): "
                    "after a ring wrap the earlier rows' keys are overwritten, so a causal "
                    "multi-row result does not exist");
    }
    return HOLO_OK;
}

int holo_hip_validate(const holo_kernel_call *call, const uint64_t *slot_bytes, uint32_t nslots) {
    SlotTable st;
    st.sizes = slot_bytes;
    st.nsizes = slot_bytes ? nslots : 0;
    return dispatch_impl(nullptr, st, call);
}

int holo_hip_decode_call(const uint8_t *wire, size_t len, holo_kernel_call *out, size_t *consumed) {
    return decode_impl(wire, len, out, consumed);
}

int holo_hip_lut_table(int act, int dtype, uint16_t *out65536) {
    if (!out65536) return fail(HOLO_ERR_DISPATCH, "lut_table: null output");
    if (dtype != HOLO_DTYPE_BF16 && dtype != HOLO_DTYPE_F16)
        return fail(HOLO_ERR_UNSUPPORTED_OP, "lut_table: dtype must be bf16 or f16");
    if (!holo::build_lut_table(act, dtype == HOLO_DTYPE_F16, out65536))
        return fail(HOLO_ERR_UNSUPPORTED_OP, "lut_table: no table for this activation id");
    return HOLO_OK;
}

const char *holo_hip_last_error_message(void) { return g_last_error.c_str(); }

}  // extern "C"
