// holo_internal.h — what the session executor (holo_session.cpp) shares with
// the dispatcher (holo_backend.cpp) inside libholo_hip.so. Not exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "holo_hip.h"

namespace holo {

// Device range a slot is bound to.
struct SlotRange {
    uint8_t *ptr = nullptr;
    uint64_t bytes = 0;
};

// Record `msg` as this thread's last error and return `code`.
int set_error(int code, const std::string &msg);
// Backend::dispatch of one call with operands resolved through `slots`
// (slot id = index) instead of the backend's own binding table.
int dispatch_with_slots(holo_backend *be, const std::vector<SlotRange> &slots,
                        const holo_kernel_call *call);
// One wire-format call (u16 discriminant + LE payload).
int decode_call(const uint8_t *wire, size_t len, holo_kernel_call *out, size_t *consumed);
// The stream the backend enqueues on, and its device.
hipStream_t backend_stream(const holo_backend *be);
void set_backend_stream(holo_backend *be, hipStream_t s);
int backend_device(const holo_backend *be);
// Exchange the backend's split-K scratch (pointer, size) with the caller's.
// A session swaps its own scratch in for its walk and back out after it, so
// a captured walk's graph holds memory only that session grows or frees.
void swap_scratch(holo_backend *be, void **ptr, size_t *bytes);
// A fused few-row MatMul group (the session's device fusion): products that
// share A, each finished by its epilogue (holo_kernels.h EpiSeg) in one more
// launch. Operands stay BufferRefs, resolved through the slot table at
// dispatch, so rebinding an input needs no new plan.
struct GroupSegDesc {
    holo_buffer_ref b{}, out{}, residual{}, cos{}, sin{}, rope_out{}, pos{}, cq{}, cs{}, mul_out{};
    uint32_t n = 0;
    uint8_t base = 0;          // kEpiStore / kEpiAct / kEpiAdd / kEpiAddAct
    uint32_t act = 0;          // fused_activation id
    bool write_out = true;
    uint32_t head_dim = 0;
    bool rope = false, write_rope = true, quant = false, skip = false;
    uint32_t bucket = 0, new_rows = 0;
    int pair = -1;
    float *ssq = nullptr;      // RmsNorm statistics of the rows (EpiSeg::ssq), session memory
    const void *bp = nullptr;  // B in MFMA fragment order (session memory) when the group is packed
};
struct GroupDesc {
    holo_buffer_ref a{};
    uint32_t m = 0, k = 0;
    uint8_t dtype = 0;
    std::vector<GroupSegDesc> segs;
    // A read as RmsNorm(A) (SkinnyNormA): a_norm; the statistics a producer
    // group left in session memory (split-K readers), gamma (absent:
    // identity) and epsilon
    bool a_norm = false;
    const float *a_ssq = nullptr;
    holo_buffer_ref a_gamma{HOLO_SLOT_ABSENT, 0, 0};
    float a_eps = 0.0f;
    // every product and epilogue in one launch over each segment's `bp`
    // (gemv_packed.hip); a normalized A's statistics are then taken in that
    // launch, not read from a_ssq
    bool packed = false;
    uint32_t packed_tw = 16;   // element-wise tile width the weights were packed with
};
struct EpiArgs;
// defer: a group that ends in the split-K epilogue launches only its product
// and leaves the epilogue's arguments in *defer (ks > 0; ks == 0: nothing
// deferred). The partials stay in the backend's scratch, so the deferred
// epilogue must run before anything grows it: with the next call
// (dispatch_with_epilogue), which takes it into a decode attention's launch
// where that applies, or on its own (launch_deferred_epilogue).
int dispatch_group(holo_backend *be, const std::vector<SlotRange> &slots, const GroupDesc &g,
                   EpiArgs *defer = nullptr);
int dispatch_with_epilogue(holo_backend *be, const std::vector<SlotRange> &slots,
                           const holo_kernel_call *call, const EpiArgs &pro);
int launch_deferred_epilogue(holo_backend *be, const EpiArgs &e);
// The LUT activation id of a fused_activation id (-1: no table).
int lut_act_of_fused(uint32_t act);
// Whether the device serves fused activation `act` for dtype (bf16 table or f32 compute);
// `after_add`: applied to an f32 sum (MatMulAddActivation), never through a table.
bool fused_act_supported(uint32_t act, uint8_t dtype, bool after_add);

// BLAKE3 (default hash mode, 32-byte digest).
void blake3_hash(const void *data, size_t len, uint8_t out[32]);

// κ-labels (holo_kappa.cpp): "blake3:" + hex digest; a call's op signature
// (opcode, LE params; false for a call this backend does not serve) and its
// label operands (input slots in derivation order, output slots).
std::string kappa_of_digest(const uint8_t d[32]);
std::string address_bytes(const void *bytes, size_t len);
std::string derive_label(uint16_t opcode, const uint8_t *params, size_t n_params,
                         const std::vector<std::string> &inputs);
bool op_signature(const holo_kernel_call &c, uint16_t *opcode, uint8_t params[64], uint32_t *len);
// derive_label_boundary (address.rs:197-221): the op's label (address_bytes of
// opcode and params) composed in order with each operand label; false when a
// label is not of the blake3 form
bool derive_label_boundary(uint16_t opcode, const uint8_t *params, size_t n_params,
                           const std::vector<std::string> &inputs, std::string *out);
bool label_operands(const holo_kernel_call &c, std::vector<uint32_t> *ins,
                    std::vector<uint32_t> *outs, bool *commutative);

}  // namespace holo
