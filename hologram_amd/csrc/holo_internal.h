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
// BLAKE3 (default hash mode, 32-byte digest).
void blake3_hash(const void *data, size_t len, uint8_t out[32]);

}  // namespace holo
