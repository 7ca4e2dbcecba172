// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// dtype sizes and launch-status translation.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "rlse_kv.h"

namespace rlse {

// Records a formatted message for rlse_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Bytes per element of an rlse_dtype, 0 for an unknown dtype.
size_t dtype_size(int dtype);

// Status of the most recent launch on this thread (hipGetLastError).
int launch_status(const char* what);

// Compute-unit count of the current device (cached per device).
int device_cu_count(int* cus);

inline hipStream_t as_stream(rlse_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Current bound on a cross-workgroup merge's wait, in 100 MHz wall-clock
// ticks (rlse_set_merge_wait_ns).
unsigned long long merge_wait_ticks();

// Synchronises `stream`, reads the sticky error flags in word 0 of a
// workspace into *flags (may be NULL), clears them when set, and maps them
// to a status: RLSE_ERR_DEVICE_TIMEOUT, RLSE_ERR_TOKEN_LIMIT or 0.
int read_and_clear_ws_flags(void* workspace, hipStream_t stream, unsigned* flags);

}  // namespace rlse
