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

}  // namespace rlse
