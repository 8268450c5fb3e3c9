// sidon_host.h -- host-side helpers shared by the library's translation units
// (error text, device check).  Not part of the C ABI: every symbol here has
// hidden visibility.
#pragma once

#include <stdint.h>

#include "sidon_flexrel.h"

namespace sidon {

// Record a printf-style message as the thread's last error; returns `code`.
int fail(int code, const char* fmt, ...);
// Clear the thread's last error (start of every entry point).
void clear_error();
// SIDON_OK when the current HIP device is a gfx950, else SIDON_E_DEVICE.
int check_device();
// Compute units of the current device (after a successful check_device).
int compute_units();

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace sidon
