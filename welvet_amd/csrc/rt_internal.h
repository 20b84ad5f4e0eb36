// rt_internal.h — runtime helpers shared by the HIP translation units of
// libwelvet_hip (defined in runtime.hip). HIP-only: includes hip_runtime.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "wv_internal.h"

namespace wv {

// Sets the calling thread's wv_last_error() text and returns `code`.
int rt_fail(int code, const char* fmt, ...);
// Maps a HIP error to WV_E_OOM / WV_E_HIP with context `what`.
int rt_hip_fail(hipError_t e, const char* what);
// Initialises device 0 unless wv_init chose one; makes it current.
int rt_ensure_init();
// Copies the device view of blob `h`; false if the handle is unknown.
bool rt_lookup(uint64_t h, DevBlob& out);
// The device wv_init selected (-1 before any init).
int rt_current_device();

}  // namespace wv
