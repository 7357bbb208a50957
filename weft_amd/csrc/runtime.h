// Host-side launch plumbing shared by the libweft_hip entry points:
// the calling thread's current stream, the sticky per-thread error, and
// cached device facts.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace weft {

hipStream_t current_stream();
// Record an error for the calling thread (first one wins until read).
void set_error(hipError_t e);
// Check the launch just made and record its error, if any; `kernel` names
// it in the calling thread's launch log (weft_hip_launch_log).
void check_launch(const char* kernel = nullptr);
// The calling thread's recorded error, left in place.
hipError_t pending_error();
// Whether the calling thread keeps a launch log (weft_hip_set_launch_log).
bool launch_log_enabled();
// The calling thread's source tile bindings (weft_hip_set_tile_binding;
// 0 = unset): nc = weight rows per workgroup and mr = activation rows per
// pass of the GEMV kernels; the Q4_K MFMA GEMM takes nc as weight rows and
// mc as activation rows per tile (64 / 128 and 32 / 64).
struct TileBindings {
  int nc = 0, mr = 0, mc = 0;
};
const TileBindings& tile_bindings();

// Compute units of the current device (cached per device).
int cu_count();
// Largest dynamic LDS a workgroup may request on the current device.
size_t max_lds_per_block();

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace weft
