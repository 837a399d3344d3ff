// Host-side helpers shared by the TR-MoE translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/trmoe.h"

namespace trmoe {

constexpr int kMaxExperts = 16;
constexpr int kMaxTopK = 4;

// Records `msg` as this thread's last error and returns `status`.
int set_error(int status, const char* msg);
// After a launch: maps a pending HIP error to TRMOE_ERR_HIP.
int check_launch(const char* what);
// Raises a kernel's dynamic LDS limit to `bytes` (> 64 KiB) once per
// (kernel, device): the runtime call is not repeated on every launch.
int set_kernel_lds(const void* kernel, int bytes);

// Compute units of the current device (cached per device; 256 when the
// runtime cannot say).  Used only to balance tile rounds.
int current_device_cus();

int64_t route_sort_blocks(int64_t n, int k, int order);
int launch_route_sort(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                      int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                      int32_t* counts, void* workspace, size_t workspace_bytes, hipStream_t stream);
int launch_route_sort_noalloc(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                              int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                              int32_t* counts, hipStream_t stream);

}  // namespace trmoe
