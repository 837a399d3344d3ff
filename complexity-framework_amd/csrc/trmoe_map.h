// Destination index of one element of a weight gradient written straight into
// a parameter's layout (trmoe_weight_grad_mapped): off + idx * stride, in
// elements of the flat output.  -1 when the row/column is skipped (off < 0)
// or the destination falls outside [0, out_elems): a bad map from a C-ABI
// caller then writes nothing instead of arbitrary device memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trmoe {

__host__ __device__ inline int64_t mapped_dest(int64_t off, int64_t idx, int64_t stride, int64_t out_elems) {
    if (off < 0) return -1;
    const int64_t d = off + idx * stride;
    return (d >= 0 && d < out_elems) ? d : -1;
}

}  // namespace trmoe
