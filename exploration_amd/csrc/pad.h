// Row padding of head dimensions (pad.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

// Head dimension the kernels run at: D rounded up to a multiple of 8.
inline int64_t padded_head_dim(int64_t D) { return (D + 7) / 8 * 8; }

// [rows, D] -> zero-filled [rows, Dp] (unpad = false), or [rows, Dp] ->
// [rows, D] (unpad = true), for 2- or 4-byte elements.
hipError_t launch_pad_rows(int elem_bytes, void* dst, const void* src, int64_t rows, int D, int Dp, bool unpad,
                           hipStream_t stream);

}  // namespace st
