// Row padding for head dimensions that are not a multiple of 8: copies of
// [rows, D] matrices into zero-filled [rows, Dp] buffers (and back), so the
// attention kernels, whose loads and LDS tiles move 16 bytes per lane, see
// rows of Dp = round_up(D, 8) elements. Zero columns change no product:
// q.k is unchanged, and the padded columns of every output come out zero.
// Grid-stride element loops; not on the hot path.
#include "pad.h"

#include "common.h"

namespace st {

template <typename T>
__global__ __launch_bounds__(256) void pad_rows_kernel(T* dst, const T* src, int64_t rows, int D, int Dp) {
  const int64_t total = rows * Dp;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / Dp;
    const int c = (int)(i - r * Dp);
    dst[i] = c < D ? src[r * D + c] : T(0);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void unpad_rows_kernel(T* dst, const T* src, int64_t rows, int D, int Dp) {
  const int64_t total = rows * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / D;
    const int c = (int)(i - r * D);
    dst[i] = src[r * Dp + c];
  }
}

static unsigned pad_grid(int64_t n) {
  const int64_t g = (n + 255) / 256;
  return (unsigned)(g < 4096 ? (g > 0 ? g : 1) : 4096);
}

template <typename T>
static hipError_t pad_t(void* dst, const void* src, int64_t rows, int D, int Dp, bool unpad, hipStream_t s) {
  if (unpad)
    hipLaunchKernelGGL(unpad_rows_kernel<T>, dim3(pad_grid(rows * D)), dim3(256), 0, s, static_cast<T*>(dst),
                       static_cast<const T*>(src), rows, D, Dp);
  else
    hipLaunchKernelGGL(pad_rows_kernel<T>, dim3(pad_grid(rows * Dp)), dim3(256), 0, s, static_cast<T*>(dst),
                       static_cast<const T*>(src), rows, D, Dp);
  return hipGetLastError();
}

hipError_t launch_pad_rows(int elem_bytes, void* dst, const void* src, int64_t rows, int D, int Dp, bool unpad,
                           hipStream_t stream) {
  switch (elem_bytes) {
    case 2: return pad_t<uint16_t>(dst, src, rows, D, Dp, unpad, stream);
    case 4: return pad_t<uint32_t>(dst, src, rows, D, Dp, unpad, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace st
