// Internal launch interface of the dense gated attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

enum DType { kF32 = 0, kF16 = 1, kBF16 = 2 };

struct DenseArgs {
  const void* q;          // [B,Q,H,D]
  const void* k;          // [B,N,H,D]
  const void* v;          // [B,N,H,D]
  const int64_t* pos;     // [B,Q], -1 = padding row
  const void* dout;       // [B,Q,H,D] (backward only)
  void* out;              // [B,Q,H,D] forward output (input dtype)
  float* rc;              // [B,Q,H,D] remote part of the output
  float* pr;              // [B,Q,H] remote probability mass
  float* zr;              // [B,Q,H] log Z_R (-inf: no remote block)
  float* z;               // [B,Q,H] logsumexp of all logits (-inf: padding)
  float* delta;           // [B,Q,H] dO.O (backward workspace)
  float* rho;             // [B,Q,H] dO.RC - delta*PR (backward workspace)
  void* dq;               // [B,Q,H,D]
  void* dk;               // [B,N,H,D]
  void* dv;               // [B,N,H,D]
  int B, Q, N, H, D;
  int block, logb;
  float scale;            // 1/sqrt(D)
  float scale_log2;       // log2(e)/sqrt(D)
};

// Each returns hipSuccess or the launch error; the arguments were validated
// by the caller (dtype, head_dim <= 256, block a power of two in [2,128]).
hipError_t launch_dense_fwd(int dtype, const DenseArgs& a, hipStream_t stream);
// Pipelined forward for 16-bit inputs with head_dim 64 or 128.
bool dense_fwd_fast_supported(int dtype, const DenseArgs& a);
hipError_t launch_dense_fwd_fast(int dtype, const DenseArgs& a, hipStream_t stream);
hipError_t launch_dense_bwd(int dtype, const DenseArgs& a, hipStream_t stream);

}  // namespace st
