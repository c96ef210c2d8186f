// Two-block window attention of the Stack model's local (halo) blocks
// (st/models/blocks.py:102-179): every block of b queries attends causally
// to [previous block ++ own block] with the split-half rotary embedding at
// window-relative positions (queries 0..b-1, keys -b..b-1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

struct HaloArgs {
  int B, G, b, H, hd;     // batch, query blocks, block size, heads, head dim
  int n;                  // real query rows (<= G*b); rows beyond are padding
  int64_t start;          // absolute position of query row 0
  int64_t first_key;      // smallest absolute key position that may be read
  float scale;            // 1/sqrt(hd)
  const void* qkv;        // [B, (G+1)*b, 3, H, hd]; raw block 0 = previous halo
  const float* cos_t;     // [2b, hd/2] cos of positions -b..b-1, rounded to the element type
  const float* sin_t;     // [2b, hd/2]
  void* out;              // [B, n, H, hd]
  const void* dout;       // [B, n, H, hd]
  void* dqkv;             // [B, (G+1)*b, 3, H, hd]
};

bool halo_supported(int b, int hd);
hipError_t launch_halo_fwd(int dtype, const HaloArgs& a, hipStream_t stream);
hipError_t launch_halo_bwd(int dtype, const HaloArgs& a, hipStream_t stream);

}  // namespace st
