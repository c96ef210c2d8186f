// Launch records of the library's kernels: what `st_launch_report` returns.
#pragma once

#include <hip/hip_runtime.h>

namespace st {

struct LaunchInfo {
  const char* kernel;   // stable kernel name (without template arguments)
  int dtype;            // ST_DTYPE_* of the inputs
  int head_dim;         // head dimension the kernel runs at
  int block_size;       // attention block size (0 where it does not apply)
  int tile_m;           // query rows (or keys) per workgroup work item
  int tile_n;           // keys (or rows) per staged tile
  int waves;            // waves per workgroup (the reference's num_warps)
  int stages;           // LDS buffers per operand (2 = double-buffered)
  unsigned workgroups;  // grid size of this launch
  const char* mode;     // scheduling mode ("pair", "slot", "grid", ...)
};

// Records (kernel, dtype, head_dim, block_size, mode) once per process and
// device, with the kernel's VGPR/AGPR count, LDS bytes and scratch bytes from
// hipFuncGetAttributes; later launches update the workgroup count. Host
// only, thread-safe, no device synchronisation.
void note_launch(const void* func, const LaunchInfo& info);

// The records as a JSON array in buf (at most cap bytes, NUL terminated);
// returns the bytes the whole text needs including its NUL.
size_t report_json(char* buf, size_t cap);

}  // namespace st
