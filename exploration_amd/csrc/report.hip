// Launch records behind st_launch_report (the counterpart of the reference's
// launch_report, st/ops/kernels/launch.py:52-56,96-98): per kernel
// configuration its tiles, waves, LDS buffers, registers and LDS bytes.
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "report.h"

namespace st {

namespace {

struct Record {
  LaunchInfo info;
  int device;
  int vgprs, lds_bytes, scratch_bytes, max_threads;
};

std::mutex g_mu;
std::map<std::tuple<std::string, int, int, int, int, std::string>, Record> g_records;
std::map<std::pair<const void*, int>, hipFuncAttributes> g_attrs;

}  // namespace

void note_launch(const void* func, const LaunchInfo& info) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(g_mu);
  auto ak = std::make_pair(func, dev);
  auto it = g_attrs.find(ak);
  if (it == g_attrs.end()) {
    hipFuncAttributes attr;
    memset(&attr, 0, sizeof(attr));
    if (hipFuncGetAttributes(&attr, func) != hipSuccess) memset(&attr, 0, sizeof(attr));
    (void)hipGetLastError();  // an attribute query failure must not surface as a launch error
    it = g_attrs.emplace(ak, attr).first;
  }
  const hipFuncAttributes& attr = it->second;
  auto key = std::make_tuple(std::string(info.kernel), dev, info.dtype, info.head_dim, info.block_size,
                             std::string(info.mode ? info.mode : ""));
  Record r = {info, dev, attr.numRegs, (int)attr.sharedSizeBytes, (int)attr.localSizeBytes,
              attr.maxThreadsPerBlock};
  g_records[key] = r;
}

size_t report_json(char* buf, size_t cap) {
  std::string out = "[";
  {
    std::lock_guard<std::mutex> lock(g_mu);
    bool first = true;
    for (const auto& kv : g_records) {
      const Record& r = kv.second;
      char line[512];
      snprintf(line, sizeof(line),
               "%s{\"kernel\": \"%s\", \"path\": \"hip\", \"device\": %d, \"dtype\": %d, \"head_dim\": %d, "
               "\"block_size\": %d, \"tile_m\": %d, \"tile_n\": %d, \"num_warps\": %d, \"num_stages\": %d, "
               "\"shared_memory_bytes\": %d, \"vgprs\": %d, \"scratch_bytes\": %d, \"workgroups\": %u, "
               "\"mode\": \"%s\"}",
               first ? "" : ", ", r.info.kernel, r.device, r.info.dtype, r.info.head_dim, r.info.block_size,
               r.info.tile_m, r.info.tile_n, r.info.waves, r.info.stages, r.lds_bytes, r.vgprs, r.scratch_bytes,
               r.info.workgroups, r.info.mode ? r.info.mode : "");
      out += line;
      first = false;
    }
  }
  out += "]";
  if (buf && cap > 0) {
    const size_t n = out.size() < cap - 1 ? out.size() : cap - 1;
    memcpy(buf, out.data(), n);
    buf[n] = '\0';
  }
  return out.size() + 1;
}

}  // namespace st
