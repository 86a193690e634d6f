// Run-time compilation of generated kernels (fused elementwise clusters).
//
// Compile turns each elementwise cluster into HIP source (graph_lower.cpp) and
// this file compiles it once per process with hipRTC for gfx950, caching the
// code object by source text (identical clusters across graphs share one) and
// loading it once on each device that runs it.  A plan-only backend compiles (which validates the generated
// source) but never loads modules.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <stdio.h>
#include <stdlib.h>

#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "graph.h"

namespace ghip {

namespace {
// One code object per source; one loaded module per device that has run it (a
// module loaded while device d is current holds functions of d's context only).
struct Entry {
  std::vector<char> code;
  std::map<int, RtcKernel> loaded;
};
std::mutex g_mu;
std::map<std::string, Entry> g_cache;

// Options: gfx950, -O3, packed-fp32 VALU ops disabled (they are not used
// anywhere in this library), and no floating-point contraction: every generated
// statement is one graph op rounded on its own, so a multiply is never fused into
// a following add (a producer's product into a reduction's running sum, say),
// and a fused kernel computes exactly what the unfused ops would store.
const char* kOpts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
                       "-target-feature", "-Xclang", "-packed-fp32-ops"};
}  // namespace

int rtc_get(GHipBackend* be, const std::string& src, const std::string& entry, RtcKernel* out,
            GHipError* err) {
  std::lock_guard<std::mutex> lk(g_mu);
  Entry& e = g_cache[src];
  // GHIP_RTC_DUMP=<dir>: keep a copy of every generated source (for reading the
  // generated code and its ISA offline), also when the compiled code is cached.
  if (const char* dir = getenv("GHIP_RTC_DUMP")) {
    const std::string path = std::string(dir) + "/" + entry + "_" +
                             std::to_string(std::hash<std::string>()(src)) + ".hip";
    if (FILE* f = fopen(path.c_str(), "w")) {
      fwrite(src.data(), 1, src.size(), f);
      fclose(f);
    }
  }
  if (e.code.empty()) {
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src.c_str(), "fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
      g_cache.erase(src);
      return set_error(err, GHIP_ERR_HIP, "hiprtcCreateProgram failed");
    }
    const hiprtcResult rc = hiprtcCompileProgram(prog, sizeof(kOpts) / sizeof(kOpts[0]), kOpts);
    if (rc != HIPRTC_SUCCESS) {
      size_t n = 0;
      hiprtcGetProgramLogSize(prog, &n);
      std::string log(n + 1, '\0');
      hiprtcGetProgramLog(prog, &log[0]);
      hiprtcDestroyProgram(&prog);
      g_cache.erase(src);
      return set_error(err, GHIP_ERR_HIP, "generated kernel failed to compile: %s\n--- source ---\n%s",
                       log.c_str(), src.c_str());
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    e.code.resize(n);
    hiprtcGetCode(prog, e.code.data());
    hiprtcDestroyProgram(&prog);
  }
  if (be->plan_only) {
    *out = RtcKernel{};
    return GHIP_OK;
  }
  auto it = e.loaded.find(be->device);
  if (it == e.loaded.end()) {
    hipSetDevice(be->device);
    RtcKernel k{};
    hipError_t h = hipModuleLoadData(&k.module, e.code.data());
    if (h != hipSuccess) return check_hip(h, err, "hipModuleLoadData(generated kernel)");
    h = hipModuleGetFunction(&k.func, k.module, entry.c_str());
    if (h != hipSuccess) {
      hipModuleUnload(k.module);
      return check_hip(h, err, "hipModuleGetFunction(generated kernel)");
    }
    it = e.loaded.emplace(be->device, k).first;
  }
  *out = it->second;
  return GHIP_OK;
}

}  // namespace ghip
