// Execute without allocating: the executable's intermediates live in one
// file-scope device array instead of an arena from the backend's allocator, and
// the caller passes the output buffers.  For callers that cannot call hipMalloc
// (serving loops that must not allocate, code run under stream capture).
//
// The array is per GPU: each device the library runs on holds its own copy for
// the life of the process, at its own address, which is looked up once per device
// with hipGetSymbolAddress (the array's name in host code is only a host-side
// stand-in).  Every call on one GPU shares that GPU's array and leaves the last
// call's contents in it; the plans never read an arena byte before writing it, so
// nothing needs clearing between calls.  Calls that overlap on one GPU (two host
// threads, or two streams) race on the array.
#include <mutex>

#include "common.h"
#include "graph.h"

namespace ghip {
namespace {

constexpr size_t kNoAllocScratchBytes = size_t{256} << 20;  // 256 MiB per GPU
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// The device address of `scratch` on `device` (which must be current).
int scratch_ptr(int device, void** out, GHipError* err) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return check_hip(e, err, "ExecuteNoAlloc: hipGetSymbolAddress(scratch)");
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return GHIP_OK;
}

}  // namespace
}  // namespace ghip

using namespace ghip;

extern "C" size_t ghip_exec_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int ghip_exec_execute_noalloc(GHipExecutable* e, GHipBuffer* const* inputs, int n,
                                         GHipBuffer* const* outputs, int nout, GHipError* err) {
  if (!e || e->finalized) return set_error(err, GHIP_ERR_STATE, "ExecuteNoAlloc: executable finalized");
  std::lock_guard<std::mutex> lk(e->mu);
  if (const int rc = check_execute_args(e, inputs, n, nout, err)) return rc;
  for (int i = 0; i < nout; ++i) {
    if (!outputs || !outputs[i] || !outputs[i]->valid)
      return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: output #%d is not a valid buffer", i);
    if (outputs[i]->backend != e->backend)
      return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: output #%d belongs to another backend", i);
    if (outputs[i]->shape != e->out_shapes[i])
      return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: output #%d shape mismatch: expected %s, got %s",
                       i, e->out_shapes[i].str().c_str(), outputs[i]->shape.str().c_str());
    for (int j = 0; j < n; ++j)
      if (outputs[i]->ptr == inputs[j]->ptr)
        return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: output #%d is input #%d", i, j);
    for (int j = 0; j < i; ++j)
      if (outputs[i]->ptr == outputs[j]->ptr)
        return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: outputs #%d and #%d are one buffer", j, i);
  }
  const Plan& plan = e->plan;
  if (!plan.subs.empty())
    return set_error(err, GHIP_ERR_UNSUPPORTED,
                     "ExecuteNoAlloc: graphs with Call / While / If run their sub-functions with their own "
                     "arenas; use Execute");
  if (plan.arena_bytes > kNoAllocScratchBytes)
    return set_error(err, GHIP_ERR_INVALID_ARG,
                     "ExecuteNoAlloc: the plan needs %zu bytes of intermediates, above the %zu-byte limit",
                     plan.arena_bytes, kNoAllocScratchBytes);
  GHipBackend* be = e->backend;
  hipSetDevice(be->device);
  void* arena = nullptr;
  if (const int rc = scratch_ptr(be->device, &arena, err)) return rc;
  void* in_ptrs[64];
  void* out_ptrs[64];
  if (n > 64 || nout > 64)
    return set_error(err, GHIP_ERR_INVALID_ARG, "ExecuteNoAlloc: at most 64 inputs and 64 outputs");
  for (int i = 0; i < n; ++i) in_ptrs[i] = inputs[i]->ptr;
  for (int i = 0; i < nout; ++i) out_ptrs[i] = outputs[i]->ptr;
  return run_plan_in(e, arena, in_ptrs, out_ptrs, err);
}
