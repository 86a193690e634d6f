// Compile and Execute (builder.go:72-109, executable.go:19-112).
//
// Compile lowers the graph once (graph_lower.cpp) and uploads constants to
// device memory owned by the executable.  Execute validates the inputs like the
// reference (executable.go:54-68), allocates the outputs from the backend's
// caching allocator, binds every plan slot to a device pointer (inputs, constants,
// the executable's arena, outputs) and launches the steps on the backend stream.
// It does not wait: buffers are device resident, and reading one back
// (BufferToFlatData) or releasing one synchronises the stream.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>

#include "common.h"
#include "graph.h"

using namespace ghip;

namespace ghip {

// Lowers fn and uploads its constants.  Inputs: fn's params, then its captures.
static GHipExecutable* compile_raw(GHipBackend* be, GHipFunction* fn, GHipError* err) {
  if (!fn->returned) {
    set_error(err, GHIP_ERR_STATE, "Compile: function %s has no Return() call", fn->name.c_str());
    return nullptr;
  }
  auto ex = std::make_unique<GHipExecutable>();
  ex->backend = be;
  for (int p : fn->params) {
    ex->in_shapes.push_back(fn->nodes[p].shape);
    ex->in_names.push_back(fn->nodes[p].name);
  }
  std::vector<int> cap(fn->captures.size(), -1);
  for (const auto& kv : fn->capture_of) cap[fn->nodes[kv.second].i0] = kv.second;
  for (int c : cap) {
    ex->in_shapes.push_back(fn->nodes[c].shape);
    ex->in_names.push_back("capture");
  }
  for (int o : fn->outputs) ex->out_shapes.push_back(fn->nodes[o].shape);
  if (lower(be, fn, &ex->plan, err) != GHIP_OK) return nullptr;
  if (!be->plan_only) {
    hipSetDevice(be->device);
    for (size_t s = 0; s < ex->plan.slots.size(); ++s) {
      Slot& sl = ex->plan.slots[s];
      if (sl.kind != SlotKind::Const) continue;
      void* p = nullptr;
      if (be->alloc(sl.bytes, &p, err) != GHIP_OK) {
        ghip_exec_finalize(ex.release());
        return nullptr;
      }
      ex->owned_consts.emplace_back(p, sl.bytes);
      sl.const_ptr = p;
      const auto& data = ex->plan.const_data[s];
      if (!data.empty()) {
        hipError_t e = hipMemcpyAsync(p, data.data(), data.size(), hipMemcpyHostToDevice, be->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(be->stream);
        if (e != hipSuccess) {
          check_hip(e, err, "Compile: constant upload");
          ghip_exec_finalize(ex.release());
          return nullptr;
        }
      }
    }
  }
  return ex.release();
}

std::shared_ptr<GHipExecutable> compile_function(GHipBackend* be, GHipFunction* fn, GHipError* err) {
  GHipExecutable* e = compile_raw(be, fn, err);
  if (!e) return nullptr;
  return std::shared_ptr<GHipExecutable>(e, [](GHipExecutable* x) { ghip_exec_finalize(x); });
}

int run_plan(GHipExecutable* e, void* const* in_ptrs, void* const* out_ptrs, GHipError* err) {
  GHipBackend* be = e->backend;
  const Plan& plan = e->plan;
  if (plan.arena_bytes > e->arena_cap) {
    if (e->arena) {
      hipStreamSynchronize(be->stream);
      be->release(e->arena, e->arena_cap);
      e->arena = nullptr;
      e->arena_cap = 0;
    }
    if (be->alloc(plan.arena_bytes, &e->arena, err) != GHIP_OK) return err ? err->code : GHIP_ERR_OOM;
    e->arena_cap = plan.arena_bytes;
  }
  return run_plan_in(e, e->arena, in_ptrs, out_ptrs, err);
}

int run_plan_in(GHipExecutable* e, void* arena, void* const* in_ptrs, void* const* out_ptrs, GHipError* err) {
  GHipBackend* be = e->backend;
  const Plan& plan = e->plan;
  ExecState st;
  st.stream = be->stream;
  st.slot_ptr.resize(plan.slots.size(), nullptr);
  for (size_t s = 0; s < plan.slots.size(); ++s) {
    const Slot& sl = plan.slots[s];
    switch (sl.kind) {
      case SlotKind::Input: st.slot_ptr[s] = static_cast<char*>(in_ptrs[sl.index]); break;
      case SlotKind::Const: st.slot_ptr[s] = static_cast<char*>(sl.const_ptr); break;
      case SlotKind::Arena: st.slot_ptr[s] = static_cast<char*>(arena) + sl.arena_off; break;
      case SlotKind::Output: st.slot_ptr[s] = static_cast<char*>(out_ptrs[sl.index]); break;
    }
  }
  for (const Step& step : plan.steps) {
    const int rc = step.run(st, err);
    if (rc != GHIP_OK) {
      if (err && err->message) {
        std::string m = std::string("Execute: ") + step.desc + ": " + err->message;
        set_error(err, rc, "%s", m.c_str());
      }
      hipStreamSynchronize(be->stream);
      return rc;
    }
  }
  return GHIP_OK;
}

}  // namespace ghip

extern "C" GHipExecutable* ghip_builder_compile(GHipBuilder* bl, GHipError* err) {
  if (!bl) { set_error(err, GHIP_ERR_INVALID_ARG, "Compile: null builder"); return nullptr; }
  if (bl->compiled) { set_error(err, GHIP_ERR_STATE, "Builder already compiled"); return nullptr; }
  if (!bl->main) { set_error(err, GHIP_ERR_STATE, "Builder has no main function"); return nullptr; }
  if (!bl->main->returned) { set_error(err, GHIP_ERR_STATE, "Main function has no Return() call"); return nullptr; }
  GHipBackend* be = bl->backend;
  if (!be || be->finalized) { set_error(err, GHIP_ERR_STATE, "Compile: backend finalized"); return nullptr; }
  bl->compiled = true;
  return compile_raw(be, bl->main.get(), err);
}

extern "C" int ghip_exec_num_inputs(GHipExecutable* e) { return e ? static_cast<int>(e->in_shapes.size()) : -1; }
extern "C" int ghip_exec_num_outputs(GHipExecutable* e) { return e ? static_cast<int>(e->out_shapes.size()) : -1; }

static int shape_out(const Shape& s, int* dtype, int64_t* dims, int max_rank) {
  if (dtype) *dtype = s.dtype;
  for (int i = 0; i < s.rank() && i < max_rank; ++i) dims[i] = s.dims[i];
  return s.rank();
}
extern "C" int ghip_exec_input_shape(GHipExecutable* e, int i, int* dtype, int64_t* dims, int max_rank) {
  if (!e || i < 0 || i >= static_cast<int>(e->in_shapes.size())) return -1;
  return shape_out(e->in_shapes[i], dtype, dims, max_rank);
}
extern "C" int ghip_exec_output_shape(GHipExecutable* e, int i, int* dtype, int64_t* dims, int max_rank) {
  if (!e || i < 0 || i >= static_cast<int>(e->out_shapes.size())) return -1;
  return shape_out(e->out_shapes[i], dtype, dims, max_rank);
}

extern "C" size_t ghip_exec_plan(GHipExecutable* e, char* buf, size_t buflen) {
  if (!e) return 0;
  std::string s;
  char head[160];
  snprintf(head, sizeof head, "# %zu steps, arena %zu bytes\n", e->plan.steps.size(), e->plan.arena_bytes);
  s += head;
  for (auto& l : e->plan.log) s += l + "\n";
  if (buf && buflen) {
    const size_t n = std::min(buflen - 1, s.size());
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return s.size();
}

namespace ghip {
// Execute's argument checks (executable.go:54-68); the caller holds e->mu.
int check_execute_args(GHipExecutable* e, GHipBuffer* const* inputs, int n, int nout, GHipError* err) {
  GHipBackend* be = e->backend;
  if (!be || be->finalized) return set_error(err, GHIP_ERR_STATE, "Execute: backend finalized");
  if (be->plan_only) return set_error(err, GHIP_ERR_STATE, "Execute: plan-only backend has no device");
  if (n != static_cast<int>(e->in_shapes.size()))
    return set_error(err, GHIP_ERR_INVALID_ARG, "Execute: expected %zu inputs, got %d", e->in_shapes.size(), n);
  if (nout != static_cast<int>(e->out_shapes.size()))
    return set_error(err, GHIP_ERR_INVALID_ARG, "Execute: expected %zu outputs, got %d", e->out_shapes.size(), nout);
  for (int i = 0; i < n; ++i) {
    if (!inputs[i] || !inputs[i]->valid)
      return set_error(err, GHIP_ERR_INVALID_ARG, "Execute: input #%d is not a valid buffer", i);
    // A buffer of another backend lives on another stream (and maybe device):
    // reading it, or taking it over by donation into this backend's allocator,
    // would race with that stream's work.
    if (inputs[i]->backend != be)
      return set_error(err, GHIP_ERR_INVALID_ARG, "Execute: input #%d belongs to another backend", i);
    if (inputs[i]->shape != e->in_shapes[i])
      return set_error(err, GHIP_ERR_INVALID_ARG, "Execute: input #%d shape mismatch: expected %s, got %s", i,
                       e->in_shapes[i].str().c_str(), inputs[i]->shape.str().c_str());
  }
  return GHIP_OK;
}
}  // namespace ghip

// Whether output o may take donated input i's memory: same shape, and the plan
// reads input i only before it first writes output o, or in that same step
// when the step is elementwise and reads input i at output o's own indices.
static bool can_donate(const GHipExecutable* e, int i, int o) {
  const Plan& plan = e->plan;
  if (e->in_shapes[i] != e->out_shapes[o]) return false;
  const int last = plan.in_last_read[i], first = plan.out_first_write[o];
  if (last < first) return true;
  if (last != first || first == INT32_MAX) return false;
  const auto& ip = plan.inplace_inputs[first];
  return std::find(ip.begin(), ip.end(), i) != ip.end();
}

extern "C" int ghip_exec_execute(GHipExecutable* e, GHipBuffer* const* inputs, int n, const uint8_t* donate,
                                 GHipBuffer** outputs, int nout, GHipError* err) {
  if (!e || e->finalized) return set_error(err, GHIP_ERR_STATE, "Execute: executable finalized");
  std::lock_guard<std::mutex> lk(e->mu);
  GHipBackend* be = e->backend;
  if (const int rc = check_execute_args(e, inputs, n, nout, err)) return rc;
  hipSetDevice(be->device);
  std::vector<GHipBuffer*> outs(nout, nullptr);
  // Donated inputs (executable.go:50): an output of the same shape takes over the
  // memory of a donated input the plan no longer needs when it writes that output
  // (the input buffer is consumed: it becomes invalid, and finalizing it is a
  // no-op).  A buffer passed as several inputs is never taken.
  std::vector<int> donor(nout, -1);
  if (donate) {
    std::vector<char> used(n, 0);
    for (int o = 0; o < nout; ++o)
      for (int i = 0; i < n && donor[o] < 0; ++i) {
        if (!donate[i] || used[i] || !can_donate(e, i, o)) continue;
        bool shared = false;
        for (int j = 0; j < n; ++j) shared = shared || (j != i && inputs[j]->ptr == inputs[i]->ptr);
        if (shared) continue;
        donor[o] = i;
        used[i] = 1;
      }
  }
  auto cleanup = [&]() {
    for (int o = 0; o < nout; ++o)
      if (outs[o] && donor[o] < 0) ghip_buffer_finalize(outs[o]);
      else delete outs[o];
  };
  for (int o = 0; o < nout; ++o) {
    if (donor[o] >= 0) {
      const GHipBuffer* in = inputs[donor[o]];
      outs[o] = new GHipBuffer();
      outs[o]->backend = be;
      outs[o]->shape = e->out_shapes[o];
      outs[o]->ptr = in->ptr;
      outs[o]->cap = in->cap;
      continue;
    }
    outs[o] = ghip_buffer_new(be, e->out_shapes[o].dtype, e->out_shapes[o].dims.data(), e->out_shapes[o].rank(), err);
    if (!outs[o]) {
      cleanup();
      return err ? err->code : GHIP_ERR_OOM;
    }
  }
  std::vector<void*> in_ptrs(std::max(n, 1)), out_ptrs(std::max(nout, 1));
  for (int i = 0; i < n; ++i) in_ptrs[i] = inputs[i]->ptr;
  for (int i = 0; i < nout; ++i) out_ptrs[i] = outs[i]->ptr;
  const int rc = run_plan(e, in_ptrs.data(), out_ptrs.data(), err);
  if (rc != GHIP_OK) {
    cleanup();
    return rc;
  }
  for (int o = 0; o < nout; ++o) {
    if (donor[o] >= 0) {  // the input's memory now belongs to the output
      inputs[donor[o]]->valid = false;
      inputs[donor[o]]->ptr = nullptr;
    }
    outputs[o] = outs[o];
  }
  return GHIP_OK;
}

extern "C" void ghip_exec_finalize(GHipExecutable* e) {
  if (!e) return;
  GHipBackend* be = e->backend;
  if (be && !be->finalized && !be->plan_only) {
    hipSetDevice(be->device);
    hipStreamSynchronize(be->stream);
    for (auto& pc : e->owned_consts) be->release(pc.first, pc.second);
    if (e->arena) be->release(e->arena, e->arena_cap);
  }
  e->finalized = true;
  delete e;
}
