// Backend, buffers and graph construction (the backends.Function surface).
//
// Each ghip_fn_* call checks its operands, infers the output shape with the
// XLA / GoMLX rules and appends one node; nothing touches the device until
// Compile.  Errors follow the reference: graph-building calls return an error
// (function.go wraps each with pkg/errors), never abort.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <set>
#include <sstream>

#include "common.h"
#include "graph.h"

using namespace ghip;

namespace ghip {

int dtype_size(int dt) {
  switch (dt) {
    case GHIP_DTYPE_BOOL: case GHIP_DTYPE_INT8: case GHIP_DTYPE_UINT8: return 1;
    case GHIP_DTYPE_INT16: case GHIP_DTYPE_UINT16: case GHIP_DTYPE_FLOAT16:
    case GHIP_DTYPE_BFLOAT16: return 2;
    case GHIP_DTYPE_INT32: case GHIP_DTYPE_UINT32: case GHIP_DTYPE_FLOAT32: return 4;
    case GHIP_DTYPE_INT64: case GHIP_DTYPE_UINT64: case GHIP_DTYPE_FLOAT64: return 8;
    default: return 0;
  }
}
bool dtype_is_float(int dt) {
  return dt == GHIP_DTYPE_FLOAT16 || dt == GHIP_DTYPE_BFLOAT16 || dt == GHIP_DTYPE_FLOAT32 ||
         dt == GHIP_DTYPE_FLOAT64;
}
bool dtype_is_unsigned(int dt) {
  return dt == GHIP_DTYPE_UINT8 || dt == GHIP_DTYPE_UINT16 || dt == GHIP_DTYPE_UINT32 ||
         dt == GHIP_DTYPE_UINT64;
}
bool dtype_is_int(int dt) {
  return dt == GHIP_DTYPE_INT8 || dt == GHIP_DTYPE_INT16 || dt == GHIP_DTYPE_INT32 ||
         dt == GHIP_DTYPE_INT64 || dtype_is_unsigned(dt);
}
const char* dtype_name(int dt) {
  static const char* n[] = {"bool", "int8", "int16", "int32", "int64", "float16", "bfloat16",
                            "float32", "float64", "uint8", "uint16", "uint32", "uint64"};
  return (dt >= 0 && dt <= 12) ? n[dt] : "invalid";
}

std::string Shape::str() const {
  std::ostringstream o;
  o << "(" << dtype_name(dtype) << ")[";
  for (size_t i = 0; i < dims.size(); ++i) o << (i ? " " : "") << dims[i];
  o << "]";
  return o.str();
}

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& dims) {
  std::vector<int64_t> s(dims.size());
  int64_t acc = 1;
  for (int i = static_cast<int>(dims.size()) - 1; i >= 0; --i) {
    s[i] = acc;
    acc *= dims[i];
  }
  return s;
}

bool View::contiguous(const Shape& s) const {
  auto c = contiguous_strides(s.dims);
  for (int i = 0; i < s.rank(); ++i)
    if (s.dims[i] != 1 && strides[i] != c[i]) return false;
  return true;
}

const char* kind_name(Kind k) {
  switch (k) {
    case Kind::Param: return "Parameter"; case Kind::Const: return "Constant";
    case Kind::Iota: return "Iota"; case Kind::Unary: return "Unary";
    case Kind::Binary: return "Binary"; case Kind::Compare: return "Compare";
    case Kind::Where: return "Where"; case Kind::Clamp: return "Clamp";
    case Kind::Convert: return "ConvertDType"; case Kind::Reshape: return "Reshape";
    case Kind::Transpose: return "Transpose"; case Kind::Broadcast: return "BroadcastInDim";
    case Kind::Slice: return "Slice"; case Kind::Concat: return "Concatenate";
    case Kind::Reverse: return "Reverse";
    case Kind::Reduce: return "Reduce"; case Kind::ArgMinMax: return "ArgMinMax";
    case Kind::Dot: return "DotGeneral"; case Kind::Gather: return "Gather";
    case Kind::Softmax: return "FusedSoftmax"; case Kind::LayerNorm: return "FusedLayerNorm";
    case Kind::SDPA: return "FusedScaledDotProductAttention";
    case Kind::DynSlice: return "DynamicSlice"; case Kind::DynUpdate: return "DynamicUpdateSlice";
    case Kind::Scatter: return "Scatter";
    default: break;
  }
  return "?";
}

bool is_elementwise(Kind k) {
  return k == Kind::Unary || k == Kind::Binary || k == Kind::Compare || k == Kind::Where ||
         k == Kind::Clamp || k == Kind::Convert;
}

}  // namespace ghip

// ===========================================================================
// Backend and device allocator
// ===========================================================================
static size_t round_alloc(size_t b) { return (b + 255) & ~size_t(255); }

int GHipBackend::alloc(size_t bytes, void** out, GHipError* err) {
  bytes = round_alloc(bytes ? bytes : 1);
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = free_blocks.find(bytes);
    if (it != free_blocks.end()) {
      *out = it->second;
      free_blocks.erase(it);
      cached_bytes -= bytes;
      return GHIP_OK;
    }
  }
  if (plan_only) return set_error(err, GHIP_ERR_STATE, "plan-only backend cannot allocate device memory");
  hipSetDevice(device);
  hipError_t e = hipMalloc(out, bytes);
  if (e != hipSuccess) {
    trim();
    e = hipMalloc(out, bytes);
  }
  if (e != hipSuccess)
    return set_error(err, GHIP_ERR_OOM, "device allocation of %zu bytes failed: %s", bytes,
                     hipGetErrorString(e));
  return GHIP_OK;
}

void GHipBackend::release(void* p, size_t bytes) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(mu);
  if (finalized) return;
  bytes = round_alloc(bytes ? bytes : 1);
  free_blocks.emplace(bytes, p);
  cached_bytes += bytes;
}

void GHipBackend::trim() {
  std::lock_guard<std::mutex> lk(mu);
  if (plan_only) return;
  hipSetDevice(device);
  hipDeviceSynchronize();
  for (auto& kv : free_blocks) hipFree(kv.second);
  free_blocks.clear();
  cached_bytes = 0;
}

extern "C" GHipBackend* ghip_backend_new(const char* config, GHipError* err) {
  auto be = std::make_unique<GHipBackend>();
  std::string cfg = config ? config : "";
  if (cfg == "plan") {
    be->plan_only = true;
    be->device_name = "plan-only (no device)";
    return be.release();
  }
  int dev = 0;
  if (!cfg.empty()) {
    const char* p = strstr(cfg.c_str(), "device=");
    if (cfg.rfind("hip", 0) != 0 || (cfg != "hip" && !p)) {
      set_error(err, GHIP_ERR_INVALID_ARG, "backend config \"%s\": expected \"hip:device=N\"", cfg.c_str());
      return nullptr;
    }
    if (p) dev = atoi(p + 7);
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    set_error(err, GHIP_ERR_HIP, "no HIP device visible");
    return nullptr;
  }
  if (dev < 0 || dev >= count) {
    set_error(err, GHIP_ERR_INVALID_ARG, "device %d out of range (have %d)", dev, count);
    return nullptr;
  }
  be->device = dev;
  hipError_t e = hipSetDevice(dev);
  if (e != hipSuccess) {
    check_hip(e, err, "hipSetDevice");
    return nullptr;
  }
  // Default-priority stream (no priority changes on this platform).
  e = hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    check_hip(e, err, "hipStreamCreate");
    return nullptr;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof buf, "%s (%s, %d CUs, %zu MiB)", prop.name, prop.gcnArchName,
             prop.multiProcessorCount, static_cast<size_t>(prop.totalGlobalMem >> 20));
    be->device_name = buf;
  }
  return be.release();
}

extern "C" void ghip_backend_finalize(GHipBackend* b) {
  if (!b || b->finalized) return;
  b->trim();
  std::lock_guard<std::mutex> lk(b->mu);
  b->finalized = true;
  if (b->stream) {
    hipSetDevice(b->device);
    hipStreamSynchronize(b->stream);
    hipStreamDestroy(b->stream);
    b->stream = nullptr;
  }
}

extern "C" int ghip_backend_is_finalized(GHipBackend* b) { return !b || b->finalized; }

extern "C" int ghip_backend_description(GHipBackend* b, char* buf, size_t buflen) {
  if (!b || !buf || !buflen) return -1;
  return snprintf(buf, buflen, "HIP GPU backend (%s)", b->device_name.c_str());
}

// Capabilities (capabilities.go:14-166): the GoMLX OpType names (without the
// "OpType" prefix) this backend builds, and the dtypes it holds.  Ops of the
// reference's list that are absent here: BatchNorm*, ConvGeneral,
// ReduceWindow, SelectAndScatterMax and RNGBitGenerator.  The dtype list is the
// reference's (capabilities.go:153-166): Float64 is not declared there, so it is
// not declared here either, although the elementwise, reduce, scatter and copy
// kernels accept it.
extern "C" int ghip_backend_capabilities(char* buf, size_t buflen) {
  static const char kCaps[] =
      "functions=1;ops="
      "Parameter,Constant,"
      "Abs,Neg,Sqrt,Rsqrt,Exp,Expm1,Log,Log1p,Sin,Cos,Tanh,Logistic,Erf,Floor,Ceil,Round,Sign,"
      "LogicalNot,BitwiseNot,IsFinite,IsNaN,Identity,"
      "Add,Sub,Mul,Div,Rem,Pow,Max,Min,Atan2,LogicalAnd,LogicalOr,LogicalXor,BitwiseAnd,BitwiseOr,"
      "BitwiseXor,ShiftLeft,ShiftRightArithmetic,ShiftRightLogical,"
      "Equal,NotEqual,GreaterThan,GreaterOrEqual,LessThan,LessOrEqual,"
      "EqualTotalOrder,NotEqualTotalOrder,GreaterThanTotalOrder,GreaterOrEqualTotalOrder,"
      "LessThanTotalOrder,LessOrEqualTotalOrder,"
      "Reshape,Transpose,ConvertDType,BroadcastInDim,Where,Clamp,Slice,Concatenate,Reverse,Iota,Pad,"
      "DotGeneral,ReduceSum,ReduceMax,ReduceMin,ReduceProduct,ReduceLogicalAnd,ReduceLogicalOr,"
      "ArgMinMax,Gather,ScatterSum,ScatterMax,ScatterMin,DynamicSlice,DynamicUpdateSlice,"
      "FusedSoftmax,FusedLayerNorm,FusedGelu,FusedDense,FusedAttentionQKVProjection,"
      "FusedScaledDotProductAttention,While,If,Sort,Call;dtypes="
      "Bool,Int8,Int16,Int32,Int64,Float16,BFloat16,Float32,Uint8,Uint16,Uint32,Uint64";
  if (buf && buflen) snprintf(buf, buflen, "%s", kCaps);
  return static_cast<int>(sizeof(kCaps) - 1);
}

extern "C" int ghip_backend_num_devices(GHipBackend* b) { return b && !b->plan_only ? 1 : 0; }
extern "C" void* ghip_backend_stream(GHipBackend* b) { return b ? b->stream : nullptr; }

// ===========================================================================
// Buffers
// ===========================================================================
static bool make_shape(int dtype, const int64_t* dims, int rank, Shape* s, GHipError* err,
                       const char* what) {
  if (dtype_size(dtype) == 0) {
    set_error(err, GHIP_ERR_INVALID_ARG, "%s: invalid dtype %d", what, dtype);
    return false;
  }
  if (rank < 0 || rank > kMaxRank || (rank > 0 && !dims)) {
    set_error(err, GHIP_ERR_INVALID_ARG, "%s: rank %d not supported (max %d)", what, rank, kMaxRank);
    return false;
  }
  s->dtype = dtype;
  s->dims.assign(dims, dims + rank);
  for (auto d : s->dims)
    if (d < 0) {
      set_error(err, GHIP_ERR_INVALID_ARG, "%s: negative dimension", what);
      return false;
    }
  return true;
}

static GHipBuffer* new_buffer(GHipBackend* b, const Shape& s, GHipError* err) {
  auto buf = std::make_unique<GHipBuffer>();
  buf->backend = b;
  buf->shape = s;
  buf->cap = s.bytes();
  if (b->alloc(buf->cap, &buf->ptr, err) != GHIP_OK) return nullptr;
  return buf.release();
}

extern "C" GHipBuffer* ghip_buffer_new(GHipBackend* b, int dtype, const int64_t* dims, int rank,
                                       GHipError* err) {
  if (!b || b->finalized) { set_error(err, GHIP_ERR_STATE, "buffer_new: backend finalized"); return nullptr; }
  Shape s;
  if (!make_shape(dtype, dims, rank, &s, err, "buffer_new")) return nullptr;
  return new_buffer(b, s, err);
}

extern "C" GHipBuffer* ghip_buffer_from_host(GHipBackend* b, int dtype, const int64_t* dims,
                                             int rank, const void* data, size_t nbytes,
                                             GHipError* err) {
  if (!b || b->finalized) { set_error(err, GHIP_ERR_STATE, "BufferFromFlatData: backend finalized"); return nullptr; }
  Shape s;
  if (!make_shape(dtype, dims, rank, &s, err, "BufferFromFlatData")) return nullptr;
  if (nbytes != s.bytes()) {
    set_error(err, GHIP_ERR_INVALID_ARG, "BufferFromFlatData: %zu bytes given for shape %s (%zu bytes)",
              nbytes, s.str().c_str(), s.bytes());
    return nullptr;
  }
  GHipBuffer* buf = new_buffer(b, s, err);
  if (!buf) return nullptr;
  if (nbytes) {
    hipSetDevice(b->device);
    hipError_t e = hipMemcpyAsync(buf->ptr, data, nbytes, hipMemcpyHostToDevice, b->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
    if (e != hipSuccess) {
      check_hip(e, err, "BufferFromFlatData copy");
      b->release(buf->ptr, buf->cap);
      delete buf;
      return nullptr;
    }
  }
  return buf;
}

extern "C" int ghip_buffer_to_host(GHipBuffer* buf, void* data, size_t nbytes, GHipError* err) {
  if (!buf || !buf->valid) return set_error(err, GHIP_ERR_STATE, "BufferToFlatData: buffer finalized");
  if (nbytes != buf->shape.bytes())
    return set_error(err, GHIP_ERR_INVALID_ARG, "BufferToFlatData: %zu bytes for shape %s (%zu bytes)",
                     nbytes, buf->shape.str().c_str(), buf->shape.bytes());
  if (!nbytes) return GHIP_OK;
  GHipBackend* b = buf->backend;
  hipSetDevice(b->device);
  GHIP_CHECK(hipMemcpyAsync(data, buf->ptr, nbytes, hipMemcpyDeviceToHost, b->stream), err);
  GHIP_CHECK(hipStreamSynchronize(b->stream), err);
  return GHIP_OK;
}

extern "C" int ghip_buffer_shape(GHipBuffer* buf, int* dtype, int64_t* dims, int max_rank) {
  if (!buf || !buf->valid) return -1;
  if (dtype) *dtype = buf->shape.dtype;
  for (int i = 0; i < buf->shape.rank() && i < max_rank; ++i) dims[i] = buf->shape.dims[i];
  return buf->shape.rank();
}

extern "C" void* ghip_buffer_device_ptr(GHipBuffer* buf) { return buf && buf->valid ? buf->ptr : nullptr; }

extern "C" void ghip_buffer_finalize(GHipBuffer* buf) {
  if (!buf) return;
  if (buf->valid && buf->backend && buf->ptr) {
    // Stream-ordered release: every use of a backend buffer (Execute's kernels,
    // BufferFromFlatData / BufferToFlatData copies) is enqueued on the backend's
    // one stream, so the block can go back to the cache now: whatever allocation
    // takes it next is used by work enqueued after everything already queued
    // against this buffer.  (A caller that used BufferData's pointer on another
    // stream must synchronise that stream before finalizing.)
    buf->backend->release(buf->ptr, buf->cap);
  }
  buf->valid = false;
  delete buf;
}

// ===========================================================================
// Builder
// ===========================================================================
extern "C" GHipBuilder* ghip_builder_new(GHipBackend* b, const char* name, GHipError* err) {
  if (!b || b->finalized) { set_error(err, GHIP_ERR_STATE, "Builder: backend finalized"); return nullptr; }
  auto bl = new GHipBuilder();
  bl->backend = b;
  bl->name = name ? name : "";
  bl->table.push_back(nullptr);  // index 0: the main function, created on demand
  return bl;
}

extern "C" void ghip_builder_finalize(GHipBuilder* bl) { delete bl; }

extern "C" GHipFunction* ghip_builder_main(GHipBuilder* bl) {
  if (!bl) return nullptr;
  if (!bl->main) {
    bl->main = std::make_unique<GHipFunction>();
    bl->main->builder = bl;
    bl->main->name = "main";
    bl->main->index = 0;
    if (bl->table.empty()) bl->table.push_back(nullptr);
    bl->table[0] = bl->main.get();
  }
  return bl->main.get();
}

// ===========================================================================
// Function: shape inference helpers
// ===========================================================================
namespace {

struct Ctx {
  GHipFunction* f;
  GHipError* err;
  const char* op;
  bool ok = true;
  int fail(int code, const char* fmt, ...) {
    char buf[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error(err, code, "%s: %s", op, buf);
    ok = false;
    return -1;
  }
  // Node index in f of the value with (builder-wide) id v; a value of an
  // enclosing function is captured (through every function in between).
  int loc(int v) {
    if (!f) { fail(GHIP_ERR_INVALID_ARG, "null function"); return -1; }
    if (v < 0) return v;
    GHipBuilder* b = f->builder;
    const int fi = v >> kFnShift, li = v & kNodeMask;
    GHipFunction* g = b && fi < static_cast<int>(b->table.size()) ? b->table[fi] : (fi == 0 ? f : nullptr);
    if (!g || li >= static_cast<int>(g->nodes.size())) {
      fail(GHIP_ERR_INVALID_ARG, "value %d does not belong to this builder", v);
      return -1;
    }
    if (g == f) return li;
    GHipFunction* p = f->parent;
    while (p && p != g) p = p->parent;
    if (!p) {
      fail(GHIP_ERR_INVALID_ARG, "value %d belongs to function %s, which does not enclose %s", v, g->name.c_str(),
           f->name.c_str());
      return -1;
    }
    return capture(f, g, li);
  }
  static int capture(GHipFunction* h, GHipFunction* g, int li) {
    if (h == g) return li;
    const int pl = capture(h->parent, g, li);
    auto it = h->capture_of.find(pl);
    if (it != h->capture_of.end()) return it->second;
    Node cn{Kind::Capture};
    cn.shape = h->parent->nodes[pl].shape;
    cn.i0 = static_cast<int64_t>(h->captures.size());
    const int id = h->add(std::move(cn));
    h->captures.push_back(pl);
    h->capture_of[pl] = id;
    return id;
  }
  const Node* node(int v) {
    if (!f) { fail(GHIP_ERR_INVALID_ARG, "null function"); return nullptr; }
    if (f->returned) { fail(GHIP_ERR_STATE, "function already returned"); return nullptr; }
    const int l = loc(v);
    if (l < 0) {
      if (ok) fail(GHIP_ERR_INVALID_ARG, "value %d does not belong to function %s", v, f->name.c_str());
      return nullptr;
    }
    return &f->nodes[l];
  }
  // Appends n (operands given as value ids) and returns its value id.
  int add(Node&& n) {
    for (auto& i : n.in) {
      if (i < 0) continue;
      i = loc(i);
      if (i < 0) return -1;
    }
    return f->global(f->add(std::move(n)));
  }
};

// Shape of the value with id v, looked up in its own function.
const Node* value_node(GHipFunction* f, int v) {
  if (!f || v < 0) return nullptr;
  GHipBuilder* b = f->builder;
  const int fi = v >> kFnShift, li = v & kNodeMask;
  GHipFunction* g = b && fi < static_cast<int>(b->table.size()) ? b->table[fi] : (fi == 0 ? f : nullptr);
  if (!g || li >= static_cast<int>(g->nodes.size())) return nullptr;
  return &g->nodes[li];
}

// numpy-style broadcast of two shapes (equal dims, size-1 dims, or rank-0 scalars).
bool broadcast_dims(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                    std::vector<int64_t>* out) {
  if (a.empty()) { *out = b; return true; }
  if (b.empty()) { *out = a; return true; }
  size_t r = std::max(a.size(), b.size());
  out->assign(r, 1);
  for (size_t i = 0; i < r; ++i) {
    int64_t da = i < r - a.size() ? 1 : a[i - (r - a.size())];
    int64_t db = i < r - b.size() ? 1 : b[i - (r - b.size())];
    if (da != db && da != 1 && db != 1) return false;
    (*out)[i] = da == 1 ? db : da;
  }
  return true;
}

bool normalize_axes(const int* axes, int n, int rank, std::vector<int64_t>* out) {
  out->clear();
  std::set<int64_t> seen;
  for (int i = 0; i < n; ++i) {
    int64_t a = axes[i] < 0 ? axes[i] + rank : axes[i];
    if (a < 0 || a >= rank || seen.count(a)) return false;
    seen.insert(a);
    out->push_back(a);
  }
  return true;
}

}  // namespace

#define FN_BEGIN(opname) Ctx c{f, err, opname}

extern "C" GHipValue ghip_fn_parameter(GHipFunction* f, const char* name, int dtype,
                                       const int64_t* dims, int rank, GHipError* err) {
  FN_BEGIN("Parameter");
  if (!f) return c.fail(GHIP_ERR_INVALID_ARG, "null function");
  if (f->returned) return c.fail(GHIP_ERR_STATE, "function already returned");
  Node n{Kind::Param};
  if (!make_shape(dtype, dims, rank, &n.shape, err, "Parameter")) return -1;
  n.name = name ? name : "";
  n.i0 = static_cast<int64_t>(f->params.size());
  int id = f->add(std::move(n));
  f->params.push_back(id);
  return f->global(id);
}

extern "C" GHipValue ghip_fn_constant(GHipFunction* f, int dtype, const int64_t* dims, int rank,
                                      const void* data, size_t nbytes, GHipError* err) {
  FN_BEGIN("Constant");
  if (!f) return c.fail(GHIP_ERR_INVALID_ARG, "null function");
  if (f->returned) return c.fail(GHIP_ERR_STATE, "function already returned");
  Node n{Kind::Const};
  if (!make_shape(dtype, dims, rank, &n.shape, err, "Constant")) return -1;
  if (nbytes != n.shape.bytes())
    return c.fail(GHIP_ERR_INVALID_ARG, "%zu bytes for shape %s", nbytes, n.shape.str().c_str());
  if (nbytes && !data) return c.fail(GHIP_ERR_INVALID_ARG, "null data");
  n.data.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + nbytes);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_iota(GHipFunction* f, int dtype, const int64_t* dims, int rank,
                                  int axis, GHipError* err) {
  FN_BEGIN("Iota");
  if (!f) return c.fail(GHIP_ERR_INVALID_ARG, "null function");
  Node n{Kind::Iota};
  if (!make_shape(dtype, dims, rank, &n.shape, err, "Iota")) return -1;
  if (dtype == GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "bool iota");
  if (axis < 0) axis += rank;
  if (axis < 0 || axis >= rank) return c.fail(GHIP_ERR_INVALID_ARG, "axis out of range");
  n.i0 = axis;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_unary(GHipFunction* f, int op, GHipValue x, GHipError* err) {
  FN_BEGIN("Unary");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (op < 0 || op >= GHIP_UNARY_COUNT) return c.fail(GHIP_ERR_INVALID_ARG, "bad unary op %d", op);
  const int dt = a->shape.dtype;
  Node n{Kind::Unary};
  n.sub = op;
  n.in = {x};
  n.shape = a->shape;
  switch (op) {
    case GHIP_UNARY_SQRT: case GHIP_UNARY_RSQRT: case GHIP_UNARY_EXP: case GHIP_UNARY_EXPM1:
    case GHIP_UNARY_LOG: case GHIP_UNARY_LOG1P: case GHIP_UNARY_SIN: case GHIP_UNARY_COS:
    case GHIP_UNARY_TANH: case GHIP_UNARY_LOGISTIC: case GHIP_UNARY_ERF: case GHIP_UNARY_FLOOR:
    case GHIP_UNARY_CEIL: case GHIP_UNARY_ROUND:
      if (!dtype_is_float(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "op %d needs a float operand, got %s", op, dtype_name(dt));
      break;
    case GHIP_UNARY_LOGICAL_NOT:
      if (dt != GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "LogicalNot needs bool");
      break;
    case GHIP_UNARY_BITWISE_NOT:
      if (!dtype_is_int(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "BitwiseNot needs an integer");
      break;
    case GHIP_UNARY_IS_FINITE: case GHIP_UNARY_IS_NAN:
      if (!dtype_is_float(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "needs a float operand");
      n.shape.dtype = GHIP_DTYPE_BOOL;
      break;
    case GHIP_UNARY_ABS: case GHIP_UNARY_NEG: case GHIP_UNARY_SIGN:
      if (dt == GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "bool operand");
      break;
    default: break;
  }
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_binary(GHipFunction* f, int op, GHipValue lhs, GHipValue rhs,
                                    GHipError* err) {
  FN_BEGIN("Binary");
  const Node* a = c.node(lhs);
  if (!a) return -1;
  const Node* b = c.node(rhs);
  if (!b) return -1;
  if (op < 0 || op >= GHIP_BINARY_COUNT) return c.fail(GHIP_ERR_INVALID_ARG, "bad binary op %d", op);
  if (a->shape.dtype != b->shape.dtype)
    return c.fail(GHIP_ERR_INVALID_ARG, "dtype mismatch %s vs %s", dtype_name(a->shape.dtype), dtype_name(b->shape.dtype));
  const int dt = a->shape.dtype;
  const bool logical = op == GHIP_BINARY_LOGICAL_AND || op == GHIP_BINARY_LOGICAL_OR || op == GHIP_BINARY_LOGICAL_XOR;
  const bool bitwise = op >= GHIP_BINARY_BITWISE_AND;
  if (logical && dt != GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "logical op needs bool");
  if (bitwise && !dtype_is_int(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "bitwise op needs integers");
  if (!logical && !bitwise && dt == GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "arithmetic on bool");
  if (op == GHIP_BINARY_ATAN2 && !dtype_is_float(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "Atan2 needs floats");
  Node n{Kind::Binary};
  n.sub = op;
  n.in = {lhs, rhs};
  n.shape.dtype = dt;
  if (!broadcast_dims(a->shape.dims, b->shape.dims, &n.shape.dims))
    return c.fail(GHIP_ERR_INVALID_ARG, "incompatible shapes %s and %s", a->shape.str().c_str(), b->shape.str().c_str());
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_compare(GHipFunction* f, int op, GHipValue lhs, GHipValue rhs,
                                     GHipError* err) {
  FN_BEGIN("Compare");
  const Node* a = c.node(lhs);
  if (!a) return -1;
  const Node* b = c.node(rhs);
  if (!b) return -1;
  if (op < 0 || op >= GHIP_CMP_COUNT) return c.fail(GHIP_ERR_INVALID_ARG, "bad comparison %d", op);
  if (a->shape.dtype != b->shape.dtype) return c.fail(GHIP_ERR_INVALID_ARG, "dtype mismatch");
  Node n{Kind::Compare};
  n.sub = op;
  n.in = {lhs, rhs};
  n.shape.dtype = GHIP_DTYPE_BOOL;
  if (!broadcast_dims(a->shape.dims, b->shape.dims, &n.shape.dims))
    return c.fail(GHIP_ERR_INVALID_ARG, "incompatible shapes %s and %s", a->shape.str().c_str(), b->shape.str().c_str());
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_where(GHipFunction* f, GHipValue cond, GHipValue on_true,
                                   GHipValue on_false, GHipError* err) {
  FN_BEGIN("Where");
  const Node* p = c.node(cond);
  if (!p) return -1;
  const Node* t = c.node(on_true);
  if (!t) return -1;
  const Node* e = c.node(on_false);
  if (!e) return -1;
  if (p->shape.dtype != GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "condition must be bool");
  if (t->shape.dtype != e->shape.dtype) return c.fail(GHIP_ERR_INVALID_ARG, "branch dtypes differ");
  Node n{Kind::Where};
  n.in = {cond, on_true, on_false};
  n.shape.dtype = t->shape.dtype;
  std::vector<int64_t> d1;
  if (!broadcast_dims(t->shape.dims, e->shape.dims, &d1) ||
      !broadcast_dims(p->shape.dims, d1, &n.shape.dims))
    return c.fail(GHIP_ERR_INVALID_ARG, "incompatible shapes");
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_clamp(GHipFunction* f, GHipValue lo, GHipValue x, GHipValue hi,
                                   GHipError* err) {
  FN_BEGIN("Clamp");
  const Node* l = c.node(lo);
  if (!l) return -1;
  const Node* v = c.node(x);
  if (!v) return -1;
  const Node* h = c.node(hi);
  if (!h) return -1;
  if (l->shape.dtype != v->shape.dtype || h->shape.dtype != v->shape.dtype)
    return c.fail(GHIP_ERR_INVALID_ARG, "dtype mismatch");
  std::vector<int64_t> tmp;
  if (!broadcast_dims(l->shape.dims, v->shape.dims, &tmp) || tmp != v->shape.dims ||
      !broadcast_dims(h->shape.dims, v->shape.dims, &tmp) || tmp != v->shape.dims)
    return c.fail(GHIP_ERR_INVALID_ARG, "min/max must be scalars or x's shape");
  Node n{Kind::Clamp};
  n.in = {lo, x, hi};
  n.shape = v->shape;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_convert_dtype(GHipFunction* f, GHipValue x, int dtype, GHipError* err) {
  FN_BEGIN("ConvertDType");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (dtype_size(dtype) == 0) return c.fail(GHIP_ERR_INVALID_ARG, "invalid dtype %d", dtype);
  Node n{Kind::Convert};
  n.in = {x};
  n.shape = a->shape;
  n.shape.dtype = dtype;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_reshape(GHipFunction* f, GHipValue x, const int64_t* dims, int rank,
                                     GHipError* err) {
  FN_BEGIN("Reshape");
  const Node* a = c.node(x);
  if (!a) return -1;
  Node n{Kind::Reshape};
  if (!make_shape(a->shape.dtype, dims, rank, &n.shape, err, "Reshape")) return -1;
  if (n.shape.size() != a->shape.size())
    return c.fail(GHIP_ERR_INVALID_ARG, "cannot reshape %s to %s", a->shape.str().c_str(), n.shape.str().c_str());
  n.in = {x};
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_transpose(GHipFunction* f, GHipValue x, const int* perm, int rank,
                                       GHipError* err) {
  FN_BEGIN("Transpose");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (rank != a->shape.rank()) return c.fail(GHIP_ERR_INVALID_ARG, "permutation rank %d vs %d", rank, a->shape.rank());
  std::vector<int64_t> p;
  if (!normalize_axes(perm, rank, rank, &p)) return c.fail(GHIP_ERR_INVALID_ARG, "invalid permutation");
  Node n{Kind::Transpose};
  n.in = {x};
  n.a0 = p;
  n.shape.dtype = a->shape.dtype;
  for (auto i : p) n.shape.dims.push_back(a->shape.dims[i]);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_broadcast_in_dim(GHipFunction* f, GHipValue x, const int64_t* dims,
                                              int rank, const int* axes, int naxes, GHipError* err) {
  FN_BEGIN("BroadcastInDim");
  const Node* a = c.node(x);
  if (!a) return -1;
  Node n{Kind::Broadcast};
  if (!make_shape(a->shape.dtype, dims, rank, &n.shape, err, "BroadcastInDim")) return -1;
  if (naxes != a->shape.rank()) return c.fail(GHIP_ERR_INVALID_ARG, "%d axes for rank-%d operand", naxes, a->shape.rank());
  std::vector<int64_t> ax;
  if (!normalize_axes(axes, naxes, rank, &ax)) return c.fail(GHIP_ERR_INVALID_ARG, "invalid broadcast axes");
  for (int i = 0; i < naxes; ++i) {
    if (i > 0 && ax[i] <= ax[i - 1]) return c.fail(GHIP_ERR_INVALID_ARG, "broadcast axes must increase");
    const int64_t d = a->shape.dims[i];
    if (d != 1 && d != n.shape.dims[ax[i]])
      return c.fail(GHIP_ERR_INVALID_ARG, "operand dim %d (%lld) vs output dim %lld", i, (long long)d,
                    (long long)n.shape.dims[ax[i]]);
  }
  n.in = {x};
  n.a0 = ax;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_reduce(GHipFunction* f, int op, GHipValue x, const int* axes, int naxes,
                                    GHipError* err) {
  FN_BEGIN("Reduce");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (op < 0 || op > GHIP_REDUCE_MIN) return c.fail(GHIP_ERR_INVALID_ARG, "bad reduce op %d", op);
  if (a->shape.dtype == GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "bool reduction");
  std::vector<int64_t> ax;
  if (naxes == 0) {  // empty axes: reduce everything (function.go:1152-1158)
    for (int i = 0; i < a->shape.rank(); ++i) ax.push_back(i);
  } else if (!normalize_axes(axes, naxes, a->shape.rank(), &ax)) {
    return c.fail(GHIP_ERR_INVALID_ARG, "invalid axes");
  }
  std::sort(ax.begin(), ax.end());
  Node n{Kind::Reduce};
  n.sub = op;
  n.in = {x};
  n.a0 = ax;
  n.shape.dtype = a->shape.dtype;
  for (int i = 0; i < a->shape.rank(); ++i)
    if (!std::binary_search(ax.begin(), ax.end(), i)) n.shape.dims.push_back(a->shape.dims[i]);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_arg_min_max(GHipFunction* f, GHipValue x, int axis, int out_dtype,
                                         int is_min, GHipError* err) {
  FN_BEGIN("ArgMinMax");
  const Node* a = c.node(x);
  if (!a) return -1;
  const int r = a->shape.rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) return c.fail(GHIP_ERR_INVALID_ARG, "axis out of range");
  if (a->shape.dims[axis] == 0) return c.fail(GHIP_ERR_INVALID_ARG, "empty reduced axis");
  if (out_dtype != GHIP_DTYPE_INT32 && out_dtype != GHIP_DTYPE_INT64)
    return c.fail(GHIP_ERR_UNSUPPORTED, "output dtype %s", dtype_name(out_dtype));
  if (!dtype_is_float(a->shape.dtype)) return c.fail(GHIP_ERR_UNSUPPORTED, "input dtype %s", dtype_name(a->shape.dtype));
  Node n{Kind::ArgMinMax};
  n.in = {x};
  n.i0 = axis;
  n.i1 = is_min ? 1 : 0;
  n.shape.dtype = out_dtype;
  for (int i = 0; i < r; ++i)
    if (i != axis) n.shape.dims.push_back(a->shape.dims[i]);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_dot_general(GHipFunction* f, GHipValue lhs, const int* lc, int nlc,
                                         const int* lb, int nlb, GHipValue rhs, const int* rc,
                                         int nrc, const int* rb, int nrb, GHipError* err) {
  FN_BEGIN("DotGeneral");
  const Node* a = c.node(lhs);
  if (!a) return -1;
  const Node* b = c.node(rhs);
  if (!b) return -1;
  if (a->shape.dtype != b->shape.dtype) return c.fail(GHIP_ERR_INVALID_ARG, "dtype mismatch");
  if (nlc != nrc || nlb != nrb) return c.fail(GHIP_ERR_INVALID_ARG, "axis count mismatch");
  std::vector<int64_t> lca, lba, rca, rba;
  std::vector<int> lall(lc, lc + nlc), rall(rc, rc + nrc);
  lall.insert(lall.end(), lb, lb + nlb);
  rall.insert(rall.end(), rb, rb + nrb);
  std::vector<int64_t> tmp;
  if (!normalize_axes(lall.data(), nlc + nlb, a->shape.rank(), &tmp) ||
      !normalize_axes(rall.data(), nrc + nrb, b->shape.rank(), &tmp))
    return c.fail(GHIP_ERR_INVALID_ARG, "invalid or repeated axes");
  normalize_axes(lc, nlc, a->shape.rank(), &lca);
  normalize_axes(lb, nlb, a->shape.rank(), &lba);
  normalize_axes(rc, nrc, b->shape.rank(), &rca);
  normalize_axes(rb, nrb, b->shape.rank(), &rba);
  for (int i = 0; i < nlc; ++i)
    if (a->shape.dims[lca[i]] != b->shape.dims[rca[i]]) return c.fail(GHIP_ERR_INVALID_ARG, "contracting dims differ");
  for (int i = 0; i < nlb; ++i)
    if (a->shape.dims[lba[i]] != b->shape.dims[rba[i]]) return c.fail(GHIP_ERR_INVALID_ARG, "batch dims differ");
  if (!dtype_is_float(a->shape.dtype) || a->shape.dtype == GHIP_DTYPE_FLOAT64)
    return c.fail(GHIP_ERR_UNSUPPORTED, "dtype %s (float32, bfloat16 and float16 are lowered)",
                  dtype_name(a->shape.dtype));
  Node n{Kind::Dot};
  n.in = {lhs, rhs};
  n.a0 = lca; n.a1 = lba; n.a2 = rca; n.a3 = rba;
  // Output: [batch..., lhs free..., rhs free...] (dotgeneral.go:15-53), lhs dtype.
  n.shape.dtype = a->shape.dtype;
  for (auto ax : lba) n.shape.dims.push_back(a->shape.dims[ax]);
  for (int i = 0; i < a->shape.rank(); ++i)
    if (std::find(lca.begin(), lca.end(), i) == lca.end() && std::find(lba.begin(), lba.end(), i) == lba.end())
      n.shape.dims.push_back(a->shape.dims[i]);
  for (int i = 0; i < b->shape.rank(); ++i)
    if (std::find(rca.begin(), rca.end(), i) == rca.end() && std::find(rba.begin(), rba.end(), i) == rba.end())
      n.shape.dims.push_back(b->shape.dims[i]);
  if (n.shape.rank() > kMaxRank) return c.fail(GHIP_ERR_UNSUPPORTED, "output rank too large");
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_gather(GHipFunction* f, GHipValue operand, GHipValue start_indices,
                                    int index_vector_axis, const int* offset_output_axes, int n_offset,
                                    const int* collapsed_slice_axes, int n_collapsed,
                                    const int* start_index_map, int n_map, const int64_t* slice_sizes,
                                    int n_sizes, int indices_are_sorted, GHipError* err) {
  FN_BEGIN("Gather");
  const Node* op = c.node(operand);
  if (!op) return -1;
  const Node* ix = c.node(start_indices);
  if (!ix) return -1;
  const int r = op->shape.rank(), ir = ix->shape.rank();
  if (!dtype_is_int(ix->shape.dtype)) return c.fail(GHIP_ERR_INVALID_ARG, "indices must be integers");
  if (n_sizes != r) return c.fail(GHIP_ERR_INVALID_ARG, "slice_sizes must have operand rank");
  if (index_vector_axis < 0 || index_vector_axis > ir) return c.fail(GHIP_ERR_INVALID_ARG, "bad index_vector_axis");
  const int64_t ivec = index_vector_axis < ir ? ix->shape.dims[index_vector_axis] : 1;
  if (ivec != n_map) return c.fail(GHIP_ERR_INVALID_ARG, "index vector size %lld vs start_index_map %d", (long long)ivec, n_map);
  for (int i = 0; i < r; ++i)
    if (slice_sizes[i] < 0 || slice_sizes[i] > op->shape.dims[i]) return c.fail(GHIP_ERR_INVALID_ARG, "slice size out of range");
  std::vector<int64_t> coll, omap, offs;
  if (!normalize_axes(collapsed_slice_axes, n_collapsed, r, &coll) || !normalize_axes(start_index_map, n_map, r, &omap))
    return c.fail(GHIP_ERR_INVALID_ARG, "invalid axes");
  for (auto a : coll)
    if (slice_sizes[a] != 1) return c.fail(GHIP_ERR_INVALID_ARG, "collapsed axes need slice size 1");
  std::vector<int64_t> offset_dims;
  for (int i = 0; i < r; ++i)
    if (std::find(coll.begin(), coll.end(), i) == coll.end()) offset_dims.push_back(slice_sizes[i]);
  if (static_cast<int>(offset_dims.size()) != n_offset) return c.fail(GHIP_ERR_INVALID_ARG, "offset_output_axes size");
  std::vector<int64_t> batch_dims;
  for (int i = 0; i < ir; ++i)
    if (i != index_vector_axis) batch_dims.push_back(ix->shape.dims[i]);
  const int orank = static_cast<int>(batch_dims.size()) + n_offset;
  if (!normalize_axes(offset_output_axes, n_offset, orank, &offs)) return c.fail(GHIP_ERR_INVALID_ARG, "bad offset_output_axes");
  Node n{Kind::Gather};
  n.in = {operand, start_indices};
  n.shape.dtype = op->shape.dtype;
  n.shape.dims.assign(orank, 0);
  size_t bi = 0, oi = 0;
  for (int i = 0; i < orank; ++i) {
    if (std::find(offs.begin(), offs.end(), i) != offs.end()) n.shape.dims[i] = offset_dims[oi++];
    else n.shape.dims[i] = batch_dims[bi++];
  }
  n.i0 = index_vector_axis;
  n.i1 = indices_are_sorted;
  n.a0 = offs;
  n.a1 = coll;
  n.a2 = omap;
  n.a3.assign(slice_sizes, slice_sizes + n_sizes);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_slice(GHipFunction* f, GHipValue x, const int64_t* starts,
                                   const int64_t* limits, const int64_t* strides, int rank,
                                   GHipError* err) {
  FN_BEGIN("Slice");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (rank != a->shape.rank()) return c.fail(GHIP_ERR_INVALID_ARG, "rank mismatch");
  Node n{Kind::Slice};
  n.in = {x};
  n.shape.dtype = a->shape.dtype;
  for (int i = 0; i < rank; ++i) {
    const int64_t st = strides ? strides[i] : 1;
    if (starts[i] < 0 || limits[i] > a->shape.dims[i] || starts[i] > limits[i] || st <= 0)
      return c.fail(GHIP_ERR_INVALID_ARG, "bad bounds on axis %d", i);
    n.a0.push_back(starts[i]);
    n.a1.push_back(limits[i]);
    n.a2.push_back(st);
    n.shape.dims.push_back((limits[i] - starts[i] + st - 1) / st);
  }
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_concatenate(GHipFunction* f, int axis, const GHipValue* operands, int cnt,
                                         GHipError* err) {
  FN_BEGIN("Concatenate");
  if (cnt <= 0) return c.fail(GHIP_ERR_INVALID_ARG, "no operands");
  const Node* first = c.node(operands[0]);
  if (!first) return -1;
  const int r = first->shape.rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) return c.fail(GHIP_ERR_INVALID_ARG, "axis out of range");
  Node n{Kind::Concat};
  n.shape = first->shape;
  n.shape.dims[axis] = 0;
  for (int i = 0; i < cnt; ++i) {
    const Node* o = c.node(operands[i]);
    if (!o) return -1;
    if (o->shape.dtype != first->shape.dtype || o->shape.rank() != r) return c.fail(GHIP_ERR_INVALID_ARG, "operand %d mismatch", i);
    for (int d = 0; d < r; ++d)
      if (d != axis && o->shape.dims[d] != first->shape.dims[d]) return c.fail(GHIP_ERR_INVALID_ARG, "operand %d dims", i);
    n.shape.dims[axis] += o->shape.dims[axis];
    n.in.push_back(operands[i]);
  }
  n.i0 = axis;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_reverse(GHipFunction* f, GHipValue x, const int* axes, int naxes,
                                     GHipError* err) {
  FN_BEGIN("Reverse");
  const Node* a = c.node(x);
  if (!a) return -1;
  std::vector<int64_t> ax;
  if (!normalize_axes(axes, naxes, a->shape.rank(), &ax)) return c.fail(GHIP_ERR_INVALID_ARG, "invalid axes");
  Node n{Kind::Reverse};
  n.in = {x};
  n.a0 = ax;
  n.shape = a->shape;
  return c.add(std::move(n));
}

namespace {
GHipValue wrap(GHipValue v, GHipError* err, const char* op);
}  // namespace

// Pad (function.go:1533-1569): edge padding with a scalar fill value; interior
// padding is refused as the reference refuses it.  Negative padding crops (XLA
// semantics).  Composed of a Slice for the crops and, per padded axis, a
// Concatenate of fill blocks around the operand.
extern "C" GHipValue ghip_fn_pad(GHipFunction* f, GHipValue x, GHipValue fill, const int64_t* start,
                                 const int64_t* end, const int64_t* interior, int rank, GHipError* err) {
  FN_BEGIN("Pad");
  const Node* a = c.node(x);
  if (!a) return -1;
  const Node* fv = c.node(fill);
  if (!fv) return -1;
  const Shape xs = a->shape;
  if (rank != xs.rank()) return c.fail(GHIP_ERR_INVALID_ARG, "%d axis configs for rank-%d operand", rank, xs.rank());
  if (fv->shape.rank() != 0 || fv->shape.dtype != xs.dtype)
    return c.fail(GHIP_ERR_INVALID_ARG, "fill value must be a %s scalar, got %s", dtype_name(xs.dtype),
                  fv->shape.str().c_str());
  for (int i = 0; i < rank; ++i)
    if (interior && interior[i] != 0)
      return c.fail(GHIP_ERR_UNSUPPORTED, "interior padding not supported (axis %d)", i);
  std::vector<int64_t> s0(rank), s1(rank), st(rank, 1);
  bool crop = false;
  for (int i = 0; i < rank; ++i) {
    s0[i] = start[i] < 0 ? -start[i] : 0;
    s1[i] = xs.dims[i] - (end[i] < 0 ? -end[i] : 0);
    if (s1[i] < s0[i]) return c.fail(GHIP_ERR_INVALID_ARG, "axis %d: padding (%lld, %lld) crops more than %lld",
                                     i, (long long)start[i], (long long)end[i], (long long)xs.dims[i]);
    crop = crop || start[i] < 0 || end[i] < 0;
  }
  GHipValue v = x;
  if (crop) v = ghip_fn_slice(f, v, s0.data(), s1.data(), st.data(), rank, err);
  std::vector<int64_t> dims(rank);
  for (int i = 0; i < rank; ++i) dims[i] = s1[i] - s0[i];
  for (int i = 0; i < rank && v >= 0; ++i) {
    const int64_t lo = start[i] > 0 ? start[i] : 0, hi = end[i] > 0 ? end[i] : 0;
    if (lo == 0 && hi == 0) continue;
    std::vector<GHipValue> parts;
    for (int side = 0; side < 3 && v >= 0; ++side) {
      if (side == 1) { parts.push_back(v); continue; }
      const int64_t w = side == 0 ? lo : hi;
      if (w == 0) continue;
      std::vector<int64_t> bd = dims;
      bd[i] = w;
      const GHipValue b = ghip_fn_broadcast_in_dim(f, fill, bd.data(), rank, nullptr, 0, err);
      if (b < 0) return wrap(b, err, "Pad");
      parts.push_back(b);
    }
    v = ghip_fn_concatenate(f, i, parts.data(), static_cast<int>(parts.size()), err);
    dims[i] += lo + hi;
  }
  return wrap(v, err, "Pad");
}

// ReduceLogicalAnd / ReduceLogicalOr (function.go:2262-2270): the minimum /
// maximum of the {0, 1} bytes a Bool holds, read back as Bool.
extern "C" GHipValue ghip_fn_reduce_logical(GHipFunction* f, int is_or, GHipValue x, const int* axes,
                                            int naxes, GHipError* err) {
  FN_BEGIN(is_or ? "ReduceLogicalOr" : "ReduceLogicalAnd");
  const Node* a = c.node(x);
  if (!a) return -1;
  if (a->shape.dtype != GHIP_DTYPE_BOOL)
    return c.fail(GHIP_ERR_INVALID_ARG, "bool operand required, got %s", dtype_name(a->shape.dtype));
  GHipValue v = ghip_fn_convert_dtype(f, x, GHIP_DTYPE_UINT8, err);
  if (v >= 0) v = ghip_fn_reduce(f, is_or ? GHIP_REDUCE_MAX : GHIP_REDUCE_MIN, v, axes, naxes, err);
  if (v >= 0) v = ghip_fn_convert_dtype(f, v, GHIP_DTYPE_BOOL, err);
  return wrap(v, err, is_or ? "ReduceLogicalOr" : "ReduceLogicalAnd");
}

extern "C" GHipValue ghip_fn_fused_softmax(GHipFunction* f, GHipValue x, int axis, GHipError* err) {
  FN_BEGIN("FusedSoftmax");
  const Node* a = c.node(x);
  if (!a) return -1;
  const int r = a->shape.rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) return c.fail(GHIP_ERR_INVALID_ARG, "axis out of range");
  if (!dtype_is_float(a->shape.dtype)) return c.fail(GHIP_ERR_INVALID_ARG, "float input required");
  Node n{Kind::Softmax};
  n.in = {x};
  n.i0 = axis;
  n.shape = a->shape;
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_fused_layer_norm(GHipFunction* f, GHipValue x, const int* axes, int naxes,
                                              double epsilon, GHipValue gamma, GHipValue beta,
                                              GHipError* err) {
  FN_BEGIN("FusedLayerNorm");
  const Node* a = c.node(x);
  if (!a) return -1;
  const int r = a->shape.rank();
  std::vector<int64_t> ax;
  if (!normalize_axes(axes, naxes, r, &ax) || naxes == 0)
    return c.fail(GHIP_ERR_INVALID_ARG, "axis out of range for rank %d", r);  // function.go:2416-2427
  std::sort(ax.begin(), ax.end());
  if (!dtype_is_float(a->shape.dtype)) return c.fail(GHIP_ERR_INVALID_ARG, "float input required");
  Node n{Kind::LayerNorm};
  n.in = {x, gamma, beta};
  n.a0 = ax;
  n.f0 = epsilon;
  n.shape = a->shape;
  int64_t norm = 1;
  for (auto d : ax) norm *= a->shape.dims[d];
  for (int which = 1; which <= 2; ++which) {
    const int v = n.in[which];
    if (v < 0) continue;
    const Node* p = c.node(v);
    if (!p) return -1;
    if (p->shape.dtype != a->shape.dtype) return c.fail(GHIP_ERR_INVALID_ARG, "gamma/beta dtype");
    if (p->shape.size() != norm) return c.fail(GHIP_ERR_INVALID_ARG, "gamma/beta must cover the normalized axes");
  }
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_fused_sdpa(GHipFunction* f, GHipValue q, GHipValue k, GHipValue v,
                                        GHipValue mask, int num_heads, int num_kv_heads, int layout,
                                        double scale, int causal, GHipError* err) {
  FN_BEGIN("FusedScaledDotProductAttention");
  const Node* qn = c.node(q);
  if (!qn) return -1;
  const Node* kn = c.node(k);
  if (!kn) return -1;
  const Node* vn = c.node(v);
  if (!vn) return -1;
  if (qn->shape.rank() != 4) return c.fail(GHIP_ERR_INVALID_ARG, "query must have rank 4, got %d", qn->shape.rank());
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads)
    return c.fail(GHIP_ERR_INVALID_ARG, "numHeads (%d) must be positive and divisible by numKVHeads (%d)", num_heads, num_kv_heads);
  if (layout != GHIP_LAYOUT_BHSD && layout != GHIP_LAYOUT_BSHD) return c.fail(GHIP_ERR_INVALID_ARG, "bad layout");
  if (kn->shape.rank() != 4 || vn->shape.rank() != 4) return c.fail(GHIP_ERR_INVALID_ARG, "k/v must have rank 4");
  if (qn->shape.dtype != kn->shape.dtype || qn->shape.dtype != vn->shape.dtype)
    return c.fail(GHIP_ERR_INVALID_ARG, "q/k/v dtypes differ");
  const int ha = layout == GHIP_LAYOUT_BHSD ? 1 : 2, sa = layout == GHIP_LAYOUT_BHSD ? 2 : 1;
  if (qn->shape.dims[ha] != num_heads || kn->shape.dims[ha] != num_kv_heads || vn->shape.dims[ha] != num_kv_heads)
    return c.fail(GHIP_ERR_INVALID_ARG, "head counts do not match the shapes");
  if (kn->shape.dims[0] != qn->shape.dims[0] || kn->shape.dims[3] != qn->shape.dims[3] ||
      kn->shape.dims[sa] != vn->shape.dims[sa] || vn->shape.dims[0] != qn->shape.dims[0])
    return c.fail(GHIP_ERR_INVALID_ARG, "q/k/v shapes are inconsistent");
  if (mask >= 0) {
    const Node* m = c.node(mask);
    if (!m) return -1;
    if (m->shape.dtype != GHIP_DTYPE_BOOL && m->shape.dtype != qn->shape.dtype)
      return c.fail(GHIP_ERR_INVALID_ARG, "mask must be bool or additive in q's dtype");
    // It must broadcast to the scores [B, H, Sq, Sk] over its trailing axes
    // (broadcastMaskToScores, function.go:2959-2974); a rank-4 mask follows Q's
    // layout (:2709-2718).
    std::vector<int64_t> md = m->shape.dims;
    if (md.size() > 4) return c.fail(GHIP_ERR_INVALID_ARG, "mask rank %zu > 4", md.size());
    if (layout == GHIP_LAYOUT_BSHD && md.size() == 4) std::swap(md[1], md[2]);
    const int64_t sd[4] = {qn->shape.dims[0], num_heads, qn->shape.dims[sa], kn->shape.dims[sa]};
    const size_t off = 4 - md.size();
    for (size_t i = 0; i < md.size(); ++i)
      if (md[i] != 1 && md[i] != sd[off + i])
        return c.fail(GHIP_ERR_INVALID_ARG, "mask %s does not broadcast to the scores [%lld,%lld,%lld,%lld]",
                      m->shape.str().c_str(), (long long)sd[0], (long long)sd[1], (long long)sd[2], (long long)sd[3]);
  }
  Node n{Kind::SDPA};
  n.in = {q, k, v, mask};
  n.i0 = num_heads;
  n.i1 = num_kv_heads;
  n.i2 = layout;
  n.i3 = causal ? 1 : 0;
  n.f0 = scale;
  n.shape = qn->shape;
  n.shape.dims[3] = vn->shape.dims[3];
  return c.add(std::move(n));
}

// ===========================================================================
// Functions and control flow (builder.go:57-70, function.go:120-133, 354-660).
// A closure is a function whose parent is the function that created it; values
// of enclosing functions it uses become Capture nodes (extra inputs after its
// params).  Call / While / If / Sort append one multi-output node and return
// its outputs as TupleGet values.
// ===========================================================================
namespace {
GHipFunction* new_function(GHipBuilder* bl, const std::string& name, GHipFunction* parent) {
  auto fn = std::make_unique<GHipFunction>();
  fn->builder = bl;
  fn->name = name;
  fn->parent = parent;
  fn->index = static_cast<int>(bl->table.size());
  bl->table.push_back(fn.get());
  bl->others.push_back(std::move(fn));
  return bl->table.back();
}

// Emits the control-flow node and one TupleGet per output; writes the value ids.
int emit_cf(Ctx& c, Node&& n, GHipValue* outs, int max_outs) {
  const int k = static_cast<int>(n.outs.size());
  if (!outs || max_outs < k) {
    c.fail(GHIP_ERR_INVALID_ARG, "room for %d outputs needed, %d given", k, max_outs);
    return -1;
  }
  std::vector<Shape> shapes = n.outs;
  const int cf = c.add(std::move(n));
  if (cf < 0) return -1;
  for (int i = 0; i < k; ++i) {
    Node t{Kind::TupleGet};
    t.in = {cf};
    t.i0 = i;
    t.shape = shapes[i];
    outs[i] = c.add(std::move(t));
    if (outs[i] < 0) return -1;
  }
  return k;
}

// The reference's validateClosure (function.go:234-248).
bool check_closure(Ctx& c, GHipFunction* f, GHipFunction* g, const char* what) {
  if (!g) return c.fail(GHIP_ERR_INVALID_ARG, "%s is null", what), false;
  if (g->parent != f) return c.fail(GHIP_ERR_INVALID_ARG, "%s must be a closure of the current function", what), false;
  if (!g->returned) return c.fail(GHIP_ERR_INVALID_ARG, "%s must have Return() called", what), false;
  return true;
}

void add_captures(Node& n, const GHipFunction* g, GHipFunction* f) {
  for (int pl : g->captures) n.in.push_back(f->global(pl));
}
}  // namespace

extern "C" GHipFunction* ghip_builder_new_function(GHipBuilder* bl, const char* name, GHipError* err) {
  if (!bl) {
    set_error(err, GHIP_ERR_INVALID_ARG, "NewFunction: null builder");
    return nullptr;
  }
  if (bl->compiled) {
    set_error(err, GHIP_ERR_STATE, "NewFunction: builder already compiled");
    return nullptr;
  }
  return new_function(bl, name ? name : "", nullptr);
}

extern "C" GHipFunction* ghip_fn_closure(GHipFunction* f, GHipError* err) {
  if (!f || !f->builder) {
    set_error(err, GHIP_ERR_INVALID_ARG, "Closure: null function");
    return nullptr;
  }
  if (f->returned) {
    set_error(err, GHIP_ERR_STATE, "Closure: function %s already returned", f->name.c_str());
    return nullptr;
  }
  return new_function(f->builder, f->name + "/closure", f);
}

extern "C" int ghip_fn_call(GHipFunction* f, GHipFunction* target, const GHipValue* inputs, int n, GHipValue* outs,
                            int max_outs, GHipError* err) {
  FN_BEGIN("Call");
  if (!f || !target) return c.fail(GHIP_ERR_INVALID_ARG, "null function");
  if (target->builder != f->builder) return c.fail(GHIP_ERR_INVALID_ARG, "target function must be from the same builder");
  if (!target->returned) return c.fail(GHIP_ERR_INVALID_ARG, "target function %s must have Return() called", target->name.c_str());
  if (target->parent && target->parent != f)
    return c.fail(GHIP_ERR_INVALID_ARG, "target closure must belong to the current function");
  if (target == f) return c.fail(GHIP_ERR_INVALID_ARG, "a function cannot call itself");
  if (n != static_cast<int>(target->params.size()))
    return c.fail(GHIP_ERR_INVALID_ARG, "function %s expects %zu parameters, got %d inputs", target->name.c_str(),
                  target->params.size(), n);
  Node node{Kind::Call};
  for (int i = 0; i < n; ++i) {
    const Node* a = c.node(inputs[i]);
    if (!a) return -1;
    if (a->shape != target->nodes[target->params[i]].shape)
      return c.fail(GHIP_ERR_INVALID_ARG, "parameter %d shape mismatch: expected %s, got %s", i,
                    target->nodes[target->params[i]].shape.str().c_str(), a->shape.str().c_str());
    node.in.push_back(inputs[i]);
  }
  add_captures(node, target, f);
  node.fns = {target};
  for (int o : target->outputs) node.outs.push_back(target->nodes[o].shape);
  node.i0 = n;
  return emit_cf(c, std::move(node), outs, max_outs);
}

extern "C" int ghip_fn_while(GHipFunction* f, GHipFunction* cond, GHipFunction* body, const GHipValue* init, int n,
                             GHipValue* outs, int max_outs, GHipError* err) {
  FN_BEGIN("While");
  if (n <= 0) return c.fail(GHIP_ERR_INVALID_ARG, "requires at least one initial state value");
  if (!check_closure(c, f, cond, "cond") || !check_closure(c, f, body, "body")) return -1;
  Node node{Kind::While};
  for (int i = 0; i < n; ++i) {
    const Node* a = c.node(init[i]);
    if (!a) return -1;
    node.in.push_back(init[i]);
    node.outs.push_back(a->shape);
  }
  if (static_cast<int>(cond->params.size()) != n)
    return c.fail(GHIP_ERR_INVALID_ARG, "cond must have %d parameters, got %zu", n, cond->params.size());
  if (static_cast<int>(body->params.size()) != n)
    return c.fail(GHIP_ERR_INVALID_ARG, "body must have %d parameters, got %zu", n, body->params.size());
  for (int i = 0; i < n; ++i) {
    if (cond->nodes[cond->params[i]].shape != node.outs[i])
      return c.fail(GHIP_ERR_INVALID_ARG, "cond parameter %d shape %s doesn't match state shape %s", i,
                    cond->nodes[cond->params[i]].shape.str().c_str(), node.outs[i].str().c_str());
    if (body->nodes[body->params[i]].shape != node.outs[i])
      return c.fail(GHIP_ERR_INVALID_ARG, "body parameter %d shape %s doesn't match state shape %s", i,
                    body->nodes[body->params[i]].shape.str().c_str(), node.outs[i].str().c_str());
  }
  if (cond->outputs.size() != 1) return c.fail(GHIP_ERR_INVALID_ARG, "cond must return exactly one value, got %zu", cond->outputs.size());
  const Shape& cs = cond->nodes[cond->outputs[0]].shape;
  if (cs.rank() != 0 || cs.dtype != GHIP_DTYPE_BOOL)
    return c.fail(GHIP_ERR_INVALID_ARG, "cond must return scalar bool, got %s", cs.str().c_str());
  if (static_cast<int>(body->outputs.size()) != n)
    return c.fail(GHIP_ERR_INVALID_ARG, "body must return %d values, got %zu", n, body->outputs.size());
  for (int i = 0; i < n; ++i)
    if (body->nodes[body->outputs[i]].shape != node.outs[i])
      return c.fail(GHIP_ERR_INVALID_ARG, "body output %d shape %s must match state shape %s", i,
                    body->nodes[body->outputs[i]].shape.str().c_str(), node.outs[i].str().c_str());
  add_captures(node, cond, f);
  add_captures(node, body, f);
  node.fns = {cond, body};
  node.i0 = n;
  node.i1 = static_cast<int64_t>(cond->captures.size());
  return emit_cf(c, std::move(node), outs, max_outs);
}

extern "C" int ghip_fn_if(GHipFunction* f, GHipValue pred, GHipFunction* true_branch, GHipFunction* false_branch,
                          GHipValue* outs, int max_outs, GHipError* err) {
  FN_BEGIN("If");
  const Node* p = c.node(pred);
  if (!p) return -1;
  if (p->shape.rank() != 0 || p->shape.dtype != GHIP_DTYPE_BOOL)
    return c.fail(GHIP_ERR_INVALID_ARG, "pred must be scalar bool, got %s", p->shape.str().c_str());
  if (!check_closure(c, f, true_branch, "trueBranch") || !check_closure(c, f, false_branch, "falseBranch")) return -1;
  if (!true_branch->params.empty())
    return c.fail(GHIP_ERR_INVALID_ARG, "trueBranch must have no parameters, got %zu", true_branch->params.size());
  if (!false_branch->params.empty())
    return c.fail(GHIP_ERR_INVALID_ARG, "falseBranch must have no parameters, got %zu", false_branch->params.size());
  if (true_branch->outputs.size() != false_branch->outputs.size())
    return c.fail(GHIP_ERR_INVALID_ARG, "branches must return same number of outputs (true=%zu, false=%zu)",
                  true_branch->outputs.size(), false_branch->outputs.size());
  Node node{Kind::If};
  for (size_t i = 0; i < true_branch->outputs.size(); ++i) {
    const Shape& a = true_branch->nodes[true_branch->outputs[i]].shape;
    const Shape& b = false_branch->nodes[false_branch->outputs[i]].shape;
    if (a != b)
      return c.fail(GHIP_ERR_INVALID_ARG, "output %zu shapes must match (true=%s, false=%s)", i, a.str().c_str(),
                    b.str().c_str());
    node.outs.push_back(a);
  }
  node.in = {pred};
  add_captures(node, true_branch, f);
  add_captures(node, false_branch, f);
  node.fns = {true_branch, false_branch};
  node.i0 = static_cast<int64_t>(true_branch->captures.size());
  return emit_cf(c, std::move(node), outs, max_outs);
}

extern "C" int ghip_fn_sort(GHipFunction* f, GHipFunction* comparator, int axis, int is_stable,
                            const GHipValue* inputs, int n, GHipValue* outs, int max_outs, GHipError* err) {
  FN_BEGIN("Sort");
  if (n <= 0) return c.fail(GHIP_ERR_INVALID_ARG, "requires at least one input tensor");
  Node node{Kind::Sort};
  const Node* first = nullptr;
  for (int i = 0; i < n; ++i) {
    const Node* a = c.node(inputs[i]);
    if (!a) return -1;
    if (!first) first = a;
    if (a->shape.dims != first->shape.dims) return c.fail(GHIP_ERR_INVALID_ARG, "all inputs must have same dimensions");
    node.in.push_back(inputs[i]);
    node.outs.push_back(a->shape);
  }
  const int rank = first->shape.rank();
  if (axis < 0) axis += rank;
  if (axis < 0 || axis >= rank) return c.fail(GHIP_ERR_INVALID_ARG, "axis %d out of range for rank %d", axis, rank);
  if (!check_closure(c, f, comparator, "comparator")) return -1;
  if (static_cast<int>(comparator->params.size()) != 2 * n)
    return c.fail(GHIP_ERR_INVALID_ARG, "comparator must have %d parameters, got %zu", 2 * n, comparator->params.size());
  for (int i = 0; i < 2 * n; ++i) {
    const Shape& ps = comparator->nodes[comparator->params[i]].shape;
    if (ps.rank() != 0) return c.fail(GHIP_ERR_INVALID_ARG, "comparator parameter %d must be scalar, got %s", i, ps.str().c_str());
    if (ps.dtype != node.outs[i / 2].dtype)
      return c.fail(GHIP_ERR_INVALID_ARG, "comparator parameter %d dtype %s must match input dtype %s", i,
                    dtype_name(ps.dtype), dtype_name(node.outs[i / 2].dtype));
  }
  if (comparator->outputs.size() != 1)
    return c.fail(GHIP_ERR_INVALID_ARG, "comparator must return exactly one value, got %zu", comparator->outputs.size());
  const Shape& rs = comparator->nodes[comparator->outputs[0]].shape;
  if (rs.rank() != 0 || rs.dtype != GHIP_DTYPE_BOOL)
    return c.fail(GHIP_ERR_INVALID_ARG, "comparator must return scalar bool, got %s", rs.str().c_str());
  add_captures(node, comparator, f);
  node.fns = {comparator};
  node.i0 = axis;
  node.i1 = is_stable ? 1 : 0;
  node.i2 = n;
  return emit_cf(c, std::move(node), outs, max_outs);
}

// ===========================================================================
// DynamicSlice / DynamicUpdateSlice (function.go:1571-1621) and ScatterSum /
// ScatterMax / ScatterMin (gather.go:441-640).
// ===========================================================================
namespace {
// Start indices: one integer scalar value per operand axis.
bool check_starts(Ctx& c, const GHipValue* starts, int n, int rank) {
  if (n != rank) {
    c.fail(GHIP_ERR_INVALID_ARG, "%d start indices for a rank-%d operand", n, rank);
    return false;
  }
  for (int i = 0; i < n; ++i) {
    const Node* s = c.node(starts[i]);
    if (!s) return false;
    if (!dtype_is_int(s->shape.dtype) || s->shape.rank() != 0) {
      c.fail(GHIP_ERR_INVALID_ARG, "startIndex[%d] must be an integer scalar, got %s", i, s->shape.str().c_str());
      return false;
    }
  }
  return true;
}
}  // namespace

extern "C" GHipValue ghip_fn_dynamic_slice(GHipFunction* f, GHipValue operand, const GHipValue* starts, int nstarts,
                                           const int64_t* sizes, int nsizes, GHipError* err) {
  FN_BEGIN("DynamicSlice");
  const Node* a = c.node(operand);
  if (!a) return -1;
  const int r = a->shape.rank();
  if (!check_starts(c, starts, nstarts, r)) return -1;
  if (nsizes != r) return c.fail(GHIP_ERR_INVALID_ARG, "%d slice sizes for a rank-%d operand", nsizes, r);
  Node n{Kind::DynSlice};
  n.shape.dtype = a->shape.dtype;
  for (int i = 0; i < r; ++i) {
    if (sizes[i] < 0 || sizes[i] > a->shape.dims[i])
      return c.fail(GHIP_ERR_INVALID_ARG, "slice size %lld out of [0, %lld] on axis %d", (long long)sizes[i],
                    (long long)a->shape.dims[i], i);
    n.shape.dims.push_back(sizes[i]);
  }
  n.in.push_back(operand);
  n.in.insert(n.in.end(), starts, starts + nstarts);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_dynamic_update_slice(GHipFunction* f, GHipValue operand, GHipValue update,
                                                  const GHipValue* starts, int nstarts, GHipError* err) {
  FN_BEGIN("DynamicUpdateSlice");
  const Node* a = c.node(operand);
  if (!a) return -1;
  const Node* u = c.node(update);
  if (!u) return -1;
  const int r = a->shape.rank();
  if (u->shape.dtype != a->shape.dtype)
    return c.fail(GHIP_ERR_INVALID_ARG, "update dtype %s differs from operand %s", dtype_name(u->shape.dtype),
                  dtype_name(a->shape.dtype));
  if (u->shape.rank() != r) return c.fail(GHIP_ERR_INVALID_ARG, "update rank %d vs operand rank %d", u->shape.rank(), r);
  for (int i = 0; i < r; ++i)
    if (u->shape.dims[i] > a->shape.dims[i])
      return c.fail(GHIP_ERR_INVALID_ARG, "update dim %lld exceeds operand dim %lld on axis %d",
                    (long long)u->shape.dims[i], (long long)a->shape.dims[i], i);
  if (!check_starts(c, starts, nstarts, r)) return -1;
  Node n{Kind::DynUpdate};
  n.shape = a->shape;
  n.in = {operand, update};
  n.in.insert(n.in.end(), starts, starts + nstarts);
  return c.add(std::move(n));
}

extern "C" GHipValue ghip_fn_scatter(GHipFunction* f, int mode, GHipValue operand, GHipValue indices,
                                     GHipValue updates, int index_vector_axis, const int* update_window_axes,
                                     int n_uwa, const int* inserted_window_axes, int n_iwa,
                                     const int* scatter_axes_to_operand_axes, int n_sato, int indices_are_sorted,
                                     int unique_indices, GHipError* err) {
  static const char* names[] = {"ScatterSum", "ScatterMax", "ScatterMin"};
  if (mode < GHIP_SCATTER_SUM || mode > GHIP_SCATTER_MIN) {
    set_error(err, GHIP_ERR_INVALID_ARG, "Scatter: bad mode %d", mode);
    return -1;
  }
  FN_BEGIN(names[mode]);
  const Node* op = c.node(operand);
  if (!op) return -1;
  const Node* ix = c.node(indices);
  if (!ix) return -1;
  const Node* up = c.node(updates);
  if (!up) return -1;
  const int r = op->shape.rank(), ir = ix->shape.rank(), ur = up->shape.rank();
  if (!dtype_is_int(ix->shape.dtype)) return c.fail(GHIP_ERR_INVALID_ARG, "indices must be integers");
  if (up->shape.dtype != op->shape.dtype) return c.fail(GHIP_ERR_INVALID_ARG, "updates dtype differs from operand");
  if (op->shape.dtype == GHIP_DTYPE_BOOL) return c.fail(GHIP_ERR_INVALID_ARG, "bool operand");
  if (index_vector_axis < 0 || index_vector_axis > ir) return c.fail(GHIP_ERR_INVALID_ARG, "bad indexVectorAxis %d", index_vector_axis);
  const int64_t ivec = index_vector_axis < ir ? ix->shape.dims[index_vector_axis] : 1;
  if (ivec != n_sato)
    return c.fail(GHIP_ERR_INVALID_ARG, "index vector size %lld vs %d scatterAxesToOperandAxes", (long long)ivec, n_sato);
  std::vector<int64_t> uwa, iwa, sato;
  if (!normalize_axes(update_window_axes, n_uwa, ur, &uwa)) return c.fail(GHIP_ERR_INVALID_ARG, "invalid updateWindowAxes");
  if (!normalize_axes(inserted_window_axes, n_iwa, r, &iwa)) return c.fail(GHIP_ERR_INVALID_ARG, "invalid insertedWindowAxes");
  if (!normalize_axes(scatter_axes_to_operand_axes, n_sato, r, &sato))
    return c.fail(GHIP_ERR_INVALID_ARG, "invalid scatterAxesToOperandAxes");
  if (!std::is_sorted(uwa.begin(), uwa.end()) || !std::is_sorted(iwa.begin(), iwa.end()))
    return c.fail(GHIP_ERR_INVALID_ARG, "window axes must be sorted");
  if (n_uwa + n_iwa != r)
    return c.fail(GHIP_ERR_INVALID_ARG, "%d update window axes + %d inserted axes != operand rank %d", n_uwa, n_iwa, r);
  const int nbatch = ir - (index_vector_axis < ir ? 1 : 0);
  if (ur != n_uwa + nbatch)
    return c.fail(GHIP_ERR_INVALID_ARG, "updates rank %d != %d window axes + %d scatter axes", ur, n_uwa, nbatch);
  // Window axes of updates map, in order, onto the operand axes not inserted.
  int wi = 0;
  for (int d = 0; d < r; ++d) {
    if (std::find(iwa.begin(), iwa.end(), d) != iwa.end()) continue;
    const int64_t ws = up->shape.dims[uwa[wi++]];
    if (ws > op->shape.dims[d])
      return c.fail(GHIP_ERR_INVALID_ARG, "update window size %lld exceeds operand dim %lld (axis %d)", (long long)ws,
                    (long long)op->shape.dims[d], d);
  }
  // Scatter axes of updates match the index batch axes, in order.
  int bi = 0;
  for (int d = 0; d < ur; ++d) {
    if (std::find(uwa.begin(), uwa.end(), d) != uwa.end()) continue;
    if (bi == index_vector_axis) ++bi;
    if (up->shape.dims[d] != ix->shape.dims[bi])
      return c.fail(GHIP_ERR_INVALID_ARG, "updates scatter dim %d (%lld) != indices batch dim %d (%lld)", d,
                    (long long)up->shape.dims[d], bi, (long long)ix->shape.dims[bi]);
    ++bi;
  }
  Node n{Kind::Scatter};
  n.sub = mode;
  n.in = {operand, indices, updates};
  n.shape = op->shape;
  n.i0 = index_vector_axis;
  n.i1 = indices_are_sorted;
  n.i2 = unique_indices;
  n.a0 = uwa;
  n.a1 = iwa;
  n.a2 = sato;
  return c.add(std::move(n));
}

// ===========================================================================
// Composite fused ops.  The reference builds these from primitive MPSGraph ops
// (function.go:2288-2408, 2567-2667, 2976-3075); here they are built from this
// Function's own primitives in the same order, so the lowering sees ordinary
// DotGeneral + elementwise graphs and fuses bias / activation / slicing into the
// GEMM epilogue like any other chain.
// ===========================================================================
namespace {

// fp32 -> bf16 / f16 bits, round to nearest even (NaN quiet).
uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// makeScalarConst (function.go:210-231): the value is taken as float32 and then
// converted to dt.  The conversion happens here, at build time, so the constant
// reaches the lowering as one literal of dt.
GHipValue scalar_const(GHipFunction* f, int dt, double val, GHipError* err) {
  const float v32 = static_cast<float>(val);
  uint8_t buf[8];
  size_t nb = 0;
  switch (dt) {
    case GHIP_DTYPE_FLOAT32: memcpy(buf, &v32, 4); nb = 4; break;
    case GHIP_DTYPE_FLOAT64: { const double d = v32; memcpy(buf, &d, 8); nb = 8; break; }
    case GHIP_DTYPE_BFLOAT16: { const uint16_t h = host_f32_to_bf16(v32); memcpy(buf, &h, 2); nb = 2; break; }
    case GHIP_DTYPE_FLOAT16: { const _Float16 h = static_cast<_Float16>(v32); memcpy(buf, &h, 2); nb = 2; break; }
    default: set_error(err, GHIP_ERR_INVALID_ARG, "scalar constant: dtype %s is not a float", dtype_name(dt)); return -1;
  }
  return ghip_fn_constant(f, dt, nullptr, 0, buf, nb, err);
}

// Prefixes err's message with "<op>: " (errors.Wrap in the reference).
GHipValue wrap(GHipValue v, GHipError* err, const char* op) {
  if (v < 0 && err && err->message) {
    std::string m = std::string(op) + ": " + err->message;
    set_error(err, err->code, "%s", m.c_str());
  }
  return v;
}

// bias broadcast over the trailing axes of `shape_of` and added (function.go:2601-2618).
GHipValue add_trailing_bias(GHipFunction* f, GHipValue v, GHipValue bias, GHipError* err) {
  const Shape rs = value_node(f, v)->shape;
  const Shape bs = value_node(f, bias)->shape;
  if (bs.rank() > rs.rank()) {
    set_error(err, GHIP_ERR_INVALID_ARG, "bias rank %d exceeds result rank %d", bs.rank(), rs.rank());
    return -1;
  }
  std::vector<int> axes(bs.rank());
  for (int i = 0; i < bs.rank(); ++i) axes[i] = rs.rank() - bs.rank() + i;
  const GHipValue b = ghip_fn_broadcast_in_dim(f, bias, rs.dims.data(), rs.rank(), axes.data(), bs.rank(), err);
  if (b < 0) return -1;
  return ghip_fn_binary(f, GHIP_BINARY_ADD, v, b, err);
}

// x [..., din] . w [din, ...] contracting x's last axis with w's first.
GHipValue dense_dot(GHipFunction* f, GHipValue x, GHipValue w, GHipError* err) {
  const int lc = value_node(f, x)->shape.rank() - 1, rc = 0;
  return ghip_fn_dot_general(f, x, &lc, 1, nullptr, 0, w, &rc, 1, nullptr, 0, err);
}

}  // namespace

extern "C" GHipValue ghip_fn_fused_gelu(GHipFunction* f, GHipValue x, int exact, GHipError* err) {
  FN_BEGIN("FusedGelu");
  const Node* a = c.node(x);
  if (!a) return -1;
  const int dt = a->shape.dtype;
  if (!dtype_is_float(dt)) return c.fail(GHIP_ERR_INVALID_ARG, "float input required, got %s", dtype_name(dt));
  auto K = [&](double v) { return scalar_const(f, dt, v, err); };
  auto mul = [&](GHipValue p, GHipValue q) { return p < 0 || q < 0 ? -1 : ghip_fn_binary(f, GHIP_BINARY_MUL, p, q, err); };
  auto add = [&](GHipValue p, GHipValue q) { return p < 0 || q < 0 ? -1 : ghip_fn_binary(f, GHIP_BINARY_ADD, p, q, err); };
  auto un = [&](int op, GHipValue p) { return p < 0 ? -1 : ghip_fn_unary(f, op, p, err); };
  GHipValue r;
  if (exact) {
    // x * 0.5 * (1 + erf(x / sqrt(2))), evaluated as (0.5 x) (1 + erf(x (1/sqrt 2))).
    const GHipValue half = K(0.5), inv_sqrt2 = K(0.7071067811865475), one = K(1.0);
    const GHipValue e = un(GHIP_UNARY_ERF, mul(x, inv_sqrt2));
    r = mul(mul(half, x), add(one, e));
  } else {
    // (0.5 x) (1 + tanh(sqrt(2/pi) (x + 0.044715 ((x x) x)))), one op at a time in
    // the reference's order (function.go:2343-2402): in 16-bit dtypes every op
    // rounds, so the association decides the result bits.
    const GHipValue half = K(0.5), one = K(1.0), coeff = K(0.044715), s2pi = K(0.7978845608);
    const GHipValue x3 = mul(mul(x, x), x);
    const GHipValue inner = add(x, mul(coeff, x3));
    const GHipValue t = un(GHIP_UNARY_TANH, mul(s2pi, inner));
    r = mul(mul(half, x), add(one, t));
  }
  return wrap(r, err, "FusedGelu");
}

extern "C" GHipValue ghip_fn_fused_dense(GHipFunction* f, GHipValue x, GHipValue weight, GHipValue bias,
                                         int activation, GHipError* err) {
  FN_BEGIN("FusedDense");
  const Node* xn = c.node(x);
  if (!xn) return -1;
  const Node* wn = c.node(weight);
  if (!wn) return -1;
  if (bias >= 0 && !c.node(bias)) return -1;
  if (xn->shape.rank() < 1 || wn->shape.rank() < 2)
    return c.fail(GHIP_ERR_INVALID_ARG, "x must have rank >= 1 (got %d), weight must have rank >= 2 (got %d)",
                  xn->shape.rank(), wn->shape.rank());
  const int64_t in_features = xn->shape.dims.back();
  if (in_features != wn->shape.dims[0])
    return c.fail(GHIP_ERR_INVALID_ARG, "x's last dim (%lld) must match weight's first dim (%lld)",
                  static_cast<long long>(in_features), static_cast<long long>(wn->shape.dims[0]));
  if (activation < GHIP_ACTIVATION_NONE || activation > GHIP_ACTIVATION_TANH)
    return c.fail(GHIP_ERR_INVALID_ARG, "unsupported activation type %d", activation);
  GHipValue r = wrap(dense_dot(f, x, weight, err), err, "FusedDense: DotGeneral");
  if (r < 0) return -1;
  if (bias >= 0) {
    r = wrap(add_trailing_bias(f, r, bias, err), err, "FusedDense: bias");
    if (r < 0) return -1;
  }
  const int dt = value_node(f, r)->shape.dtype;
  switch (activation) {
    case GHIP_ACTIVATION_GELU:
      return wrap(ghip_fn_fused_gelu(f, r, 0, err), err, "FusedDense: GELU activation");
    case GHIP_ACTIVATION_RELU: {
      const GHipValue zero = scalar_const(f, dt, 0.0, err);
      return wrap(zero < 0 ? -1 : ghip_fn_binary(f, GHIP_BINARY_MAX, r, zero, err), err, "FusedDense: ReLU");
    }
    case GHIP_ACTIVATION_SILU: {
      const GHipValue s = ghip_fn_unary(f, GHIP_UNARY_LOGISTIC, r, err);
      return wrap(s < 0 ? -1 : ghip_fn_binary(f, GHIP_BINARY_MUL, r, s, err), err, "FusedDense: SiLU");
    }
    case GHIP_ACTIVATION_TANH:
      return wrap(ghip_fn_unary(f, GHIP_UNARY_TANH, r, err), err, "FusedDense: Tanh");
    default:
      return r;
  }
}

extern "C" int ghip_fn_fused_qkv_projection(GHipFunction* f, GHipValue x, GHipValue w_qkv, GHipValue bias_q,
                                            GHipValue bias_k, GHipValue bias_v, int query_dim, int key_value_dim,
                                            GHipValue* query, GHipValue* key, GHipValue* value, GHipError* err) {
  FN_BEGIN("FusedAttentionQKVProjection");
  auto code = [&]() { return err && err->code ? err->code : GHIP_ERR_INVALID_ARG; };
  if (!query || !key || !value) {
    c.fail(GHIP_ERR_INVALID_ARG, "null output pointer");
    return GHIP_ERR_INVALID_ARG;
  }
  *query = *key = *value = -1;
  const Node* xn = c.node(x);
  if (!xn || !c.node(w_qkv)) return code();
  for (GHipValue b : {bias_q, bias_k, bias_v})
    if (b >= 0 && !c.node(b)) return code();
  if (xn->shape.rank() < 1) {
    c.fail(GHIP_ERR_INVALID_ARG, "x must have rank >= 1, got %d", xn->shape.rank());
    return GHIP_ERR_INVALID_ARG;
  }
  if (query_dim < 0 || key_value_dim < 0) {
    c.fail(GHIP_ERR_INVALID_ARG, "negative queryDim (%d) or keyValueDim (%d)", query_dim, key_value_dim);
    return GHIP_ERR_INVALID_ARG;
  }
  const int64_t q = query_dim, kv = key_value_dim;
  const int64_t lo[3] = {0, q, q + kv}, hi[3] = {q, q + kv, q + 2 * kv};
  const char* what[3] = {"FusedAttentionQKVProjection: slice Q", "FusedAttentionQKVProjection: slice K",
                         "FusedAttentionQKVProjection: slice V"};
  auto slice_last = [&](GHipValue t, int64_t a, int64_t b, const char* msg) -> GHipValue {
    const Shape ts = value_node(f, t)->shape;
    const int r = ts.rank();
    std::vector<int64_t> st(r, 0), lim = ts.dims, str(r, 1);
    st[r - 1] = a;
    lim[r - 1] = b;
    return wrap(ghip_fn_slice(f, t, st.data(), lim.data(), str.data(), r, err), err, msg);
  };
  GHipValue out[3] = {-1, -1, -1};
  const bool any_bias = bias_q >= 0 || bias_k >= 0 || bias_v >= 0;
  if (any_bias && value_node(f, w_qkv)->shape.rank() >= 2) {
    // With biases: one product per output over the matching columns of wQKV.
    // Every output element is the same K-sum as in x . wQKV (the GEMM's
    // summation order does not depend on N), and each product's bias add runs
    // in its GEMM epilogue instead of as a separate pass over a strided slice.
    for (int i = 0; i < 3; ++i) {
      const GHipValue ws = slice_last(w_qkv, lo[i], hi[i], what[i]);
      if (ws < 0) return code();
      out[i] = wrap(dense_dot(f, x, ws, err), err, "FusedAttentionQKVProjection: DotGeneral");
      if (out[i] < 0) return code();
    }
  } else {
    // One product x . wQKV -> [..., queryDim + 2 keyValueDim], sliced on its last
    // axis (zero-copy views of the product).
    const GHipValue comb = wrap(dense_dot(f, x, w_qkv, err), err, "FusedAttentionQKVProjection: DotGeneral");
    if (comb < 0) return code();
    for (int i = 0; i < 3; ++i) {
      out[i] = slice_last(comb, lo[i], hi[i], what[i]);
      if (out[i] < 0) return code();
    }
  }
  const GHipValue biases[3] = {bias_q, bias_k, bias_v};
  const char* names[3] = {"FusedAttentionQKVProjection: biasQ", "FusedAttentionQKVProjection: biasK",
                          "FusedAttentionQKVProjection: biasV"};
  for (int i = 0; i < 3; ++i) {
    if (biases[i] < 0) continue;
    out[i] = wrap(add_trailing_bias(f, out[i], biases[i], err), err, names[i]);
    if (out[i] < 0) return code();
  }
  *query = out[0];
  *key = out[1];
  *value = out[2];
  return GHIP_OK;
}

extern "C" int ghip_fn_return(GHipFunction* f, const GHipValue* outputs, int cnt, GHipError* err) {
  FN_BEGIN("Return");
  if (!f) return c.fail(GHIP_ERR_INVALID_ARG, "null function");
  if (f->returned) return set_error(err, GHIP_ERR_STATE, "Return: called twice");
  std::vector<int> loc(cnt);
  for (int i = 0; i < cnt; ++i) {
    loc[i] = outputs[i] < 0 ? -1 : c.loc(outputs[i]);  // a closure may return a captured value
    if (loc[i] < 0) {
      ghip_error_clear(err);
      return set_error(err, GHIP_ERR_INVALID_ARG, "Return: output %d is not a value of this function", i);
    }
    if (f->nodes[loc[i]].kind == Kind::Call || f->nodes[loc[i]].kind == Kind::While ||
        f->nodes[loc[i]].kind == Kind::If || f->nodes[loc[i]].kind == Kind::Sort)
      return set_error(err, GHIP_ERR_INVALID_ARG, "Return: output %d is a control-flow tuple", i);
  }
  f->outputs = loc;
  f->returned = true;
  return GHIP_OK;
}

extern "C" int ghip_fn_value_shape(GHipFunction* f, GHipValue v, int* dtype, int64_t* dims, int max_rank) {
  const Node* n = value_node(f, v);
  if (!n) return -1;
  const Shape& s = n->shape;
  if (dtype) *dtype = s.dtype;
  for (int i = 0; i < s.rank() && i < max_rank; ++i) dims[i] = s.dims[i];
  return s.rank();
}
