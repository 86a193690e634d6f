// Graph IR, builder, lowering plan and executor of the GoMLX backend.
//
// Mirrors the reference backend's object model (mpsgraph/gomlx): a Backend owns
// the device context (backend.go:22-27), a Builder owns one Function graph
// (builder.go:16-24), Function methods append nodes with inferred shapes
// (function.go), Compile lowers the graph to a launch plan (builder.go:72-109) and
// an Executable runs it (executable.go:19-112).  Unlike the reference, which hands
// the graph to MPSGraph, lowering and fusion happen here (graph_lower.cpp) and
// every buffer stays in device memory.
#pragma once

#include <hip/hip_runtime.h>

#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gomlx_hip.h"

struct GHipBackend;
struct GHipBuilder;
struct GHipFunction;
struct GHipExecutable;
struct GHipBuffer;

namespace ghip {

// The first half of a split contraction (k_gemm.hip), for the graph lowering,
// which folds the sum of the partials into the consumer's generated kernel:
// writes the s fp32 partial products [s][M][N] of a (batch 1, 16-bit operands)
// into ws, exactly as ghip_gemm_batched_ws does before its sum kernel.  Reports
// an error when the product would not take that path with s ranges (the
// lowering checks the same conditions when it compiles the plan).
int gemm_split_partials(int ab_dtype, int64_t M, int64_t N, int64_t K, const void* a, int64_t sa_m, int64_t sa_k,
                        const void* b, int64_t sb_k, int64_t sb_n, float* ws, int64_t ws_bytes, int s, void* stream,
                        GHipError* err);

int dtype_size(int dt);
bool dtype_is_float(int dt);
bool dtype_is_int(int dt);      // signed or unsigned integer (not bool)
bool dtype_is_unsigned(int dt);
const char* dtype_name(int dt);

struct Shape {
  int dtype = GHIP_DTYPE_FLOAT32;
  std::vector<int64_t> dims;
  int rank() const { return static_cast<int>(dims.size()); }
  int64_t size() const {
    int64_t n = 1;
    for (auto d : dims) n *= d;
    return n;
  }
  size_t bytes() const { return static_cast<size_t>(size()) * dtype_size(dtype); }
  bool operator==(const Shape& o) const { return dtype == o.dtype && dims == o.dims; }
  bool operator!=(const Shape& o) const { return !(*this == o); }
  std::string str() const;
};

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& dims);

enum class Kind {
  Param, Const, Iota, Unary, Binary, Compare, Where, Clamp, Convert,
  Reshape, Transpose, Broadcast, Slice, Concat, Reverse,
  Reduce, ArgMinMax, Dot, Gather, Softmax, LayerNorm, SDPA,
  DynSlice, DynUpdate, Scatter,
  Capture,    // a closure's copy of an ancestor's value (an extra input after the params)
  Call, While, If, Sort,  // control flow: multi-output, read through TupleGet
  TupleGet,   // output i0 of a control-flow node
};
const char* kind_name(Kind k);

struct Node {
  Kind kind;
  int sub = 0;                 // unary / binary / compare / reduce op code
  Shape shape;
  std::vector<int> in;         // operand value ids
  std::vector<int64_t> a0, a1, a2, a3, a4;  // op attributes (see graph_build.cpp)
  double f0 = 0.0;
  int64_t i0 = 0, i1 = 0, i2 = 0, i3 = 0;
  std::vector<uint8_t> data;   // Const payload
  std::string name;            // Param name
  std::vector<GHipFunction*> fns;   // control flow: called / cond+body / true+false / comparator
  std::vector<Shape> outs;          // control flow: output shapes
};

bool is_elementwise(Kind k);

}  // namespace ghip

// ---------------------------------------------------------------------------
// Public handle types (opaque in the C header).
// ---------------------------------------------------------------------------
struct GHipBackend {
  int device = 0;
  bool plan_only = false;
  bool finalized = false;
  hipStream_t stream = nullptr;
  std::string device_name;
  std::mutex mu;
  // Caching device allocator: exact-size free lists (sizes rounded to 256 B).
  std::multimap<size_t, void*> free_blocks;
  size_t cached_bytes = 0;
  int alloc(size_t bytes, void** out, GHipError* err);
  void release(void* p, size_t bytes);
  void trim();
};

struct GHipBuffer {
  GHipBackend* backend = nullptr;
  ghip::Shape shape;
  void* ptr = nullptr;
  size_t cap = 0;      // allocated bytes (>= shape.bytes())
  bool valid = true;
};

// Value ids handed out by the graph API are unique within a builder:
// (function index << kFnShift) | node index, the main function being index 0
// (so its ids are plain node indices).  Nodes refer to their operands by node
// index inside their own function.
constexpr int kFnShift = 24;
constexpr int kNodeMask = (1 << kFnShift) - 1;

struct GHipFunction {
  GHipBuilder* builder = nullptr;
  std::string name;
  int index = 0;                    // position in the builder's function table
  GHipFunction* parent = nullptr;   // closures: the function that created them
  std::deque<ghip::Node> nodes;     // stable addresses: nodes are only appended
  std::vector<int> params;
  std::vector<int> outputs;
  std::vector<int> captures;        // per Capture node: the parent's node index it copies
  std::map<int, int> capture_of;    // parent node index -> local Capture node
  bool returned = false;
  int add(ghip::Node&& n) {
    nodes.push_back(std::move(n));
    return static_cast<int>(nodes.size()) - 1;
  }
  int global(int local) const { return (index << kFnShift) | local; }
};

struct GHipBuilder {
  GHipBackend* backend = nullptr;
  std::string name;
  std::unique_ptr<GHipFunction> main;
  std::vector<std::unique_ptr<GHipFunction>> others;  // closures and named functions
  std::vector<GHipFunction*> table;                   // index -> function (main first)
  bool compiled = false;
};

namespace ghip {

// A device view of a value: base slot + element offset + per-dim element strides.
struct View {
  int slot = -1;
  int64_t offset = 0;
  std::vector<int64_t> strides;
  bool contiguous(const Shape& s) const;
};

// Execution-time state: one device pointer per memory slot.
struct ExecState {
  std::vector<char*> slot_ptr;
  hipStream_t stream = nullptr;
  char* ptr(const View& v, int dt) const { return slot_ptr[v.slot] + v.offset * dtype_size(dt); }
};

using StepFn = std::function<int(ExecState&, GHipError*)>;

struct Step {
  std::string desc;
  StepFn run;
};

enum class SlotKind { Input, Const, Arena, Output };

struct Slot {
  SlotKind kind;
  size_t bytes = 0;
  int index = 0;          // input / output index
  size_t arena_off = 0;   // Arena
  void* const_ptr = nullptr;
};

struct Plan {
  std::vector<std::shared_ptr<GHipExecutable>> subs;  // compiled closures / called functions
  std::vector<Slot> slots;
  std::vector<Step> steps;
  size_t arena_bytes = 0;
  std::vector<View> out_views;  // where each output value lives
  std::vector<int> out_slot;    // output slot for each output
  // Donation (Execute's `donate`): the last step that reads each input (-1: none)
  // and the first step that writes each output; an output may take a donated
  // input's memory when that input is read only before the output's first write,
  // or in the same step when that step is elementwise with the input read at the
  // output's own element index (inplace_inputs of the step).
  std::vector<int> in_last_read;
  std::vector<int> out_first_write;
  std::vector<std::vector<int>> inplace_inputs;  // per step: input indices it may overwrite
  std::vector<std::string> log;
  std::vector<std::vector<uint8_t>> const_data;  // per slot (Const slots only)
};

int lower(GHipBackend* be, GHipFunction* fn, Plan* plan, GHipError* err);
// Compiles one function (main, closure or named function) into an executable:
// inputs are its params followed by its captures.
std::shared_ptr<GHipExecutable> compile_function(GHipBackend* be, GHipFunction* fn, GHipError* err);
// Runs an executable's plan on its backend's stream with the given device
// pointers for its inputs and (contiguous, pre-allocated) outputs.
int run_plan(GHipExecutable* e, void* const* in_ptrs, void* const* out_ptrs, GHipError* err);
// The same with the intermediates in `arena` (at least plan.arena_bytes, 256-byte
// aligned) instead of the executable's own arena.
int run_plan_in(GHipExecutable* e, void* arena, void* const* in_ptrs, void* const* out_ptrs, GHipError* err);
// Execute's checks of the input buffers and the input / output counts.
int check_execute_args(GHipExecutable* e, GHipBuffer* const* inputs, int n, int nout, GHipError* err);

// Generated elementwise kernels (rtc.cpp).
struct RtcKernel {
  hipModule_t module = nullptr;
  hipFunction_t func = nullptr;
};
int rtc_get(GHipBackend* be, const std::string& src, const std::string& entry, RtcKernel* out,
            GHipError* err);

// Generic kernels (k_generic.hip).
constexpr int kMaxRank = 8;
// dst[...] = src[...] over `dims`, both sides addressed by element strides.
struct CopyDesc {
  int rank = 0;
  int64_t dims[kMaxRank];
  int64_t sst[kMaxRank];  // source strides
  int64_t dst[kMaxRank];  // destination strides
};
int launch_strided_copy(int elem_bytes, const void* src, void* dst, const CopyDesc& d,
                        hipStream_t s, GHipError* err);
// out[o] = reduce over r of src[o-offset + r-offset]; out is contiguous over odims.
struct ReduceDesc {
  int orank = 0, rrank = 0;
  int64_t odims[kMaxRank], ost[kMaxRank];
  int64_t rdims[kMaxRank], rst[kMaxRank];
};
int launch_reduce(int dtype, int op, const void* src, const ReduceDesc& d, void* dst,
                  hipStream_t s, GHipError* err);
// Gather rows with int32 or int64 ids (clamped).
int launch_gather_rows(const void* table, int64_t V, int64_t row_bytes, const void* ids,
                       int id_dtype, int64_t n, void* out, hipStream_t s, GHipError* err);
// Window copy at run-time starts (DynamicSlice: window on the source side,
// at_dst = 0; DynamicUpdateSlice: window on the destination side, at_dst = 1).
// Starts are integer scalars in device memory, clamped to [0, dims - win].
struct DynDesc {
  int rank = 0;
  int64_t dims[kMaxRank];   // operand dims (the side the window lives in)
  int64_t win[kMaxRank];    // window dims
  int64_t sst[kMaxRank];    // source strides
  int64_t dst[kMaxRank];    // destination strides
  const void* start[kMaxRank];
  int sdt[kMaxRank];        // start dtypes
};
int launch_window_copy(int elem_bytes, const void* src, void* dst, const DynDesc& d, int at_dst, hipStream_t s,
                       GHipError* err);
// XLA scatter into `acc` (dtype scatter_acc_dtype(dtype), contiguous operand
// dims): one thread per update element.
struct ScatterDesc {
  int ur = 0;                  // updates rank
  int64_t udims[kMaxRank], ust[kMaxRank];
  int uwin_od[kMaxRank];       // operand dim of each window dim of updates; -1: scatter dim
  int64_t ibatch_st[kMaxRank]; // scatter dims: element stride in the indices tensor
  int nidx = 0;                // index vector length
  int64_t ivec_st = 0;         // element stride of the index vector axis
  int sato[kMaxRank];          // operand dim of each index vector component
  int r = 0;                   // operand rank
  int64_t odims[kMaxRank], ost[kMaxRank], wsize[kMaxRank];
  int idx_dt = 0, idx_es = 0;
};
int scatter_acc_dtype(int dtype);
int launch_scatter(int dtype, int mode, const void* updates, const void* indices, void* acc, const ScatterDesc& d,
                   hipStream_t s, GHipError* err);
// Deterministic scatter-add of n update rows (row stride upd_row elements) into
// rows ids[i] (stride id_stride elements, int32 / int64; out of range skipped) of
// the contiguous [V, D] float32 / bfloat16 / float16 table `out`, each row's
// updates folded in their original order in fp32 and rounded once.  scratch:
// scatter_rows_scratch(n) bytes.  n <= kScatterRowsMax, V <= kScatterRowsMaxTable.
constexpr int64_t kScatterRowsMax = 16384;
constexpr int64_t kScatterRowsMaxTable = (1 << 18) - 1;
inline size_t scatter_rows_scratch(int64_t n) { return static_cast<size_t>(2 * n + 2) * 4; }
// copy_src: when not null, the contiguous operand (16-byte aligned, size a
// multiple of 16 bytes), copied into `out` by the same launch that sorts.
int launch_scatter_rows(int dtype, const void* updates, int64_t upd_row, const void* ids, int id_dt, int64_t id_stride,
                        int64_t n, void* out, int64_t V, int64_t D, void* scratch, const void* copy_src, hipStream_t s,
                        GHipError* err);
// dst (contiguous) = convert(src viewed through d.sst); widening / narrowing pairs
// used around scatter accumulators.
int launch_convert(int src_dt, int dst_dt, const void* src, void* dst, const CopyDesc& d, hipStream_t s,
                   GHipError* err);
// Whether the fused attention kernel (ghip_sdpa_fwd) takes these operands; strides
// in elements ordered (batch, head, sequence), head dim contiguous.
bool sdpa_fused_supported(int dtype, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                          const int64_t* qs, const int64_t* ks, const int64_t* vs, const int64_t* os,
                          float scale, int mask_dtype);

}  // namespace ghip

struct GHipExecutable {
  GHipBackend* backend = nullptr;
  std::vector<ghip::Shape> in_shapes, out_shapes;
  std::vector<std::string> in_names;
  ghip::Plan plan;
  std::vector<std::pair<void*, size_t>> owned_consts;
  void* arena = nullptr;
  size_t arena_cap = 0;
  std::mutex mu;
  bool finalized = false;
};
