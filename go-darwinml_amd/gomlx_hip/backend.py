"""Python mirror of the GoMLX `backends` plugin API over libgomlx_hip.so.

Same object model and method names as the Go interfaces the reference
registers (mpsgraph/gomlx: backend.go, builder.go, function.go,
dotgeneral.go, gather.go, executable.go): a Backend hands out Builders, a
Builder's Main() Function collects ops, Compile() returns an Executable whose
Execute() maps device Buffers to device Buffers.  Errors the Go code returns as
`error` raise BackendError here; Backend.Builder raises like the Go code panics
(backend.go:72-75).  Every call goes through the C ABI of include/gomlx_hip.h.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import BackendError, GHipError

# ---------------------------------------------------------------- dtypes / shapes
class dtypes:
    Bool, Int8, Int16, Int32, Int64 = 0, 1, 2, 3, 4
    Float16, BFloat16, Float32, Float64 = 5, 6, 7, 8
    Uint8, Uint16, Uint32, Uint64 = 9, 10, 11, 12


_NP = {
    dtypes.Bool: np.bool_, dtypes.Int8: np.int8, dtypes.Int16: np.int16, dtypes.Int32: np.int32,
    dtypes.Int64: np.int64, dtypes.Float16: np.float16, dtypes.BFloat16: np.uint16,
    dtypes.Float32: np.float32, dtypes.Float64: np.float64, dtypes.Uint8: np.uint8,
    dtypes.Uint16: np.uint16, dtypes.Uint32: np.uint32, dtypes.Uint64: np.uint64,
}
_FROM_NP = {np.dtype(v): k for k, v in _NP.items() if k != dtypes.BFloat16}


def np_dtype(dt: int):
    """Host storage dtype (bf16 is carried as its uint16 bit pattern)."""
    return _NP[dt]


@dataclass(frozen=True)
class Shape:
    dtype: int
    dims: tuple

    def size(self) -> int:
        return int(np.prod(self.dims, dtype=np.int64)) if self.dims else 1

    def rank(self) -> int:
        return len(self.dims)


@dataclass(frozen=True)
class PadAxis:
    """backends.PadAxis: elements added before / after an axis and between its
    elements (interior)."""
    start: int = 0
    end: int = 0
    interior: int = 0


@dataclass(frozen=True)
class Capabilities:
    """backends.Capabilities (capabilities.go:14-166): control-flow functions,
    the OpType names (without the "OpType" prefix) and the DType names."""
    functions: bool
    operations: frozenset
    dtypes: frozenset


def make_shape(dtype: int, *dims: int) -> Shape:
    """shapes.Make(dtype, dims...)."""
    return Shape(dtype, tuple(int(d) for d in dims))


class ActivationType:
    NONE, GELU, RELU, SILU, TANH = range(5)


class AxesLayout:
    BHSD = 0
    BSHD = 1


UNARY = ["Abs", "Neg", "Sqrt", "Rsqrt", "Exp", "Expm1", "Log", "Log1p", "Sin", "Cos", "Tanh",
         "Logistic", "Erf", "Floor", "Ceil", "Round", "Sign", "LogicalNot", "BitwiseNot",
         "IsFinite", "IsNaN", "Identity"]
BINARY = ["Add", "Sub", "Mul", "Div", "Rem", "Pow", "Max", "Min", "Atan2", "LogicalAnd",
          "LogicalOr", "LogicalXor", "BitwiseAnd", "BitwiseOr", "BitwiseXor", "ShiftLeft",
          "ShiftRightArithmetic", "ShiftRightLogical"]
COMPARE = ["Equal", "NotEqual", "GreaterThan", "GreaterOrEqual", "LessThan", "LessOrEqual"]
REDUCE = {"ReduceSum": 0, "ReduceProduct": 1, "ReduceMax": 2, "ReduceMin": 3}


# ---------------------------------------------------------------- C signatures
_vp, _i64, _int, _dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
_errp = ctypes.POINTER(GHipError)
_i64p = ctypes.POINTER(ctypes.c_int64)
_intp = ctypes.POINTER(ctypes.c_int)
_GRAPH_SIGS = {
    "ghip_backend_new": ([ctypes.c_char_p, _errp], _vp),
    "ghip_backend_finalize": ([_vp], None),
    "ghip_backend_is_finalized": ([_vp], _int),
    "ghip_backend_description": ([_vp, ctypes.c_char_p, ctypes.c_size_t], _int),
    "ghip_backend_num_devices": ([_vp], _int),
    "ghip_backend_stream": ([_vp], _vp),
    "ghip_backend_capabilities": ([ctypes.c_char_p, ctypes.c_size_t], _int),
    "ghip_buffer_from_host": ([_vp, _int, _i64p, _int, _vp, ctypes.c_size_t, _errp], _vp),
    "ghip_buffer_new": ([_vp, _int, _i64p, _int, _errp], _vp),
    "ghip_buffer_to_host": ([_vp, _vp, ctypes.c_size_t, _errp], _int),
    "ghip_buffer_shape": ([_vp, _intp, _i64p, _int], _int),
    "ghip_buffer_device_ptr": ([_vp], _vp),
    "ghip_buffer_finalize": ([_vp], None),
    "ghip_builder_new": ([_vp, ctypes.c_char_p, _errp], _vp),
    "ghip_builder_finalize": ([_vp], None),
    "ghip_builder_main": ([_vp], _vp),
    "ghip_builder_compile": ([_vp, _errp], _vp),
    "ghip_fn_parameter": ([_vp, ctypes.c_char_p, _int, _i64p, _int, _errp], _int),
    "ghip_fn_constant": ([_vp, _int, _i64p, _int, _vp, ctypes.c_size_t, _errp], _int),
    "ghip_fn_iota": ([_vp, _int, _i64p, _int, _int, _errp], _int),
    "ghip_fn_unary": ([_vp, _int, _int, _errp], _int),
    "ghip_fn_binary": ([_vp, _int, _int, _int, _errp], _int),
    "ghip_fn_compare": ([_vp, _int, _int, _int, _errp], _int),
    "ghip_fn_where": ([_vp, _int, _int, _int, _errp], _int),
    "ghip_fn_clamp": ([_vp, _int, _int, _int, _errp], _int),
    "ghip_fn_convert_dtype": ([_vp, _int, _int, _errp], _int),
    "ghip_fn_reshape": ([_vp, _int, _i64p, _int, _errp], _int),
    "ghip_fn_transpose": ([_vp, _int, _intp, _int, _errp], _int),
    "ghip_fn_broadcast_in_dim": ([_vp, _int, _i64p, _int, _intp, _int, _errp], _int),
    "ghip_fn_reduce": ([_vp, _int, _int, _intp, _int, _errp], _int),
    "ghip_fn_arg_min_max": ([_vp, _int, _int, _int, _int, _errp], _int),
    "ghip_fn_dot_general": ([_vp, _int, _intp, _int, _intp, _int, _int, _intp, _int, _intp, _int,
                             _errp], _int),
    "ghip_fn_gather": ([_vp, _int, _int, _int, _intp, _int, _intp, _int, _intp, _int, _i64p, _int,
                        _int, _errp], _int),
    "ghip_fn_slice": ([_vp, _int, _i64p, _i64p, _i64p, _int, _errp], _int),
    "ghip_fn_concatenate": ([_vp, _int, _intp, _int, _errp], _int),
    "ghip_fn_reverse": ([_vp, _int, _intp, _int, _errp], _int),
    "ghip_fn_pad": ([_vp, _int, _int, _i64p, _i64p, _i64p, _int, _errp], _int),
    "ghip_fn_reduce_logical": ([_vp, _int, _int, _intp, _int, _errp], _int),
    "ghip_fn_fused_softmax": ([_vp, _int, _int, _errp], _int),
    "ghip_fn_fused_layer_norm": ([_vp, _int, _intp, _int, _dbl, _int, _int, _errp], _int),
    "ghip_fn_fused_sdpa": ([_vp, _int, _int, _int, _int, _int, _int, _int, _dbl, _int, _errp], _int),
    "ghip_fn_dynamic_slice": ([_vp, _int, _intp, _int, _i64p, _int, _errp], _int),
    "ghip_fn_dynamic_update_slice": ([_vp, _int, _int, _intp, _int, _errp], _int),
    "ghip_fn_scatter": ([_vp, _int, _int, _int, _int, _int, _intp, _int, _intp, _int, _intp, _int, _int, _int,
                         _errp], _int),
    "ghip_fn_fused_gelu": ([_vp, _int, _int, _errp], _int),
    "ghip_fn_fused_dense": ([_vp, _int, _int, _int, _int, _errp], _int),
    "ghip_fn_fused_qkv_projection": ([_vp, _int, _int, _int, _int, _int, _int, _int, _intp, _intp,
                                      _intp, _errp], _int),
    "ghip_builder_new_function": ([_vp, ctypes.c_char_p, _errp], _vp),
    "ghip_fn_closure": ([_vp, _errp], _vp),
    "ghip_fn_call": ([_vp, _vp, _intp, _int, _intp, _int, _errp], _int),
    "ghip_fn_while": ([_vp, _vp, _vp, _intp, _int, _intp, _int, _errp], _int),
    "ghip_fn_if": ([_vp, _int, _vp, _vp, _intp, _int, _errp], _int),
    "ghip_fn_sort": ([_vp, _vp, _int, _int, _intp, _int, _intp, _int, _errp], _int),
    "ghip_fn_return": ([_vp, _intp, _int, _errp], _int),
    "ghip_fn_value_shape": ([_vp, _int, _intp, _i64p, _int], _int),
    "ghip_exec_num_inputs": ([_vp], _int),
    "ghip_exec_num_outputs": ([_vp], _int),
    "ghip_exec_input_shape": ([_vp, _int, _intp, _i64p, _int], _int),
    "ghip_exec_output_shape": ([_vp, _int, _intp, _i64p, _int], _int),
    "ghip_exec_execute": ([_vp, ctypes.POINTER(_vp), _int, ctypes.POINTER(ctypes.c_uint8),
                           ctypes.POINTER(_vp), _int, _errp], _int),
    "ghip_exec_execute_noalloc": ([_vp, ctypes.POINTER(_vp), _int, ctypes.POINTER(_vp), _int, _errp], _int),
    "ghip_exec_noalloc_scratch_bytes": ([], ctypes.c_size_t),
    "ghip_exec_plan": ([_vp, ctypes.c_char_p, ctypes.c_size_t], ctypes.c_size_t),
    "ghip_exec_finalize": ([_vp], None),
}
_SIGNED = False


def _L():
    global _SIGNED
    L = _lib.load()
    if not _SIGNED:
        for name, (args, res) in _GRAPH_SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _SIGNED = True
    return L


def _raise(err: GHipError, rc: int = None):
    msg = err.message.decode() if err.message else "(no message)"
    code = err.code if rc is None else rc
    _lib.load().ghip_error_clear(ctypes.byref(err))
    raise BackendError(code, msg)


def _i64arr(xs):
    xs = [int(x) for x in xs]
    return (ctypes.c_int64 * max(len(xs), 1))(*xs), len(xs)


def _intarr(xs):
    xs = [int(x) for x in xs]
    return (ctypes.c_int * max(len(xs), 1))(*xs), len(xs)


# ---------------------------------------------------------------- Backend
class Buffer:
    """A device-resident buffer (buffer.go's gpuBuffer, but in HBM)."""

    def __init__(self, backend: "Backend", handle):
        self.backend, self.handle = backend, handle

    def shape(self) -> Shape:
        return self.backend.BufferShape(self)

    def device_ptr(self) -> int:
        return _L().ghip_buffer_device_ptr(self.handle)

    def __del__(self):
        try:
            if self.handle and not self.backend.IsFinalized():
                _L().ghip_buffer_finalize(self.handle)
        except Exception:
            pass
        self.handle = None


class Backend:
    """backends.Backend (backend.go:22-167).  New(config) == Backend(config)."""

    def __init__(self, config: str = ""):
        err = GHipError(0, None)
        h = _L().ghip_backend_new(config.encode(), ctypes.byref(err))
        if not h:
            _raise(err)
        self.handle = h

    # --- identity
    def Name(self) -> str:
        return "hip"

    def String(self) -> str:
        return self.Name()

    def Description(self) -> str:
        buf = ctypes.create_string_buffer(512)
        _L().ghip_backend_description(self.handle, buf, 512)
        return buf.value.decode()

    def NumDevices(self) -> int:
        return _L().ghip_backend_num_devices(self.handle)

    def DeviceDescription(self, device_num: int = 0) -> str:
        return self.Description()

    def Capabilities(self) -> Capabilities:
        n = _L().ghip_backend_capabilities(None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        _L().ghip_backend_capabilities(buf, n + 1)
        fields = dict(kv.split("=", 1) for kv in buf.value.decode().split(";"))
        return Capabilities(fields["functions"] == "1", frozenset(fields["ops"].split(",")),
                            frozenset(fields["dtypes"].split(",")))

    def Builder(self, name: str) -> "Builder":
        err = GHipError(0, None)
        h = _L().ghip_builder_new(self.handle, name.encode(), ctypes.byref(err))
        if not h:
            _raise(err)
        return Builder(self, h, name)

    def Finalize(self):
        if self.handle:
            _L().ghip_backend_finalize(self.handle)

    def IsFinalized(self) -> bool:
        return bool(_L().ghip_backend_is_finalized(self.handle))

    def stream(self) -> int:
        return _L().ghip_backend_stream(self.handle) or 0

    # --- DataInterface
    def BufferFromFlatData(self, device_num: int, flat, shape: Shape) -> Buffer:
        flat = np.asarray(flat)
        if shape.dtype == dtypes.BFloat16 and flat.dtype != np.uint16:
            from .synth import to_bf16_bits
            flat = to_bf16_bits(np.asarray(flat, np.float32))
        flat = np.ascontiguousarray(flat, dtype=np_dtype(shape.dtype))
        dims, r = _i64arr(shape.dims)
        err = GHipError(0, None)
        h = _L().ghip_buffer_from_host(self.handle, shape.dtype, dims, r,
                                       flat.ctypes.data_as(ctypes.c_void_p), flat.nbytes,
                                       ctypes.byref(err))
        if not h:
            _raise(err)
        return Buffer(self, h)

    def NewSharedBuffer(self, device_num: int, shape: Shape) -> Buffer:
        dims, r = _i64arr(shape.dims)
        err = GHipError(0, None)
        h = _L().ghip_buffer_new(self.handle, shape.dtype, dims, r, ctypes.byref(err))
        if not h:
            _raise(err)
        return Buffer(self, h)

    def BufferShape(self, buf: Buffer) -> Shape:
        dt = ctypes.c_int(0)
        dims = (ctypes.c_int64 * 8)()
        r = _L().ghip_buffer_shape(buf.handle, ctypes.byref(dt), dims, 8)
        if r < 0:
            raise BackendError(5, "BufferShape: buffer finalized")
        return Shape(dt.value, tuple(dims[i] for i in range(r)))

    def BufferDeviceNum(self, buf: Buffer) -> int:
        """Always 0: one device (backend.go:125-128)."""
        return 0

    def BufferToFlatData(self, buf: Buffer, flat: Optional[np.ndarray] = None) -> np.ndarray:
        s = self.BufferShape(buf)
        if flat is None:
            flat = np.empty(s.size(), dtype=np_dtype(s.dtype))
        if not flat.flags.c_contiguous:
            raise ValueError("BufferToFlatData: flat must be contiguous")
        err = GHipError(0, None)
        rc = _L().ghip_buffer_to_host(buf.handle, flat.ctypes.data_as(ctypes.c_void_p), flat.nbytes,
                                      ctypes.byref(err))
        if rc:
            _raise(err, rc)
        return flat

    def BufferData(self, buf: Buffer) -> int:
        """Direct (zero-copy) access: the device pointer."""
        return buf.device_ptr()

    def BufferFinalize(self, buf: Buffer):
        if buf.handle:
            _L().ghip_buffer_finalize(buf.handle)
            buf.handle = None

    def HasSharedBuffers(self) -> bool:
        return False

    def BufferCopyToDevice(self, source: Buffer, device_num: int):
        raise BackendError(2, "BufferCopyToDevice: only one device supported")


# ---------------------------------------------------------------- Builder / Function
class Value:
    __slots__ = ("fn", "id")

    def __init__(self, fn, vid):
        self.fn, self.id = fn, vid

    def __repr__(self):
        return f"Value({self.id}, {self.fn.OpShape(self)})"


class Builder:
    """backends.Builder (builder.go:16-109)."""

    def __init__(self, backend: Backend, handle, name: str):
        self.backend, self.handle, self.name = backend, handle, name
        self._main = None

    def Name(self) -> str:
        return self.name

    def Main(self) -> "Function":
        if self._main is None:
            self._main = Function(self, _L().ghip_builder_main(self.handle))
        return self._main

    def OpShape(self, v: Value) -> Shape:
        return self.Main().OpShape(v)

    def NewFunction(self, name: str) -> "Function":
        """Builder.NewFunction (builder.go:57-70): a named function, the target of Call."""
        err = GHipError(0, None)
        h = _L().ghip_builder_new_function(self.handle, name.encode(), ctypes.byref(err))
        if not h:
            _raise(err)
        return Function(self, h)

    def Compile(self) -> "Executable":
        err = GHipError(0, None)
        h = _L().ghip_builder_compile(self.handle, ctypes.byref(err))
        if not h:
            _raise(err)
        return Executable(self.backend, h)

    def Finalize(self):
        if self.handle:
            _L().ghip_builder_finalize(self.handle)
            self.handle = None


def _vid(v) -> int:
    return -1 if v is None else v.id


class Function:
    """backends.Function: one method per op (function.go, dotgeneral.go, gather.go)."""

    def __init__(self, builder: Builder, handle):
        self.builder, self.handle = builder, handle

    def _call(self, name, *args) -> Value:
        err = GHipError(0, None)
        vid = getattr(_L(), name)(self.handle, *args, ctypes.byref(err))
        if vid < 0:
            _raise(err)
        return Value(self, vid)

    def OpShape(self, v: Value) -> Shape:
        dt = ctypes.c_int(0)
        dims = (ctypes.c_int64 * 8)()
        r = _L().ghip_fn_value_shape(self.handle, v.id, ctypes.byref(dt), dims, 8)
        if r < 0:
            raise BackendError(1, "OpShape: invalid value")
        return Shape(dt.value, tuple(dims[i] for i in range(r)))

    # lifecycle
    def Parameter(self, name: str, shape: Shape, sharding=None) -> Value:
        dims, r = _i64arr(shape.dims)
        return self._call("ghip_fn_parameter", name.encode(), shape.dtype, dims, r)

    def Constant(self, flat, *dims, dtype: Optional[int] = None) -> Value:
        arr = np.asarray(flat)
        if dtype is None:
            dtype = _FROM_NP[arr.dtype]
        if dtype == dtypes.BFloat16 and arr.dtype != np.uint16:
            from .synth import to_bf16_bits
            arr = to_bf16_bits(np.asarray(arr, np.float32))
        arr = np.ascontiguousarray(arr, dtype=np_dtype(dtype))
        d, r = _i64arr(dims)
        return self._call("ghip_fn_constant", dtype, d, r, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)

    def Return(self, outputs: Sequence[Value], shardings=None):
        ids, n = _intarr([o.id for o in outputs])
        err = GHipError(0, None)
        rc = _L().ghip_fn_return(self.handle, ids, n, ctypes.byref(err))
        if rc:
            _raise(err, rc)

    # creation
    def Iota(self, shape: Shape, iota_axis: int) -> Value:
        dims, r = _i64arr(shape.dims)
        return self._call("ghip_fn_iota", shape.dtype, dims, r, iota_axis)

    # elementwise
    def Where(self, cond, on_true, on_false) -> Value:
        return self._call("ghip_fn_where", cond.id, on_true.id, on_false.id)

    def Clamp(self, lo, x, hi) -> Value:
        return self._call("ghip_fn_clamp", lo.id, x.id, hi.id)

    def ConvertDType(self, x, dtype: int) -> Value:
        return self._call("ghip_fn_convert_dtype", x.id, dtype)

    # shape ops
    def Reshape(self, x, *dims) -> Value:
        d, r = _i64arr(dims)
        return self._call("ghip_fn_reshape", x.id, d, r)

    def Transpose(self, x, *permutation) -> Value:
        p, r = _intarr(permutation)
        return self._call("ghip_fn_transpose", x.id, p, r)

    def BroadcastInDim(self, x, output_shape: Shape, broadcast_axes: Sequence[int]) -> Value:
        d, r = _i64arr(output_shape.dims)
        a, na = _intarr(broadcast_axes)
        return self._call("ghip_fn_broadcast_in_dim", x.id, d, r, a, na)

    def Slice(self, x, starts, limits, strides=None) -> Value:
        s, r = _i64arr(starts)
        lim, _ = _i64arr(limits)
        st, _ = _i64arr(strides if strides is not None else [1] * len(starts))
        return self._call("ghip_fn_slice", x.id, s, lim, st, r)

    def Concatenate(self, axis: int, *operands) -> Value:
        ids, n = _intarr([o.id for o in operands])
        return self._call("ghip_fn_concatenate", axis, ids, n)

    def Reverse(self, x, *axes) -> Value:
        a, n = _intarr(axes)
        return self._call("ghip_fn_reverse", x.id, a, n)

    def Pad(self, operand, fill_value, *axes_config) -> Value:
        """axes_config: one PadAxis (or (start, end[, interior]) tuple) per axis."""
        cfg = [a if isinstance(a, PadAxis) else PadAxis(*a) for a in axes_config]
        st, r = _i64arr([a.start for a in cfg])
        en, _ = _i64arr([a.end for a in cfg])
        it, _ = _i64arr([a.interior for a in cfg])
        return self._call("ghip_fn_pad", operand.id, fill_value.id, st, en, it, r)

    # reductions
    def ReduceLogicalAnd(self, x, *axes) -> Value:
        a, n = _intarr(axes)
        return self._call("ghip_fn_reduce_logical", 0, x.id, a, n)

    def ReduceLogicalOr(self, x, *axes) -> Value:
        a, n = _intarr(axes)
        return self._call("ghip_fn_reduce_logical", 1, x.id, a, n)

    def _reduce(self, op, x, axes):
        a, n = _intarr(axes)
        return self._call("ghip_fn_reduce", op, x.id, a, n)

    def ArgMinMax(self, x, axis: int, output_dtype: int, is_min: bool) -> Value:
        return self._call("ghip_fn_arg_min_max", x.id, axis, output_dtype, int(is_min))

    # matrix / indexing
    def DotGeneral(self, lhs, lhs_contracting, lhs_batch, rhs, rhs_contracting, rhs_batch,
                   config=None) -> Value:
        lc, nlc = _intarr(lhs_contracting or [])
        lb, nlb = _intarr(lhs_batch or [])
        rc, nrc = _intarr(rhs_contracting or [])
        rb, nrb = _intarr(rhs_batch or [])
        return self._call("ghip_fn_dot_general", lhs.id, lc, nlc, lb, nlb, rhs.id, rc, nrc, rb, nrb)

    def Gather(self, operand, start_indices, index_vector_axis, offset_output_axes,
               collapsed_slice_axes, start_index_map, slice_sizes, indices_are_sorted=False) -> Value:
        o, no = _intarr(offset_output_axes)
        c, nc = _intarr(collapsed_slice_axes)
        m, nm = _intarr(start_index_map)
        s, ns = _i64arr(slice_sizes)
        return self._call("ghip_fn_gather", operand.id, start_indices.id, index_vector_axis, o, no,
                          c, nc, m, nm, s, ns, int(indices_are_sorted))

    def DynamicSlice(self, operand, start_indices, slice_sizes) -> Value:
        s, ns = _intarr([v.id for v in start_indices])
        z, nz = _i64arr(slice_sizes)
        return self._call("ghip_fn_dynamic_slice", operand.id, s, ns, z, nz)

    def DynamicUpdateSlice(self, operand, update, start_indices) -> Value:
        s, ns = _intarr([v.id for v in start_indices])
        return self._call("ghip_fn_dynamic_update_slice", operand.id, update.id, s, ns)

    def _scatter(self, mode, operand, scatter_indices, updates, index_vector_axis, update_window_axes,
                 inserted_window_axes, scatter_axes_to_operand_axes, indices_are_sorted=False,
                 unique_indices=False) -> Value:
        u, nu = _intarr(update_window_axes)
        i, ni = _intarr(inserted_window_axes)
        a, na = _intarr(scatter_axes_to_operand_axes)
        return self._call("ghip_fn_scatter", mode, operand.id, scatter_indices.id, updates.id, index_vector_axis,
                          u, nu, i, ni, a, na, int(indices_are_sorted), int(unique_indices))

    def ScatterSum(self, *args, **kw) -> Value:
        return self._scatter(0, *args, **kw)

    def ScatterMax(self, *args, **kw) -> Value:
        return self._scatter(1, *args, **kw)

    def ScatterMin(self, *args, **kw) -> Value:
        return self._scatter(2, *args, **kw)

    # functions and control flow
    def Closure(self) -> "Function":
        """Function.Closure (function.go:120-133)."""
        err = GHipError(0, None)
        h = _L().ghip_fn_closure(self.handle, ctypes.byref(err))
        if not h:
            _raise(err)
        return Function(self.builder, h)

    def _cf(self, name, *args, max_outs=64):
        outs = (ctypes.c_int * max_outs)()
        err = GHipError(0, None)
        n = getattr(_L(), name)(self.handle, *args, outs, max_outs, ctypes.byref(err))
        if n < 0:
            _raise(err)
        return [Value(self, outs[i]) for i in range(n)]

    def Call(self, fn: "Function", *inputs):
        a, n = _intarr([v.id for v in inputs])
        return self._cf("ghip_fn_call", fn.handle, a, n)

    def While(self, cond: "Function", body: "Function", *initial_state):
        a, n = _intarr([v.id for v in initial_state])
        return self._cf("ghip_fn_while", cond.handle, body.handle, a, n)

    def If(self, pred, true_branch: "Function", false_branch: "Function"):
        return self._cf("ghip_fn_if", pred.id, true_branch.handle, false_branch.handle)

    def Sort(self, comparator: "Function", axis: int, is_stable: bool, *inputs):
        a, n = _intarr([v.id for v in inputs])
        return self._cf("ghip_fn_sort", comparator.handle, int(axis), int(is_stable), a, n)

    # fused ops
    def FusedSoftmax(self, x, axis: int) -> Value:
        return self._call("ghip_fn_fused_softmax", x.id, axis)

    def FusedLayerNorm(self, x, axes, epsilon: float, gamma=None, beta=None) -> Value:
        a, n = _intarr(axes)
        return self._call("ghip_fn_fused_layer_norm", x.id, a, n, float(epsilon), _vid(gamma), _vid(beta))

    def FusedScaledDotProductAttention(self, query, key, value, mask, num_heads: int,
                                       num_kv_heads: int, axes_layout: int, scale: float,
                                       causal: bool, options=None) -> Value:
        return self._call("ghip_fn_fused_sdpa", query.id, key.id, value.id, _vid(mask), num_heads,
                          num_kv_heads, axes_layout, float(scale), int(causal))

    def FusedGelu(self, x, exact: bool) -> Value:
        return self._call("ghip_fn_fused_gelu", x.id, int(exact))

    def FusedDense(self, x, weight, bias, activation: int) -> Value:
        return self._call("ghip_fn_fused_dense", x.id, weight.id, _vid(bias), int(activation))

    def FusedAttentionQKVProjection(self, x, w_qkv, bias_q, bias_k, bias_v, query_dim: int,
                                    key_value_dim: int):
        """Returns (query, key, value)."""
        out = [ctypes.c_int(-1) for _ in range(3)]
        err = GHipError(0, None)
        rc = _L().ghip_fn_fused_qkv_projection(self.handle, x.id, w_qkv.id, _vid(bias_q), _vid(bias_k),
                                                _vid(bias_v), int(query_dim), int(key_value_dim),
                                                *(ctypes.byref(o) for o in out), ctypes.byref(err))
        if rc != 0:
            _raise(err, rc)
        return tuple(Value(self, o.value) for o in out)


def _add_unary(name, code):
    def f(self, x):
        return self._call("ghip_fn_unary", code, x.id)
    f.__name__ = name
    setattr(Function, name, f)


def _add_binary(name, code, cfn):
    def f(self, lhs, rhs):
        return self._call(cfn, code, lhs.id, rhs.id)
    f.__name__ = name
    setattr(Function, name, f)


def _add_reduce(name, code):
    def f(self, x, *axes):
        return self._reduce(code, x, axes)
    f.__name__ = name
    setattr(Function, name, f)


for _i, _n in enumerate(UNARY):
    _add_unary(_n, _i)
for _i, _n in enumerate(BINARY):
    _add_binary(_n, _i, "ghip_fn_binary")
for _i, _n in enumerate(COMPARE):
    _add_binary(_n, _i, "ghip_fn_compare")
for _n, _c in REDUCE.items():
    _add_reduce(_n, _c)
# EqualTotalOrder ... LessOrEqualTotalOrder: the plain comparisons, as the
# reference delegates them (function.go:2227-2256); they differ from a total
# order only for NaN and for -0 vs +0.
for _i, _n in enumerate(COMPARE):
    _add_binary(_n + "TotalOrder", _i, "ghip_fn_compare")


# ---------------------------------------------------------------- Executable
class Executable:
    """backends.Executable (executable.go:19-112)."""

    def __init__(self, backend: Backend, handle):
        self.backend, self.handle = backend, handle

    def _shape(self, fn, i):
        dt = ctypes.c_int(0)
        dims = (ctypes.c_int64 * 8)()
        r = fn(self.handle, i, ctypes.byref(dt), dims, 8)
        return Shape(dt.value, tuple(dims[k] for k in range(r)))

    def Inputs(self):
        n = _L().ghip_exec_num_inputs(self.handle)
        return [self._shape(_L().ghip_exec_input_shape, i) for i in range(n)]

    def Outputs(self):
        n = _L().ghip_exec_num_outputs(self.handle)
        return [self._shape(_L().ghip_exec_output_shape, i) for i in range(n)]

    def Execute(self, inputs: Sequence[Buffer], donate=None, default_device: int = 0):
        n = len(inputs)
        arr = (ctypes.c_void_p * max(n, 1))(*[b.handle for b in inputs])
        nout = _L().ghip_exec_num_outputs(self.handle)
        outs = (ctypes.c_void_p * max(nout, 1))()
        don = None
        if donate is not None:
            don = (ctypes.c_uint8 * max(n, 1))(*[int(bool(d)) for d in donate])
        err = GHipError(0, None)
        rc = _L().ghip_exec_execute(self.handle, arr, n, don, outs, nout, ctypes.byref(err))
        if rc:
            _raise(err, rc)
        return [Buffer(self.backend, outs[i]) for i in range(nout)]

    def ExecuteNoAlloc(self, inputs: Sequence[Buffer], outputs: Sequence[Buffer]) -> None:
        """Execute into caller-allocated output buffers with the intermediates in the
        library's per-GPU scratch array: no device memory is allocated."""
        n, nout = len(inputs), len(outputs)
        arr = (ctypes.c_void_p * max(n, 1))(*[b.handle for b in inputs])
        outs = (ctypes.c_void_p * max(nout, 1))(*[b.handle for b in outputs])
        err = GHipError(0, None)
        rc = _L().ghip_exec_execute_noalloc(self.handle, arr, n, outs, nout, ctypes.byref(err))
        if rc:
            _raise(err, rc)

    def Plan(self) -> str:
        n = _L().ghip_exec_plan(self.handle, None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        _L().ghip_exec_plan(self.handle, buf, n + 1)
        return buf.value.decode()

    def Finalize(self):
        if self.handle:
            _L().ghip_exec_finalize(self.handle)
            self.handle = None


def New(config: str = "") -> Backend:
    """backends.Register(name, New) constructor (backend.go:33-43)."""
    return Backend(config)
