"""Direct-op front end: device tensors in, device tensors out, via the C ABI.

torch is used only as the allocator of device memory and as the source of the
current HIP stream; every computation runs in libgomlx_hip.so.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call

_DT = {
    torch.float32: _lib.DT_FLOAT32,
    torch.bfloat16: _lib.DT_BFLOAT16,
    torch.float16: _lib.DT_FLOAT16,
    torch.int32: _lib.DT_INT32,
    torch.int64: _lib.DT_INT64,
    torch.bool: _lib.DT_BOOL,
    torch.uint8: _lib.DT_UINT8,
    torch.int8: _lib.DT_INT8,
    torch.int16: _lib.DT_INT16,
}
for _name, _code in (("uint16", "DT_UINT16"), ("uint32", "DT_UINT32"), ("uint64", "DT_UINT64")):
    if hasattr(torch, _name) and hasattr(_lib, _code):
        _DT[getattr(torch, _name)] = getattr(_lib, _code)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"gomlx_hip: unsupported dtype {dt}") from None


def _stream(stream=None) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return int(stream)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check_dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("gomlx_hip ops take device tensors")


def _rows(x: torch.Tensor):
    if not x.is_contiguous():
        raise ValueError("row kernels need a contiguous input")
    n = x.shape[-1] if x.dim() else 1
    return x.numel() // max(n, 1), n


def softmax(x: torch.Tensor, log: bool = False, out=None, stream=None) -> torch.Tensor:
    """Softmax (log-softmax) over the last axis."""
    _check_dev(x)
    rows, n = _rows(x)
    y = torch.empty_like(x) if out is None else out
    call("ghip_softmax_rows", dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), rows, n,
         int(log), _stream(stream))
    return y


def scale_mask_softmax(x: torch.Tensor, scale: float, causal: bool, bmask=None, out=None,
                       stream=None) -> torch.Tensor:
    """softmax(x * scale + mask) over the last axis of x [..., sq, sk]."""
    _check_dev(x, bmask)
    sq, sk = x.shape[-2], x.shape[-1]
    rows = x.numel() // sk
    y = torch.empty_like(x) if out is None else out
    call("ghip_scale_mask_softmax_rows", dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), rows,
         sq, sk, float(scale), int(causal), _ptr(bmask), _stream(stream))
    return y


def rmsnorm(x: torch.Tensor, gamma=None, eps: float = 1e-6, out=None, stream=None):
    _check_dev(x, gamma)
    rows, n = _rows(x)
    y = torch.empty_like(x) if out is None else out
    call("ghip_rmsnorm_rows", dtype_code(x.dtype), x.data_ptr(), _ptr(gamma), y.data_ptr(),
         rows, n, float(eps), _stream(stream))
    return y


def layernorm(x: torch.Tensor, gamma=None, beta=None, eps: float = 1e-5, out=None, stream=None):
    _check_dev(x, gamma, beta)
    rows, n = _rows(x)
    y = torch.empty_like(x) if out is None else out
    call("ghip_layernorm_rows", dtype_code(x.dtype), x.data_ptr(), _ptr(gamma), _ptr(beta),
         y.data_ptr(), rows, n, float(eps), _stream(stream))
    return y


def gemm_workspace(a_dtype, out_dtype, B: int, M: int, N: int, K: int, device):
    """Workspace for ghip_gemm_batched_ws / ghip_gemm_grouped_ws (None when a
    product of these sizes never splits its contraction)."""
    n = _lib.load().ghip_gemm_workspace_bytes(dtype_code(a_dtype), dtype_code(out_dtype or a_dtype), B, M, N, K)
    return torch.empty((n,), dtype=torch.uint8, device=device) if n > 0 else None


def gemm(a: torch.Tensor, b: torch.Tensor, out_dtype=None, out=None, stream=None, k_split: bool = True,
         workspace=None):
    """c[b] = a[b] @ b[b] for a [B,M,K] / [M,K], b [B,K,N] / [K,N]; any strides.
    k_split: with a workspace (`workspace`, or one allocated here), so few-tile
    products with a long contraction split it (ghip_gemm_batched_ws)."""
    _check_dev(a, b)
    squeeze = a.dim() == 2
    a3 = a.unsqueeze(0) if a.dim() == 2 else a
    b3 = b.unsqueeze(0) if b.dim() == 2 else b
    B, M, K = a3.shape
    B2, K2, N = b3.shape
    if K != K2 or (B2 != B and B2 != 1):
        raise ValueError(f"gemm: shapes {tuple(a.shape)} x {tuple(b.shape)}")
    odt = out_dtype or a.dtype
    c = torch.empty((B, M, N), dtype=odt, device=a.device) if out is None else out.view(B, M, N)
    sb_b = b3.stride(0) if B2 == B else 0
    if k_split and workspace is None:
        workspace = gemm_workspace(a.dtype, odt, B, M, N, K, a.device)
    ws_ptr = workspace.data_ptr() if (k_split and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if ws_ptr is not None else 0
    call("ghip_gemm_batched_ws", dtype_code(a.dtype), dtype_code(odt), B, M, N, K,
         a3.data_ptr(), a3.stride(0), a3.stride(1), a3.stride(2),
         b3.data_ptr(), sb_b, b3.stride(1), b3.stride(2),
         c.data_ptr(), c.stride(0), c.stride(1), c.stride(2), ws_ptr, ws_bytes, _stream(stream))
    return c[0] if squeeze else c


def gemm_grouped(a: torch.Tensor, bs, out_dtype=None, outs=None, stream=None, k_split: bool = True,
                 workspace=None):
    """[a @ b for b in bs] in one call (ghip_gemm_grouped_ws): a [M,K], every b [K,N]
    with the same strides; returns the list of [M,N] results.  k_split as in gemm."""
    import ctypes
    _check_dev(a, *bs)
    M, K = a.shape
    K2, N = bs[0].shape
    if K != K2 or any(b.shape != bs[0].shape or b.stride() != bs[0].stride() for b in bs):
        raise ValueError("gemm_grouped: every b must be [K, N] with the same strides")
    odt = out_dtype or a.dtype
    cs = [torch.empty((M, N), dtype=odt, device=a.device) for _ in bs] if outs is None else list(outs)
    if any(c.stride() != cs[0].stride() or c.stride(1) != 1 for c in cs):
        raise ValueError("gemm_grouped: outputs need one row stride and unit column stride")
    bp = (ctypes.c_void_p * len(bs))(*[b.data_ptr() for b in bs])
    cp = (ctypes.c_void_p * len(cs))(*[c.data_ptr() for c in cs])
    if k_split and workspace is None:
        workspace = gemm_workspace(a.dtype, odt, 1, M, N, K, a.device)
    ws_ptr = workspace.data_ptr() if (k_split and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if ws_ptr is not None else 0
    call("ghip_gemm_grouped_ws", dtype_code(a.dtype), dtype_code(odt), len(bs), M, N, K, a.data_ptr(),
         a.stride(0), a.stride(1), bp, bs[0].stride(0), bs[0].stride(1), cp, cs[0].stride(0), ws_ptr, ws_bytes,
         _stream(stream))
    return cs


def softmax_axis(x: torch.Tensor, axis: int, log: bool = False, out=None, stream=None) -> torch.Tensor:
    """Softmax (log-softmax) over a middle axis of a contiguous tensor (the column
    kernel: x read as [outer, n, inner])."""
    _check_dev(x)
    if not x.is_contiguous():
        raise ValueError("softmax_axis: contiguous input required")
    axis = axis % x.dim()
    outer = 1
    for d in x.shape[:axis]:
        outer *= d
    inner = 1
    for d in x.shape[axis + 1:]:
        inner *= d
    y = torch.empty_like(x) if out is None else out
    call("ghip_softmax_cols", dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), outer, x.shape[axis], inner,
         int(log), _stream(stream))
    return y


def copy(src: torch.Tensor, out: torch.Tensor, stream=None) -> torch.Tensor:
    """out[...] = src[...] for tensors of one shape and element size, any strides."""
    import ctypes
    _check_dev(src, out)
    if tuple(src.shape) != tuple(out.shape) or src.element_size() != out.element_size():
        raise ValueError(f"copy: {tuple(src.shape)} x{src.element_size()} -> {tuple(out.shape)} x{out.element_size()}")
    r = src.dim()
    arr = ctypes.c_int64 * max(r, 1)
    call("ghip_copy_strided", src.element_size(), src.data_ptr(), out.data_ptr(), r,
         arr(*src.shape), arr(*src.stride()), arr(*out.stride()), _stream(stream))
    return out


def _strides3(t: torch.Tensor):
    """(batch, head, sequence) element strides of a [B, H, S, D] view."""
    import ctypes
    if t.stride(3) != 1:
        raise ValueError("sdpa: the head dim must be contiguous")
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


def sdpa_workspace(q: torch.Tensor, Hkv: int, Sk: int, causal: bool):
    """Workspace for ghip_sdpa_fwd_masked_ws (None when the shape takes no key split)."""
    B, H, Sq, D = q.shape
    n = _lib.load().ghip_sdpa_workspace_bytes(dtype_code(q.dtype), B, H, Hkv, Sq, Sk, D, int(causal))
    return torch.empty((n,), dtype=torch.uint8, device=q.device) if n > 0 else None


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, causal: bool,
         out=None, stream=None, kv_split: bool = True, workspace=None):
    """Fused attention: q [B,H,Sq,D], k / v [B,Hkv,Sk,D] (any strides with a contiguous
    head dim, e.g. BSHD storage viewed as BHSD) -> out [B,H,Sq,D].  kv_split: with a
    workspace (`workspace`, or one allocated here), so small grids split their key
    range (ghip_sdpa_fwd_masked_ws)."""
    return sdpa_masked(q, k, v, None, scale, causal, out=out, stream=stream, kv_split=kv_split,
                       workspace=workspace)


def _mask_strides(mask: torch.Tensor, B, H, Sq, Sk):
    """Element strides of `mask` broadcast to [B, H, Sq, Sk] over its trailing axes
    (0 on missing and size-1 axes)."""
    import ctypes
    st = [0, 0, 0, 0]
    off = 4 - mask.dim()
    for i in range(mask.dim()):
        if mask.shape[i] != 1:
            if mask.shape[i] != (B, H, Sq, Sk)[off + i]:
                raise ValueError(f"mask {tuple(mask.shape)} does not broadcast to {(B, H, Sq, Sk)}")
            st[off + i] = mask.stride(i)
    return (ctypes.c_int64 * 4)(*st)


def sdpa_masked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask, scale: float, causal: bool,
                out=None, stream=None, kv_split: bool = True, workspace=None):
    """sdpa with a bool keep-mask or an additive mask (q's dtype) of any rank that
    broadcasts to the scores [B, H, Sq, Sk] (mask None: none)."""
    _check_dev(q, k, v, *([mask] if mask is not None else []))
    B, H, Sq, D = q.shape
    _, Hkv, Sk, _ = k.shape
    o = torch.empty((B, H, Sq, D), dtype=q.dtype, device=q.device) if out is None else out
    mdt = -1 if mask is None else dtype_code(mask.dtype)
    ms = None if mask is None else _mask_strides(mask, B, H, Sq, Sk)
    ws = (workspace if workspace is not None else sdpa_workspace(q, Hkv, Sk, causal)) if kv_split else None
    call("ghip_sdpa_fwd_masked_ws", dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
         o.data_ptr(), B, H, Hkv, Sq, Sk, D, _strides3(q), _strides3(k), _strides3(v),
         _strides3(o), _ptr(mask), mdt, ms, float(scale), int(causal), _ptr(ws),
         0 if ws is None else ws.numel(), _stream(stream))
    return o


def scale_mask_softmax_ex(x: torch.Tensor, scale: float, causal: bool, mask=None, out=None, stream=None):
    """softmax(x * scale + mask) over the last axis of scores x [B, H, Sq, Sk]."""
    _check_dev(x, mask)
    B, H, Sq, Sk = x.shape
    y = torch.empty_like(x) if out is None else out
    mdt = -1 if mask is None else dtype_code(mask.dtype)
    ms = None if mask is None else _mask_strides(mask, B, H, Sq, Sk)
    call("ghip_scale_mask_softmax_rows_ex", dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), B, H, Sq, Sk,
         float(scale), int(causal), _ptr(mask), mdt, ms, _stream(stream))
    return y


def gather_rows(table: torch.Tensor, ids: torch.Tensor, out=None, stream=None):
    """out[i] = table[clamp(ids[i])] for an embedding table [V, ...]."""
    _check_dev(table, ids)
    if ids.dtype != torch.int32 or not ids.is_contiguous() or not table.is_contiguous():
        raise ValueError("gather_rows: contiguous table and int32 ids required")
    V = table.shape[0]
    row_bytes = table[0].numel() * table.element_size()
    o = torch.empty((ids.numel(),) + tuple(table.shape[1:]), dtype=table.dtype,
                    device=table.device) if out is None else out
    call("ghip_gather_rows", table.data_ptr(), V, row_bytes, ids.data_ptr(), ids.numel(),
         o.data_ptr(), _stream(stream))
    return o.view(tuple(ids.shape) + tuple(table.shape[1:])) if out is None else o


def argminmax(x: torch.Tensor, axis: int, is_min: bool = False, out_dtype=torch.int32,
              stream=None):
    _check_dev(x)
    if not x.is_contiguous():
        raise ValueError("argminmax: contiguous input required")
    ax = axis % x.dim()
    outer = 1
    for d in x.shape[:ax]:
        outer *= d
    inner = 1
    for d in x.shape[ax + 1:]:
        inner *= d
    o = torch.empty(tuple(x.shape[:ax]) + tuple(x.shape[ax + 1:]), dtype=out_dtype,
                    device=x.device)
    call("ghip_argminmax", dtype_code(x.dtype), x.data_ptr(), outer, x.shape[ax], inner,
         int(is_min), dtype_code(out_dtype), o.data_ptr(), _stream(stream))
    return o


def iota(shape, axis: int, dtype=torch.int32, device="cuda", stream=None):
    o = torch.empty(tuple(shape), dtype=dtype, device=device)
    ax = axis % len(shape)
    outer = 1
    for d in shape[:ax]:
        outer *= d
    inner = 1
    for d in shape[ax + 1:]:
        inner *= d
    call("ghip_iota", dtype_code(dtype), o.data_ptr(), outer, shape[ax], inner, _stream(stream))
    return o
