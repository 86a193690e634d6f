"""ctypes front end of the CPU oracle (oracle/oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py
import this module, as the checker.  Every function returns fp64 results computed
by the C restatement; inputs are fp32 numpy arrays (bf16 data is passed widened,
which is exact).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

MODE_F64 = 0
MODE_F32SEQ = 1

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def build() -> str:
    """Compile liboracle.so (gcc + OpenMP) and return its path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_softmax.argtypes = [_f32p, _f64p, _i64, _i64, _i64, _int, _int]
        L.orc_layernorm.argtypes = [_f32p, _vp, _vp, _f64p, _i64, _i64, ctypes.c_double, _int]
        L.orc_rmsnorm.argtypes = [_f32p, _vp, _f64p, _i64, _i64, ctypes.c_double, _int]
        L.orc_rmsnorm_f32.argtypes = [_f32p, _vp, _f32p, _i64, _i64, ctypes.c_double]
        L.orc_dot_general.argtypes = [_f32p, _int, _i64p, _vp, _int, _vp, _int,
                                      _f32p, _int, _i64p, _vp, _int, _vp, _int, _f64p, _int]
        L.orc_dot_general.restype = _int
        L.orc_dot_sampled.argtypes = [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                      _i64p, _i64p, _i64p, _i64, _f64p]
        L.orc_sdpa.argtypes = [_f32p, _f32p, _f32p, _vp, _int, _i64p, _i64, _i64, _i64, _i64, _i64, _i64,
                               ctypes.c_double, _int, _f64p]
        L.orc_gather_rows.argtypes = [_vp, _i64, _i64, _i32p, _i64, _vp]
        L.orc_argminmax.argtypes = [_f32p, _i64, _i64, _i64, _int, _i64p]
        L.orc_argminmax_int.argtypes = [_i64p, _i64, _i64, _i64, _int, _int, _i64p]
        L.orc_iota.argtypes = [_f64p, _i64, _i64, _i64]
        L.orc_f32_to_bf16.argtypes = [_f32p, _u16p, _i64]
        L.orc_activation.argtypes = [_f64p, _f64p, _i64, _int]
        L.orc_dynamic_slice.argtypes = [_vp, _int, _int, _i64p, _i64p, _i64p, _vp]
        L.orc_dynamic_update_slice.argtypes = [_vp, _int, _int, _i64p, _vp, _i64p, _i64p, _vp]
        L.orc_scatter.argtypes = [_int, _f64p, _int, _i64p, _i64p, _int, _i64p, _int, _f64p, _int, _i64p,
                                  _vp, _int, _vp, _int, _vp, _int, _f64p]
        _lib = L
    return _lib


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _split(shape, axis):
    axis = axis % len(shape)
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    return outer, int(shape[axis]), inner


def softmax(x, axis=-1, log=False, mode=MODE_F64) -> np.ndarray:
    x = _f32(x)
    y = np.empty(x.shape, np.float64)
    outer, n, inner = _split(x.shape, axis)
    lib().orc_softmax(x, y, outer, n, inner, int(log), mode)
    return y


def log_softmax(x, axis=-1, mode=MODE_F64) -> np.ndarray:
    return softmax(x, axis, log=True, mode=mode)


def _opt(a):
    if a is None:
        return None, None
    a = _f32(a).reshape(-1)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def layernorm(x, gamma=None, beta=None, eps=1e-5, mode=MODE_F64) -> np.ndarray:
    """LayerNorm over the last axis; gamma/beta broadcast over it ([n] or [1, n])."""
    x = _f32(x)
    n = x.shape[-1]
    g, gp = _opt(gamma)
    b, bp = _opt(beta)
    y = np.empty(x.shape, np.float64)
    lib().orc_layernorm(x, gp, bp, y, x.size // n, n, eps, mode)
    return y


def rmsnorm(x, gamma=None, eps=1e-6, mode=MODE_F64) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    g, gp = _opt(gamma)
    y = np.empty(x.shape, np.float64)
    lib().orc_rmsnorm(x, gp, y, x.size // n, n, eps, mode)
    return y


def rmsnorm_f32(x, gamma=None, eps=1e-6, out=None) -> np.ndarray:
    """RMSNorm in fp32 end to end (fp32 sequential statistics, fp32 output)."""
    x = _f32(x)
    n = x.shape[-1]
    g, gp = _opt(gamma)
    y = np.empty(x.shape, np.float32) if out is None else out
    lib().orc_rmsnorm_f32(x, gp, y, x.size // n, n, eps)
    return y


def _int_arr(lst):
    a = np.ascontiguousarray(np.asarray(list(lst), dtype=np.int32))
    return a, (a.ctypes.data_as(ctypes.c_void_p) if a.size else None)


def dot_general_shape(lshape, lc, lb, rshape, rc, rb):
    """Output dims [batch..., lhs free..., rhs free...] (dotgeneral.go:15-53)."""
    dims = [lshape[a] for a in lb]
    dims += [d for i, d in enumerate(lshape) if i not in lc and i not in lb]
    dims += [d for i, d in enumerate(rshape) if i not in rc and i not in rb]
    return tuple(dims)


def dot_general(lhs, lc, lb, rhs, rc, rb, mode=MODE_F64) -> np.ndarray:
    lhs, rhs = _f32(lhs), _f32(rhs)
    oshape = dot_general_shape(lhs.shape, lc, lb, rhs.shape, rc, rb)
    out = np.empty(oshape, np.float64)
    ld = np.asarray(lhs.shape, np.int64)
    rd = np.asarray(rhs.shape, np.int64)
    a1, p1 = _int_arr(lc)
    a2, p2 = _int_arr(lb)
    a3, p3 = _int_arr(rc)
    a4, p4 = _int_arr(rb)
    rc_ = lib().orc_dot_general(lhs, lhs.ndim, ld, p1, len(lc), p2, len(lb),
                                rhs, rhs.ndim, rd, p3, len(rc), p4, len(rb), out, mode)
    if rc_ != 0:
        raise ValueError("orc_dot_general: invalid axes")
    return out


def dot_sampled(a, b, bs, ms, ns) -> np.ndarray:
    """Sampled fp64 entries of C[b] = A[b] @ B[b] for A [B,M,K], B [B,K,N] (fp32)."""
    a, b = _f32(a), _f32(b)
    Bn, M, K = a.shape
    _, K2, N = b.shape
    assert K == K2
    bs = np.ascontiguousarray(bs, np.int64)
    ms = np.ascontiguousarray(ms, np.int64)
    ns = np.ascontiguousarray(ns, np.int64)
    out = np.empty(bs.shape, np.float64)
    lib().orc_dot_sampled(a.ctypes.data, M * K, K, 1, b.ctypes.data, K * N, N, 1, K,
                          bs, ms, ns, bs.size, out)
    return out


def sdpa(q, k, v, mask=None, scale=None, causal=False, additive=None) -> np.ndarray:
    """Attention in BHSD layout; q [B,H,Sq,D], k/v [B,Hkv,Sk,D].  mask: a bool
    keep-mask, additive: an additive mask (fp32); either of any rank that
    broadcasts (numpy rules, trailing axes) to the scores [B,H,Sq,Sk]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Sq, D = q.shape
    _, Hkv, Sk, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    kind, mp, keep = 0, None, None
    strides = np.zeros(4, np.int64)
    m = mask if mask is not None else additive
    if m is not None:
        kind = 1 if mask is not None else 2
        keep = np.ascontiguousarray(np.asarray(m, bool if kind == 1 else np.float32))
        if kind == 1:
            keep = keep.astype(np.uint8)
        view = np.broadcast_to(keep, (B, H, Sq, Sk))      # strides 0 on broadcast axes
        strides = np.asarray([st // keep.itemsize for st in view.strides], np.int64)
        mp = keep.ctypes.data_as(ctypes.c_void_p)
    out = np.empty((B, H, Sq, D), np.float64)
    lib().orc_sdpa(q, k, v, mp, kind, strides, B, H, Hkv, Sq, Sk, D, float(scale), int(causal), out)
    return out


def gather_rows(table: np.ndarray, ids) -> np.ndarray:
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(np.asarray(ids, np.int32).reshape(-1))
    V = table.shape[0]
    row_bytes = table.nbytes // V
    out = np.empty((ids.size,) + table.shape[1:], table.dtype)
    lib().orc_gather_rows(table.ctypes.data, V, row_bytes, ids, ids.size, out.ctypes.data)
    return out


def argminmax(x, axis, is_min=False) -> np.ndarray:
    """Index of the max (min) along `axis`: floats compare as fp32 with NaN
    winning, integers compare exactly (as int64 / uint64); ties -> lowest index."""
    x = np.asarray(x)
    outer, n, inner = _split(x.shape, axis)
    out = np.empty(outer * inner, np.int64)
    if x.dtype.kind in "iu":
        unsigned = x.dtype.kind == "u"
        xi = np.ascontiguousarray(x.astype(np.uint64 if unsigned else np.int64)).view(np.int64)
        lib().orc_argminmax_int(xi, outer, n, inner, int(is_min), int(unsigned), out)
    else:
        x = _f32(x)
        lib().orc_argminmax(x, outer, n, inner, int(is_min), out)
    ax = axis % x.ndim
    return out.reshape(x.shape[:ax] + x.shape[ax + 1:])


def iota(shape, axis) -> np.ndarray:
    outer, n, inner = _split(tuple(shape), axis)
    out = np.empty(tuple(shape), np.float64)
    lib().orc_iota(out, outer, n, inner)
    return out


def dynamic_slice(x, starts, sizes) -> np.ndarray:
    """DynamicSlice (function.go:1571-1594), starts clamped to [0, dim - size]; any dtype, bit-exact."""
    x = np.ascontiguousarray(x)
    out = np.empty(tuple(int(s) for s in sizes), x.dtype)
    lib().orc_dynamic_slice(x.ctypes.data, x.itemsize, x.ndim, np.asarray(x.shape, np.int64),
                            np.asarray(starts, np.int64).reshape(-1), np.asarray(sizes, np.int64).reshape(-1),
                            out.ctypes.data)
    return out


def dynamic_update_slice(x, upd, starts) -> np.ndarray:
    """DynamicUpdateSlice (function.go:1596-1621), starts clamped to [0, dim - update dim]."""
    x = np.ascontiguousarray(x)
    upd = np.ascontiguousarray(upd, x.dtype)
    out = np.empty_like(x)
    lib().orc_dynamic_update_slice(x.ctypes.data, x.itemsize, x.ndim, np.asarray(x.shape, np.int64), upd.ctypes.data,
                                   np.asarray(upd.shape, np.int64), np.asarray(starts, np.int64).reshape(-1),
                                   out.ctypes.data)
    return out


SCATTER_SUM, SCATTER_MAX, SCATTER_MIN = 0, 1, 2


def scatter(mode, operand, indices, updates, index_vector_axis, update_window_axes, inserted_window_axes,
            scatter_axes_to_operand_axes) -> np.ndarray:
    """ScatterSum / Max / Min (gather.go:441-640) in fp64, XLA semantics; out-of-range windows skipped."""
    op = np.ascontiguousarray(np.asarray(operand, np.float64))
    ix = np.ascontiguousarray(np.asarray(indices, np.int64))
    up = np.ascontiguousarray(np.asarray(updates, np.float64))
    out = np.empty_like(op)
    keep = []

    def arr(a):
        a = np.ascontiguousarray(np.asarray(list(a), np.int32))
        keep.append(a)
        return a.ctypes.data_as(ctypes.c_void_p) if a.size else None, len(a)

    u, nu = arr(update_window_axes)
    i, ni = arr(inserted_window_axes)
    s, ns = arr(scatter_axes_to_operand_axes)
    lib().orc_scatter(int(mode), op.reshape(-1), op.ndim, np.asarray(op.shape, np.int64), ix.reshape(-1), ix.ndim,
                      np.asarray(ix.shape if ix.ndim else (1,), np.int64), int(index_vector_axis), up.reshape(-1),
                      up.ndim, np.asarray(up.shape if up.ndim else (1,), np.int64), u, nu, i, ni, s, ns, out.reshape(-1))
    return out


ACT_NONE, ACT_GELU, ACT_RELU, ACT_SILU, ACT_TANH, ACT_GELU_EXACT = range(6)


def activation(x, act: int) -> np.ndarray:
    """FusedDense / FusedGelu activations in fp64 (function.go:2288-2408, 2620-2664)."""
    x = np.ascontiguousarray(np.asarray(x, np.float64))
    y = np.empty_like(x)
    lib().orc_activation(x.reshape(-1), y.reshape(-1), x.size, int(act))
    return y


def gelu(x, exact: bool) -> np.ndarray:
    """FusedGelu (function.go:2288-2408)."""
    return activation(x, ACT_GELU_EXACT if exact else ACT_GELU)


def round_16(x, dtype: str) -> np.ndarray:
    """fp32 -> bf16 / f16 (round to nearest even) -> fp32."""
    x = np.asarray(x, np.float32)
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(np.float32)
    bits = f32_to_bf16_bits(x).astype(np.uint32) << 16
    return bits.view(np.float32).reshape(x.shape)


def _rounded_16_pair(t64, dtype: str, rel: float):
    """The 16-bit roundings of t * (1 - rel) and t * (1 + rel): any value within
    relative distance `rel` of t rounds (to nearest even) to one of the two, and
    they differ only where t lies that close to a rounding midpoint."""
    lo = round_16((t64 * (1.0 - rel)).astype(np.float32), dtype)
    hi = round_16((t64 * (1.0 + rel)).astype(np.float32), dtype)
    return lo, hi


def gelu_chain_16(x, exact: bool, dtype: str = "bf16", rel: float = 1e-5):
    """FusedGelu as the reference composes it (function.go:2343-2402 tanh form,
    :2299-2341 exact form), with x, every op result and every scalar constant held
    in the 16-bit dtype: each op is evaluated in fp32 on 16-bit operands and its
    result rounded to nearest even, in the reference's order.  The scalar constants
    are float32 values converted to the dtype (makeScalarConst, function.go:210-231).
    The transcendental (tanh / erf) step is the exact value rounded to the dtype,
    evaluated by any routine within relative error `rel`: near a rounding midpoint
    either side is allowed, so two results come back (lo, hi: equal everywhere
    else).  Returns float32 arrays."""
    x = round_16(x, dtype)
    np_err = np.seterr(over="ignore", invalid="ignore")  # x^3 overflows for |x| >~ 2^42, as in the graph
    r = lambda a: round_16(a, dtype)  # noqa: E731
    c = lambda v: r(np.float32(v))    # noqa: E731
    half, one = c(0.5), c(1.0)
    if exact:
        xs = r(x * c(0.7071067811865475))
        from scipy.special import erf
        tl, th = _rounded_16_pair(erf(xs.astype(np.float64)), dtype, rel)
    else:
        x3 = r(r(x * x) * x)
        inner = r(x + r(c(0.044715) * x3))
        scaled = r(c(0.7978845608) * inner)
        tl, th = _rounded_16_pair(np.tanh(scaled.astype(np.float64)), dtype, rel)
    hx = r(half * x)
    out = r(hx * r(one + tl)), r(hx * r(one + th))
    np.seterr(**np_err)
    return out


def dense(x, w, bias=None, act: int = ACT_NONE) -> np.ndarray:
    """FusedDense (function.go:2567-2667): x's last axis contracted with w's first,
    plus bias broadcast over the trailing axes, then the activation."""
    x = _f32(x)
    y = dot_general(x, [x.ndim - 1], [], w, [0], [])
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return activation(y, act)


def qkv_projection(x, w, bq, bk, bv, query_dim: int, key_value_dim: int):
    """FusedAttentionQKVProjection (function.go:2976-3075): x . w sliced on the last
    axis into Q [0, q), K [q, q+kv), V [q+kv, q+2kv), each plus its bias."""
    x = _f32(x)
    y = dot_general(x, [x.ndim - 1], [], w, [0], [])
    q, kv = query_dim, key_value_dim
    outs = [y[..., :q], y[..., q:q + kv], y[..., q + kv:q + 2 * kv]]
    return tuple(o if b is None else o + np.asarray(b, np.float64) for o, b in zip(outs, (bq, bk, bv)))


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(x.reshape(-1), y.reshape(-1), x.size)
    return y


def block_tokens(P, b, toks, d_model, heads, head_dim, eps):
    """fp64 output of the decoder block (gather, RMSNorm, Q/K/V projections, causal
    attention, O projection + residual, RMSNorm, SwiGLU FFN + residual: the graph
    gomlx_hip.graphs.transformer_block builds) at tokens `toks` of batch row b.  K
    and V are computed for the tokens up to the last one asked for, then attention,
    the O projection and the FFN for the asked tokens only (token t sees keys
    0..t).  P: "ids" [B, S] int32, "embedding", "wq", "wk", "wv", "wo", "w_gate",
    "w_up", "w_down" (values widened to fp32), "g_attn", "g_ffn".  Returns
    (out [len(toks), d_model], flops of this evaluation)."""
    d, H, Dh = d_model, heads, head_dim
    last = max(toks) + 1
    x = gather_rows(P["embedding"], P["ids"][b, :last]).astype(np.float64)
    h = rmsnorm(x.astype(np.float32), P["g_attn"], eps)
    proj = lambda a, w: dot_general(np.asarray(a, np.float32), [a.ndim - 1], [], P[w], [0], [])  # noqa: E731
    hd = lambda t: np.ascontiguousarray(t.reshape(1, -1, H, Dh).transpose(0, 2, 1, 3), np.float32)  # noqa: E731
    k, v = hd(proj(h, "wk")), hd(proj(h, "wv"))
    q = hd(proj(h[toks], "wq"))
    a = np.concatenate([sdpa(q[:, :, i:i + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=Dh ** -0.5, causal=False)
                        for i, t in enumerate(toks)], axis=2)
    x2 = x[toks] + proj(a.transpose(0, 2, 1, 3).reshape(len(toks), d), "wo")
    h2 = rmsnorm(x2.astype(np.float32), P["g_ffn"], eps)
    gate, up = proj(h2, "w_gate"), proj(h2, "w_up")
    out = x2 + proj(gate / (1.0 + np.exp(-gate)) * up, "w_down")
    ff = P["w_up"].shape[1]
    n = len(toks)
    flops = 2 * 2 * last * d * d + n * (2 * 2 * d * d + 3 * 2 * d * ff) + sum(4 * H * Dh * (t + 1) for t in toks)
    return out, flops


def decode_step(P, rows, heads, kv_heads, head_dim, eps):
    """fp64 outputs of the decoding step gomlx_hip.graphs.decode_step builds, for
    the sequences `rows`: RMSNorm, Q / K / V projections, grouped-query attention of
    each sequence's query over its whole K / V cache (no mask), O projection +
    residual, RMSNorm, SwiGLU FFN + residual.  P: "x" [B, d], "w_qkv" ([Wq | Wk |
    Wv], [d, (H + 2 Hkv) Dh]), "k_cache" / "v_cache" [B, Hkv, S, Dh], "wo", "w_gate",
    "w_up", "w_down" (values widened to fp32), "g_attn", "g_ffn".  Returns
    (x' [n, d], k_new, v_new [n, Hkv*Dh])."""
    H, Hkv, Dh = heads, kv_heads, head_dim
    x = np.asarray(P["x"][rows], np.float64)
    n, d = x.shape
    h = rmsnorm(x.astype(np.float32), P["g_attn"], eps)
    proj = lambda a, w: dot_general(np.asarray(a, np.float32), [a.ndim - 1], [], P[w], [0], [])  # noqa: E731
    qkv = proj(h, "w_qkv")
    q = qkv[:, :H * Dh].reshape(n, H, 1, Dh)
    k_new, v_new = qkv[:, H * Dh:(H + Hkv) * Dh], qkv[:, (H + Hkv) * Dh:]
    kc = np.ascontiguousarray(P["k_cache"][rows], np.float32)  # [n, Hkv, S, Dh]: head h reads kv head h // (H / Hkv)
    vc = np.ascontiguousarray(P["v_cache"][rows], np.float32)
    a = sdpa(np.ascontiguousarray(q, np.float32), kc, vc, scale=Dh ** -0.5, causal=False)
    x2 = x + proj(a.reshape(n, H * Dh), "wo")
    h2 = rmsnorm(x2.astype(np.float32), P["g_ffn"], eps)
    gate, up = proj(h2, "w_gate"), proj(h2, "w_up")
    out = x2 + proj(gate / (1.0 + np.exp(-gate)) * up, "w_down")
    return out, k_new, v_new
