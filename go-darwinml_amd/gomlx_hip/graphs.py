"""The BASELINE workloads as GoMLX graphs, built through the backend API.

Each builder emits the ops a GoMLX graph program sends to a backend for that
workload (the same primitive / fused ops the reference backend receives), so
running them exercises the full Builder -> Compile -> Execute path.
"""
from __future__ import annotations

import numpy as np

from .backend import AxesLayout, Backend, dtypes, make_shape


def rms_norm(f, x, gamma, eps: float):
    """RMSNorm as the primitive chain GoMLX emits (no fused backend op exists):
    x * rsqrt(ReduceSum(x*x, -1) / n + eps) * gamma."""
    s = f.OpShape(x)
    dt, dims = s.dtype, s.dims
    n = dims[-1]
    rows = dims[:-1]
    ss = f.ReduceSum(f.Mul(x, x), len(dims) - 1)
    inv_n = f.Constant(np.array(1.0 / n, np.float32), dtype=dt)
    mean = f.Mul(ss, f.BroadcastInDim(inv_n, make_shape(dt, *rows), []))
    e = f.Constant(np.array(eps, np.float32), dtype=dt)
    r = f.Rsqrt(f.Add(mean, f.BroadcastInDim(e, make_shape(dt, *rows), [])))
    rb = f.BroadcastInDim(r, make_shape(dt, *dims), list(range(len(dims) - 1)))
    y = f.Mul(x, rb)
    if gamma is not None:
        y = f.Mul(y, f.BroadcastInDim(gamma, make_shape(dt, *dims), [len(dims) - 1]))
    return y


def layer_norm_chain(f, x, gamma, beta, eps: float):
    """LayerNorm over the last axis as primitives, in the reference's op order
    (function.go:2429-2562): mean = sum / n, d = x - mean, var = sum(d * d) / n,
    y = d * rsqrt(var + eps) [* gamma] [+ beta]."""
    s = f.OpShape(x)
    dt, dims = s.dtype, s.dims
    r = len(dims)
    rows = make_shape(dt, *dims[:-1])
    keep = list(range(r - 1))
    count = f.BroadcastInDim(f.Constant(np.array(dims[-1], np.float32), dtype=dt), rows, [])
    mean = f.Div(f.ReduceSum(x, r - 1), count)
    d = f.Sub(x, f.BroadcastInDim(mean, s, keep))
    var = f.Div(f.ReduceSum(f.Mul(d, d), r - 1), count)
    e = f.BroadcastInDim(f.Constant(np.array(eps, np.float32), dtype=dt), rows, [])
    y = f.Mul(d, f.BroadcastInDim(f.Rsqrt(f.Add(var, e)), s, keep))
    if gamma is not None:
        y = f.Mul(y, f.BroadcastInDim(gamma, s, [r - 1]))
    if beta is not None:
        y = f.Add(y, f.BroadcastInDim(beta, s, [r - 1]))
    return y


def softmax_chain(f, x):
    """Softmax over the last axis as the primitive chain (max, sub, exp, sum, div)."""
    s = f.OpShape(x)
    r = len(s.dims)
    m = f.ReduceMax(x, r - 1)
    e = f.Exp(f.Sub(x, f.BroadcastInDim(m, s, list(range(r - 1)))))
    z = f.ReduceSum(e, r - 1)
    return f.Div(e, f.BroadcastInDim(z, s, list(range(r - 1))))


def log_softmax_chain(f, x):
    """Log-softmax over the last axis as primitives: (x - max) - log(sum(exp(x - max)))."""
    s = f.OpShape(x)
    r = len(s.dims)
    keep = list(range(r - 1))
    d = f.Sub(x, f.BroadcastInDim(f.ReduceMax(x, r - 1), s, keep))
    z = f.ReduceSum(f.Exp(d), r - 1)
    return f.Sub(d, f.BroadcastInDim(f.Log(z), s, keep))


def dense(f, x, w):
    """x [..., din] @ w [din, dout] -> [..., dout] (DotGeneral, no batch axes)."""
    rx = len(f.OpShape(x).dims)
    return f.DotGeneral(x, [rx - 1], [], w, [0], [])


class TransformerBlockConfig:
    def __init__(self, batch=8, seq=1024, vocab=32000, d_model=2048, heads=16, head_dim=128,
                 ffn=8192, eps=1e-6, dtype=dtypes.BFloat16):
        self.batch, self.seq, self.vocab = batch, seq, vocab
        self.d_model, self.heads, self.head_dim, self.ffn = d_model, heads, head_dim, ffn
        self.eps, self.dtype = eps, dtype

    def flops(self) -> int:
        """Algorithmic flops of the block forward (GEMMs + full attention matrices)."""
        T, d, f = self.batch * self.seq, self.d_model, self.ffn
        S, H, Dh = self.seq, self.heads, self.head_dim
        proj = 2 * T * d * d * 4          # Q, K, V, O
        attn = 2 * 2 * self.batch * H * S * S * Dh
        ffn = 2 * T * d * f * 3           # gate, up, down
        return proj + attn + ffn

    def param_shapes(self):
        dt, d, f = self.dtype, self.d_model, self.ffn
        return [
            ("ids", make_shape(dtypes.Int32, self.batch, self.seq)),
            ("embedding", make_shape(dt, self.vocab, d)),
            ("g_attn", make_shape(dt, d)),
            ("wq", make_shape(dt, d, d)), ("wk", make_shape(dt, d, d)),
            ("wv", make_shape(dt, d, d)), ("wo", make_shape(dt, d, d)),
            ("g_ffn", make_shape(dt, d)),
            ("w_gate", make_shape(dt, d, f)), ("w_up", make_shape(dt, d, f)),
            ("w_down", make_shape(dt, f, d)),
        ]


def transformer_block(backend: Backend, cfg: TransformerBlockConfig):
    """Decoder-only block forward:
    embedding gather -> RMSNorm -> 16-head causal attention -> residual ->
    RMSNorm -> SwiGLU FFN -> residual.  Returns the compiled Executable."""
    b = backend.Builder("transformer_block")
    f = b.Main()
    P = {name: f.Parameter(name, shape) for name, shape in cfg.param_shapes()}
    B, S, d, H, Dh = cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.head_dim
    ids = f.Reshape(P["ids"], B, S, 1)
    x = f.Gather(P["embedding"], ids, 2, [2], [0], [0], [1, d], False)      # [B, S, d]
    h = rms_norm(f, x, P["g_attn"], cfg.eps)
    q = f.Reshape(dense(f, h, P["wq"]), B, S, H, Dh)
    k = f.Reshape(dense(f, h, P["wk"]), B, S, H, Dh)
    v = f.Reshape(dense(f, h, P["wv"]), B, S, H, Dh)
    a = f.FusedScaledDotProductAttention(q, k, v, None, H, H, AxesLayout.BSHD, Dh ** -0.5, True)
    x2 = f.Add(x, dense(f, f.Reshape(a, B, S, d), P["wo"]))
    h2 = rms_norm(f, x2, P["g_ffn"], cfg.eps)
    gate = dense(f, h2, P["w_gate"])
    up = dense(f, h2, P["w_up"])
    act = f.Mul(f.Mul(gate, f.Logistic(gate)), up)                          # SiLU(gate) * up
    out = f.Add(x2, dense(f, act, P["w_down"]))
    f.Return([out])
    return b.Compile()


class DecodeStepConfig:
    """One decoding step of a decoder block for `batch` sequences, each with a KV
    cache of `cache` positions (grouped-query attention, kv_heads <= heads)."""

    def __init__(self, batch=16, cache=4096, d_model=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336,
                 eps=1e-6, dtype=dtypes.BFloat16):
        self.batch, self.cache, self.d_model = batch, cache, d_model
        self.heads, self.kv_heads, self.head_dim, self.ffn = heads, kv_heads, head_dim, ffn
        self.eps, self.dtype = eps, dtype

    def param_shapes(self):
        dt, d, f = self.dtype, self.d_model, self.ffn
        B, S, H, Hkv, Dh = self.batch, self.cache, self.heads, self.kv_heads, self.head_dim
        return [
            ("x", make_shape(dt, B, d)),
            ("g_attn", make_shape(dt, d)),
            ("w_qkv", make_shape(dt, d, (H + 2 * Hkv) * Dh)),  # [Wq | Wk | Wv]
            ("k_cache", make_shape(dt, B, Hkv, S, Dh)), ("v_cache", make_shape(dt, B, Hkv, S, Dh)),
            ("wo", make_shape(dt, H * Dh, d)),
            ("g_ffn", make_shape(dt, d)),
            ("w_gate", make_shape(dt, d, f)), ("w_up", make_shape(dt, d, f)),
            ("w_down", make_shape(dt, f, d)),
        ]

    def bytes(self) -> int:
        """HBM bytes a step must move at least: every parameter read once (weights,
        caches, x, gammas) and the outputs (x' and the Q / K / V projections) written;
        2 bytes an element."""
        n = sum(int(np.prod(s.dims)) for _, s in self.param_shapes())
        out = self.batch * (self.d_model + (self.heads + 2 * self.kv_heads) * self.head_dim)
        return 2 * (n + out)


def decode_step(backend: Backend, cfg: DecodeStepConfig):
    """One decoding step: x [B, d] (the sequences' current hidden states) ->
    RMSNorm -> Q, K, V projections (one product with the [Wq | Wk | Wv] weight, Q a
    column view of it, as FusedAttentionQKVProjection lowers) -> grouped-query
    attention of the B queries over their K / V caches [B, Hkv, S, Dh] (BHSD; the
    caller has already written the current position into them) -> O projection +
    residual -> RMSNorm -> SwiGLU FFN + residual.  Returns the compiled Executable,
    whose outputs are (x' [B, d], qkv [B, (H + 2 Hkv) Dh]): the current position's
    projections, whose K columns [H Dh, (H + Hkv) Dh) and V columns [(H + Hkv) Dh,
    (H + 2 Hkv) Dh) the caller writes into the caches for the next step.  Every
    product has B rows (decoding), so the GEMMs are few-tile products."""
    b = backend.Builder("decode_step")
    f = b.Main()
    P = {name: f.Parameter(name, shape) for name, shape in cfg.param_shapes()}
    B, d, H, Hkv, Dh = cfg.batch, cfg.d_model, cfg.heads, cfg.kv_heads, cfg.head_dim
    x = P["x"]
    h = rms_norm(f, x, P["g_attn"], cfg.eps)
    qkv = dense(f, h, P["w_qkv"])
    q = f.Reshape(f.Slice(qkv, [0, 0], [B, H * Dh]), B, H, 1, Dh)
    a = f.FusedScaledDotProductAttention(q, P["k_cache"], P["v_cache"], None, H, Hkv, AxesLayout.BHSD,
                                         Dh ** -0.5, False)
    x2 = f.Add(x, dense(f, f.Reshape(a, B, H * Dh), P["wo"]))
    h2 = rms_norm(f, x2, P["g_ffn"], cfg.eps)
    gate = dense(f, h2, P["w_gate"])
    up = dense(f, h2, P["w_up"])
    act = f.Mul(f.Mul(gate, f.Logistic(gate)), up)
    out = f.Add(x2, dense(f, act, P["w_down"]))
    f.Return([out, qkv])
    return b.Compile()
