"""ExecuteNoAlloc (ghip_exec_execute_noalloc): the Execute variant that allocates
nothing, with the intermediates in the library's per-GPU scratch array and the
outputs in caller-made buffers.  Checked bit for bit against Execute on the same
executable, for two calls in a row (the second graph smaller), and for its
errors."""
import numpy as np
import pytest

from gomlx_hip import graphs, synth
from gomlx_hip.backend import AxesLayout, Backend, BackendError, dtypes, make_shape

pytestmark = pytest.mark.gpu

F32, BF16, I32 = dtypes.Float32, dtypes.BFloat16, dtypes.Int32


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def _block_case(be, cfg, seed):
    ex = graphs.transformer_block(be, cfg)
    bufs = []
    for i, (name, shape) in enumerate(cfg.param_shapes()):
        if name == "ids":
            host = synth.uniform_int(seed, (cfg.batch, cfg.seq), 0, cfg.vocab)
        elif name.startswith("g_"):
            host = synth.uniform_f32(seed + 50 + i, shape.dims, 0.5, 1.5)
        else:
            host = synth.round_bf16(synth.normal(seed + i, shape.dims, std=0.02))
        bufs.append(be.BufferFromFlatData(0, host, shape))
    return ex, bufs


def _scatter_case(be, V, D, n, seed):
    """Embedding-gradient ScatterSum plus a row softmax of the result: the scatter
    sorts its row ids in the arena, the softmax reads the scatter's output there."""
    b = be.Builder("scatter_noalloc")
    f = b.Main()
    t = f.Parameter("t", make_shape(F32, V, D))
    i = f.Parameter("i", make_shape(I32, n))
    u = f.Parameter("u", make_shape(F32, n, D))
    s = f.ScatterSum(t, i, u, 1, [1], [0], [0])
    f.Return([f.FusedSoftmax(s, 1), f.Add(s, s)])
    ex = b.Compile()
    host = [(synth.normal(seed, (V, D)), make_shape(F32, V, D)),
            (synth.uniform_int(seed + 1, (n,), 0, V), make_shape(I32, n)),
            (synth.normal(seed + 2, (n, D)), make_shape(F32, n, D))]
    return ex, [be.BufferFromFlatData(0, a, sh) for a, sh in host]


def _decode_case(be, B, H, Hkv, Sk, D, seed):
    """One decoding step of grouped-query attention: its key range splits over a
    workspace in the arena (the scratch array here)."""
    b = be.Builder("decode_noalloc")
    f = b.Main()
    q = f.Parameter("q", make_shape(BF16, B, H, 1, D))
    k = f.Parameter("k", make_shape(BF16, B, Hkv, Sk, D))
    v = f.Parameter("v", make_shape(BF16, B, Hkv, Sk, D))
    f.Return([f.FusedScaledDotProductAttention(q, k, v, None, H, Hkv, AxesLayout.BHSD, D ** -0.5, False)])
    ex = b.Compile()
    assert "key range split" in ex.Plan(), ex.Plan()
    host = [synth.normal(seed, (B, H, 1, D)), synth.normal(seed + 1, (B, Hkv, Sk, D)),
            synth.normal(seed + 2, (B, Hkv, Sk, D))]
    return ex, [be.BufferFromFlatData(0, a, make_shape(BF16, *a.shape)) for a in host]


def _dot_case(be, M, N, K, seed):
    """A few-tile DotGeneral with a long contraction plus a bias: the contraction
    splits over a workspace in the arena (the scratch array here)."""
    b = be.Builder("dot_split_noalloc")
    f = b.Main()
    x = f.Parameter("x", make_shape(BF16, M, K))
    w = f.Parameter("w", make_shape(BF16, K, N))
    c = f.Parameter("c", make_shape(BF16, N))
    d = f.DotGeneral(x, [1], [], w, [0], [])
    f.Return([f.Add(d, f.BroadcastInDim(c, make_shape(BF16, M, N), [1]))])
    ex = b.Compile()
    assert "contraction split" in ex.Plan(), ex.Plan()
    host = [synth.round_bf16(synth.normal(seed, (M, K), std=0.125)),
            synth.round_bf16(synth.normal(seed + 1, (K, N), std=0.125)), synth.round_bf16(synth.normal(seed + 2, (N,)))]
    return ex, [be.BufferFromFlatData(0, a, make_shape(BF16, *a.shape)) for a in host]


def _compare(be, ex, bufs):
    ref = ex.Execute(bufs, None, 0)
    outs = [be.NewSharedBuffer(0, s) for s in ex.Outputs()]
    ex.ExecuteNoAlloc(bufs, outs)
    for r, o in zip(ref, outs):
        assert be.BufferShape(r) == be.BufferShape(o)
        assert np.array_equal(be.BufferToFlatData(r), be.BufferToFlatData(o))
    return outs


def test_noalloc_matches_execute_two_calls_second_smaller(be):
    """A transformer block (intermediates in the scratch array), then a smaller one;
    then a scatter graph, then a smaller scatter graph, then two decoding attention
    steps, then two few-tile products with a split contraction: each bit-identical
    to Execute on the same executable and inputs."""
    big = graphs.TransformerBlockConfig(batch=2, seq=256, vocab=2000, d_model=512, heads=4, head_dim=128, ffn=2048)
    small = graphs.TransformerBlockConfig(batch=1, seq=128, vocab=1000, d_model=256, heads=2, head_dim=128, ffn=1024)
    for cfg, seed in ((big, 7100), (small, 7200)):
        ex, bufs = _block_case(be, cfg, seed)
        assert int(ex.Plan().splitlines()[0].split("arena ")[1].split()[0]) > 0
        _compare(be, ex, bufs)
    for (V, D, n), seed in (((4000, 512, 3000), 7300), ((500, 256, 700), 7400)):
        ex, bufs = _scatter_case(be, V, D, n, seed)
        _compare(be, ex, bufs)
    # decoding attention: the split key range's partial outputs in the arena
    for (B, H, Hkv, Sk, D), seed in (((4, 16, 4, 6000, 128), 7500), ((1, 8, 2, 1500, 64), 7600)):
        ex, bufs = _decode_case(be, B, H, Hkv, Sk, D, seed)
        _compare(be, ex, bufs)
    # few-tile products: the contraction split's fp32 partials in the arena
    for (M, N, K), seed in (((16, 4096, 4096), 7700), ((8, 2048, 2048), 7800)):
        ex, bufs = _dot_case(be, M, N, K, seed)
        _compare(be, ex, bufs)


def test_noalloc_errors(be):
    ex, bufs = _scatter_case(be, 64, 32, 40, 7500)
    outs = [be.NewSharedBuffer(0, s) for s in ex.Outputs()]
    with pytest.raises(BackendError, match="shape mismatch"):
        ex.ExecuteNoAlloc(bufs, [be.NewSharedBuffer(0, make_shape(F32, 3, 3)), outs[1]])
    with pytest.raises(BackendError, match="is input"):
        ex.ExecuteNoAlloc(bufs, [bufs[0], outs[1]])
    with pytest.raises(BackendError, match="expected 2 outputs"):
        ex.ExecuteNoAlloc(bufs, outs[:1])
    other = Backend("")
    try:
        with pytest.raises(BackendError, match="another backend"):
            ex.ExecuteNoAlloc(bufs, [other.NewSharedBuffer(0, ex.Outputs()[0]), outs[1]])
    finally:
        other.Finalize()
    # While runs sub-functions with arenas of their own: refused, Execute still works
    b = be.Builder("loop")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 4))
    cond = f.Closure()
    cx = cond.Parameter("c", make_shape(F32, 4))
    cond.Return([cond.LessThan(cond.ReduceSum(cx, 0), cond.Constant(np.float32(100)))])
    body = f.Closure()
    bx = body.Parameter("c", make_shape(F32, 4))
    body.Return([body.Add(bx, bx)])
    (y,) = f.While(cond, body, x)
    f.Return([y])
    wex = b.Compile()
    xb = be.BufferFromFlatData(0, np.ones(4, np.float32), make_shape(F32, 4))
    with pytest.raises(BackendError, match="Call / While / If"):
        wex.ExecuteNoAlloc([xb], [be.NewSharedBuffer(0, make_shape(F32, 4))])
    (r,) = wex.Execute([xb], None, 0)
    assert be.BufferToFlatData(r).tolist() == [32.0] * 4
