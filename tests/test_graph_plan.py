"""Graph API host logic on the plan-only backend (no GPU): shape inference,
error paths the reference's Go code returns, and the lowering decisions."""
import numpy as np
import pytest

from gomlx_hip.backend import AxesLayout, Backend, BackendError, dtypes, make_shape
from gomlx_hip import graphs


@pytest.fixture(scope="module")
def be():
    b = Backend("plan")
    yield b
    b.Finalize()


F32 = dtypes.Float32
BF16 = dtypes.BFloat16


def test_backend_identity(be):
    assert be.Name() == "hip"
    assert "plan-only" in be.Description()
    assert be.NumDevices() == 0
    with pytest.raises(BackendError):
        Backend("mpsgraph:whatever")


def test_shape_inference(be):
    f = be.Builder("shapes").Main()
    x = f.Parameter("x", make_shape(F32, 2, 3, 4))
    assert f.OpShape(f.Transpose(x, 2, 0, 1)).dims == (4, 2, 3)
    assert f.OpShape(f.ReduceSum(x, 1)).dims == (2, 4)
    assert f.OpShape(f.ReduceMax(x)).dims == ()
    assert f.OpShape(f.ArgMinMax(x, 2, dtypes.Int32, False)) == make_shape(dtypes.Int32, 2, 3)
    assert f.OpShape(f.GreaterThan(x, x)).dtype == dtypes.Bool
    y = f.Parameter("y", make_shape(F32, 5, 4, 7))
    # DotGeneral output order [batch..., lhs free..., rhs free...] (dotgeneral.go:15-53)
    assert f.OpShape(f.DotGeneral(x, [2], [], y, [1], [])).dims == (2, 3, 5, 7)
    z = f.Parameter("z", make_shape(F32, 2, 4, 6))
    assert f.OpShape(f.DotGeneral(x, [2], [0], z, [1], [0])).dims == (2, 3, 6)
    assert f.OpShape(f.Slice(x, [0, 1, 0], [2, 3, 4], [1, 1, 2])).dims == (2, 2, 2)
    assert f.OpShape(f.Concatenate(1, x, x)).dims == (2, 6, 4)
    emb = f.Parameter("emb", make_shape(BF16, 100, 16))
    ids = f.Parameter("ids", make_shape(dtypes.Int32, 3, 5, 1))
    assert f.OpShape(f.Gather(emb, ids, 2, [2], [0], [0], [1, 16])).dims == (3, 5, 16)
    q = f.Parameter("q", make_shape(BF16, 2, 4, 8, 16))
    kv = f.Parameter("kv", make_shape(BF16, 2, 2, 8, 16))
    o = f.FusedScaledDotProductAttention(q, kv, kv, None, 4, 2, AxesLayout.BHSD, 0.25, True)
    assert f.OpShape(o).dims == (2, 4, 8, 16)


def test_build_errors(be):
    f = be.Builder("errors").Main()
    x = f.Parameter("x", make_shape(F32, 2, 3))
    i = f.Parameter("i", make_shape(dtypes.Int32, 2, 3))
    with pytest.raises(BackendError, match="dtype mismatch"):
        f.Add(x, i)
    with pytest.raises(BackendError):
        f.Reshape(x, 7)
    with pytest.raises(BackendError):
        f.DotGeneral(x, [1], [], x, [1], [0])
    q = f.Parameter("q", make_shape(F32, 2, 3, 4))
    with pytest.raises(BackendError, match="rank 4"):  # function.go:2695-2697
        f.FusedScaledDotProductAttention(q, q, q, None, 1, 1, AxesLayout.BHSD, 1.0, False)
    with pytest.raises(BackendError, match="divisible"):
        q4 = f.Parameter("q4", make_shape(F32, 1, 3, 2, 4))
        f.FusedScaledDotProductAttention(q4, q4, q4, None, 3, 2, AxesLayout.BHSD, 1.0, False)
    with pytest.raises(BackendError, match="out of range"):  # function.go:2420-2424
        f.FusedLayerNorm(x, [5], 1e-5)


def test_compile_state_errors(be):
    b = be.Builder("state")
    with pytest.raises(BackendError, match="no main"):      # builder.go:76-78
        b.Compile()
    b = be.Builder("state2")
    f = b.Main()
    f.Parameter("x", make_shape(F32, 2))
    with pytest.raises(BackendError, match="Return"):       # builder.go:79-81
        b.Compile()
    x = f.Parameter("y", make_shape(F32, 2))
    f.Return([f.Neg(x)])
    b.Compile()
    with pytest.raises(BackendError, match="already compiled"):  # builder.go:73-75
        b.Compile()


def plan_of(be, build):
    b = be.Builder("p")
    f = b.Main()
    outs = build(f)
    f.Return(outs)
    return b.Compile().Plan()


def test_rmsnorm_chain_is_fused(be):
    def build(f):
        x = f.Parameter("x", make_shape(BF16, 64, 256))
        g = f.Parameter("g", make_shape(BF16, 256))
        return [graphs.rms_norm(f, x, g, 1e-6)]
    p = plan_of(be, build)
    assert "rmsnorm_rows bfloat16 rows=64 n=256 +gamma" in p
    assert "reduce" not in p and "fused_elementwise" not in p


@pytest.mark.parametrize("gb", ["both", "gamma", "beta", "none"])
def test_layernorm_chain_is_fused(be, gb):
    """The reference's LayerNorm composition (function.go:2429-2562) sent as
    primitives becomes one layernorm_rows launch, with or without gamma / beta."""
    def build(f):
        x = f.Parameter("x", make_shape(BF16, 64, 512))
        g = f.Parameter("g", make_shape(BF16, 512)) if gb in ("both", "gamma") else None
        b = f.Parameter("b", make_shape(BF16, 512)) if gb in ("both", "beta") else None
        return [graphs.layer_norm_chain(f, x, g, b, 1e-5)]
    p = plan_of(be, build)
    assert p.count("layernorm_rows bfloat16 rows=64 n=512") == 1, p
    assert ("+gamma" in p) == (gb in ("both", "gamma")) and ("+beta" in p) == (gb in ("both", "beta"))
    assert "(fused primitive LayerNorm chain)" in p
    assert "reduce" not in p and "fused_elementwise" not in p


def _reduce_chains(f, dt=F32):
    """Elementwise -> Reduce -> elementwise chains none of the row patterns match."""
    x = f.Parameter("x", make_shape(dt, 96, 1000))
    n = f.BroadcastInDim(f.Constant(np.array(1000, np.float32), dtype=dt), make_shape(dt, 96), [])
    rms = f.Sqrt(f.Div(f.ReduceSum(f.Mul(x, x), 1), n))                 # producer + consumer, wave form
    z = f.Parameter("z", make_shape(dt, 6, 40, 5))
    two = f.BroadcastInDim(f.Constant(np.array(2, np.float32), dtype=dt), make_shape(dt, 40), [])
    amax = f.Mul(f.ReduceMax(f.Abs(z), 0, 2), two)                      # thread form, two reduced axes
    t = f.ReduceSum(f.Exp(f.Transpose(x, 1, 0)), 0)                       # strided producer, no consumer
    return [rms, amax, t]


def test_reduce_chains_fuse_into_one_kernel(be, monkeypatch):
    """Reduce absorbs its elementwise producer and consumer: one launch per chain
    (the unfused plan runs producer, reduce and consumer as three)."""
    p = plan_of(be, _reduce_chains)
    assert p.count("fused_reduce_sum (float32)[96 1000] -> (float32)[96] (producer fused) (consumer fused)") == 1, p
    assert p.count("fused_reduce_max (float32)[6 40 5] -> (float32)[40] (producer fused) (consumer fused)") == 1, p
    assert p.count("fused_reduce_sum (float32)[1000 96] -> (float32)[96] (producer fused)") == 1, p
    assert "fused_elementwise" not in p and "reduce_sum (" not in p.replace("fused_reduce_sum", "")
    monkeypatch.setenv("GHIP_REDUCE_FUSION", "0")
    u = plan_of(be, _reduce_chains)
    assert "fused_reduce" not in u and u.count("fused_elementwise") == 5, u


def test_reduce_fusion_leaves_shared_and_output_values(be):
    """A producer that is also a graph output, or read by a second user, stays
    materialised; the Reduce then reads it."""
    def build(f):
        x = f.Parameter("x", make_shape(F32, 64, 128))
        sq = f.Mul(x, x)
        return [f.ReduceSum(sq, 1), sq]
    p = plan_of(be, build)
    assert "fused_reduce" not in p and p.count("fused_elementwise") == 1 and "reduce_sum" in p
    def build2(f):
        x = f.Parameter("x", make_shape(dtypes.Int32, 64, 50))
        return [f.ReduceSum(f.Mul(x, x), 1), f.ReduceMin(f.Neg(x))]
    p = plan_of(be, build2)
    assert "fused_reduce_sum (int32)[64 50] -> (int32)[64] (producer fused)" in p
    assert "fused_reduce_min (int32)[64 50] -> (int32)[] (producer fused)" in p


def test_softmax_chain_and_fused_softmax(be):
    def build(f):
        x = f.Parameter("x", make_shape(F32, 4096, 1024))
        return [graphs.softmax_chain(f, x), f.FusedSoftmax(x, 1)]
    p = plan_of(be, build)
    assert p.count("softmax_rows float32 rows=4096 n=1024") == 2
    assert "reduce" not in p


def test_middle_axis_softmax_and_layernorm_use_column_kernels(be):
    """FusedSoftmax / FusedLayerNorm over an axis before the last run the column
    kernels on x as it lies in memory: one step each, no transposing copy of x or
    of the result."""
    def build(f):
        x = f.Parameter("x", make_shape(F32, 8, 300, 64))
        g = f.Parameter("g", make_shape(F32, 300))
        b = f.Parameter("b", make_shape(F32, 1, 300, 1))
        return [f.FusedSoftmax(x, 1), f.FusedLayerNorm(x, [1], 1e-5, g, b), f.FusedSoftmax(x, 0)]
    p = plan_of(be, build)
    assert "softmax_cols float32 outer=8 n=300 inner=64" in p, p
    assert "layernorm_cols float32 outer=8 n=300 inner=64 +gamma +beta" in p, p
    assert "softmax_cols float32 outer=1 n=8 inner=19200" in p, p
    assert "strided_copy" not in p, p


@pytest.mark.parametrize("dt", [F32, BF16, dtypes.Float16])
def test_log_softmax_chain_is_fused(be, dt):
    def build(f):
        x = f.Parameter("x", make_shape(dt, 4096, 1024))
        return [graphs.log_softmax_chain(f, x)]
    p = plan_of(be, build)
    assert p.count("log_softmax_rows") == 1, p
    assert "(fused primitive log-softmax chain)" in p
    assert "reduce" not in p and "fused_elementwise" not in p


def test_float16_chains_fuse_and_float64_chains_stay_unfused(be):
    """The row kernels take f32 / bf16 / f16; an f64 chain (a dtype the reference
    does not declare) must still compile, as plain reduce + elementwise kernels."""
    def build(dt):
        def b(f):
            x = f.Parameter("x", make_shape(dt, 64, 256))
            g = f.Parameter("g", make_shape(dt, 256))
            return [graphs.softmax_chain(f, x), graphs.rms_norm(f, x, g, 1e-6), graphs.log_softmax_chain(f, x)]
        return b
    p = plan_of(be, build(dtypes.Float16))
    assert "softmax_rows float16" in p and "rmsnorm_rows float16" in p and "log_softmax_rows float16" in p
    p = plan_of(be, build(dtypes.Float64))
    assert "_rows" not in p and "reduce" in p, p
    with pytest.raises(BackendError, match="row kernels take"):
        plan_of(be, lambda f: [f.FusedSoftmax(f.Parameter("x", make_shape(dtypes.Float64, 4, 8)), 1)])


def test_dot_general_folds_transposes(be):
    def build(f):
        a = f.Parameter("a", make_shape(BF16, 8, 2048, 4096))
        b = f.Parameter("b", make_shape(BF16, 8, 4096, 4096))
        bt = f.Transpose(b, 0, 2, 1)                    # [8, N, K] view of the same data
        return [f.DotGeneral(a, [2], [0], b, [1], [0]), f.DotGeneral(a, [2], [0], bt, [2], [0])]
    p = plan_of(be, build)
    assert p.count("strides folded") == 2 and "strided_copy" not in p
    assert "arena 0 bytes" in p  # both products written straight into the outputs


def test_elementwise_chain_is_one_kernel(be):
    def build(f):
        x = f.Parameter("x", make_shape(F32, 128, 64))
        w = f.Parameter("w", make_shape(F32, 64))
        c = f.Constant(np.array(0.5, np.float32))
        y = f.Logistic(f.Add(f.Mul(x, f.BroadcastInDim(w, make_shape(F32, 128, 64), [1])),
                             f.BroadcastInDim(c, make_shape(F32, 128, 64), [])))
        return [y]
    p = plan_of(be, build)
    assert p.count("fused_elementwise") == 1 and "ops=3 inputs=2" in p


def test_transformer_block_plan(be, monkeypatch):
    cfg = graphs.TransformerBlockConfig(batch=2, seq=64, vocab=100, d_model=128, heads=2, head_dim=64, ffn=256)
    e = graphs.transformer_block(be, cfg)
    p = e.Plan()
    assert p.count("rmsnorm_rows") == 2
    # Q, K, V are one grouped launch (three products sharing the normed x),
    # attention (head dim 64) is one fused kernel; the residual adds and
    # SiLU(gate) * up run as GEMM epilogues (gate and up in one kernel).
    assert p.count("gemm_grouped bfloat16 G=3") == 1 and "gemm_batched bfloat16" not in p
    assert p.count("sdpa_fwd bfloat16") == 1 and "causal=1 mask=none (fused attention)" in p
    assert p.count("gemm_batched+epilogue") == 3 and p.count("dots=2") == 1
    assert "fused_elementwise" not in p
    # head dim 96: the fused kernel (padded to 128)
    c96 = graphs.TransformerBlockConfig(batch=2, seq=64, vocab=100, d_model=192, heads=2, head_dim=96, ffn=256)
    p96 = graphs.transformer_block(be, c96).Plan()
    assert "sdpa_fwd bfloat16" in p96 and "D=96 causal=1 mask=none (fused attention)" in p96
    assert "scale_mask_softmax_rows" not in p96 and p96.count("gemm_grouped bfloat16 G=3") == 1
    # head dim 100 (not a multiple of 8) has no fused kernel: GEMM, scale + causal
    # softmax, GEMM
    c100 = graphs.TransformerBlockConfig(batch=2, seq=64, vocab=100, d_model=200, heads=2, head_dim=100, ffn=256)
    p100 = graphs.transformer_block(be, c100).Plan()
    assert "sdpa_fwd" not in p100 and "scale_mask_softmax_rows" in p100 and "causal=1" in p100
    assert p100.count("gemm_batched bfloat16") == 2 and p100.count("gemm_grouped bfloat16 G=3") == 1
    monkeypatch.setenv("GHIP_EPILOGUE_FUSION", "0")
    u = graphs.transformer_block(be, cfg).Plan()
    assert u.count("gemm_batched bfloat16") == 4 and "gemm_batched+epilogue" not in u
    assert u.count("gemm_grouped bfloat16 G=3") == 1
    monkeypatch.setenv("GHIP_DOT_GROUPING", "0")
    g0 = graphs.transformer_block(be, cfg).Plan()
    assert g0.count("gemm_batched bfloat16") == 7 and "gemm_grouped" not in g0
    assert u.count("fused_elementwise") == 3
    assert "gather_rows" in p
    assert e.Outputs()[0].dims == (2, 64, 128)
    assert [s.dims for s in e.Inputs()][:2] == [(2, 64), (100, 128)]


def test_plan_backend_cannot_execute(be):
    b = be.Builder("noexec")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 4))
    f.Return([f.Exp(x)])
    e = b.Compile()
    with pytest.raises(BackendError):
        be.BufferFromFlatData(0, np.zeros(4, np.float32), make_shape(F32, 4))


def _plan(be, build, shapes):
    b = be.Builder("p")
    f = b.Main()
    ps = [f.Parameter(f"p{i}", s) for i, s in enumerate(shapes)]
    f.Return(build(f, *ps))
    return b.Compile().Plan()


def test_reshape_of_strided_views_is_zero_copy(be):
    # Splitting the last axis of a column slice: a view (no copy) feeding SDPA.
    def build(f, x, w):
        q, k, v = f.FusedAttentionQKVProjection(x, w, None, None, None, 512, 256)
        heads = lambda t, h: f.Reshape(t, 2, 64, h, 128)
        return [f.FusedScaledDotProductAttention(heads(q, 4), heads(k, 2), heads(v, 2), None, 4, 2,
                                                 AxesLayout.BSHD, 0.125, True)]
    plan = _plan(be, build, [make_shape(BF16, 2, 64, 256), make_shape(BF16, 256, 1024)])
    assert "strided_copy" not in plan and "materialise" not in plan, plan
    assert plan.count("gemm_batched") == 1 and "N=1024" in plan and "fused attention" in plan, plan
    # Merging axes that a transpose separated cannot be a view: one copy.
    def merged(f, x):
        t = f.Reshape(f.Transpose(x, 1, 0), 12)
        return [f.Add(t, t)]
    plan = _plan(be, merged, [make_shape(F32, 3, 4)])
    assert plan.count("strided_copy") == 1, plan
    # Reshape of a reversed / broadcast view that keeps the stride runs stays a view.
    plan = _plan(be, lambda f, x: [f.ReduceSum(f.Reshape(f.Reverse(x, 0), 2, 3, 4), 0)], [make_shape(F32, 6, 4)])
    assert "strided_copy" not in plan, plan


def test_fused_dense_and_qkv_plans(be):
    plan = _plan(be, lambda f, x, w, b: [f.FusedDense(x, w, b, 1)],
                 [make_shape(BF16, 4, 128, 256), make_shape(BF16, 256, 512), make_shape(BF16, 512)])
    assert plan.count("gemm_batched+epilogue") == 1 and "fused_elementwise" not in plan, plan
    plan = _plan(be, lambda f, x, w, bq, bk, bv: list(f.FusedAttentionQKVProjection(x, w, bq, bk, bv, 256, 128)),
                 [make_shape(BF16, 4, 128, 256), make_shape(BF16, 256, 512), make_shape(BF16, 256),
                  make_shape(BF16, 128), make_shape(BF16, 128)])
    assert plan.count("gemm_batched+epilogue") == 3 and "fused_elementwise" not in plan, plan
    f = be.Builder("e").Main()
    x = f.Parameter("x", make_shape(F32, 2, 3))
    with pytest.raises(BackendError, match="FusedGelu: float input required"):
        f.FusedGelu(f.Parameter("i", make_shape(dtypes.Int32, 3)), False)


def test_epilogue_core_follows_layout_and_epilogue_weight(be):
    """Large products with A K-contiguous and B N-contiguous (x . W, the DotGeneral
    config's layout) run the 4-wave 128 x 128-wave core for a light epilogue (a
    residual add) or two products (SwiGLU) and the 8-wave 32-deep core for a
    VALU-heavy epilogue of one product (tanh-GELU: a transcendental in a 10-op
    chain); B K-contiguous layouts the 8-wave 64-deep core; both operands
    MN-contiguous the 4-wave 32-deep core for a light epilogue and the 8-wave 64-deep
    core for a VALU-heavy one."""
    x = make_shape(BF16, 8, 1024, 2048)
    gelu = _plan(be, lambda f, xx, w, b: [f.FusedDense(xx, w, b, 1)], [x, make_shape(BF16, 2048, 8192), make_shape(BF16, 8192)])
    assert "gemm_batched+epilogue" in gelu and "waves=8" in gelu, gelu
    resid = _plan(be, lambda f, xx, w, r: [f.Add(f.DotGeneral(xx, [2], [], w, [0], []), r)],
                  [x, make_shape(BF16, 2048, 2048), x])
    assert "gemm_batched+epilogue" in resid and "waves=4" in resid, resid
    # W stored [N, K] (x . W^T): B K-contiguous
    resid_t = _plan(be, lambda f, xx, w, r: [f.Add(f.DotGeneral(xx, [2], [], w, [1], []), r)],
                    [x, make_shape(BF16, 2048, 2048), x])
    assert "gemm_batched+epilogue" in resid_t and "waves=8" in resid_t, resid_t
    gelu_t = _plan(be, lambda f, xx, w: [f.FusedGelu(f.DotGeneral(xx, [2], [], w, [1], []), False)],
                   [x, make_shape(BF16, 8192, 2048)])
    assert "gemm_batched+epilogue" in gelu_t and "waves=8" in gelu_t and "core=8w-k64" in gelu_t, gelu_t
    assert "core=8w-km32" in gelu and "core=4w-km32" in resid and "core=8w-k64" in resid_t
    # x^T . dY (both MN-contiguous): light epilogue on 4 waves, heavy on 8
    xt = make_shape(BF16, 2048, 8192)
    resid_mm = _plan(be, lambda f, xx, w, r: [f.Add(f.DotGeneral(xx, [0], [], w, [0], []), r)],
                     [xt, make_shape(BF16, 2048, 2048), make_shape(BF16, 8192, 2048)])
    assert "core=4w-mn32" in resid_mm and "waves=4" in resid_mm, resid_mm
    gelu_mm = _plan(be, lambda f, xx, w: [f.FusedGelu(f.DotGeneral(xx, [0], [], w, [0], []), False)],
                    [xt, make_shape(BF16, 2048, 2048)])
    assert "core=8w-k64" in gelu_mm, gelu_mm

    # SwiGLU: two products sharing x in one kernel, on the 4-wave core for x . W
    def swiglu(f, xx, wg, wu):
        g = f.DotGeneral(xx, [2], [], wg, [0], [])
        return [f.Mul(f.Mul(g, f.Logistic(g)), f.DotGeneral(xx, [2], [], wu, [0], []))]
    w = make_shape(BF16, 2048, 8192)
    sw = _plan(be, swiglu, [x, w, w])
    assert "dots=2" in sw and "core=4w-km32" in sw and "tile=256x256" in sw, sw
    small = _plan(be, swiglu, [make_shape(BF16, 1, 1024, 2048), w, w])
    assert "dots=2" in small and "core=4w-km32" in small, small  # 4 x 64 tiles
    tiny = _plan(be, swiglu, [make_shape(BF16, 1, 256, 512), make_shape(BF16, 512, 1024), make_shape(BF16, 512, 1024)])
    assert "dots=2" in tiny and "core=8w-k64" in tiny, tiny  # 8 tiles
    # The same 8 tiles with K = 2048: each product splits its contraction (8 ranges
    # of 256 steps), so the products stay unfused and the gate runs as its own
    # elementwise kernel.
    split = _plan(be, swiglu, [make_shape(BF16, 1, 256, 2048), make_shape(BF16, 2048, 1024),
                               make_shape(BF16, 2048, 1024)])
    assert split.count("contraction split in 8") == 2 and "epilogue" not in split, split
    assert "fused_elementwise" in split, split


def test_dynamic_slice_and_scatter_shapes_and_errors(be):
    f = be.Builder("ds").Main()
    x = f.Parameter("x", make_shape(F32, 5, 6))
    i0 = f.Parameter("i0", make_shape(dtypes.Int32))
    i1 = f.Parameter("i1", make_shape(dtypes.Int64))
    assert f.OpShape(f.DynamicSlice(x, [i0, i1], [2, 3])).dims == (2, 3)
    u = f.Parameter("u", make_shape(F32, 2, 6))
    assert f.OpShape(f.DynamicUpdateSlice(x, u, [i0, i1])).dims == (5, 6)
    with pytest.raises(BackendError, match="3 start indices for a rank-2"):
        f.DynamicSlice(x, [i0, i1, i0], [1, 1])
    with pytest.raises(BackendError, match="slice size 7 out of"):
        f.DynamicSlice(x, [i0, i1], [2, 7])
    with pytest.raises(BackendError, match="integer scalar"):
        f.DynamicSlice(x, [i0, f.Parameter("v", make_shape(dtypes.Int32, 2))], [2, 2])
    with pytest.raises(BackendError, match="exceeds operand dim"):
        f.DynamicUpdateSlice(x, f.Parameter("u2", make_shape(F32, 6, 1)), [i0, i1])
    ids = f.Parameter("ids", make_shape(dtypes.Int32, 7, 1))
    upd = f.Parameter("upd", make_shape(F32, 7, 6))
    assert f.OpShape(f.ScatterSum(x, ids, upd, 1, [1], [0], [0])).dims == (5, 6)
    with pytest.raises(BackendError, match="ScatterMax: updates scatter dim"):
        f.ScatterMax(x, ids, f.Parameter("upd2", make_shape(F32, 6, 6)), 1, [1], [0], [0])
    with pytest.raises(BackendError, match="index vector size"):
        f.ScatterMin(x, ids, upd, 1, [1], [0], [0, 1])
    with pytest.raises(BackendError, match="window size 9 exceeds"):
        f.ScatterSum(x, ids, f.Parameter("upd3", make_shape(F32, 7, 9)), 1, [1], [0], [0])


def test_control_flow_plans_and_errors(be):
    b = be.Builder("cf")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 3))
    n = f.Parameter("n", make_shape(dtypes.Int32))
    cond = f.Closure()
    i = cond.Parameter("i", make_shape(dtypes.Int32))
    cond.Parameter("v", make_shape(F32, 3))
    cond.Return([cond.LessThan(i, n)])                  # n captured from main
    body = f.Closure()
    i = body.Parameter("i", make_shape(dtypes.Int32))
    v = body.Parameter("v", make_shape(F32, 3))
    body.Return([body.Add(i, body.Constant(np.array(1, np.int32))), body.Mul(v, x)])   # x captured
    outs = f.While(cond, body, f.Constant(np.array(0, np.int32)), x)
    assert [f.OpShape(o) for o in outs] == [make_shape(dtypes.Int32), make_shape(F32, 3)]
    with pytest.raises(BackendError, match="body must have 1 parameters|cond must have 1 parameters"):
        f.While(cond, body, x)
    with pytest.raises(BackendError, match="pred must be scalar bool"):
        f.If(x, cond, body)
    callee = b.NewFunction("callee")
    a = callee.Parameter("a", make_shape(F32, 3))
    callee.Return([callee.Neg(a)])
    with pytest.raises(BackendError, match="expects 1 parameters, got 2"):
        f.Call(callee, x, x)
    with pytest.raises(BackendError, match="parameter 0 shape mismatch"):
        f.Call(callee, n)
    (neg,) = f.Call(callee, outs[1])
    f.Return([neg])
    plan = b.Compile().Plan()
    assert "while (2 state values" in plan and "call callee" in plan, plan


def test_sort_picks_lds_or_global_network(be):
    """Rows whose keys and index array fit one workgroup's LDS use the LDS kernel;
    longer rows (or wide multi-operand keys) the global-memory network; both
    generated kernels compile (hipRTC runs on the plan-only backend too)."""
    def plan_of(dims, dts):
        b = be.Builder("sort")
        f = b.Main()
        xs = [f.Parameter(f"x{i}", make_shape(dt, *dims)) for i, dt in enumerate(dts)]
        c = f.Closure()
        ps = []
        for i, dt in enumerate(dts):
            ps += [c.Parameter(f"l{i}", make_shape(dt)), c.Parameter(f"r{i}", make_shape(dt))]
        c.Return([c.LessThan(ps[0], ps[1])])
        f.Return(f.Sort(c, len(dims) - 1, True, *xs))
        return b.Compile().Plan()
    assert "sort_rows " in plan_of((4, 16384), [F32])                     # 64 KiB keys + 64 KiB indices
    p = plan_of((4, 16385), [F32])
    assert "sort_rows_global" in p and "chunks of 16384" in p, p
    p = plan_of((2, 1000000), [F32, dtypes.Int32])
    assert "sort_rows_global" in p, p
    assert "sort_rows_global" in plan_of((2, 8000), [dtypes.Int64, dtypes.Int64, dtypes.Int32])


# The reference's declared ops (capabilities.go:17-150) minus the ones this
# backend does not build (CNN / batch-norm / RNG ops, outside the hot path).
_REFERENCE_OPS = set("""Parameter Constant Abs Neg Sqrt Rsqrt Exp Expm1 Log Log1p Sin Cos Tanh
Logistic Erf Floor Ceil Round Sign LogicalNot BitwiseNot IsFinite IsNaN Identity Add Sub Mul Div
Rem Pow Max Min Atan2 LogicalAnd LogicalOr LogicalXor BitwiseAnd BitwiseOr BitwiseXor ShiftLeft
ShiftRightArithmetic ShiftRightLogical Equal NotEqual GreaterThan GreaterOrEqual LessThan
LessOrEqual Reshape Transpose ConvertDType BroadcastInDim Where Clamp Slice Concatenate Reverse
Iota Pad DotGeneral ReduceSum ReduceMax ReduceMin ReduceProduct ArgMinMax BatchNormForInference
Gather ScatterSum ScatterMax ScatterMin DynamicSlice DynamicUpdateSlice RNGBitGenerator
ConvGeneral ReduceWindow SelectAndScatterMax EqualTotalOrder NotEqualTotalOrder
GreaterThanTotalOrder GreaterOrEqualTotalOrder LessThanTotalOrder LessOrEqualTotalOrder
ReduceLogicalAnd ReduceLogicalOr FusedSoftmax FusedLayerNorm FusedGelu FusedDense
FusedAttentionQKVProjection FusedScaledDotProductAttention BatchNormForTraining
BatchNormGradient While If Sort Call""".split())
_ABSENT = {"BatchNormForInference", "BatchNormForTraining", "BatchNormGradient", "RNGBitGenerator",
           "ConvGeneral", "ReduceWindow", "SelectAndScatterMax"}


def test_capabilities_match_reference_list_and_methods():
    from gomlx_hip.backend import Backend, Function
    caps = Backend("plan").Capabilities()
    assert caps.functions
    assert caps.operations == _REFERENCE_OPS - _ABSENT
    # every declared op is a Function method of the same name
    assert [op for op in caps.operations if not hasattr(Function, op)] == []
    # the reference's dtype list exactly (capabilities.go:153-166): no Float64
    assert caps.dtypes == {"Float32", "Float16", "Bool", "Int8", "Int16", "Int32", "Int64", "Uint8",
                           "Uint16", "Uint32", "Uint64", "BFloat16"}


def test_pad_and_logical_reduce_shapes():
    from gomlx_hip.backend import Backend, BackendError, dtypes, make_shape
    import numpy as np
    b = Backend("plan").Builder("pad")
    f = b.Main()
    x = f.Parameter("x", make_shape(dtypes.Float32, 3, 4))
    z = f.Constant(np.float32(0))
    assert f.OpShape(f.Pad(x, z, (1, 2), (0, -1))).dims == (6, 3)
    assert f.OpShape(f.Pad(x, z, (0, 0), (0, 0))).dims == (3, 4)
    with pytest.raises(BackendError, match="interior"):
        f.Pad(x, z, (1, 2, 1), (0, 0))
    with pytest.raises(BackendError, match="2 axis configs for rank-2|axis configs"):
        f.Pad(x, z, (1, 2))
    bl = f.Parameter("b", make_shape(dtypes.Bool, 3, 4))
    assert f.OpShape(f.ReduceLogicalAnd(bl, 1)).dims == (3,)
    assert f.OpShape(f.ReduceLogicalOr(bl)).dtype == dtypes.Bool
    with pytest.raises(BackendError, match="bool operand required"):
        f.ReduceLogicalOr(x)


def test_dot_grouping_rule(be):
    """DotGenerals sharing a left operand run as one grouped launch when none feeds
    an elementwise op (which may absorb it as a GEMM epilogue), they fold without
    copies, and their right operands are leaves; the rest stay separate steps."""
    sx, sw = make_shape(BF16, 512, 256), make_shape(BF16, 256, 384)
    dense = graphs.dense
    # three plain products + one feeding an Add: G=3 and a fused epilogue
    p = _plan(be, lambda f, x, a, b, c, d, r: [dense(f, x, a), dense(f, x, b), dense(f, x, c),
                                                f.Add(r, dense(f, x, d))],
              [sx, sw, sw, sw, sw, make_shape(BF16, 512, 384)])
    assert p.count("gemm_grouped bfloat16 G=3 M=512 N=384 K=256") == 1 and "gemm_batched+epilogue" in p, p
    # a right operand computed from another product's output is not a leaf: that
    # product runs alone, the other two are grouped
    def chained(f, x, a, b):
        y = dense(f, x, a)
        return [y, dense(f, x, b), dense(f, x, f.Slice(y, [0, 0], [256, 384], [1, 1]))]
    p = _plan(be, chained, [sx, sw, sw])
    assert p.count("gemm_grouped bfloat16 G=2") == 1 and p.count("gemm_batched bfloat16") == 1, p
    w_sq = make_shape(BF16, 256, 256)
    p = _plan(be, lambda f, x, a, b: [dense(f, x, a), dense(f, x, f.Mul(b, b))], [sx, w_sq, w_sq])
    assert "gemm_grouped" not in p and p.count("gemm_batched bfloat16") == 2, p
    # different right-operand layouts (one transposed view): separate
    p = _plan(be, lambda f, x, a, b: [dense(f, x, a), f.DotGeneral(x, [1], [], b, [1], [])], [sx, w_sq, w_sq])
    assert "gemm_grouped" not in p and p.count("gemm_batched bfloat16") == 2, p
    # fp32 products: not grouped (the grouped core is the 16-bit one)
    p = _plan(be, lambda f, x, a, b: [dense(f, x, a), dense(f, x, b)],
              [make_shape(F32, 512, 256), make_shape(F32, 256, 384), make_shape(F32, 256, 384)])
    assert "gemm_grouped" not in p and p.count("gemm_batched float32") == 2, p
    # more than four siblings: groups of at most four
    p = _plan(be, lambda f, x, *ws: [dense(f, x, w) for w in ws], [sx] + [sw] * 6)
    assert p.count("gemm_grouped bfloat16 G=4") == 1 and p.count("gemm_grouped bfloat16 G=2") == 1, p


def test_decode_step_plan(be):
    """The decoding block step (16 sequences, 8B-class shapes) plans every projection
    as a contraction split: the QKV product with its own sum (a graph output, Q read
    by the attention), the O / gate / up / down partials summed inside the residual
    and SwiGLU kernels; the attention as one fused launch with a split key range."""
    from gomlx_hip import graphs
    plan = graphs.decode_step(be, graphs.DecodeStepConfig()).Plan()
    assert plan.startswith("# 11 steps"), plan
    assert "gemm_batched bfloat16 B=1 M=16 N=6144 K=4096" in plan and "contraction split in 8)" in plan, plan
    assert plan.count("gemm_split_partials") == 4, plan
    assert "sums the split partials of 2 products" in plan and plan.count("sums the split partials of 1 product") == 2
    assert plan.count("sdpa_fwd") == 1 and "key range split" in plan, plan
    assert "strided_copy" not in plan and "epilogue" not in plan, plan
