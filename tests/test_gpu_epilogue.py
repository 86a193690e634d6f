"""DotGeneral -> elementwise chains fused into the GEMM epilogue.

The lowering runs an elementwise cluster that consumes one DotGeneral (or two
sharing the left operand, e.g. SiLU(x.Wg) * (x.Wu)) as one GEMM whose epilogue
evaluates the cluster.  The Dot value enters the epilogue rounded to the Dot's
dtype and the members run the same generated code as the stand-alone cluster
kernel, so every case here must be bit-identical to the unfused plan
(GHIP_EPILOGUE_FUSION=0), which the rest of the suite checks against the
oracle; one case per pattern is also checked against the oracle directly."""
import os

import numpy as np
import pytest

from oracle import oracle as orc
from gomlx_hip import synth
from gomlx_hip.backend import Backend, dtypes, make_shape
from gomlx_hip import graphs
from conftest import rel_err, norm_err

pytestmark = pytest.mark.gpu

F32, BF16 = dtypes.Float32, dtypes.BFloat16


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def _bf(a):
    return synth.round_bf16(np.asarray(a, np.float32))


def _compile_run(be, build, inputs, fuse):
    old = os.environ.get("GHIP_EPILOGUE_FUSION")
    os.environ["GHIP_EPILOGUE_FUSION"] = "1" if fuse else "0"
    try:
        b = be.Builder("epi")
        f = b.Main()
        params = [f.Parameter(f"p{i}", s) for i, (_, s) in enumerate(inputs)]
        f.Return(build(f, *params))
        ex = b.Compile()
    finally:
        if old is None:
            del os.environ["GHIP_EPILOGUE_FUSION"]
        else:
            os.environ["GHIP_EPILOGUE_FUSION"] = old
    plan = ex.Plan()
    bufs = [be.BufferFromFlatData(0, a, s) for a, s in inputs]
    outs = []
    for r in ex.Execute(bufs, None, 0):
        s = be.BufferShape(r)
        outs.append((s.dtype, be.BufferToFlatData(r).reshape(s.dims).copy()))
    ex.Finalize()
    return plan, outs


def _check_fused_equals_unfused(be, build, inputs, dots=1, core=None):
    plan_f, out_f = _compile_run(be, build, inputs, True)
    plan_u, out_u = _compile_run(be, build, inputs, False)
    print(plan_f)
    assert f"gemm_batched+epilogue bf16" in plan_f and f"dots={dots}" in plan_f
    assert core is None or f"core={core}" in plan_f, plan_f
    assert "gemm_batched+epilogue" not in plan_u
    assert len(out_f) == len(out_u)
    for (dt_f, a), (dt_u, b) in zip(out_f, out_u):
        assert dt_f == dt_u
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), "fused epilogue differs from the unfused plan"
    return [synth.bf16_bits_to_f32(a) if dt == BF16 else a for dt, a in out_f]


def _bf16_in(seed, shape, std=1.0):
    x = _bf(synth.normal(seed, shape, std=std))
    return x, make_shape(BF16, *shape)


def test_residual_add_ragged(be):
    """x2 = r + x.W with M, N not multiples of the tile (rows 300, cols 264)."""
    x, sx = _bf16_in(11, (2, 150, 136))
    w, sw = _bf16_in(12, (136, 264), std=136 ** -0.5)
    r, sr = _bf16_in(13, (2, 150, 264))
    (y,) = _check_fused_equals_unfused(be, lambda f, x, w, r: [f.Add(r, graphs.dense(f, x, w))],
                                       [(x, sx), (w, sw), (r, sr)])
    dot = _bf(orc.dot_general(x, [2], [], w, [0], []))
    want = _bf(r.astype(np.float64) + dot)
    assert rel_err(y, want) <= 2.0 ** -7 and norm_err(y, want) <= 1e-3


def test_bias_relu_broadcast(be):
    """max(x.W + bias, 0): a [N] operand broadcast along the rows and a literal."""
    x, sx = _bf16_in(21, (300, 136))
    w, sw = _bf16_in(22, (136, 264), std=136 ** -0.5)
    bias, sb = _bf16_in(23, (264,))

    def build(f, x, w, b):
        d = graphs.dense(f, x, w)
        bb = f.BroadcastInDim(b, make_shape(BF16, 300, 264), [1])
        zero = f.BroadcastInDim(f.Constant(np.array(0.0, np.float32), dtype=BF16), make_shape(BF16, 300, 264), [])
        return [f.Max(f.Add(d, bb), zero)]
    (y,) = _check_fused_equals_unfused(be, build, [(x, sx), (w, sw), (bias, sb)])
    dot = _bf(orc.dot_general(x, [1], [], w, [0], []))
    want = np.maximum(_bf(dot.astype(np.float64) + bias), 0)
    assert rel_err(y, want) <= 2.0 ** -7 and norm_err(y, want) <= 1e-3


@pytest.mark.parametrize("rows,cols,k,core", [(300, 264, 136, "8w-k64"), (1024, 512, 136, "8w-k64"),
                                              (2000, 2000, 1000, "4w-km32"), (2048, 2048, 512, "4w-km32")])
def test_swiglu_two_products(be, rows, cols, k, core):
    """SiLU(x.Wg) * (x.Wu): both products in one kernel sharing the x tile.  Grids
    of >= 128 tiles run the 4-wave 128 x 128-wave core (ragged: rows, cols and k not
    multiples of the tile), smaller ones the 64-deep core; the large cases are
    checked bit for bit against the unfused plan, whose products the DotGeneral
    tests check against the oracle."""
    x, sx = _bf16_in(31, (rows, k))
    wg, sg = _bf16_in(32, (k, cols), std=k ** -0.5)
    wu, su = _bf16_in(33, (k, cols), std=k ** -0.5)

    def build(f, x, wg, wu):
        g, u = graphs.dense(f, x, wg), graphs.dense(f, x, wu)
        return [f.Mul(f.Mul(g, f.Logistic(g)), u)]
    (y,) = _check_fused_equals_unfused(be, build, [(x, sx), (wg, sg), (wu, su)], dots=2, core=core)
    if rows * cols * k > 1024 * 512 * 136:
        return
    g = _bf(orc.dot_general(x, [1], [], wg, [0], [])).astype(np.float64)
    u = _bf(orc.dot_general(x, [1], [], wu, [0], []))
    want = _bf(_bf(g * _bf(1.0 / (1.0 + np.exp(-g)))) * u)
    assert rel_err(y, want) <= 2.0 ** -7 and norm_err(y, want) <= 1e-3


def test_batched_scale_add(be):
    """Batch axes: 0.5 * (a[b].B[b]) + c[b] over [3, 64, 72]."""
    a, sa = _bf16_in(41, (3, 64, 136))
    b, sb = _bf16_in(42, (3, 136, 72), std=136 ** -0.5)
    c, sc = _bf16_in(43, (3, 64, 72))

    def build(f, a, b, c):
        d = f.DotGeneral(a, [2], [0], b, [1], [0])
        half = f.BroadcastInDim(f.Constant(np.array(0.5, np.float32), dtype=BF16), make_shape(BF16, 3, 64, 72), [])
        return [f.Add(f.Mul(d, half), c)]
    (y,) = _check_fused_equals_unfused(be, build, [(a, sa), (b, sb), (c, sc)])
    dot = _bf(orc.dot_general(a, [2], [0], b, [1], [0]))
    want = _bf(_bf(dot * 0.5).astype(np.float64) + c)
    assert rel_err(y, want) <= 2.0 ** -7 and norm_err(y, want) <= 1e-3


def test_convert_to_f32_add(be):
    """The cluster's output dtype differs from the Dot's: f32(x.W) + y."""
    x, sx = _bf16_in(51, (256, 136))
    w, sw = _bf16_in(52, (136, 136), std=136 ** -0.5)
    y32 = synth.normal(53, (256, 136))
    (y,) = _check_fused_equals_unfused(
        be, lambda f, x, w, y: [f.Add(f.ConvertDType(graphs.dense(f, x, w), F32), y)],
        [(x, sx), (w, sw), (y32, make_shape(F32, 256, 136))])
    want = _bf(orc.dot_general(x, [1], [], w, [0], [])).astype(np.float64) + y32
    assert np.max(np.abs(y - want) / np.maximum(np.abs(want), 1.0)) <= 1e-6


def test_rhs_k_contiguous(be):
    """rhs stored [N, K] (contracting its last axis): the K-major B tile path."""
    x, sx = _bf16_in(61, (384, 136))
    wt, sw = _bf16_in(62, (264, 136), std=136 ** -0.5)
    r, sr = _bf16_in(63, (384, 264))
    (y,) = _check_fused_equals_unfused(
        be, lambda f, x, w, r: [f.Add(f.DotGeneral(x, [1], [], w, [1], []), r)], [(x, sx), (wt, sw), (r, sr)])
    want = _bf(_bf(orc.dot_general(x, [1], [], wt, [1], [])).astype(np.float64) + r)
    assert rel_err(y, want) <= 2.0 ** -7 and norm_err(y, want) <= 1e-3


def test_dot_also_returned_is_not_fused(be):
    """A Dot with a consumer outside the cluster (here: a graph output) stays a
    stand-alone GEMM."""
    x, sx = _bf16_in(71, (256, 136))
    w, sw = _bf16_in(72, (136, 264), std=136 ** -0.5)
    r, sr = _bf16_in(73, (256, 264))

    def build(f, x, w, r):
        d = graphs.dense(f, x, w)
        return [d, f.Add(d, r)]
    plan, outs = _compile_run(be, build, [(x, sx), (w, sw), (r, sr)], True)
    assert "gemm_batched+epilogue" not in plan
    d = synth.bf16_bits_to_f32(outs[0][1])
    s = synth.bf16_bits_to_f32(outs[1][1])
    assert np.array_equal(s, _bf(d.astype(np.float64) + r))


def test_transformer_block_fused_equals_unfused(be):
    """The block's SwiGLU and the wo residual add run as GEMM epilogues; the down
    projection (M 256, N 256, K 1024: four tiles of 128 x 128) splits its
    contraction and stays unfused; the whole block is bit-identical to the unfused
    plan."""
    cfg = graphs.TransformerBlockConfig(batch=2, seq=128, vocab=1000, d_model=256, heads=2, head_dim=128, ffn=1024)
    P = {"ids": synth.uniform_int(5001, (cfg.batch, cfg.seq), 0, cfg.vocab)}
    for i, (name, shape) in enumerate(cfg.param_shapes()[1:]):
        P[name] = np.ones(shape.dims, np.float32) if name.startswith("g_") else _bf(
            synth.normal(5002 + i, shape.dims, std=0.02))
    outs = {}
    for fuse in (True, False):
        os.environ["GHIP_EPILOGUE_FUSION"] = "1" if fuse else "0"
        try:
            ex = graphs.transformer_block(be, cfg)
        finally:
            del os.environ["GHIP_EPILOGUE_FUSION"]
        plan = ex.Plan()
        assert ("dots=2" in plan) == fuse and (plan.count("gemm_batched+epilogue") == (2 if fuse else 0)), plan
        assert "M=256 N=256 K=1024" in plan and "contraction split in" in plan, plan
        bufs = [be.BufferFromFlatData(0, P[name], shape) for name, shape in cfg.param_shapes()]
        (out,) = ex.Execute(bufs, None, 0)
        outs[fuse] = be.BufferToFlatData(out).copy()
        ex.Finalize()
    assert np.array_equal(outs[True], outs[False])


@pytest.mark.parametrize("rows,cols,k", [(2304, 4096, 512), (2000, 4104, 520)])
def test_gelu_both_operands_mn_contiguous(be, rows, cols, k):
    """FusedGelu(DotGeneral(x, [0], [], w, [0], [])) with x stored [K, M] and w
    [K, N]: both operands MN-contiguous and a VALU-heavy (tanh) epilogue, which
    runs on the 8-wave 64-deep core with both tiles read by transpose reads.  More
    than 128 tiles of 256 x 256 (fewer run the 128 x 128 core), even and ragged (rows, cols and k not multiples
    of the tile); bit for bit against the unfused plan and 2048 sampled outputs
    against the reference's bf16 GELU chain on the fp64 product (row strides stay
    multiples of 8 elements, which the MFMA path needs)."""
    xt, sx = _bf16_in(81, (k, rows))
    w, sw = _bf16_in(82, (k, cols), std=k ** -0.5)

    def build(f, xt, w):
        return [f.FusedGelu(f.DotGeneral(xt, [0], [], w, [0], []), False)]
    (y,) = _check_fused_equals_unfused(be, build, [(xt, sx), (w, sw)], core="8w-k64")
    rng = np.random.default_rng(rows + cols)
    mi, ni = rng.integers(0, rows, 2048), rng.integers(0, cols, 2048)
    dot = _bf(np.einsum("km,km->m", xt[:, mi].astype(np.float64), w[:, ni].astype(np.float64)))
    lo, hi = orc.gelu_chain_16(dot, False)
    got = y[mi, ni]
    want = lo.astype(np.float64)
    assert rel_err(got, want) <= 3e-2 and norm_err(got, want) <= 1e-2
    # the chain's result exactly, except where the fp32-accumulated product rounds
    # to the other bf16 neighbour of the fp64 one
    assert np.mean((got == lo) | (got == hi)) >= 0.95


def test_grouped_projections_equal_separate(be):
    """Three DotGenerals sharing x (the Q, K, V projections of a block) compile to
    one grouped launch (gemm_grouped G=3) whose outputs equal the stand-alone GEMMs
    (GHIP_DOT_GROUPING=0) bit for bit; a fourth Dot on x with an elementwise user
    stays outside the group (it is the residual epilogue's)."""
    M, D = 2048, 1024
    x, sx = _bf16_in(5101, (M, D), std=0.5)
    ws = [_bf16_in(5102 + i, (D, D), std=0.03) for i in range(4)]
    r, sr = _bf16_in(5110, (M, D))

    def build(f, xx, w0, w1, w2, w3, rr):
        dots = [graphs.dense(f, xx, w) for w in (w0, w1, w2)]
        return dots + [f.Add(rr, graphs.dense(f, xx, w3))]

    inputs = [(x, sx)] + ws + [(r, sr)]
    outs = {}
    for grouping in ("1", "0"):
        old = os.environ.get("GHIP_DOT_GROUPING")
        os.environ["GHIP_DOT_GROUPING"] = grouping
        try:
            plan, out = _compile_run(be, build, inputs, True)
        finally:
            if old is None:
                del os.environ["GHIP_DOT_GROUPING"]
            else:
                os.environ["GHIP_DOT_GROUPING"] = old
        outs[grouping] = out
        if grouping == "1":
            assert plan.count("gemm_grouped bfloat16 G=3") == 1 and "gemm_batched+epilogue" in plan, plan
        else:
            assert "gemm_grouped" not in plan and plan.count("gemm_batched bfloat16") == 3, plan
    for (dt_g, a), (dt_s, b) in zip(outs["1"], outs["0"]):
        assert dt_g == dt_s and np.array_equal(a.view(np.uint8), b.view(np.uint8))
    for i in range(3):
        y = synth.bf16_bits_to_f32(outs["1"][i][1])
        rows = np.arange(0, M, 97)
        ref = orc.dot_general(x[rows], [1], [], ws[i][0], [0], [])
        assert rel_err(y[rows], ref) <= 1e-2

