"""Graph API on the GPU: Builder -> Compile -> Execute through the C ABI.

The first block mirrors the reference's own backend tests
(mpsgraph/gomlx/mpsgraph_test.go, cited per test) with the same inputs,
expected values and tolerances; the rest checks fused lowerings and the
transformer block against the CPU oracle."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from gomlx_hip import synth
from gomlx_hip.backend import AxesLayout, Backend, BackendError, dtypes, make_shape
from gomlx_hip import graphs
from conftest import rel_err, norm_err

pytestmark = pytest.mark.gpu

F32, BF16, I32, I64 = dtypes.Float32, dtypes.BFloat16, dtypes.Int32, dtypes.Int64


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def run(be, build, inputs, name="t"):
    """build(f, params) -> list of outputs; inputs: list of (np array, Shape)."""
    b = be.Builder(name)
    f = b.Main()
    params = [f.Parameter(f"p{i}", s) for i, (_, s) in enumerate(inputs)]
    outs = build(f, *params)
    f.Return(outs)
    ex = b.Compile()
    bufs = [be.BufferFromFlatData(0, a, s) for a, s in inputs]
    res = ex.Execute(bufs, None, 0)
    out = []
    for r in res:
        s = be.BufferShape(r)
        a = be.BufferToFlatData(r).reshape(s.dims)
        if s.dtype == BF16:
            a = synth.bf16_bits_to_f32(a)
        out.append(a)
    ex.Finalize()
    return out


def close(got, want, tol):
    assert np.max(np.abs(np.asarray(got, np.float64).reshape(-1) - np.asarray(want, np.float64).reshape(-1))) <= tol


# ------------------------------------------------------------ reference Tier A mirrors
def test_backend_creation(be):                                    # :27-42
    assert be.Name() == "hip" and be.NumDevices() == 1
    assert "gfx950" in be.Description()


def test_buffer_operations(be):                                   # :44-81
    s = make_shape(F32, 2, 3)
    buf = be.BufferFromFlatData(0, np.arange(1, 7, dtype=np.float32), s)
    assert be.BufferShape(buf) == s
    assert be.BufferToFlatData(buf).tolist() == [1, 2, 3, 4, 5, 6]
    be.BufferFinalize(buf)
    with pytest.raises(BackendError):
        be.BufferFromFlatData(0, np.zeros(5, np.float32), s)     # size mismatch


def test_add_operation(be):                                       # :223-239
    s = make_shape(F32, 2, 3)
    (y,) = run(be, lambda f, x, y: [f.Add(x, y)],
               [(np.array([1, 2, 3, 4, 5, 6], np.float32), s), (np.array([10, 20, 30, 40, 50, 60], np.float32), s)])
    close(y, [11, 22, 33, 44, 55, 66], 1e-5)


@pytest.mark.parametrize("name,inp,exp,tol", [                    # :241-276
    ("Abs", [-1, 2, -3, 4], [1, 2, 3, 4], 1e-5),
    ("Neg", [-1, 2, -3, 4], [1, -2, 3, -4], 1e-5),
    ("Sqrt", [1, 4, 9, 16], [1, 2, 3, 4], 1e-5),
    ("Exp", [0, 1], [1, math.e], 1e-5),
    ("Log", [1, math.e], [0, 1], 1e-4),
    ("Tanh", [0, 1], [0, math.tanh(1)], 1e-5),
])
def test_unary_operations(be, name, inp, exp, tol):
    x = np.array(inp, np.float32)
    (y,) = run(be, lambda f, a: [getattr(f, name)(a)], [(x, make_shape(F32, len(inp)))])
    close(y, exp, tol)


@pytest.mark.parametrize("name,exp,tol", [                        # :278-324
    ("Add", [13, 25, 40, 48], 1e-5), ("Sub", [7, 15, 20, 32], 1e-5), ("Mul", [30, 100, 300, 320], 1e-5),
    ("Div", [10 / 3, 4, 3, 5], 1e-4), ("Max", [10, 20, 30, 40], 1e-5), ("Min", [3, 5, 10, 8], 1e-5),
])
def test_binary_operations(be, name, exp, tol):
    s = make_shape(F32, 4)
    (y,) = run(be, lambda f, a, b: [getattr(f, name)(a, b)],
               [(np.array([10, 20, 30, 40], np.float32), s), (np.array([3, 5, 10, 8], np.float32), s)])
    close(y, exp, tol)


def test_reshape_constant_reduce(be):                             # :326-487
    (r,) = run(be, lambda f, x: [f.Reshape(x, 3, 2)], [(np.arange(6, dtype=np.float32), make_shape(F32, 2, 3))])
    assert r.shape == (3, 2) and r.reshape(-1).tolist() == list(range(6))
    (c,) = run(be, lambda f, x: [f.Add(x, f.Constant(np.array([10, 20, 30], np.float32), 3))],
               [(np.array([1, 2, 3], np.float32), make_shape(F32, 3))])
    close(c, [11, 22, 33], 1e-5)
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    s, p, mx, mn = run(be, lambda f, a: [f.ReduceSum(a, 1), f.ReduceProduct(a, 1), f.ReduceMax(a, 0), f.ReduceMin(a)],
                       [(x, make_shape(F32, 2, 3))])
    close(s, [6, 15], 1e-5)
    close(p, [6, 120], 1e-5)                                       # :1318-1365
    close(mx, [4, 5, 6], 0)
    close(mn, [1], 0)


def test_dot_general_known_answers(be, known):                    # :489-596
    for name in ("dot_simple", "dot_batched"):
        c = known[name]
        (y,) = run(be, lambda f, a, b: [f.DotGeneral(a, c["lc"], c["lb"], b, c["rc"], c["rb"])],
                   [(np.array(c["lhs"], np.float32), make_shape(F32, *c["lhs_shape"])),
                    (np.array(c["rhs"], np.float32), make_shape(F32, *c["rhs_shape"]))])
        close(y, c["expected"], c["tol"])


def test_gather_known_answer(be, known):                          # :599-674
    c = known["gather_embedding"]
    (y,) = run(be, lambda f, t, i: [f.Gather(t, i, 1, [1], [0], [0], [1, 3], False)],
               [(np.array(c["table"], np.float32), make_shape(F32, 4, 3)),
                (np.array(c["ids"], np.int32), make_shape(I32, 2, 1))])
    assert y.reshape(-1).tolist() == c["expected"]


def test_slice_concat_broadcast_reverse_transpose(be):            # :677-876, :1269-1316, :1535-1582
    x = np.arange(12, dtype=np.float32)
    (s,) = run(be, lambda f, a: [f.Slice(a, [1, 1], [3, 3], [1, 1])], [(x, make_shape(F32, 3, 4))])
    close(s, [5, 6, 9, 10], 0)  # arange(12) (the reference fills 1..12 and expects [6,7,10,11])
    (c,) = run(be, lambda f, a, b: [f.Concatenate(1, a, b)],
               [(np.array([1, 2, 3, 4], np.float32), make_shape(F32, 2, 2)),
                (np.array([5, 6, 7, 8, 9, 10], np.float32), make_shape(F32, 2, 3))])
    close(c, [1, 2, 5, 6, 7, 3, 4, 8, 9, 10], 0)
    (b,) = run(be, lambda f, a: [f.BroadcastInDim(a, make_shape(F32, 2, 3), [1])],
               [(np.array([10, 20, 30], np.float32), make_shape(F32, 3))])
    close(b, [10, 20, 30, 10, 20, 30], 0)
    v = np.array([1, 2, 3, 4, 5, 6], np.float32)
    r, t = run(be, lambda f, a: [f.Reverse(a, 1), f.Transpose(a, 1, 0)], [(v, make_shape(F32, 2, 3))])
    close(r, [3, 2, 1, 6, 5, 4], 0)
    close(t, [1, 4, 2, 5, 3, 6], 0)


def test_iota_argmax_convert(be, known):                          # :785-822, :941-991, :1485-1532
    b = be.Builder("iota")
    f = b.Main()
    f.Return([f.Iota(make_shape(F32, 2, 3), 1)])
    ex = b.Compile()
    (out,) = ex.Execute([], None, 0)
    assert be.BufferToFlatData(out).tolist() == known["iota"]["expected"]
    (a,) = run(be, lambda f, x: [f.ArgMinMax(x, 1, I32, False)],
               [(np.array([1, 5, 3, 8, 2, 6], np.float32), make_shape(F32, 2, 3))])
    assert a.tolist() == [1, 0]
    (cv,) = run(be, lambda f, x: [f.ConvertDType(x, I32)], [(np.array([1.7, 2.3, -0.9], np.float32), make_shape(F32, 3))])
    assert cv.tolist() == [1, 2, 0]


def test_comparisons_and_where(be):                               # :1367-1483
    s = make_shape(F32, 4)
    l, r = np.array([1, 2, 3, 4], np.float32), np.array([2, 2, 2, 2], np.float32)
    outs = run(be, lambda f, a, b: [f.Equal(a, b), f.NotEqual(a, b), f.GreaterThan(a, b), f.LessThan(a, b),
                                    f.GreaterOrEqual(a, b), f.LessOrEqual(a, b)], [(l, s), (r, s)])
    for got, want in zip(outs, [l == r, l != r, l > r, l < r, l >= r, l <= r]):
        assert got.astype(bool).tolist() == want.tolist()
    (w,) = run(be, lambda f, c, t, e: [f.Where(c, t, e)],
               [(np.array([True, False, True, False]), make_shape(dtypes.Bool, 4)),
                (np.array([10, 20, 30, 40], np.float32), s), (np.array([1, 2, 3, 4], np.float32), s)])
    close(w, [10, 2, 30, 4], 0)


def test_multiple_outputs_and_chained_ops(be):                    # :1584-1634, :1727-1803
    s = make_shape(F32, 3)
    a, d = run(be, lambda f, x, y: [f.Add(x, y), f.Sub(x, y)],
               [(np.array([10, 20, 30], np.float32), s), (np.array([1, 2, 3], np.float32), s)])
    close(a, [11, 22, 33], 1e-5)
    close(d, [9, 18, 27], 1e-5)
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    w = np.array([0.5, -0.5, 1.0, -1.0], np.float32)
    bb = np.array([0.1, 0.2, -0.1, 0.0], np.float32)
    (y,) = run(be, lambda f, xx: [f.Logistic(f.Add(f.Mul(xx, f.Constant(w, 4)), f.Constant(bb, 4)))],
               [(x, make_shape(F32, 4))])
    close(y, 1 / (1 + np.exp(-(x.astype(np.float64) * w + bb))), 1e-5)


def test_transformer_block_attention_chain(be, known):            # :1638-1724
    c = known["attention_dot_chain"]
    s = make_shape(F32, 2, 3)

    def build(f, q, k, v):
        scores = f.DotGeneral(q, [1], [], k, [1], [])
        sc = f.Constant(np.array([c["scale"]], np.float32), 1)
        scores = f.Mul(scores, f.BroadcastInDim(sc, make_shape(F32, 2, 2), [1]))
        w = f.FusedSoftmax(scores, 1)
        return [f.DotGeneral(w, [1], [], v, [0], [])]
    (y,) = run(be, build, [(np.array(c["q"], np.float32), s), (np.array(c["k"], np.float32), s),
                           (np.array(c["v"], np.float32), s)])
    close(y, c["expected"], c["tol"])


def test_int64_and_uint8(be):                                     # :2746-2804
    (a,) = run(be, lambda f, x, y: [f.Add(x, y)], [(np.array([1, 2, 3], np.int64), make_shape(I64, 3)),
                                                   (np.array([10, 20, 30], np.int64), make_shape(I64, 3))])
    assert a.tolist() == [11, 22, 33]
    (cv,) = run(be, lambda f, x: [f.ConvertDType(x, I64)], [(np.array([1.5, 2.7, -3.2], np.float32), make_shape(F32, 3))])
    assert cv.tolist() == [1, 2, -3]
    (u,) = run(be, lambda f, x, y: [f.Add(x, y)], [(np.array([250, 3], np.uint8), make_shape(dtypes.Uint8, 2)),
                                                   (np.array([10, 4], np.uint8), make_shape(dtypes.Uint8, 2))])
    assert u.tolist() == [4, 7]  # wraps like Go's uint8


# ------------------------------------------------------------ reference Tier D mirrors
def test_fused_softmax_known_answer(be, known):                   # :1133-1190
    c = known["softmax"]
    (y,) = run(be, lambda f, x: [f.FusedSoftmax(x, 1)], [(np.array(c["x"], np.float32), make_shape(F32, 2, 3))])
    close(y, c["expected"], c["tol"])


def test_fused_layer_norm_known_answers(be, known):               # :2595-2623
    c = known["layernorm_basic"]
    (y,) = run(be, lambda f, x: [f.FusedLayerNorm(x, [-1], c["eps"])],
               [(np.array(c["x"], np.float32), make_shape(F32, 2, 4))])
    close(y, c["expected"], c["tol"])
    c = known["layernorm_gamma_beta"]
    (y,) = run(be, lambda f, x, g, b: [f.FusedLayerNorm(x, [-1], c["eps"], g, b)],
               [(np.array(c["x"], np.float32), make_shape(F32, 2, 4)),
                (np.array(c["gamma"], np.float32), make_shape(F32, 1, 4)),
                (np.array(c["beta"], np.float32), make_shape(F32, 1, 4))])
    close(y[0], c["expected_first_row"], c["tol"])


def test_fused_sdpa_known_answers(be, known):                     # :2966-3058
    c = known["sdpa_causal"]
    sh = make_shape(F32, *c["shape"])
    (y,) = run(be, lambda f, q, k, v: [f.FusedScaledDotProductAttention(q, k, v, None, 1, 1, AxesLayout.BHSD, c["scale"], True)],
               [(np.array(c[n], np.float32), sh) for n in "qkv"])
    close(y[0, 0, 0], c["expected_first_row"], c["tol"])
    c = known["sdpa_bool_mask"]
    sh = make_shape(F32, *c["shape"])
    (y,) = run(be, lambda f, q, k, v, m: [f.FusedScaledDotProductAttention(q, k, v, m, 1, 1, AxesLayout.BHSD, 1.0, False)],
               [(np.array(c[n], np.float32), sh) for n in "qkv"] +
               [(np.array(c["mask"], bool), make_shape(dtypes.Bool, 1, 1, 2, 2))])
    close(y[0, 0, 0], c["expected_first_row"], c["tol"])
    c = known["sdpa_basic_range"]
    (y,) = run(be, lambda f, q, k, v: [f.FusedScaledDotProductAttention(q, k, v, None, 1, 1, AxesLayout.BSHD, c["scale"], False)],
               [(np.array(c[n], np.float32), make_shape(F32, 1, 2, 1, 2)) for n in "qkv"])
    assert y.shape == (1, 2, 1, 2) and np.all(y > -0.1) and np.all(y < 1.1)


def test_bfloat16_add_and_matmul(be):                             # :3128-3156
    (y,) = run(be, lambda f, x: [f.ConvertDType(f.Add(f.ConvertDType(x, BF16), f.ConvertDType(x, BF16)), F32)],
               [(np.array([1, 2, 3, 4], np.float32), make_shape(F32, 4))])
    close(y, [2, 4, 6, 8], 0.1)

    def mm(f, a, b):
        c = f.DotGeneral(f.ConvertDType(a, BF16), [1], [], f.ConvertDType(b, BF16), [0], [])
        return [f.ConvertDType(c, F32)]
    (y,) = run(be, mm, [(np.array([1, 2, 3, 4], np.float32), make_shape(F32, 2, 2)),
                        (np.array([5, 6, 7, 8], np.float32), make_shape(F32, 2, 2))])
    close(y, [19, 22, 43, 50], 1.0)


# ------------------------------------------------------------ fused lowerings vs the oracle
def test_graph_softmax_chain_and_rmsnorm_chain(be):
    x = synth.normal(1001, (4096, 1024), std=2.0)
    y1, y2 = run(be, lambda f, a: [graphs.softmax_chain(f, a), f.FusedSoftmax(a, -1)], [(x, make_shape(F32, 4096, 1024))])
    ref = orc.softmax(x)
    assert rel_err(y1, ref) <= 1e-5 and rel_err(y2, ref) <= 1e-5
    x = synth.normal(2001, (512, 4096))
    g = synth.uniform_f32(2002, (4096,), 0.5, 1.5)
    (y,) = run(be, lambda f, a, gg: [graphs.rms_norm(f, a, gg, 1e-6)],
               [(x, make_shape(F32, 512, 4096)), (g, make_shape(F32, 4096))])
    assert rel_err(y, orc.rmsnorm(x, g, 1e-6)) <= 1e-5


@pytest.mark.parametrize("dt", [F32, BF16])
def test_graph_log_softmax_chain(be, dt):
    """The primitive log-softmax chain (one fused row kernel) at configs[0]'s shape."""
    x = synth.normal(1001, (4096, 1024), std=2.0)
    if dt == BF16:
        x = synth.round_bf16(x)
    (y,) = run(be, lambda f, a: [graphs.log_softmax_chain(f, a)],
               [(x if dt == F32 else synth.to_bf16_bits(x), make_shape(dt, 4096, 1024))])
    ref = orc.log_softmax(x)
    # bf16: one rounding of the fp32 result (RMS-floored)
    assert rel_err(y, ref) <= (1e-5 if dt == F32 else 2.0 ** -8 + 1e-5)


def _reduce_chain_graph(f, x, z, dt):
    """Elementwise -> Reduce -> elementwise chains that no row pattern matches: the
    generated fused reduce kernel (wave form, thread form over two axes, strided
    producer, full reduction with a scalar consumer)."""
    n = f.BroadcastInDim(f.Constant(np.array(1000, np.float32), dtype=dt), make_shape(dt, 96), [])
    rms = f.Sqrt(f.Div(f.ReduceSum(f.Mul(x, x), 1), n))
    two = f.BroadcastInDim(f.Constant(np.array(2, np.float32), dtype=dt), make_shape(dt, 40), [])
    amax = f.Mul(f.ReduceMax(f.Abs(z), 0, 2), two)
    t = f.ReduceSum(f.Exp(f.Transpose(x, 1, 0)), 0)
    tot = f.Mul(f.ReduceSum(f.Mul(z, z)), f.Constant(np.array(0.5, np.float32), dtype=dt))
    return [rms, amax, t, tot]


@pytest.mark.parametrize("dt", [F32, BF16, dtypes.Float16])
def test_reduce_fusion_matches_unfused_and_oracle(be, dt, monkeypatch):
    """The fused reduce kernels give the unfused plan's results bit for bit (same
    accumulation order, the reduced value rounded to its dtype before the
    consumer), and match a float64 restatement within the dtype's rounding."""
    x = synth.normal(2101, (96, 1000), std=0.5)
    z = synth.normal(2102, (6, 40, 5), std=2.0)
    if dt == BF16:
        x, z = synth.round_bf16(x), synth.round_bf16(z)
        feed = synth.to_bf16_bits
    elif dt == dtypes.Float16:
        x, z = x.astype(np.float16).astype(np.float32), z.astype(np.float16).astype(np.float32)
        feed = lambda a: a.astype(np.float16)  # noqa: E731
    else:
        feed = lambda a: a  # noqa: E731
    ins = [(feed(x), make_shape(dt, 96, 1000)), (feed(z), make_shape(dt, 6, 40, 5))]
    build = lambda f, a, b: _reduce_chain_graph(f, a, b, dt)  # noqa: E731
    fused = run(be, build, ins)
    monkeypatch.setenv("GHIP_REDUCE_FUSION", "0")
    plain = run(be, build, ins)
    for a, b in zip(fused, plain):
        assert np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32), equal_nan=True)
    x64, z64 = x.astype(np.float64), z.astype(np.float64)
    refs = [np.sqrt(np.sum(x64 * x64, 1) / 1000), 2 * np.max(np.abs(z64), (0, 2)), np.sum(np.exp(x64), 1),
            0.5 * np.sum(z64 * z64)]
    tol = {F32: 1e-5, BF16: 2.0 ** -6, dtypes.Float16: 2.0 ** -8}[dt]
    for got, ref in zip(fused, refs):
        assert rel_err(np.asarray(got, np.float32), ref) <= tol


def test_reduce_fusion_integers(be, monkeypatch):
    """Integer chains accumulate in 64 bits and wrap to the output type, as the
    unfused reduce does."""
    x = (synth.uniform_f32(2103, (64, 50), -300, 300)).astype(np.int32)
    build = lambda f, a: [f.ReduceSum(f.Mul(a, a), 1), f.ReduceMin(f.Neg(a)),  # noqa: E731
                          f.ReduceMax(f.Mul(a, a), 0)]
    got = run(be, build, [(x, make_shape(I32, 64, 50))])
    monkeypatch.setenv("GHIP_REDUCE_FUSION", "0")
    plain = run(be, build, [(x, make_shape(I32, 64, 50))])
    x64 = x.astype(np.int64)
    want = [np.sum(x64 * x64, 1).astype(np.int32), np.min(-x64).astype(np.int32), np.max(x64 * x64, 0).astype(np.int32)]
    for g, p_, w in zip(got, plain, want):
        assert np.array_equal(g, w) and np.array_equal(p_, w)


@pytest.mark.parametrize("dt", [F32, BF16])
def test_graph_layer_norm_chain(be, dt):
    """The reference's LayerNorm composition sent as primitives (one fused row
    kernel) against the oracle: fp32 within 1e-5, bf16 within one rounding."""
    x = synth.normal(2201, (512, 2048), std=1.5, mean=0.25)
    g = synth.uniform_f32(2202, (2048,), 0.5, 1.5)
    bt = synth.normal(2203, (2048,), std=0.1)
    if dt == BF16:
        x, g, bt = synth.round_bf16(x), synth.round_bf16(g), synth.round_bf16(bt)
        feed = synth.to_bf16_bits
    else:
        feed = lambda a: a  # noqa: E731
    ys = run(be, lambda f, a, gg, bb: [graphs.layer_norm_chain(f, a, gg, bb, 1e-5), graphs.layer_norm_chain(f, a, None, None, 1e-5)],
             [(feed(x), make_shape(dt, 512, 2048)), (feed(g), make_shape(dt, 2048)), (feed(bt), make_shape(dt, 2048))])
    tol = 1e-5 if dt == F32 else 2.0 ** -8 + 1e-5
    assert rel_err(ys[0], orc.layernorm(x, g, bt, 1e-5)) <= tol
    assert rel_err(ys[1], orc.layernorm(x, None, None, 1e-5)) <= tol


@pytest.mark.parametrize("dt", [F32, BF16, dtypes.Float16])
@pytest.mark.parametrize("shape,axis", [((6, 700, 130), 1), ((300, 5, 7), 0), ((2, 3, 257, 64), 2)])
def test_graph_softmax_layernorm_middle_axis(be, dt, shape, axis):
    """FusedSoftmax and FusedLayerNorm over an axis before the last (the column
    kernels: 64 adjacent columns per workgroup, ragged column counts) against the
    fp64 oracle on the same values: fp32 within 1e-5, 16-bit outputs within one
    rounding of the dtype (RMS-floored)."""
    np_dt = {F32: np.float32, BF16: None, dtypes.Float16: np.float16}[dt]
    x = synth.normal(2101, shape, std=2.0)
    n = shape[axis]
    g = synth.uniform_f32(2102, (n,), 0.5, 1.5)
    bt = synth.normal(2103, (n,), std=0.1)
    if dt == BF16:
        x, g, bt = _bf(x), _bf(g), _bf(bt)
        host = lambda a: synth.to_bf16_bits(a)  # noqa: E731
    else:
        x, g, bt = (a.astype(np_dt).astype(np.float32) for a in (x, g, bt))
        host = lambda a: a.astype(np_dt)  # noqa: E731
    bshape = [1] * len(shape)
    bshape[axis] = n
    ys = run(be, lambda f, a, gg, bb: [f.FusedSoftmax(a, axis), f.FusedLayerNorm(a, [axis], 1e-5, gg, bb)],
             [(host(x), make_shape(dt, *shape)), (host(g), make_shape(dt, n)),
              (host(bt.reshape(bshape)), make_shape(dt, *bshape))])
    ys = [y.astype(np.float32) for y in ys]  # run() has widened bf16 already
    ref_sm = orc.softmax(x, axis)
    ref_ln = np.moveaxis(orc.layernorm(np.ascontiguousarray(np.moveaxis(x, axis, -1)), g, bt, 1e-5), -1, axis)
    tol = 1e-5 if dt == F32 else (2.0 ** -8 if dt == BF16 else 2.0 ** -11) + 1e-5
    assert rel_err(ys[0], ref_sm) <= tol
    assert rel_err(ys[1], ref_ln) <= tol


def test_softmax_columns_direct_log_and_masked(cuda):
    """ghip_softmax_cols through the C ABI: log-softmax, a column of -inf (NaN, as
    the row kernels give), and columns with some -inf entries (those get 0)."""
    import torch
    from gomlx_hip import ops
    x = synth.normal(2111, (4, 96, 200), std=3.0)
    x[1, :, 7] = -np.inf
    x[2, ::3, 9] = -np.inf
    t = torch.from_numpy(x).cuda()
    y = ops.softmax_axis(t, 1).cpu().numpy()
    ly = ops.softmax_axis(t, 1, log=True).cpu().numpy()
    assert np.all(np.isnan(y[1, :, 7]))
    assert np.all(y[2, ::3, 9] == 0) and abs(y[2, :, 9].sum() - 1) < 1e-5
    ok = np.ones(x.shape, bool)
    ok[1, :, 7] = False
    ref = orc.softmax(x, 1)
    assert rel_err(y[ok], ref[ok]) <= 1e-5
    finite = ok & np.isfinite(x)
    assert rel_err(ly[finite], orc.log_softmax(x, 1)[finite]) <= 1e-5


def test_graph_float16_hot_ops(be):
    """Float16 (a dtype the reference declares, capabilities.go:153-166) through the
    graph API: FusedSoftmax, FusedLayerNorm, the RMSNorm chain and DotGeneral, each
    within one f16 rounding (RMS-floored) of the fp64 oracle."""
    F16 = dtypes.Float16
    h = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    x = h(synth.normal(1901, (512, 1024), std=2.0))
    g = h(synth.uniform_f32(1902, (1024,), 0.5, 1.5))
    bt = h(synth.normal(1903, (1024,), std=0.1))
    s = make_shape(F16, 512, 1024)
    v = make_shape(F16, 1024)
    ys = run(be, lambda f, a, gg, bb: [f.FusedSoftmax(a, 1), f.FusedLayerNorm(a, [1], 1e-5, gg, bb),
                                        graphs.rms_norm(f, a, gg, 1e-6), graphs.log_softmax_chain(f, a)],
             [(x, s), (g, v), (bt, v)])
    xf, gf, bf = (a.astype(np.float32) for a in (x, g, bt))
    refs = [orc.softmax(xf), orc.layernorm(xf, gf, bf, 1e-5), orc.rmsnorm(xf, gf, 1e-6), orc.log_softmax(xf)]
    for y, r in zip(ys, refs):
        assert y.dtype == np.float16
        assert rel_err(y.astype(np.float32), r) <= 2.0 ** -11 + 1e-5
    a = h(synth.normal(1904, (2, 300, 256), std=0.125))
    b = h(synth.normal(1905, (2, 256, 520), std=0.125))
    (y,) = run(be, lambda f, p, q: [f.DotGeneral(p, [2], [0], q, [1], [0])],
               [(a, make_shape(F16, 2, 300, 256)), (b, make_shape(F16, 2, 256, 520))])
    assert y.dtype == np.float16
    assert rel_err(y.astype(np.float32), orc.dot_general(a.astype(np.float32), [2], [0], b.astype(np.float32), [1], [0])) <= 1e-3


def test_graph_dot_general_layouts(be):
    a = synth.round_bf16(synth.normal(3001, (2, 64, 96), std=0.125))
    b = synth.round_bf16(synth.normal(3002, (96, 2, 80), std=0.125))
    # contracting lhs axis 2 with rhs axis 0, batch lhs 0 / rhs 1 (rhs layout needs a stride fold)
    (y,) = run(be, lambda f, x, w: [f.DotGeneral(x, [2], [0], w, [0], [1])],
               [(a, make_shape(BF16, 2, 64, 96)), (b, make_shape(BF16, 96, 2, 80))])
    assert rel_err(y, orc.dot_general(a, [2], [0], b, [0], [1])) <= 1e-2
    c = synth.normal(3003, (4, 3, 5, 6))
    d = synth.normal(3004, (6, 4, 7, 5))
    (y,) = run(be, lambda f, x, w: [f.DotGeneral(x, [3, 2], [0], w, [0, 3], [1])],
               [(c, make_shape(F32, 4, 3, 5, 6)), (d, make_shape(F32, 6, 4, 7, 5))])
    assert rel_err(y, orc.dot_general(c, [3, 2], [0], d, [0, 3], [1])) <= 1e-5


@pytest.mark.parametrize("layout", [AxesLayout.BHSD, AxesLayout.BSHD])
def test_graph_sdpa_gqa_causal(be, layout):
    B, H, Hkv, S, D = 2, 8, 2, 128, 64
    q = synth.normal(4001, (B, H, S, D))
    k = synth.normal(4002, (B, Hkv, S, D))
    v = synth.normal(4003, (B, Hkv, S, D))
    ref = orc.sdpa(q, k, v, scale=D ** -0.5, causal=True)
    t = (lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))) if layout == AxesLayout.BSHD else (lambda a: a)
    (y,) = run(be, lambda f, qq, kk, vv: [f.FusedScaledDotProductAttention(qq, kk, vv, None, H, Hkv, layout, D ** -0.5, True)],
               [(t(q), make_shape(F32, *t(q).shape)), (t(k), make_shape(F32, *t(k).shape)), (t(v), make_shape(F32, *t(v).shape))])
    if layout == AxesLayout.BSHD:
        y = y.transpose(0, 2, 1, 3)
    assert rel_err(y, ref) <= 1e-4


@pytest.mark.parametrize("layout", [AxesLayout.BHSD, AxesLayout.BSHD])
def test_graph_sdpa_decoding(be, layout):
    """One decoding step through the graph API: Q of one query against a 3000-token
    KV cache, GQA 4:1, no causal mask.  The plan splits each workgroup's key range
    (its workspace in the arena) and packs the four query heads of a kv head into
    one workgroup; the result against the oracle."""
    B, H, Hkv, Sq, Sk, D = 2, 8, 2, 1, 3000, 128
    q = _bf(synth.normal(4901, (B, H, Sq, D)))
    k = _bf(synth.normal(4902, (B, Hkv, Sk, D)))
    v = _bf(synth.normal(4903, (B, Hkv, Sk, D)))
    ref = orc.sdpa(q, k, v, scale=D ** -0.5, causal=False)
    t = (lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))) if layout == AxesLayout.BSHD else (lambda a: a)
    b = be.Builder("decode")
    f = b.Main()
    ps = [f.Parameter(n, make_shape(BF16, *t(a).shape)) for n, a in (("q", q), ("k", k), ("v", v))]
    f.Return([f.FusedScaledDotProductAttention(*ps, None, H, Hkv, layout, D ** -0.5, False)])
    ex = b.Compile()
    plan = ex.Plan()
    assert "fused attention, key range split" in plan, plan
    (r,) = ex.Execute([be.BufferFromFlatData(0, t(a), make_shape(BF16, *t(a).shape)) for a in (q, k, v)], None, 0)
    s = be.BufferShape(r)
    y = synth.bf16_bits_to_f32(be.BufferToFlatData(r).reshape(s.dims))
    ex.Finalize()
    if layout == AxesLayout.BSHD:
        y = y.transpose(0, 2, 1, 3)
    assert norm_err(y, ref) <= 1e-2
    assert rel_err(y, ref) <= 2.5e-2


@pytest.mark.parametrize("layout", [AxesLayout.BHSD, AxesLayout.BSHD])
@pytest.mark.parametrize("dt,D,kind", [(BF16, 128, "bool"), (BF16, 64, "add"), (dtypes.Float16, 128, "add"),
                                       (BF16, 96, "bool"), (F32, 64, "add"), (F32, 96, "bool"),
                                       (BF16, 100, "add"), (F32, 144, "bool")])
def test_graph_sdpa_masks(be, layout, dt, D, kind):
    """FusedScaledDotProductAttention with a mask through the graph API: rank-4
    masks in Q's layout (BSHD masks are [B, Sq, H, Sk], transposed as the reference
    does, function.go:2709-2718), lower ranks broadcast over the trailing axes;
    bf16 / f16 with a head dim that is a multiple of 8 up to 256 and fp32 with a
    multiple of 4 up to 128 take the fused kernel, the others (bf16 100, fp32 144)
    the composite (GEMM, masked softmax, GEMM)."""
    B, H, Hkv, S, Sk = 2, 4, 2, 136, 136
    q = synth.normal(4801, (B, H, S, D))
    k = synth.normal(4802, (B, Hkv, Sk, D))
    v = synth.normal(4803, (B, Hkv, Sk, D))
    if dt == BF16:
        q, k, v = (synth.round_bf16(a) for a in (q, k, v))
    elif dt == dtypes.Float16:
        q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
    m_bhsd = (synth.uniform(4804, B * H * S * Sk).reshape(B, H, S, Sk) > 0.3) if kind == "bool" else \
        synth.normal(4804, (B, H, S, Sk), std=1.0)
    if kind == "bool":
        m_bhsd[..., 0] = True
    elif dt == BF16:
        m_bhsd = synth.round_bf16(m_bhsd)
    elif dt == dtypes.Float16:
        m_bhsd = m_bhsd.astype(np.float16).astype(np.float32)
    ref = orc.sdpa(q, k, v, scale=D ** -0.5, causal=True,
                   **({"mask": m_bhsd} if kind == "bool" else {"additive": m_bhsd}))
    t = (lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))) if layout == AxesLayout.BSHD else (lambda a: a)
    host = lambda a: synth.to_bf16_bits(a) if dt == BF16 else (a.astype(np.float16) if dt == dtypes.Float16 else a)  # noqa: E731
    mt = t(m_bhsd)
    mdt = dtypes.Bool if kind == "bool" else dt
    mh = mt.astype(np.bool_) if kind == "bool" else host(mt)
    b = be.Builder("sdpa_mask")
    f = b.Main()
    ps = [f.Parameter(f"p{i}", make_shape(dt, *t(a).shape)) for i, a in enumerate((q, k, v))]
    pm = f.Parameter("m", make_shape(mdt, *mt.shape))
    f.Return([f.FusedScaledDotProductAttention(*ps, pm, H, Hkv, layout, D ** -0.5, True)])
    ex = b.Compile()
    plan = ex.Plan()
    fused = (D % 8 == 0 and D <= 256) if dt != F32 else (D % 4 == 0 and D <= 128)
    assert ("fused attention" in plan) == fused, plan
    bufs = [be.BufferFromFlatData(0, host(t(a)), make_shape(dt, *t(a).shape)) for a in (q, k, v)]
    bufs.append(be.BufferFromFlatData(0, mh, make_shape(mdt, *mt.shape)))
    (r,) = ex.Execute(bufs, None, 0)
    y = be.BufferToFlatData(r).reshape(be.BufferShape(r).dims)
    y = synth.bf16_bits_to_f32(y) if dt == BF16 else y.astype(np.float32)
    if layout == AxesLayout.BSHD:
        y = y.transpose(0, 2, 1, 3)
    # fp32: scores and probabilities in fp32; 16-bit: P and the output rounded
    assert norm_err(y, ref) <= (1e-4 if dt == F32 else 1e-2)
    ex.Finalize()
    # a key-padding mask [B, 1, 1, Sk] (rank 4 in BHSD, where BSHD and BHSD agree)
    if layout == AxesLayout.BHSD and kind == "bool":
        kp = np.ones((B, 1, 1, Sk), bool)
        kp[0, ..., 100:] = False
        ref = orc.sdpa(q, k, v, scale=D ** -0.5, causal=False, mask=kp)
        (y,) = run(be, lambda f, qq, kk, vv, mm: [f.FusedScaledDotProductAttention(qq, kk, vv, mm, H, Hkv, layout,
                                                                                    D ** -0.5, False)],
                   [(host(q), make_shape(dt, *q.shape)), (host(k), make_shape(dt, *k.shape)),
                    (host(v), make_shape(dt, *v.shape)), (kp, make_shape(dtypes.Bool, B, 1, 1, Sk))])
        assert norm_err(np.asarray(y, np.float32), ref) <= (1e-4 if dt == F32 else 1e-2)


def test_graph_sdpa_mask_shape_errors(be):
    b = be.Builder("sdpa_bad_mask")
    f = b.Main()
    q = f.Parameter("q", make_shape(BF16, 1, 2, 8, 64))
    with pytest.raises(BackendError, match="does not broadcast"):
        f.FusedScaledDotProductAttention(q, q, q, f.Parameter("m", make_shape(dtypes.Bool, 3, 8)), 2, 2,
                                         AxesLayout.BHSD, 0.1, False)
    with pytest.raises(BackendError, match="bool or additive"):
        f.FusedScaledDotProductAttention(q, q, q, f.Parameter("m2", make_shape(F32, 8, 8)), 2, 2,
                                         AxesLayout.BHSD, 0.1, False)


def test_graph_elementwise_semantics(be):
    x = np.array([-2.5, -0.5, 0.5, 1.5, 2.5, np.nan, np.inf, -np.inf], np.float32)
    s = make_shape(F32, 8)
    outs = run(be, lambda f, a: [f.Round(a), f.Sign(a), f.Floor(a), f.IsNaN(a), f.IsFinite(a),
                                 f.ConvertDType(a, I32)], [(x, s)])
    assert np.array_equal(outs[0], np.rint(x), equal_nan=True)
    assert np.array_equal(outs[1], np.sign(x), equal_nan=True)
    assert np.array_equal(outs[2], np.floor(x), equal_nan=True)
    assert outs[3].astype(bool).tolist() == np.isnan(x).tolist()
    assert outs[4].astype(bool).tolist() == np.isfinite(x).tolist()
    assert outs[5].tolist() == [-2, 0, 0, 1, 2, 0, 2147483647, -2147483648]
    i = np.array([7, -7, 7, -7, 5], np.int32)
    j = np.array([2, 2, -2, -2, 0], np.int32)
    d, r, sh = run(be, lambda f, a, b: [f.Div(a, b), f.Rem(a, b), f.ShiftRightLogical(a, f.Abs(b))],
                   [(i, make_shape(I32, 5)), (j, make_shape(I32, 5))])
    assert d.tolist() == [3, -3, -3, 3, -1]          # truncating division; x/0 = -1
    assert r.tolist() == [1, -1, 1, -1, 5]           # sign of the dividend; x%0 = x
    assert sh.tolist() == [1, (np.uint32(-7 & 0xFFFFFFFF) >> 2).astype(np.int32), 1,
                           (np.uint32(-7 & 0xFFFFFFFF) >> 2).astype(np.int32), 5]


def test_execute_errors(be):                                      # executable.go:54-68
    b = be.Builder("err")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 3))
    f.Return([f.Exp(x)])
    ex = b.Compile()
    with pytest.raises(BackendError, match="expected 1 inputs"):
        ex.Execute([], None, 0)
    bad = be.BufferFromFlatData(0, np.zeros(4, np.float32), make_shape(F32, 4))
    with pytest.raises(BackendError, match="shape mismatch"):
        ex.Execute([bad], None, 0)


def test_bf16_rounding_all_upper_halves(be):
    """fp32 -> bf16 in generated kernels (gfx950 v_cvt_pk_bf16_f32) against the
    oracle's integer round-to-nearest-even: every one of the 2^16 upper halves
    (all signs, exponents, mantissa tops: zeros, denormals, carries into the
    exponent, overflow to inf, every NaN payload) with lower halves that are
    exact, below / at / above the tie, and odd/even-tie cases, bit for bit."""
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lo = np.array([0, 1, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xFFFF, 0x4000, 0xC000, 0x0002, 0x7FFE,
                   0x1234, 0x9ABC, 0x5555, 0xAAAA], np.uint32)
    u = (hi[:, None] | lo[None, :]).reshape(-1)
    x = u.view(np.float32)
    s = make_shape(F32, x.size)
    (y,) = run(be, lambda f, a: [f.ConvertDType(a, BF16)], [(x, s)])
    want = orc.f32_to_bf16_bits(x)
    got = synth.to_bf16_bits(y)  # y holds the bf16 values widened exactly to fp32
    assert np.array_equal(got, want)


# ------------------------------------------------------------ transformer block
def _bf(a):
    return synth.round_bf16(np.asarray(a, np.float32))


def _tb_reference(cfg, P, emulate_bf16=True):
    """Block forward composed from oracle primitives in fp64; with emulate_bf16
    every op output the graph holds in bf16 is rounded to bf16 (the graph's
    semantics), with the fused RMSNorm / attention softmax rounded once."""
    r = _bf if emulate_bf16 else (lambda a: np.asarray(a, np.float64))
    B, S, d, H, Dh = cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.head_dim
    x = orc.gather_rows(P["embedding"], P["ids"].reshape(-1)).reshape(B, S, d).astype(np.float64)
    h = r(orc.rmsnorm(x.astype(np.float32), P["g_attn"], cfg.eps))
    def proj(a, w):
        return r(orc.dot_general(np.asarray(a, np.float32), [a.ndim - 1], [], w, [0], []))
    q, k, v = (proj(h, P[w]).reshape(B, S, H, Dh).transpose(0, 2, 1, 3) for w in ("wq", "wk", "wv"))
    if emulate_bf16:
        s = r(orc.dot_general(np.ascontiguousarray(q, np.float32), [3], [0, 1], np.ascontiguousarray(k, np.float32), [3], [0, 1]))
        p = orc.softmax(np.where(np.tril(np.ones((S, S), bool)), s * (Dh ** -0.5), -np.inf).astype(np.float32))
        a = r(orc.dot_general(r(p).astype(np.float32), [3], [0, 1], np.ascontiguousarray(v, np.float32), [2], [0, 1]))
    else:
        a = orc.sdpa(q, k, v, scale=Dh ** -0.5, causal=True)
    a = a.transpose(0, 2, 1, 3).reshape(B, S, d)
    x2 = r(x + proj(a, P["wo"]))
    h2 = r(orc.rmsnorm(np.asarray(x2, np.float32), P["g_ffn"], cfg.eps))
    gate, up = proj(h2, P["w_gate"]), proj(h2, P["w_up"])
    act = r(r(gate * r(1.0 / (1.0 + np.exp(-gate)))) * up)
    return r(x2 + proj(act, P["w_down"]))


def _tb_inputs(cfg, seed=5001):
    P = {"ids": synth.uniform_int(seed, (cfg.batch, cfg.seq), 0, cfg.vocab)}
    for i, (name, shape) in enumerate(cfg.param_shapes()[1:]):
        if name.startswith("g_"):
            P[name] = np.ones(shape.dims, np.float32)
        else:
            P[name] = _bf(synth.normal(seed + 1 + i, shape.dims, std=0.02))
    return P


def _tb_run(be, cfg, P):
    ex = graphs.transformer_block(be, cfg)
    bufs = [be.BufferFromFlatData(0, P[name], shape) for name, shape in cfg.param_shapes()]
    (out,) = ex.Execute(bufs, None, 0)
    y = synth.bf16_bits_to_f32(be.BufferToFlatData(out)).reshape(cfg.batch, cfg.seq, cfg.d_model)
    return ex, y


def _tb_stages(be, cfg, P):
    """Builds the block with every stage as an output (same ops as
    graphs.transformer_block) and returns {stage: GPU result}."""
    b = be.Builder("tb_stages")
    f = b.Main()
    V = {name: f.Parameter(name, shape) for name, shape in cfg.param_shapes()}
    B, S, d, H, Dh = cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.head_dim
    x = f.Gather(V["embedding"], f.Reshape(V["ids"], B, S, 1), 2, [2], [0], [0], [1, d], False)
    h = graphs.rms_norm(f, x, V["g_attn"], cfg.eps)
    q, k, v = (graphs.dense(f, h, V[w]) for w in ("wq", "wk", "wv"))
    a = f.FusedScaledDotProductAttention(f.Reshape(q, B, S, H, Dh), f.Reshape(k, B, S, H, Dh),
                                         f.Reshape(v, B, S, H, Dh), None, H, H, AxesLayout.BSHD,
                                         Dh ** -0.5, True)
    o = graphs.dense(f, f.Reshape(a, B, S, d), V["wo"])
    x2 = f.Add(x, o)
    h2 = graphs.rms_norm(f, x2, V["g_ffn"], cfg.eps)
    gate, up = graphs.dense(f, h2, V["w_gate"]), graphs.dense(f, h2, V["w_up"])
    act = f.Mul(f.Mul(gate, f.Logistic(gate)), up)
    out = f.Add(x2, graphs.dense(f, act, V["w_down"]))
    names = ["x", "h", "q", "k", "v", "a", "o", "x2", "h2", "gate", "up", "act", "out"]
    f.Return([x, h, q, k, v, a, o, x2, h2, gate, up, act, out])
    ex = b.Compile()
    bufs = [be.BufferFromFlatData(0, P[name], shape) for name, shape in cfg.param_shapes()]
    res = ex.Execute(bufs, None, 0)
    return {n: synth.bf16_bits_to_f32(be.BufferToFlatData(r)).reshape(be.BufferShape(r).dims)
            for n, r in zip(names, res)}


def test_transformer_block_small_stagewise(be):
    """Every stage of the block against the oracle, each fed the GPU's own bf16
    inputs to that stage (so one stage's rounding flips do not cascade): the
    fp64 oracle result rounded to bf16, i.e. the graph's per-op semantics."""
    cfg = graphs.TransformerBlockConfig(batch=2, seq=128, vocab=1000, d_model=256, heads=2, head_dim=128, ffn=1024)
    P = _tb_inputs(cfg)
    G = _tb_stages(be, cfg, P)
    B, S, d, H, Dh = cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.head_dim
    f32 = lambda a: np.asarray(a, np.float32)
    proj = lambda a, w: _bf(orc.dot_general(f32(a), [a.ndim - 1], [], P[w], [0], []))
    checks = {
        "x": orc.gather_rows(P["embedding"], P["ids"].reshape(-1)).reshape(B, S, d),
        "h": _bf(orc.rmsnorm(G["x"], P["g_attn"], cfg.eps)),
        "q": proj(G["h"], "wq"), "k": proj(G["h"], "wk"), "v": proj(G["h"], "wv"),
    }
    bhsd = lambda t: np.ascontiguousarray(t.reshape(B, S, H, Dh).transpose(0, 2, 1, 3), np.float32)
    q, k, v = bhsd(G["q"]), bhsd(G["k"]), bhsd(G["v"])
    # FusedScaledDotProductAttention lowers to one kernel that keeps the scores in
    # fp32 and rounds only P (before P.V) and the output: it is checked against
    # exact attention rounded once, with the fused kernel's bounds (below).
    checks["a"] = _bf(orc.sdpa(q, k, v, scale=Dh ** -0.5, causal=True)).transpose(0, 2, 1, 3)
    checks["o"] = proj(G["a"].reshape(B, S, d), "wo")
    checks["x2"] = _bf(G["x"].astype(np.float64) + G["o"])
    checks["h2"] = _bf(orc.rmsnorm(G["x2"], P["g_ffn"], cfg.eps))
    checks["gate"], checks["up"] = proj(G["h2"], "w_gate"), proj(G["h2"], "w_up")
    g = G["gate"].astype(np.float64)
    checks["act"] = _bf(_bf(g * _bf(1.0 / (1.0 + np.exp(-g)))) * G["up"])
    down = orc.dot_general(f32(G["act"]), [2], [], P["w_down"], [0], [])
    checks["out"] = _bf(G["x2"].astype(np.float64) + _bf(down))
    for name, want in checks.items():
        got = G[name]
        assert got.shape == want.shape, name
        if name == "a":
            # two bf16 roundings (P, output) of up to 2^-9 each
            assert rel_err(got, want) <= 2.5e-2, name
            assert norm_err(got, want) <= 1e-2, name
            continue
        if name == "out":
            # x2 + bf16(act . w_down): the GPU's fp32 sum order may round the
            # product the other way (one bf16 ulp of the product, <= 2^-7 |down|),
            # which cancellation against x2 can make large next to the result.
            err = np.abs(got.astype(np.float64) - want)
            assert np.all(err <= 2.0 ** -7 * (np.abs(want) + np.abs(down)) + 1e-30), name
            assert norm_err(got, want) <= 1e-3, name
            continue
        # bf16 results: isolated one-ulp rounding flips only
        assert rel_err(got, want) <= 2.0 ** -7, name
        assert norm_err(got, want) <= 1e-3, name
    # end to end against fp64 truth (no intermediate rounding)
    exact = _tb_reference(cfg, P, emulate_bf16=False)
    assert norm_err(G["out"], exact) <= 1e-2


def _tb_reference_tokens(cfg, P, b, toks):
    """fp64 block output at tokens `toks` of batch row b (the oracle's composition
    of the block; token t sees keys 0..t)."""
    return orc.block_tokens(P, b, toks, cfg.d_model, cfg.heads, cfg.head_dim, cfg.eps)[0]


def test_transformer_block_config_sampled(be):
    """BASELINE configs[4] end to end (ids [8,1024], d_model 2048, 16 heads,
    FFN 8192), checked against the fp64 oracle composition on 12 tokens of every
    one of the 8 batch rows (first, last and seeded positions in between)."""
    cfg = graphs.TransformerBlockConfig()
    P = _tb_inputs(cfg)
    ex, y = _tb_run(be, cfg, P)
    assert np.all(np.isfinite(y))
    for b in range(cfg.batch):
        mid = synth.uniform_int(5100 + b, (10,), 1, cfg.seq - 1)
        toks = sorted({0, cfg.seq - 1, *map(int, mid)})
        exact = _tb_reference_tokens(cfg, P, b, toks)
        assert norm_err(y[b, toks], exact) <= 1e-2, (b, toks)


def test_reshape_of_strided_views(be):
    """Reshapes of reversed, transposed and broadcast views (zero-copy where the
    stride runs allow it, one copy otherwise) give numpy's results."""
    x = np.arange(24, dtype=np.float32).reshape(6, 4) * 0.5 - 3
    (a, b, c) = run(be, lambda f, p: [f.ReduceSum(f.Reshape(f.Reverse(p, 0), 2, 3, 4), 0),
                                      f.Add(f.Reshape(f.Transpose(p, 1, 0), 24), f.Reshape(p, 24)),
                                      f.Mul(f.Reshape(f.BroadcastInDim(f.Reshape(f.Slice(p, [0, 1], [6, 2]), 6), make_shape(F32, 2, 6, 3), [1]), 4, 9),
                                            f.Reshape(f.BroadcastInDim(f.Slice(p, [0, 0], [6, 3]), make_shape(F32, 2, 6, 3), [1, 2]), 4, 9))],
                    [(x, make_shape(F32, 6, 4))])
    assert np.array_equal(a, x[::-1].reshape(2, 3, 4).sum(0))
    assert np.array_equal(b, x.T.reshape(24) + x.reshape(24))
    want = (np.broadcast_to(x[:, 1][None, :, None], (2, 6, 3)) * np.broadcast_to(x[None, :, :3], (2, 6, 3))).reshape(4, 9)
    assert np.array_equal(c, want)


def test_pad_known_answer(be, known):                             # :876-939
    k = known["pad"]
    (y,) = run(be, lambda f, x: [f.Pad(x, f.Constant(np.float32(k["fill"])),
                                       *zip(k["start"], k["end"]))],
               [(np.array(k["x"], np.float32), make_shape(F32, *k["shape"]))])
    assert list(y.shape) == k["expected_shape"]
    assert y.reshape(-1).tolist() == k["expected"]


@pytest.mark.parametrize("dt", [F32, BF16, I32, dtypes.Uint8])
def test_pad_crop_vs_numpy(be, dt):
    """Edge padding with a non-zero fill on several axes at once, negative
    padding cropping (XLA semantics), bit-exact against numpy.pad."""
    rng = np.random.default_rng(11)
    x = rng.integers(0, 100, (3, 5, 4)).astype(np.float32)
    cfg = [(1, 2), (0, 0), (-1, 3)]
    want = np.pad(x[:, :, 1:], [(1, 2), (0, 0), (0, 3)], constant_values=7)
    host = x if dt in (F32, BF16) else x.astype(np.int32 if dt == I32 else np.uint8)
    fill = np.array(7, host.dtype)
    (y,) = run(be, lambda f, p: [f.Pad(p, f.Constant(fill) if dt != BF16 else
                                       f.ConvertDType(f.Constant(np.float32(7)), BF16), *cfg)],
               [(host, make_shape(dt, 3, 5, 4))])
    assert y.shape == want.shape and np.array_equal(y.astype(np.float32), want)


def test_pad_errors(be):
    b = be.Builder("pad_err")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 2, 3))
    z = f.Constant(np.float32(0))
    with pytest.raises(BackendError, match="interior padding not supported"):
        f.Pad(x, z, (0, 0, 1), (0, 0))
    with pytest.raises(BackendError, match="scalar"):
        f.Pad(x, f.Constant(np.zeros(2, np.float32), 2), (0, 0), (0, 0))
    with pytest.raises(BackendError, match="crops more than"):
        f.Pad(x, z, (0, 0), (-2, -2))
    b.Finalize()


def test_reduce_logical_and_or(be):                               # function.go:2262-2270
    rng = np.random.default_rng(12)
    x = rng.random((4, 5, 6)) < 0.8
    x[0, :, 0] = True          # a column that is all true
    x[1, :, 1] = False         # and one that is all false
    s = make_shape(dtypes.Bool, 4, 5, 6)
    outs = run(be, lambda f, p: [f.ReduceLogicalAnd(p, 1), f.ReduceLogicalOr(p, 1),
                                 f.ReduceLogicalAnd(p, 0, 2), f.ReduceLogicalOr(p), f.ReduceLogicalAnd(p)],
               [(x, s)])
    wants = [x.all(1), x.any(1), x.all((0, 2)), x.any(), x.all()]
    for got, want in zip(outs, wants):
        assert got.dtype == np.bool_ and np.array_equal(got, want)


def test_total_order_comparisons_follow_plain_ones(be):           # function.go:2227-2256
    s = make_shape(F32, 6)
    l = np.array([1, 2, 3, -0.0, -np.inf, 5], np.float32)
    r = np.array([2, 2, 2, 0.0, -np.inf, -1], np.float32)
    outs = run(be, lambda f, a, b: [f.EqualTotalOrder(a, b), f.NotEqualTotalOrder(a, b),
                                    f.GreaterThanTotalOrder(a, b), f.GreaterOrEqualTotalOrder(a, b),
                                    f.LessThanTotalOrder(a, b), f.LessOrEqualTotalOrder(a, b)],
               [(l, s), (r, s)])
    for got, want in zip(outs, [l == r, l != r, l > r, l >= r, l < r, l <= r]):
        assert got.astype(bool).tolist() == want.tolist()


def test_layer_norm_gradient_known_answer(be):                    # :2625-2642
    """d/dx sum(LayerNorm(x)) for x = [1, 2, 3, 4] (no gamma / beta) is ~0: the
    reference's check, here on the backward chain of primitive ops a graph layer
    emits for it (mean, centre, variance, rsqrt and their adjoints)."""
    n, eps = 4, 1e-5

    def build(f, x):
        K = lambda v: f.Constant(np.float32(v))
        bc = lambda v: f.BroadcastInDim(v, make_shape(F32, 1, n), [0])
        mean = f.Div(f.ReduceSum(x, 1), K(n))
        d = f.Sub(x, bc(mean))
        var = f.Div(f.ReduceSum(f.Mul(d, d), 1), K(n))
        rstd = f.Rsqrt(f.Add(var, K(eps)))
        dy = f.BroadcastInDim(K(1.0), make_shape(F32, 1, n), [])
        g_rstd = f.ReduceSum(f.Mul(dy, d), 1)
        g_var = f.Mul(f.Mul(g_rstd, K(-0.5)), f.Mul(rstd, f.Mul(rstd, rstd)))
        g_d = f.Add(f.Mul(dy, bc(rstd)), f.Mul(f.Mul(d, K(2.0 / n)), bc(g_var)))
        g_x = f.Sub(g_d, bc(f.Div(f.ReduceSum(g_d, 1), K(n))))
        normed = f.Mul(d, bc(rstd))
        return [g_x, normed]

    g, y = run(be, build, [(np.array([[1, 2, 3, 4]], np.float32), make_shape(F32, 1, n))])
    close(y, [-1.3416, -0.4472, 0.4472, 1.3416], 1e-3)
    assert np.max(np.abs(g)) <= 1e-4


def test_gomlx_graph_layer_cases(be):                             # :1955-2060
    """The reference's GoMLX-level tests, as the backend ops the graph layer emits
    for them (Ones / ZerosLike: constant + broadcast; ExpandDims: reshape;
    Gather: the XLA gather of an embedding lookup)."""
    s3 = make_shape(F32, 3)
    (y,) = run(be, lambda f, a, b: [f.Add(a, b)],
               [(np.array([1, 2, 3], np.float32), s3), (np.array([10, 20, 30], np.float32), s3)])
    close(y, [11, 22, 33], 1e-5)                                  # TestGoMLXAdd
    (y,) = run(be, lambda f, x: [f.Exp(f.Add(f.Log(x), f.BroadcastInDim(f.Constant(np.float32(1)), s3, [])))],
               [(np.array([1, 2, 4], np.float32), s3)])
    close(y, [math.e, 2 * math.e, 4 * math.e], 1e-4)              # TestGoMLXMathChain
    m = np.arange(1, 7, dtype=np.float32)
    (y,) = run(be, lambda f, a, b: [f.DotGeneral(a, [1], [], b, [0], [])],
               [(m, make_shape(F32, 2, 3)), (m, make_shape(F32, 3, 2))])
    close(y, [22, 28, 49, 64], 1e-4)                              # TestGoMLXMatMul
    (y,) = run(be, lambda f, x: [f.Sub(x, f.BroadcastInDim(
        f.Reshape(f.Div(f.ReduceSum(x, 1), f.Constant(np.float32(3))), 2, 1), make_shape(F32, 2, 3), [0, 1]))],
               [(m, make_shape(F32, 2, 3))])
    close(y, [-1, 0, 1, -1, 0, 1], 1e-4)                          # TestGoMLXReduceAndBroadcast
    table = np.array([10, 11, 12, 20, 21, 22, 30, 31, 32, 40, 41, 42], np.float32)
    (y,) = run(be, lambda f, t, i: [f.Gather(t, i, 1, [1], [0], [0], [1, 3], False)],
               [(table, make_shape(F32, 4, 3)), (np.array([1, 3], np.int32), make_shape(I32, 2, 1))])
    close(y, [20, 21, 22, 40, 41, 42], 0)                         # TestGoMLXGatherAndSlice
    s5 = make_shape(F32, 5)

    def relu(f, x):
        zero = f.BroadcastInDim(f.Constant(np.float32(0)), s5, [])
        return [f.Where(f.GreaterThan(x, zero), x, zero)]
    (y,) = run(be, relu, [(np.array([-2, -1, 0, 1, 2], np.float32), s5)])
    close(y, [0, 0, 0, 1, 2], 1e-5)                               # TestGoMLXWhereAndCompare


def test_pad_crop_whole_axis_then_pad_back(be):
    """An axis cropped to nothing and padded back: the empty intermediate slice
    takes no copy, the output is all fill."""
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    (y,) = run(be, lambda f, p: [f.Pad(p, f.Constant(np.float32(5)), (0, 0), (-3, 2))],
               [(x, make_shape(F32, 2, 3))])
    assert y.shape == (2, 2) and np.all(y == 5)
