"""Call / While / If and closures with captured values on the GPU, against the
reference's known answers (mpsgraph_test.go:3376-3588: sum 1..10 = 55, 5! = 120,
If(10 > 5) = 1, If(3 > 5) = -1, the captured 3 * 10 = 30, Call(10 + 32) = 42) and
numpy on tensor-valued loops, nested closures and calls."""
import numpy as np
import pytest

from gomlx_hip import synth
from gomlx_hip.backend import Backend, BackendError, dtypes, make_shape
from oracle import oracle as orc
from conftest import rel_err

pytestmark = pytest.mark.gpu

F32, I32, BF16 = dtypes.Float32, dtypes.Int32, dtypes.BFloat16


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def run(be, build, inputs):
    b = be.Builder("cf")
    f = b.Main()
    params = [f.Parameter(f"p{i}", s) for i, (_, s) in enumerate(inputs)]
    f.Return(build(b, f, *params))
    ex = b.Compile()
    bufs = [be.BufferFromFlatData(0, np.ascontiguousarray(a), s) for a, s in inputs]
    outs = [be.BufferToFlatData(r).reshape(be.BufferShape(r).dims).copy() for r in ex.Execute(bufs, None, 0)]
    plan = ex.Plan()
    ex.Finalize()
    return plan, outs


def i32(v):
    return np.array(v, np.int32)


def test_while_sum_and_factorial(be):                            # mpsgraph_test.go:3376-3443
    def sum_1_to_10(b, f, _):
        cond = f.Closure()
        counter = cond.Parameter("counter", make_shape(I32))
        cond.Parameter("sum", make_shape(I32))
        cond.Return([cond.LessOrEqual(counter, cond.Constant(i32(10)))])
        body = f.Closure()
        c, s = body.Parameter("counter", make_shape(I32)), body.Parameter("sum", make_shape(I32))
        body.Return([body.Add(c, body.Constant(i32(1))), body.Add(s, c)])
        return [f.While(cond, body, f.Constant(i32(1)), f.Constant(i32(0)))[1]]

    def factorial(b, f, _):
        cond = f.Closure()
        n = cond.Parameter("n", make_shape(I32))
        cond.Parameter("result", make_shape(I32))
        cond.Return([cond.GreaterThan(n, cond.Constant(i32(1)))])
        body = f.Closure()
        n, r = body.Parameter("n", make_shape(I32)), body.Parameter("result", make_shape(I32))
        body.Return([body.Sub(n, body.Constant(i32(1))), body.Mul(r, n)])
        return [f.While(cond, body, f.Constant(i32(5)), f.Constant(i32(1)))[1]]

    plan, (y,) = run(be, sum_1_to_10, [(i32(0), make_shape(I32))])
    assert int(y) == 55 and "while" in plan
    _, (y,) = run(be, factorial, [(i32(0), make_shape(I32))])
    assert int(y) == 120


@pytest.mark.parametrize("x, want", [(10.0, 1.0), (3.0, -1.0)])
def test_if_branches(be, x, want):                                # mpsgraph_test.go:3446-3490
    def build(b, f, xx):
        pred = f.GreaterThan(xx, f.Constant(np.array(5, np.float32)))
        t = f.Closure()
        t.Return([t.Constant(np.array(1, np.float32))])
        e = f.Closure()
        e.Return([e.Constant(np.array(-1, np.float32))])
        return f.If(pred, t, e)
    _, (y,) = run(be, build, [(np.array(x, np.float32), make_shape(F32))])
    assert float(y) == want


@pytest.mark.parametrize("x", [3.0, -2.0])
def test_if_with_captured_values(be, x):                          # mpsgraph_test.go:3492-3523
    def build(b, f, xx):
        factor = f.Constant(np.array(10, np.float32))
        pred = f.GreaterThan(xx, f.Constant(np.array(0, np.float32)))
        t = f.Closure()
        t.Return([t.Mul(xx, factor)])
        e = f.Closure()
        e.Return([e.Neg(e.Mul(xx, factor))])
        return f.If(pred, t, e)
    _, (y,) = run(be, build, [(np.array(x, np.float32), make_shape(F32))])
    assert float(y) == (30.0 if x > 0 else -(x * 10))


def test_call_named_function(be):                                 # mpsgraph_test.go:3553-3588
    def build(b, f, _):
        add = b.NewFunction("add")
        a, c = add.Parameter("a", make_shape(F32)), add.Parameter("b", make_shape(F32))
        add.Return([add.Add(a, c)])
        return f.Call(add, f.Constant(np.array(10, np.float32)), f.Constant(np.array(32, np.float32)))
    _, (y,) = run(be, build, [(np.array(0, np.float32), make_shape(F32))])
    assert float(y) == 42.0


@pytest.mark.parametrize("limit", [0, 1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 100])
def test_while_trip_counts_across_speculative_batches(be, limit):
    """While runs cond and body in speculative batches (1, 2, 4, 8, 8, ...
    iterations) and keeps the state before the first false predicate: every trip
    count, including 0 and counts on either side of a batch boundary, gives
    exactly the sequential loop's state (a counter, a running sum and a product
    that any extra iteration would change)."""
    def build(b, f, lim):
        cond = f.Closure()
        c = cond.Parameter("c", make_shape(I32))
        cond.Parameter("s", make_shape(I32))
        cond.Parameter("p", make_shape(F32))
        cond.Return([cond.LessThan(c, lim)])  # lim: a captured value of the enclosing function
        body = f.Closure()
        c, s2, pr = (body.Parameter("c", make_shape(I32)), body.Parameter("s", make_shape(I32)),
                     body.Parameter("p", make_shape(F32)))
        body.Return([body.Add(c, body.Constant(i32(1))), body.Add(s2, body.Mul(c, c)),
                     body.Mul(pr, body.Constant(np.array(1.5, np.float32)))])
        return list(f.While(cond, body, f.Constant(i32(0)), f.Constant(i32(0)),
                            f.Constant(np.array(1.0, np.float32))))
    _, outs = run(be, build, [(i32(limit), make_shape(I32))])
    assert int(outs[0]) == limit
    assert int(outs[1]) == sum(i * i for i in range(limit))
    p = np.float32(1.0)
    for _ in range(limit):
        p = np.float32(p * np.float32(1.5))
    assert outs[2].reshape(()) == p


def test_while_large_state_uses_a_smaller_batch_ring(be):
    """A state too large for eight speculative copies within the ring's byte budget
    runs with a smaller batch and the same result."""
    n = 40 * (1 << 20) // 4  # 40 MiB of float32 state: 9 copies exceed the 256 MiB budget
    def build(b, f, x):
        cond = f.Closure()
        k = cond.Parameter("k", make_shape(I32))
        cond.Parameter("v", make_shape(F32, n))
        cond.Return([cond.LessThan(k, cond.Constant(i32(11)))])
        body = f.Closure()
        k, v = body.Parameter("k", make_shape(I32)), body.Parameter("v", make_shape(F32, n))
        body.Return([body.Add(k, body.Constant(i32(1))),
                     body.Add(v, body.BroadcastInDim(body.ConvertDType(k, F32), make_shape(F32, n), []))])
        return [f.While(cond, body, f.Constant(i32(0)), x)[1]]
    x = synth.normal(77, (n,))
    plan, outs = run(be, build, [(x, make_shape(F32, n))])
    assert "speculative batches of up to 4 iterations" in plan, plan
    want = x.astype(np.float64) + sum(range(11))
    assert np.max(np.abs(outs[0] - want)) <= 1e-4


def test_while_tensor_state_with_captures(be):
    """A loop over tensors: x <- W x / ||W x||_inf ... run k times (power iteration with
    a captured matrix and iteration count), against numpy with the same fp32 steps."""
    rng = np.random.default_rng(3)
    n, k = 96, 7
    W = rng.standard_normal((n, n)).astype(np.float32)
    x0 = rng.standard_normal((n, 1)).astype(np.float32)

    def build(b, f, w, x, kk):
        cond = f.Closure()
        i = cond.Parameter("i", make_shape(I32))
        cond.Parameter("x", make_shape(F32, n, 1))
        cond.Return([cond.LessThan(i, kk)])                      # captures kk
        body = f.Closure()
        i = body.Parameter("i", make_shape(I32))
        xv = body.Parameter("x", make_shape(F32, n, 1))
        y = body.DotGeneral(w, [1], [], xv, [0], [])            # captures W
        m = body.ReduceMax(body.Abs(y), 0, 1)
        body.Return([body.Add(i, body.Constant(i32(1))), body.Div(y, body.BroadcastInDim(m, make_shape(F32, n, 1), []))])
        out = f.While(cond, body, f.Constant(i32(0)), x)
        return [out[0], out[1]]

    plan, (it, xk) = run(be, build, [(W, make_shape(F32, n, n)), (x0, make_shape(F32, n, 1)), (i32(k), make_shape(I32))])
    assert int(it) == k
    want = x0.astype(np.float64)
    for _ in range(k):
        y = W.astype(np.float64) @ want
        want = y / np.max(np.abs(y))
    assert rel_err(xk, want) <= 1e-4


def test_nested_closures_and_calls(be):
    """If inside a While body, a Call inside the If branch, and a value captured from
    the main function two levels up (the closures in between capture it too)."""
    def build(b, f, x, lim):
        scale = b.NewFunction("scale")
        a, s = scale.Parameter("a", make_shape(F32, 4)), scale.Parameter("s", make_shape(F32))
        scale.Return([scale.Mul(a, scale.BroadcastInDim(s, make_shape(F32, 4), []))])
        two = f.Constant(np.array(2, np.float32))
        cond = f.Closure()
        v = cond.Parameter("v", make_shape(F32, 4))
        cond.Return([cond.LessThan(cond.ReduceSum(v, 0), lim)])      # captures lim
        body = f.Closure()
        v = body.Parameter("v", make_shape(F32, 4))
        big = body.GreaterThan(body.ReduceMax(v, 0), body.Constant(np.array(3, np.float32)))
        t = body.Closure()
        t.Return(t.Call(scale, v, two))                              # captures v (body) and two (main)
        e = body.Closure()
        e.Return([e.Add(v, e.Constant(np.ones(4, np.float32), 4))])
        body.Return(body.If(big, t, e))
        return f.While(cond, body, x)

    x0 = np.array([0.5, -1.0, 0.25, 1.0], np.float32)
    _, (y,) = run(be, build, [(x0, make_shape(F32, 4)), (np.array(100, np.float32), make_shape(F32))])
    want = x0.copy()
    while want.sum() < 100:
        want = want * 2 if want.max() > 3 else want + 1
    assert np.array_equal(y, want)


def test_while_with_nested_loop_runs_without_speculation(be):
    """An outer loop whose body runs an inner While that terminates for every state
    the sequential loop reaches (i = 0, 1, 2: count j up from i to 2) but not on the
    state after the exit (i = 3: j never equals 2, so the inner loop would hit the
    iteration limit).  The outer loop must not evaluate its body past the exit: the
    result is the sequential loop's, with no error."""
    def build(b, f, _):
        cond = f.Closure()
        i = cond.Parameter("i", make_shape(I32))
        cond.Parameter("total", make_shape(I32))
        cond.Return([cond.LessThan(i, cond.Constant(i32(3)))])
        body = f.Closure()
        i, tot = body.Parameter("i", make_shape(I32)), body.Parameter("total", make_shape(I32))
        icond = body.Closure()
        j = icond.Parameter("j", make_shape(I32))
        icond.Return([icond.NotEqual(j, icond.Constant(i32(2)))])
        ibody = body.Closure()
        j = ibody.Parameter("j", make_shape(I32))
        ibody.Return([ibody.Add(j, ibody.Constant(i32(1)))])
        (jend,) = body.While(icond, ibody, i)
        body.Return([body.Add(i, body.Constant(i32(1))), body.Add(tot, jend)])
        return list(f.While(cond, body, f.Constant(i32(0)), f.Constant(i32(0))))

    plan, (i_end, total) = run(be, build, [(i32(0), make_shape(I32))])
    assert "no speculation" in plan, plan
    assert int(i_end) == 3 and int(total) == 6


def test_control_flow_errors(be):
    b = be.Builder("err")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 3))
    cond = f.Closure()
    cond.Parameter("v", make_shape(F32, 3))
    cond.Return([cond.Constant(np.array(1.0, np.float32))])
    body = f.Closure()
    v = body.Parameter("v", make_shape(F32, 3))
    body.Return([v])
    with pytest.raises(BackendError, match="cond must return scalar bool"):
        f.While(cond, body, x)
    unreturned = f.Closure()
    with pytest.raises(BackendError, match="must have Return"):
        f.If(f.Constant(np.array(True)), unreturned, unreturned)
    other = be.Builder("other").Main()
    with pytest.raises(BackendError, match="does not belong|does not enclose"):
        other.Add(x, x)
    b.Finalize()


# ------------------------------------------------------------ Sort
def _comparator(f, dtypes_, rule):
    """A comparator closure over len(dtypes_) inputs: rule(c, params) -> bool value."""
    c = f.Closure()
    ps = []
    for i, dt in enumerate(dtypes_):
        ps.append(c.Parameter(f"lhs{i}", make_shape(dt)))
        ps.append(c.Parameter(f"rhs{i}", make_shape(dt)))
    c.Return([rule(c, ps)])
    return c


@pytest.mark.parametrize("ascending", [True, False])
def test_sort_known_answers(be, known, ascending):                 # mpsgraph_test.go:3526-3551
    c = known["sort"]

    def build(b, f, x):
        rule = (lambda k, p: k.LessThan(p[0], p[1])) if ascending else (lambda k, p: k.GreaterThan(p[0], p[1]))
        return f.Sort(_comparator(f, [F32], rule), 0, True, x)
    plan, (y,) = run(be, build, [(np.array(c["x"], np.float32), make_shape(F32, 6))])
    assert "sort_rows" in plan
    assert y.tolist() == c["ascending" if ascending else "descending"]


def test_sort_payload_axis_and_stability(be):
    """Keys with many ties plus an int32 payload, sorted along the middle axis of
    [3, 700, 5] (rows strided by 5): equals numpy's stable argsort applied to both."""
    rng = np.random.default_rng(2)
    keys = rng.integers(0, 20, (3, 700, 5)).astype(np.float32)
    payload = np.broadcast_to(np.arange(700, dtype=np.int32)[None, :, None], (3, 700, 5)).copy()

    def build(b, f, k, p):
        return f.Sort(_comparator(f, [F32, I32], lambda c, q: c.LessThan(q[0], q[1])), 1, True, k, p)
    _, (ks, ps) = run(be, build, [(keys, make_shape(F32, 3, 700, 5)), (payload, make_shape(I32, 3, 700, 5))])
    order = np.argsort(keys, axis=1, kind="stable")
    assert np.array_equal(ks, np.take_along_axis(keys, order, 1))
    assert np.array_equal(ps, np.take_along_axis(payload, order, 1))


def test_sort_bf16_lexicographic_with_captured_scalar(be):
    """Two keys compared lexicographically (by |a - c|, c captured from the main
    function, then by b descending), bf16 and int32, rows of 4096 along the last axis."""
    rng = np.random.default_rng(4)
    a = synth.round_bf16(rng.standard_normal((2, 4096)).astype(np.float32))
    bk = rng.integers(0, 8, (2, 4096)).astype(np.int32)
    center = np.array(0.25, np.float32)

    def build(b, f, aa, bb, cc):
        def rule(c, q):
            da, db = c.Abs(c.Sub(q[0], c.ConvertDType(cc, BF16))), c.Abs(c.Sub(q[1], c.ConvertDType(cc, BF16)))
            first = c.LessThan(da, db)
            tie = c.Equal(da, db)
            return c.LogicalOr(first, c.LogicalAnd(tie, c.GreaterThan(q[2], q[3])))
        return f.Sort(_comparator(f, [BF16, I32], rule), -1, True, aa, bb)
    _, (ya, yb) = run(be, build, [(synth.to_bf16_bits(a), make_shape(BF16, 2, 4096)), (bk, make_shape(I32, 2, 4096)),
                                  (center, make_shape(F32))])
    d = np.abs(synth.round_bf16(a - synth.round_bf16(center)))
    for r in range(2):
        order = np.lexsort((np.arange(4096), -bk[r], d[r]))     # primary |a-c|, then b desc, then index
        assert np.array_equal(synth.bf16_bits_to_f32(ya[r]), a[r][order])
        assert np.array_equal(yb[r], bk[r][order])


def test_sort_rows_longer_than_lds(be):
    """Rows of 40000 keys (an index network of 65536: four 16384-index chunks sorted in
    LDS, then stages 32768 and 65536 with exchanges across chunks in global memory),
    keys with many ties plus an int32 payload: equal to numpy's stable argsort, both
    ascending along the last axis and descending along a strided middle axis."""
    rng = np.random.default_rng(21)
    L = 40000
    keys = rng.integers(0, 500, (3, L)).astype(np.float32)
    payload = np.broadcast_to(np.arange(L, dtype=np.int32)[None, :], (3, L)).copy()

    def build(b, f, k, p):
        return f.Sort(_comparator(f, [F32, I32], lambda c, q: c.LessThan(q[0], q[1])), 1, True, k, p)
    plan, (ks, ps) = run(be, build, [(keys, make_shape(F32, 3, L)), (payload, make_shape(I32, 3, L))])
    assert "sort_rows_global" in plan, plan
    order = np.argsort(keys, axis=1, kind="stable")
    assert np.array_equal(ks, np.take_along_axis(keys, order, 1))
    assert np.array_equal(ps, np.take_along_axis(payload, order, 1))

    x = rng.standard_normal((2, 20001, 3)).astype(np.float32)
    x[0, ::7, 1] = 0.5                      # a run of ties inside one strided row

    def build_desc(b, f, xx):
        return f.Sort(_comparator(f, [F32], lambda c, q: c.GreaterThan(q[0], q[1])), 1, True, xx)
    plan, (y,) = run(be, build_desc, [(x, make_shape(F32, 2, 20001, 3))])
    assert "sort_rows_global" in plan
    assert np.array_equal(y, np.take_along_axis(x, np.argsort(-x, axis=1, kind="stable"), 1))


def test_sort_wide_keys_take_the_global_path(be):
    """Three operands of 8000 (int64, int64, int32: 160 KB of keys per row) do not fit
    one workgroup's LDS with the index array; the global-memory network with a single
    LDS chunk sorts them lexicographically like numpy.lexsort (ties by index)."""
    rng = np.random.default_rng(22)
    a = rng.integers(-3, 3, (2, 8000)).astype(np.int64)
    bk = rng.integers(0, 1 << 40, (2, 8000)).astype(np.int64)
    c = np.broadcast_to(np.arange(8000, dtype=np.int32), (2, 8000)).copy()

    def build(b, f, aa, bb, cc):
        def rule(k, q):
            return k.LogicalOr(k.LessThan(q[0], q[1]), k.LogicalAnd(k.Equal(q[0], q[1]), k.LessThan(q[2], q[3])))
        return f.Sort(_comparator(f, [dtypes.Int64, dtypes.Int64, I32], rule), 1, True, aa, bb, cc)
    plan, (ya, yb, yc) = run(be, build, [(a, make_shape(dtypes.Int64, 2, 8000)), (bk, make_shape(dtypes.Int64, 2, 8000)),
                                         (c, make_shape(I32, 2, 8000))])
    assert "sort_rows_global" in plan, plan
    for r in range(2):
        order = np.lexsort((np.arange(8000), bk[r], a[r]))
        assert np.array_equal(ya[r], a[r][order]) and np.array_equal(yb[r], bk[r][order])
        assert np.array_equal(yc[r], c[r][order])


def test_sort_errors(be):
    b = be.Builder("se")
    f = b.Main()
    x = f.Parameter("x", make_shape(F32, 8))
    cmp = _comparator(f, [F32], lambda c, p: c.LessThan(p[0], p[1]))
    with pytest.raises(BackendError, match="comparator must have 4 parameters"):
        f.Sort(cmp, 0, True, x, x)
    with pytest.raises(BackendError, match="axis 1 out of range"):
        f.Sort(cmp, 1, True, x)
    b.Finalize()
