"""DynamicSlice, DynamicUpdateSlice and ScatterSum / ScatterMax / ScatterMin on
the GPU (function.go:1571-1621, gather.go:441-640), against the reference's known
answers (mpsgraph_test.go:993-1131, 1192-1262) and the CPU oracle.

Window copies are bit-exact for every dtype.  Scatter with integer data, with
max / min, and with integer-valued floats is exact; fp32 sums of arbitrary values
differ from the fp64 oracle only by the fp32 rounding of the atomics (any order);
bf16 sums accumulate in fp32 and round once, so they sit within one bf16 rounding
of the exact sum."""
import numpy as np
import pytest

from oracle import oracle as orc
from gomlx_hip import synth
from gomlx_hip.backend import Backend, dtypes, make_shape
from conftest import rel_err

pytestmark = pytest.mark.gpu

F32, BF16, I32, I64 = dtypes.Float32, dtypes.BFloat16, dtypes.Int32, dtypes.Int64
NP = {dtypes.Float32: np.float32, dtypes.Float64: np.float64, dtypes.Int32: np.int32, dtypes.Int64: np.int64,
      dtypes.Int8: np.int8, dtypes.Uint16: np.uint16, dtypes.Uint8: np.uint8, dtypes.Int16: np.int16,
      dtypes.Uint32: np.uint32, dtypes.Uint64: np.uint64, dtypes.BFloat16: np.uint16}


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def run(be, build, inputs):
    b = be.Builder("sc")
    f = b.Main()
    params = [f.Parameter(f"p{i}", s) for i, (_, s) in enumerate(inputs)]
    f.Return(build(f, *params))
    ex = b.Compile()
    plan = ex.Plan()
    bufs = [be.BufferFromFlatData(0, np.ascontiguousarray(a), s) for a, s in inputs]
    outs = [be.BufferToFlatData(r).reshape(be.BufferShape(r).dims).copy() for r in ex.Execute(bufs, None, 0)]
    ex.Finalize()
    return plan, outs


def scalar(v, dt=I32):
    return (np.array(v, NP[dt]), make_shape(dt))


# ------------------------------------------------------------ reference known answers
def test_dynamic_slice_known_answer(be, known):                  # mpsgraph_test.go:993-1062
    c = known["dynamic_slice"]
    _, (y,) = run(be, lambda f, x, s0, s1: [f.DynamicSlice(x, [s0, s1], c["sizes"])],
                  [(np.array(c["x"], np.float32), make_shape(F32, *c["shape"])), scalar(c["starts"][0]),
                   scalar(c["starts"][1])])
    assert y.reshape(-1).tolist() == c["expected"]


def test_dynamic_update_slice_known_answer(be, known):           # mpsgraph_test.go:1064-1131
    c = known["dynamic_update_slice"]
    _, (y,) = run(be, lambda f, x, u, s0, s1: [f.DynamicUpdateSlice(x, u, [s0, s1])],
                  [(np.array(c["x"], np.float32), make_shape(F32, *c["shape"])),
                   (np.array(c["update"], np.float32), make_shape(F32, *c["update_shape"])),
                   scalar(c["starts"][0]), scalar(c["starts"][1])])
    assert y.reshape(-1).tolist() == c["expected"]


def test_scatter_sum_known_answer(be, known):                    # mpsgraph_test.go:1192-1262
    c = known["scatter_sum"]
    _, (y,) = run(be, lambda f, o, i, u: [f.ScatterSum(o, i, u, c["index_vector_axis"], c["update_window_axes"],
                                                       c["inserted_window_axes"], c["scatter_axes_to_operand_axes"])],
                  [(np.array(c["operand"], np.float32), make_shape(F32, *c["operand_shape"])),
                   (np.array(c["indices"], np.int32), make_shape(I32, *c["indices_shape"])),
                   (np.array(c["updates"], np.float32), make_shape(F32, *c["updates_shape"]))])
    assert y.reshape(-1).tolist() == c["expected"]


# ------------------------------------------------------------ window copies, bit-exact
@pytest.mark.parametrize("dt", [dtypes.Float32, dtypes.BFloat16, dtypes.Int8, dtypes.Int64])
@pytest.mark.parametrize("starts", [(1, 2, 0), (3, -5, 9), (-1, 100, 2)])
def test_dynamic_slice_and_update_vs_oracle(be, dt, starts):
    rng = np.random.default_rng(abs(hash((dt, starts))) % 1000)
    shape, sizes = (5, 9, 7), (3, 4, 7)
    info = np.iinfo(NP[dt]) if dt not in (F32,) else None
    x = (rng.standard_normal(shape).astype(np.float32) if dt == F32
         else rng.integers(info.min, info.max, shape, dtype=NP[dt], endpoint=True))
    u = (rng.standard_normal(sizes).astype(np.float32) if dt == F32
         else rng.integers(info.min, info.max, sizes, dtype=NP[dt], endpoint=True))
    sdts = (I32, I64, dtypes.Int16)
    ins = [(x, make_shape(dt, *shape)), (u, make_shape(dt, *sizes))] + [scalar(s, sd) for s, sd in zip(starts, sdts)]
    # operand read through a transposed view, update through a reversed one
    build = lambda f, xx, uu, a, b, c: [
        f.DynamicSlice(xx, [a, b, c], sizes),
        f.DynamicUpdateSlice(xx, uu, [a, b, c]),
        f.DynamicSlice(f.Transpose(xx, 2, 0, 1), [c, a, b], (7, 3, 4)),
        f.DynamicUpdateSlice(xx, f.Reverse(uu, 1), [a, b, c])]
    _, (ys, yu, yt, yr) = run(be, build, ins)
    assert np.array_equal(ys, orc.dynamic_slice(x, starts, sizes))
    assert np.array_equal(yu, orc.dynamic_update_slice(x, u, starts))
    assert np.array_equal(yt, orc.dynamic_slice(np.ascontiguousarray(x.transpose(2, 0, 1)), (starts[2], starts[0], starts[1]), (7, 3, 4)))
    assert np.array_equal(yr, orc.dynamic_update_slice(x, np.ascontiguousarray(u[:, ::-1]), starts))


# ------------------------------------------------------------ scatter
def _emb_case(rng, V, D, n, dt):
    ids = rng.integers(-2, V + 2, n).astype(np.int32)      # duplicates and a few out of range
    if dt in (F32, BF16):
        op = rng.standard_normal((V, D)).astype(np.float32)
        up = rng.standard_normal((n, D)).astype(np.float32)
        if dt == BF16:
            op, up = synth.round_bf16(op), synth.round_bf16(up)
    else:
        info = np.iinfo(NP[dt])
        lo, hi = max(info.min, -100), min(info.max, 100)
        op = rng.integers(lo, hi, (V, D)).astype(NP[dt])
        up = rng.integers(lo, hi, (n, D)).astype(NP[dt])
    return ids, op, up


def _raw(a, dt):
    return synth.to_bf16_bits(a) if dt == BF16 else a


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("dt", [F32, BF16, I32, dtypes.Int8, dtypes.Uint16, I64])
def test_scatter_embedding_gradient_vs_oracle(be, dt, mode):
    rng = np.random.default_rng(100 + 3 * mode + dt)
    V, D, n = 300, 72, 1000
    ids, op, up = _emb_case(rng, V, D, n, dt)
    fn = [lambda f: f.ScatterSum, lambda f: f.ScatterMax, lambda f: f.ScatterMin][mode]
    plan, (y,) = run(be, lambda f, o, i, u: [fn(f)(o, i, u, 1, [1], [0], [0])],
                     [(_raw(op, dt), make_shape(dt, V, D)), (ids.reshape(n, 1), make_shape(I32, n, 1)),
                      (_raw(up, dt), make_shape(dt, n, D))])
    ref = orc.scatter(mode, op.astype(np.float64), ids.reshape(n, 1), up.astype(np.float64), 1, [1], [0], [0])
    if mode == 0 and dt in (F32, BF16):
        # sorted-row path: each row's updates folded in their original order in fp32 and
        # rounded once -- exactly numpy's sequential float32 add.at, then one rounding
        assert "scatter_rows_sum" in plan, plan
        acc = op.astype(np.float32).copy()
        ok = (ids >= 0) & (ids < V)
        np.add.at(acc, ids[ok], up.astype(np.float32)[ok])
        want = synth.to_bf16_bits(acc) if dt == BF16 else acc
        assert np.array_equal(y, want)
    if dt == BF16:
        got = synth.bf16_bits_to_f32(y)
        if mode == 0:
            # one rounding of an fp32 sum: within 2^-8 relative of the exact sum (RMS floor)
            assert rel_err(got, ref) <= 2.0 ** -8
        else:
            assert np.array_equal(got, ref.astype(np.float32))
    elif dt == F32:
        if mode == 0:
            assert rel_err(y, ref) <= 1e-5
        else:
            assert np.array_equal(y, ref.astype(np.float32))
    else:
        want = ref.astype(np.int64)
        if mode == 0:   # integer sums wrap like Go's fixed-width integers
            want = want.astype(NP[dt])
        assert np.array_equal(y, want.astype(NP[dt]))


def test_scatter_general_multi_axis_exact(be):
    """Index vectors along axis 0 of [2, 3, 4] indices, two scatter axes, an inserted
    operand axis and window dims interleaved with scatter dims in the updates."""
    rng = np.random.default_rng(11)
    op = rng.integers(-5, 5, (6, 4, 5)).astype(np.float64)
    idx = np.stack([rng.integers(-1, 5, (3, 4)), rng.integers(0, 6, (3, 4))]).astype(np.int64)
    upd = rng.integers(-9, 9, (3, 2, 4, 2)).astype(np.float64)
    args = (0, [1, 3], [0], [2, 0])
    for mode, name in enumerate(("ScatterSum", "ScatterMax", "ScatterMin")):
        _, (y,) = run(be, lambda f, o, i, u: [getattr(f, name)(o, i, u, *args)],
                      [(op, make_shape(dtypes.Float64, 6, 4, 5)), (idx, make_shape(I64, 2, 3, 4)),
                       (upd, make_shape(dtypes.Float64, 3, 2, 4, 2))])
        assert np.array_equal(y, orc.scatter(mode, op, idx, upd, *args)), name


def test_scatter_rows_batched_ids_and_atomic_fallback(be):
    """Ids [B, S] with updates [B, S, D] (the batched embedding-gradient form) take the
    sorted-row path; more rows than one sort holds fall back to atomics."""
    rng = np.random.default_rng(9)
    V, D = 500, 40
    for B, S, path in ((4, 300, "scatter_rows_sum"), (3, 6000, "scatter_sum")):
        ids = rng.integers(0, V, (B, S)).astype(np.int64)
        op = rng.standard_normal((V, D)).astype(np.float32)
        up = rng.standard_normal((B, S, D)).astype(np.float32)
        plan, (y,) = run(be, lambda f, o, i, u: [f.ScatterSum(o, i, u, 2, [2], [0], [0])],
                         [(op, make_shape(F32, V, D)), (ids, make_shape(I64, B, S)), (up, make_shape(F32, B, S, D))])
        assert path in plan, plan
        ref = orc.scatter(0, op, ids, up, 2, [2], [0], [0])
        assert rel_err(y, ref) <= 1e-5
        if path == "scatter_rows_sum":
            acc = op.copy()
            np.add.at(acc, ids.reshape(-1), up.reshape(-1, D))
            assert np.array_equal(y, acc)


def test_scatter_embedding_gradient_large_bf16(be):
    """The embedding-gradient shape of a transformer: 4096 token rows of width 1024
    into an 8000-row table (many duplicate ids)."""
    rng = np.random.default_rng(5)
    V, D, n = 8000, 1024, 4096
    ids = rng.integers(0, 600, n).astype(np.int32)          # heavy duplication: ~7 updates per row
    op = synth.round_bf16(rng.standard_normal((V, D)).astype(np.float32))
    up = synth.round_bf16(rng.standard_normal((n, D)).astype(np.float32))
    _, (y,) = run(be, lambda f, o, i, u: [f.ScatterSum(o, i, u, 1, [1], [0], [0])],
                  [(synth.to_bf16_bits(op), make_shape(BF16, V, D)), (ids, make_shape(I32, n)),
                   (synth.to_bf16_bits(up), make_shape(BF16, n, D))])
    ref = orc.scatter(0, op, ids, up, 1, [1], [0], [0])
    assert rel_err(synth.bf16_bits_to_f32(y), ref) <= 2.0 ** -8
