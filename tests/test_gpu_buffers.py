"""Buffer lifecycle on the GPU (executable.go:50 donate, buffer.go BufferFinalize):
donated inputs reused for outputs when the plan allows it, refused when it does
not, and many Executes / finalizes in a row with no host synchronisation, checked
against numpy closed forms."""
import numpy as np
import pytest

from gomlx_hip import synth
from gomlx_hip.backend import Backend, BackendError, dtypes, make_shape

pytestmark = pytest.mark.gpu

F32 = dtypes.Float32


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def _compile(be, name, build, shapes):
    b = be.Builder(name)
    f = b.Main()
    ps = [f.Parameter(f"p{i}", s) for i, s in enumerate(shapes)]
    f.Return(build(f, *ps))
    return b.Compile()


def test_donated_input_becomes_the_output(be):
    """y = 0.5 x + 1 is one elementwise kernel that reads x at y's own indices:
    with x donated, y takes x's memory (same device pointer) and x is consumed."""
    s = make_shape(F32, 1024, 333)
    ex = _compile(be, "affine", lambda f, x: [f.Add(f.Mul(x, f.Constant(np.float32(0.5))), f.Constant(np.float32(1)))],
                  [s])
    host = synth.normal(5101, (1024, 333))
    x = be.BufferFromFlatData(0, host, s)
    px = be.BufferData(x)
    (y,) = ex.Execute([x], [True], 0)
    assert be.BufferData(y) == px
    assert np.array_equal(be.BufferToFlatData(y).reshape(1024, 333), host * np.float32(0.5) + np.float32(1))
    with pytest.raises(BackendError):
        be.BufferShape(x)                      # consumed by the donation
    be.BufferFinalize(x)                       # finalizing a consumed buffer is a no-op
    be.BufferFinalize(y)
    # not donated: a fresh output, the input stays valid
    x = be.BufferFromFlatData(0, host, s)
    (y,) = ex.Execute([x], [False], 0)
    assert be.BufferData(y) != be.BufferData(x)
    assert np.array_equal(be.BufferToFlatData(x).reshape(1024, 333), host)
    be.BufferFinalize(y)
    be.BufferFinalize(x)


def test_donation_refused_when_the_input_is_read_later(be):
    """y = x + 1 is written before z = y . x reads x again: x's memory cannot hold y
    (the plan would overwrite it first), so the donation is declined and both
    results are correct; a transposed read (y = x + x^T) is not at y's own
    indices, so it is declined too."""
    s = make_shape(F32, 64, 64)
    ex = _compile(be, "later", lambda f, x: [f.Add(x, f.Constant(np.float32(1))),
                                             f.DotGeneral(f.Add(x, f.Constant(np.float32(1))), [1], [], x, [0], [])],
                  [s])
    host = synth.normal(5201, (64, 64))
    x = be.BufferFromFlatData(0, host, s)
    y, z = ex.Execute([x], [True], 0)
    assert be.BufferData(y) != be.BufferData(x) and be.BufferData(z) != be.BufferData(x)
    yy = host + np.float32(1)
    assert np.array_equal(be.BufferToFlatData(y).reshape(64, 64), yy)
    ref = yy.astype(np.float64) @ host.astype(np.float64)
    assert np.max(np.abs(be.BufferToFlatData(z).reshape(64, 64) - ref)) <= 1e-4 * np.max(np.abs(ref))
    ex2 = _compile(be, "transposed", lambda f, x: [f.Add(x, f.Transpose(x, 1, 0))], [s])
    x2 = be.BufferFromFlatData(0, host, s)
    (w,) = ex2.Execute([x2], [True], 0)
    assert be.BufferData(w) != be.BufferData(x2)
    assert np.array_equal(be.BufferToFlatData(w).reshape(64, 64), host + host.T)
    for b in (x, y, z, x2, w):
        be.BufferFinalize(b)


def test_many_executes_and_finalizes_without_sync(be):
    """A state update (w <- 0.5 w + 1, n <- n + 1) run 200 times, each Execute
    donating the previous state, with no host synchronisation until the end: both
    outputs reuse the donated memory every time, w matches numpy's fp32 sequence
    bit for bit (and the closed form 2 + (w0 - 2) / 2^t), n counts the steps.
    Fresh buffers made and finalized between the Executes (stream-ordered reuse)
    never disturb the state."""
    s = make_shape(F32, 4096, 257)
    ex = _compile(be, "step", lambda f, w, n: [f.Add(f.Mul(w, f.Constant(np.float32(0.5))), f.Constant(np.float32(1))),
                                               f.Add(n, f.Constant(np.float32(1)))],
                  [s, s])
    w0 = synth.normal(5301, (4096, 257), std=4.0)
    w = be.BufferFromFlatData(0, w0, s)
    n = be.BufferFromFlatData(0, np.zeros_like(w0), s)
    ref_w = w0.copy()
    reused = 0
    for t in range(200):
        pw, pn = be.BufferData(w), be.BufferData(n)
        w_new, n_new = ex.Execute([w, n], [True, True], 0)
        reused += (be.BufferData(w_new) == pw) + (be.BufferData(n_new) == pn)
        be.BufferFinalize(w)
        be.BufferFinalize(n)
        w, n = w_new, n_new
        junk = be.NewSharedBuffer(0, s)        # takes a cached block, released again unused
        be.BufferFinalize(junk)
        ref_w = ref_w * np.float32(0.5) + np.float32(1)
    assert reused == 400
    assert np.array_equal(be.BufferToFlatData(w).reshape(4096, 257), ref_w)
    assert np.all(be.BufferToFlatData(n) == 200.0)
    assert np.max(np.abs(ref_w - 2.0)) <= np.max(np.abs(w0 - 2.0)) * 2.0 ** -20 + 1e-6
    be.BufferFinalize(w)
    be.BufferFinalize(n)


def test_finalize_does_not_wait_and_reuse_is_ordered(be):
    """Outputs finalized right after their Execute while a long queue of work is
    still pending, and new inputs uploaded into the recycled blocks: every result
    read back at the end is that of its own inputs."""
    s = make_shape(F32, 2048, 2048)
    ex = _compile(be, "scale", lambda f, x: [f.Mul(x, f.Constant(np.float32(3)))], [s])
    keep = []
    for t in range(12):
        host = np.full((2048, 2048), np.float32(t), np.float32)
        x = be.BufferFromFlatData(0, host, s)
        (y,) = ex.Execute([x], None, 0)
        (y2,) = ex.Execute([x], None, 0)
        be.BufferFinalize(y2)                  # back to the cache at once
        be.BufferFinalize(x)
        keep.append((t, y))
    for t, y in keep:
        assert np.all(be.BufferToFlatData(y) == np.float32(3 * t))
        be.BufferFinalize(y)


def test_buffers_of_another_backend_are_refused(be):
    """A buffer made by a second backend lives on that backend's stream: Execute
    refuses it as an input (donated or not) instead of reading it, or moving it
    into this backend's allocator, unordered with the other stream."""
    s = make_shape(F32, 64, 64)
    ex = _compile(be, "neg", lambda f, x: [f.Neg(x)], [s])
    other = Backend("")
    try:
        host = synth.normal(5301, (64, 64))
        xo = other.BufferFromFlatData(0, host, s)
        for donate in (None, [True]):
            with pytest.raises(BackendError, match="another backend"):
                ex.Execute([xo], donate, 0)
        assert np.array_equal(other.BufferToFlatData(xo).reshape(64, 64), host)  # still valid
        other.BufferFinalize(xo)
        x = be.BufferFromFlatData(0, host, s)
        (y,) = ex.Execute([x], None, 0)
        assert np.array_equal(be.BufferToFlatData(y).reshape(64, 64), -host)
        be.BufferFinalize(y)
        be.BufferFinalize(x)
    finally:
        other.Finalize()
