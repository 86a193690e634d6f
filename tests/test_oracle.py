"""Pins the CPU oracle: the reference's known answers, invariants, and
independent textbook computations (numpy) chosen so that a dropped term, a
wrong sign/index or a transposed operand fails."""
import itertools

import numpy as np
import pytest

from oracle import oracle as orc
from gomlx_hip import synth
from conftest import rel_err


# ---------------------------------------------------------------- known answers
def test_softmax_known_answer(known):
    c = known["softmax"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    y = orc.softmax(x, c["axis"])
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]
    y32 = orc.softmax(x, c["axis"], mode=orc.MODE_F32SEQ)
    assert np.max(np.abs(y32.reshape(-1) - np.array(c["expected"]))) <= c["tol"]


def test_layernorm_known_answers(known):
    c = known["layernorm_basic"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    y = orc.layernorm(x, eps=c["eps"])
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]
    c = known["layernorm_gamma_beta"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    g = np.array(c["gamma"], np.float32).reshape(c["gamma_shape"])
    b = np.array(c["beta"], np.float32).reshape(c["gamma_shape"])
    y = orc.layernorm(x, g, b, eps=c["eps"])
    assert np.max(np.abs(y[0] - np.array(c["expected_first_row"]))) <= c["tol"]


@pytest.mark.parametrize("name", ["dot_simple", "dot_batched", "dot_bf16"])
def test_dot_general_known_answers(known, name):
    c = known[name]
    lhs = np.array(c["lhs"], np.float32).reshape(c["lhs_shape"])
    rhs = np.array(c["rhs"], np.float32).reshape(c["rhs_shape"])
    y = orc.dot_general(lhs, c["lc"], c["lb"], rhs, c["rc"], c["rb"])
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= min(c["tol"], 1e-9)


def test_attention_chain_known_answer(known):
    c = known["attention_dot_chain"]
    q = np.array(c["q"], np.float32).reshape(1, 1, *c["shape"])
    k = np.array(c["k"], np.float32).reshape(1, 1, *c["shape"])
    v = np.array(c["v"], np.float32).reshape(1, 1, *c["shape"])
    y = orc.sdpa(q, k, v, scale=c["scale"])
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]


def test_sdpa_known_answers(known):
    c = known["sdpa_causal"]
    sh = c["shape"]
    q, k, v = (np.array(c[n], np.float32).reshape(sh) for n in "qkv")
    y = orc.sdpa(q, k, v, scale=c["scale"], causal=True)
    assert np.max(np.abs(y[0, 0, 0] - np.array(c["expected_first_row"]))) <= c["tol"]
    c = known["sdpa_bool_mask"]
    sh = c["shape"]
    q, k, v = (np.array(c[n], np.float32).reshape(sh) for n in "qkv")
    m = np.array(c["mask"], bool).reshape(sh[2], sh[3])
    y = orc.sdpa(q, k, v, mask=m, scale=c["scale"])
    assert np.max(np.abs(y[0, 0, 0] - np.array(c["expected_first_row"]))) <= c["tol"]
    c = known["sdpa_basic_range"]
    sh = c["shape"]
    q, k, v = (np.array(c[n], np.float32).reshape(sh) for n in "qkv")
    y = orc.sdpa(q, k, v, scale=c["scale"])
    lo, hi = c["expected_range"]
    assert np.all(y >= lo) and np.all(y <= hi)


def test_gather_known_answer(known):
    c = known["gather_embedding"]
    t = np.array(c["table"], np.float32).reshape(c["table_shape"])
    out = orc.gather_rows(t, c["ids"])
    assert out.reshape(-1).tolist() == c["expected"]


def test_argmax_iota_known_answers(known):
    c = known["argmax"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    assert orc.argminmax(x, c["axis"]).tolist() == c["expected"]
    c = known["iota"]
    assert orc.iota(c["shape"], c["axis"]).reshape(-1).tolist() == c["expected"]


# ---------------------------------------------------------------- invariants / brute force
def test_softmax_invariants_and_numpy():
    x = synth.normal(7, (37, 53), std=3.0)
    y = orc.softmax(x)
    assert np.allclose(y.sum(-1), 1.0, atol=1e-12)
    assert np.all(y > 0) and np.all(y <= 1)
    y2 = orc.softmax(x + np.float32(5.0))   # shift invariance (5.0 is exact in fp32 here)
    assert np.max(np.abs(y - y2)) < 1e-6
    xd = x.astype(np.float64)
    ref = np.exp(xd - xd.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    assert np.max(np.abs(y - ref)) < 1e-14
    # middle-axis softmax equals last-axis softmax of the transposed tensor
    x3 = synth.normal(8, (4, 9, 5))
    ym = orc.softmax(x3, axis=1)
    yt = orc.softmax(np.ascontiguousarray(x3.transpose(0, 2, 1)), axis=-1).transpose(0, 2, 1)
    assert np.max(np.abs(ym - yt)) < 1e-14
    ls = orc.log_softmax(x)
    assert np.max(np.abs(ls - np.log(ref))) < 1e-12


def test_layernorm_invariants():
    x = synth.normal(11, (16, 256), std=3.0, mean=2.0)
    y = orc.layernorm(x, eps=0.0)
    assert np.max(np.abs(y.mean(-1))) < 1e-12
    assert np.max(np.abs(y.var(-1) - 1.0)) < 1e-10
    g = synth.uniform_f32(12, (256,), 0.5, 1.5)
    b = synth.normal(13, (256,), std=0.1)
    yg = orc.layernorm(x, g, b, eps=1e-5)
    xd = x.astype(np.float64)
    mu = xd.mean(-1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * g + b
    assert np.max(np.abs(yg - ref)) < 1e-12


def test_rmsnorm_invariants():
    x = synth.normal(21, (16, 512), std=2.0)
    y = orc.rmsnorm(x, eps=0.0)
    assert np.max(np.abs((y ** 2).mean(-1) - 1.0)) < 1e-12
    # scale invariance: rmsnorm(c x) == rmsnorm(x) when eps = 0
    y4 = orc.rmsnorm(x * np.float32(4.0), eps=0.0)
    assert np.max(np.abs(y - y4)) < 1e-12
    # hand-computed row [3, 4]: rms = sqrt(12.5)
    y = orc.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), eps=0.0)
    r = np.sqrt(12.5)
    assert np.allclose(y, [[3 / r, 8 / r]], atol=1e-12)


def test_rmsnorm_f32_output_form():
    """The CPU baseline's fp32 form: identical to the fp32-sequential mode, within
    fp32 rounding of the fp64 truth, and the hand-computed row [3, 4]."""
    x = synth.normal(22, (64, 1024), std=1.5)
    g = synth.uniform_f32(23, (1024,), 0.5, 1.5)
    y = orc.rmsnorm_f32(x, g, 1e-6)
    assert y.dtype == np.float32
    assert np.array_equal(y, orc.rmsnorm(x, g, 1e-6, mode=orc.MODE_F32SEQ).astype(np.float32))
    assert np.max(np.abs(y - orc.rmsnorm(x, g, 1e-6))) < 1e-5
    y = orc.rmsnorm_f32(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), 0.0)
    assert np.allclose(y, [[3 / np.sqrt(12.5), 8 / np.sqrt(12.5)]], atol=1e-6)


DOT_LAYOUTS = [
    # (lhs shape, lc, lb, rhs shape, rc, rb)
    ((5, 7), [1], [], (7, 3), [0], []),
    ((5, 7), [1], [], (3, 7), [1], []),          # rhs transposed
    ((7, 5), [0], [], (7, 3), [0], []),          # lhs transposed
    ((2, 5, 7), [2], [0], (2, 7, 3), [1], [0]),  # DotGeneral config layout
    ((2, 3, 5, 4), [3], [0, 1], (2, 3, 6, 4), [3], [0, 1]),  # attention Q.K^T
    ((4, 2, 5, 3), [0, 3], [1], (3, 2, 4, 6), [2, 0], [1]),  # multi-contract, odd order
]


@pytest.mark.parametrize("layout", DOT_LAYOUTS)
def test_dot_general_vs_einsum(layout):
    ls, lc, lb, rs, rc, rb = layout
    lhs = synth.normal(31, ls)
    rhs = synth.normal(32, rs)
    got = orc.dot_general(lhs, lc, lb, rhs, rc, rb)
    letters = iter("abcdefghijklmnop")
    lsub = [None] * len(ls)
    rsub = [None] * len(rs)
    for a, b in zip(lb, rb):
        lsub[a] = rsub[b] = next(letters)
    for a, b in zip(lc, rc):
        lsub[a] = rsub[b] = next(letters)
    for i in range(len(ls)):
        if lsub[i] is None:
            lsub[i] = next(letters)
    for i in range(len(rs)):
        if rsub[i] is None:
            rsub[i] = next(letters)
    out = [lsub[a] for a in lb] + [lsub[i] for i in range(len(ls)) if i not in lc and i not in lb] \
        + [rsub[i] for i in range(len(rs)) if i not in rc and i not in rb]
    spec = "".join(lsub) + "," + "".join(rsub) + "->" + "".join(out)
    ref = np.einsum(spec, lhs.astype(np.float64), rhs.astype(np.float64))
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 1e-10


def test_dot_sampled_matches_dot_general():
    a = synth.normal(41, (2, 9, 13))
    b = synth.normal(42, (2, 13, 11))
    full = orc.dot_general(a, [2], [0], b, [1], [0])
    idx = np.array(list(itertools.product(range(2), range(9), range(11))))
    s = orc.dot_sampled(a, b, idx[:, 0], idx[:, 1], idx[:, 2])
    assert np.max(np.abs(s - full.reshape(-1))) < 1e-12


def test_sdpa_vs_numpy_gqa_causal():
    B, H, Hkv, S, D = 2, 4, 2, 7, 5
    q = synth.normal(51, (B, H, S, D))
    k = synth.normal(52, (B, Hkv, S, D))
    v = synth.normal(53, (B, Hkv, S, D))
    got = orc.sdpa(q, k, v, causal=True, scale=0.3)
    kr = np.repeat(k.astype(np.float64), H // Hkv, axis=1)
    vr = np.repeat(v.astype(np.float64), H // Hkv, axis=1)
    s = q.astype(np.float64) @ kr.transpose(0, 1, 3, 2) * 0.3
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.max(np.abs(got - p @ vr)) < 1e-12


def _np_attention(q, k, v, scale, keep=None, add=None, causal=False):
    H, Hkv = q.shape[1], k.shape[1]
    kr = np.repeat(k.astype(np.float64), H // Hkv, axis=1)
    vr = np.repeat(v.astype(np.float64), H // Hkv, axis=1)
    s = q.astype(np.float64) @ kr.transpose(0, 1, 3, 2) * scale
    if add is not None:
        s = s + np.asarray(add, np.float64)
    if keep is not None:
        s = np.where(keep, s, -np.inf)
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ vr


@pytest.mark.parametrize("mshape", [(5,), (6, 5), (1, 6, 5), (2, 1, 1, 5), (2, 4, 6, 5), (1, 4, 1, 5)])
def test_sdpa_masks_of_every_rank_vs_numpy(mshape):
    """Boolean and additive masks of every rank broadcast to [B, H, Sq, Sk]
    (broadcastMaskToScores, function.go:2959-2974), with and without causal, against
    a numpy composition; and the closed forms: an all-zero additive mask is no mask,
    an additive mask of 0 / -inf is the boolean mask, and a per-row additive constant
    changes nothing (softmax shift invariance)."""
    B, H, Hkv, Sq, Sk, D = 2, 4, 2, 6, 5, 3
    q = synth.normal(81, (B, H, Sq, D))
    k = synth.normal(82, (B, Hkv, Sk, D))
    v = synth.normal(83, (B, Hkv, Sk, D))
    keep = synth.uniform(84, int(np.prod(mshape))).reshape(mshape) > 0.3
    keep[..., 0] = True                                   # every row keeps a key
    add = synth.normal(85, mshape, std=2.0)
    for causal in (False, True):
        got = orc.sdpa(q, k, v, mask=keep, scale=0.4, causal=causal)
        assert np.max(np.abs(got - _np_attention(q, k, v, 0.4, keep=keep, causal=causal))) < 1e-12
        got = orc.sdpa(q, k, v, additive=add, scale=0.4, causal=causal)
        assert np.max(np.abs(got - _np_attention(q, k, v, 0.4, add=add, causal=causal))) < 1e-12
        zero = orc.sdpa(q, k, v, additive=np.zeros(mshape, np.float32), scale=0.4, causal=causal)
        assert np.max(np.abs(zero - orc.sdpa(q, k, v, scale=0.4, causal=causal))) < 1e-12
        as_add = np.where(keep, 0.0, -np.inf).astype(np.float32)
        assert np.max(np.abs(orc.sdpa(q, k, v, additive=as_add, scale=0.4, causal=causal) -
                             orc.sdpa(q, k, v, mask=keep, scale=0.4, causal=causal))) < 1e-12
    row_const = synth.normal(86, (B, H, Sq, 1), std=3.0)
    assert np.max(np.abs(orc.sdpa(q, k, v, additive=row_const, scale=0.4) - orc.sdpa(q, k, v, scale=0.4))) < 1e-12
    # a row whose keys are all masked is NaN, as the reference's softmax of -inf is
    none = np.zeros((Sq, Sk), bool)
    assert np.all(np.isnan(orc.sdpa(q, k, v, mask=none, scale=0.4)))


@pytest.mark.parametrize("dt", [np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16, np.uint32, np.uint64])
def test_argminmax_integers_vs_numpy(dt):
    """Integer inputs compare exactly (numpy's argmax / argmin return the first
    occurrence of the extreme): few distinct values so ties are everywhere, and
    the type's extremes, including uint64 values above INT64_MAX."""
    rng = np.random.default_rng(17)
    info = np.iinfo(dt)
    pool = np.array([info.min, info.max, 0, 1, info.max - 1, info.min + 1], dtype=dt)
    x = pool[rng.integers(0, len(pool), size=(5, 37, 3))]
    for ax in range(3):
        assert np.array_equal(orc.argminmax(x, ax), np.argmax(x, axis=ax))
        assert np.array_equal(orc.argminmax(x, ax, is_min=True), np.argmin(x, axis=ax))


def test_argminmax_vs_numpy_and_rules():
    x = synth.normal(61, (6, 17, 5))
    for ax in range(3):
        assert np.array_equal(orc.argminmax(x, ax), np.argmax(x, axis=ax))
        assert np.array_equal(orc.argminmax(x, ax, is_min=True), np.argmin(x, axis=ax))
    t = np.array([[1, 3, 3, 2], [np.nan, 1, np.nan, 5], [-np.inf, -np.inf, 0, 0]], np.float32)
    assert orc.argminmax(t, 1).tolist() == [1, 0, 2]          # ties -> first, NaN wins
    assert orc.argminmax(t, 1, is_min=True).tolist() == [0, 0, 0]


def test_gather_clamps_out_of_range():
    t = np.arange(12, dtype=np.float32).reshape(4, 3)
    out = orc.gather_rows(t, [-5, 0, 3, 99])
    assert out.tolist() == [t[0].tolist(), t[0].tolist(), t[3].tolist(), t[3].tolist()]


def test_bf16_rounding_matches_numpy_port():
    x = np.concatenate([synth.normal(71, (4096,), std=100.0),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.inf, -np.inf, 0.0, -0.0],
                                 np.float32)])
    a = orc.f32_to_bf16_bits(x)
    b = synth.to_bf16_bits(x)
    assert np.array_equal(a, b)
    # ties to even: 1 + 2^-8 -> 1.0, 1 + 3*2^-8 -> 1 + 2^-6
    assert synth.bf16_bits_to_f32(a[4096:4098]).tolist() == [1.0, 1.0 + 2 ** -6]


# ---------------------------------------------------------------- FusedGelu / FusedDense / QKV
def test_gelu_known_answer(known):
    c = known["gelu"]
    x = np.array(c["x"])
    for exact in (False, True):
        assert np.max(np.abs(orc.gelu(x, exact) - np.array(c["expected"]))) <= c["tol"]


def test_activation_identities():
    from scipy.special import erf, ndtr
    x = np.linspace(-8, 8, 4001)
    for act in (orc.ACT_GELU, orc.ACT_GELU_EXACT):
        g = orc.activation(x, act)
        # odd part: g(x) - g(-x) = x for x*Phi(x) and for its tanh approximation
        assert np.max(np.abs(g - orc.activation(-x, act) - x)) < 1e-12
    ex = orc.gelu(x, True)
    assert np.max(np.abs(ex - x * ndtr(x))) < 1e-12               # x * Phi(x), normal CDF
    assert np.max(np.abs(ex - 0.5 * x * (1 + erf(x / np.sqrt(2))))) < 1e-12
    assert np.max(np.abs(orc.gelu(x, False) - ex)) < 1e-3          # tanh form tracks the exact one
    assert np.max(np.abs(orc.activation(x, orc.ACT_SILU) - x / (1 + np.exp(-x)))) < 1e-12
    assert np.array_equal(orc.activation(x, orc.ACT_RELU), np.maximum(x, 0))
    assert np.max(np.abs(orc.activation(x, orc.ACT_TANH) - np.tanh(x))) < 1e-15
    assert np.array_equal(orc.activation(x, orc.ACT_NONE), x)


@pytest.mark.parametrize("name", ["dense_no_bias", "dense_bias", "dense_relu"])
def test_dense_known_answers(known, name):
    c = known[name]
    x = np.array(c["x"], np.float32).reshape(c["x_shape"])
    w = np.array(c["w"], np.float32).reshape(c["w_shape"])
    act = {"none": orc.ACT_NONE, "relu": orc.ACT_RELU}[c["activation"]]
    y = orc.dense(x, w, c.get("bias"), act)
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]


def test_dense_against_numpy():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 5, 7)).astype(np.float32)
    w = rng.standard_normal((7, 2, 4)).astype(np.float32)   # rank-3 weight: trailing dims kept
    b = rng.standard_normal((2, 4)).astype(np.float32)
    y = orc.dense(x, w, b, orc.ACT_TANH)
    ref = np.tanh(np.tensordot(x.astype(np.float64), w.astype(np.float64), axes=([2], [0])) + b)
    assert y.shape == (3, 5, 2, 4) and np.max(np.abs(y - ref)) < 1e-12


@pytest.mark.parametrize("name", ["qkv_identity", "qkv_biases"])
def test_qkv_projection_known_answers(known, name):
    c = known[name]
    x = np.array(c["x"], np.float32).reshape(c["x_shape"])
    w = np.array(c["w"], np.float32).reshape(c["w_shape"])
    outs = orc.qkv_projection(x, w, c.get("bias_q"), c.get("bias_k"), c.get("bias_v"),
                              c["query_dim"], c["key_value_dim"])
    for o, key in zip(outs, "qkv"):
        assert np.max(np.abs(o.reshape(-1) - np.array(c[key]))) <= c["tol"]


# ---------------------------------------------------------------- DynamicSlice / UpdateSlice / Scatter
def test_dynamic_slice_known_answers(known):
    c = known["dynamic_slice"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    assert orc.dynamic_slice(x, c["starts"], c["sizes"]).reshape(-1).tolist() == c["expected"]
    c = known["dynamic_update_slice"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    u = np.array(c["update"], np.float32).reshape(c["update_shape"])
    assert orc.dynamic_update_slice(x, u, c["starts"]).reshape(-1).tolist() == c["expected"]


def test_dynamic_slices_against_numpy():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 1 << 16, (5, 7, 6)).astype(np.uint16)
    for starts in ([0, 0, 0], [2, 3, 1], [9, -4, 5], [-1, 100, -100]):
        sizes = (3, 4, 2)
        cl = [min(max(s, 0), d - z) for s, d, z in zip(starts, x.shape, sizes)]
        want = x[cl[0]:cl[0] + 3, cl[1]:cl[1] + 4, cl[2]:cl[2] + 2]
        assert np.array_equal(orc.dynamic_slice(x, starts, sizes), want)
        u = rng.integers(0, 1 << 16, sizes).astype(np.uint16)
        want = x.copy()
        want[cl[0]:cl[0] + 3, cl[1]:cl[1] + 4, cl[2]:cl[2] + 2] = u
        assert np.array_equal(orc.dynamic_update_slice(x, u, starts), want)


def test_scatter_known_answer(known):
    c = known["scatter_sum"]
    out = orc.scatter(orc.SCATTER_SUM, np.array(c["operand"], np.float64).reshape(c["operand_shape"]),
                      np.array(c["indices"]).reshape(c["indices_shape"]),
                      np.array(c["updates"], np.float64).reshape(c["updates_shape"]), c["index_vector_axis"],
                      c["update_window_axes"], c["inserted_window_axes"], c["scatter_axes_to_operand_axes"])
    assert out.reshape(-1).tolist() == c["expected"]


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_scatter_embedding_pattern_against_numpy(mode):
    rng = np.random.default_rng(7 + mode)
    V, D, n = 50, 6, 200
    op = rng.standard_normal((V, D))
    ids = rng.integers(-3, V + 3, n)          # some out of range: skipped
    upd = rng.standard_normal((n, D))
    got = orc.scatter(mode, op, ids.reshape(n, 1), upd, 1, [1], [0], [0])
    want = op.copy()
    ok = (ids >= 0) & (ids < V)
    fn = [np.add, np.maximum, np.minimum][mode]
    fn.at(want, ids[ok], upd[ok])
    assert np.allclose(got, want, rtol=0, atol=1e-12) if mode == 0 else np.array_equal(got, want)
    # implicit trailing index vector axis (iva == indices rank) gives the same result
    got2 = orc.scatter(mode, op, ids, upd, 1, [1], [0], [0])
    assert np.array_equal(got, got2)


def test_scatter_general_invariants():
    rng = np.random.default_rng(11)
    op = rng.integers(-5, 5, (6, 4, 5)).astype(np.float64)
    # index vectors of length 2 on axis 0 of indices [2, 3, 4] -> starts on operand axes (2, 0)
    idx = np.stack([rng.integers(0, 4, (3, 4)), rng.integers(0, 5, (3, 4))])
    # updates: scatter dims [3, 4] then window dims over operand axes 1 (size 2) and 2 (size 2);
    # operand axis 0 inserted
    upd = rng.integers(-9, 9, (3, 2, 4, 2)).astype(np.float64)
    args = (0, [1, 3], [0], [2, 0])
    got = orc.scatter(orc.SCATTER_SUM, op, idx, upd, *args)
    # in-bounds windows: start on axis 2 <= 5-2, on axis 0 <= 6-1
    starts2, starts0 = idx[0], idx[1]
    ok = (starts2 <= 3) & (starts0 <= 5)
    assert got.sum() == op.sum() + upd.transpose(0, 2, 1, 3)[ok].sum()
    # brute force over the windows, in a different enumeration order
    want = op.copy()
    for i in range(3):
        for j in range(4):
            if not ok[i, j]:
                continue
            for a in range(2):
                for b in range(2):
                    want[idx[1, i, j], a, idx[0, i, j] + b] += upd[i, a, j, b]
    assert np.array_equal(got, want)


def _all_bf16(limit=None):
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    x = x[np.isfinite(x)]
    return x if limit is None else x[np.abs(x) <= limit]


def test_gelu_chain_16_hand_computed():
    """The per-op bf16 chain at points worked by hand.  bf16 constants:
    0.044715 -> 0.044677734375, sqrt(2/pi) 0.7978845608 -> 0.796875.
    x = -3: x^3 = -27, 0.0446777 * -27 = -1.2063 -> -1.203125, inner -4.203125 ->
    -4.1875 (tie, even), scaled -3.3369 -> -3.34375, tanh = -0.99751 -> -0.99609375,
    1 + t = 2^-8, 0.5 x = -1.5, result -1.5 * 2^-8 = -0.005859375.
    x = 1: inner 1.0447 -> 1.046875, scaled 0.83423 -> 0.8359375, tanh 0.68366 ->
    0.68359375, 1 + t = 1.68359375 -> 1.6875 (tie, even), result 0.84375.
    x = -4: scaled -> -5.96875 (bf16), tanh rounds to -1, so the result is -0."""
    x = np.array([-3.0, 1.0, -4.0], np.float32)
    lo, hi = orc.gelu_chain_16(x, False)
    assert lo.tolist() == hi.tolist() == [-0.005859375, 0.84375, -0.0]
    assert np.signbit(lo[2])


def test_gelu_chain_16_tracks_exact_gelu():
    """Over every bf16 input with |x| <= 8 the chain stays within |x| 2^-7 of the
    fp64 GELU (both forms), while the tanh form with its cubic term dropped leaves
    that bound by 2x; only near a rounding midpoint of erf is the step ambiguous."""
    x = _all_bf16(8.0)
    for exact in (False, True):
        lo, hi = orc.gelu_chain_16(x, exact)
        ref = orc.gelu(x.astype(np.float64), exact)
        for r in (lo, hi):
            assert np.all(np.abs(r - ref) <= np.abs(x) * 2.0 ** -7 + 2.0 ** -133)
    xx = x.astype(np.float64)
    no_cubic = 0.5 * xx * (1 + np.tanh(0.7978845608 * xx))
    assert np.max(np.abs(no_cubic - orc.gelu(xx, False)) / (np.abs(xx) * 2.0 ** -7 + 2.0 ** -133)) > 2
    lo, hi = orc.gelu_chain_16(_all_bf16(), False)
    assert np.array_equal(lo.view(np.uint32), hi.view(np.uint32))   # tanh never lands near a midpoint
