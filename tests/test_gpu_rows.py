"""Parity of the row kernels (softmax, log-softmax, attention-score softmax,
RMSNorm, LayerNorm) against the CPU oracle, through the C ABI.

Tolerances (north star): fp32 outputs <= 1e-5 relative error (max elementwise,
RMS-floored, see conftest.rel_err) against the fp64 oracle.  bf16 outputs must be
within one bf16 ulp of the fp64 truth rounded to bf16 (statistics are fp32)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import ops, synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2.0 ** -8 + 1e-5   # one bf16 rounding of the fp32 result


def bf16_ulps(got_bf16: torch.Tensor, ref: np.ndarray) -> int:
    """Max distance in bf16 ulps between a bf16 result and the fp64 reference
    rounded to bf16 (ordered-integer distance, sign-aware)."""
    g = got_bf16.view(torch.int16).cpu().numpy().astype(np.int32)
    r = synth.to_bf16_bits(ref.astype(np.float32)).astype(np.int16).astype(np.int32)
    def ordered(b):
        return np.where(b < 0, -(b & 0x7FFF), b)
    return int(np.max(np.abs(ordered(g) - ordered(r)))) if g.size else 0


def f16_ulps(got_f16: torch.Tensor, ref: np.ndarray) -> int:
    """Max distance in float16 ulps between a float16 result and the fp64 reference
    rounded to float16 (numpy's conversion rounds to nearest even)."""
    g = got_f16.view(torch.int16).cpu().numpy().astype(np.int32)
    r = ref.astype(np.float16).view(np.int16).astype(np.int32)
    def ordered(b):
        return np.where(b < 0, -(b & 0x7FFF), b)
    return int(np.max(np.abs(ordered(g) - ordered(r)))) if g.size else 0


def to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


# ---------------------------------------------------------------- softmax
def test_softmax_known_answer(known, cuda):
    c = known["softmax"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    y = ops.softmax(to_dev(x, cuda)).cpu().numpy()
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]


def test_softmax_config_f32(cuda):
    """BASELINE config: fp32 [4096, 1024], x ~ N(0, 2^2), seed 1001."""
    x = synth.normal(1001, (4096, 1024), std=2.0)
    y = ops.softmax(to_dev(x, cuda)).cpu().numpy()
    ref = orc.softmax(x)
    assert rel_err(y, ref) <= F32_TOL
    assert np.max(np.abs(y.astype(np.float64).sum(-1) - 1.0)) < 1e-5
    # reported alongside: distance to a sequential-fp32 restatement
    assert rel_err(y, orc.softmax(x, mode=orc.MODE_F32SEQ)) <= 1e-4


@pytest.mark.parametrize("n", [1, 3, 64, 100, 256, 1000, 1024, 2048, 4096, 5000, 8192,
                               12288, 16384, 20000])
def test_softmax_shapes_f32(cuda, n):
    rows = 37
    x = synth.normal(1100 + n, (rows, n), std=3.0)
    y = ops.softmax(to_dev(x, cuda)).cpu().numpy()
    assert rel_err(y, orc.softmax(x)) <= F32_TOL


@pytest.mark.parametrize("n", [8, 1000, 1024, 2048, 8192, 20000])
def test_log_softmax_f32(cuda, n):
    x = synth.normal(1200 + n, (19, n), std=2.0)
    y = ops.softmax(to_dev(x, cuda), log=True).cpu().numpy()
    assert rel_err(y, orc.log_softmax(x)) <= F32_TOL


@pytest.mark.parametrize("n", [8, 1024, 2048, 4100])
def test_softmax_bf16(cuda, n):
    x = synth.round_bf16(synth.normal(1300 + n, (29, n), std=2.0))
    y = ops.softmax(to_dev(x, cuda, torch.bfloat16))
    assert bf16_ulps(y, orc.softmax(x)) <= 1


def test_softmax_empty_and_large_values(cuda):
    assert ops.softmax(torch.empty((0, 16), device=cuda)).shape == (0, 16)
    x = np.array([[1e30, 1e30, -1e30, 0.0], [-np.inf, 0.0, 1.0, -np.inf]], np.float32)
    y = ops.softmax(to_dev(x, cuda)).cpu().numpy()
    assert rel_err(y, orc.softmax(x)) <= F32_TOL


# ---------------------------------------------------------------- attention-score softmax
def _masked_ref(x, scale, causal, mask):
    s = x.astype(np.float64) * scale
    sq, sk = s.shape[-2:]
    keep = np.ones((sq, sk), bool)
    if causal:
        keep &= np.tril(np.ones((sq, sk), bool))
    if mask is not None:
        keep &= mask
    s = np.where(keep, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    return p / p.sum(-1, keepdims=True)


@pytest.mark.parametrize("sk", [64, 2048, 100])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scale_mask_softmax_causal(cuda, sk, dtype):
    x = synth.round_bf16(synth.normal(1400 + sk, (2, 3, sk, sk)))
    y = ops.scale_mask_softmax(to_dev(x, cuda, dtype), 1 / np.sqrt(128), True)
    ref = _masked_ref(x, 1 / np.sqrt(128), True, None)
    if dtype == torch.float32:
        assert rel_err(y.cpu().numpy(), ref) <= F32_TOL
    else:
        assert bf16_ulps(y, ref) <= 1
    # reference composition through the oracle's own softmax (Where(-inf) then softmax)
    xs = np.where(np.tril(np.ones((sk, sk), bool)), x * np.float32(1 / np.sqrt(128)), -np.inf)
    assert rel_err(orc.softmax(xs.astype(np.float32)), ref) <= 1e-6


def test_scale_mask_softmax_bool_mask(cuda):
    x = synth.normal(1500, (4, 16, 32))
    m = synth.uniform(1501, 16 * 32) > 0.3
    m = m.reshape(16, 32)
    m[:, 0] = True
    y = ops.scale_mask_softmax(to_dev(x, cuda), 0.5, False,
                               torch.from_numpy(m.astype(np.uint8)).to(cuda)).cpu().numpy()
    assert rel_err(y, _masked_ref(x, 0.5, False, m)) <= F32_TOL


# ---------------------------------------------------------------- RMSNorm / LayerNorm
def test_rmsnorm_config_f32(cuda):
    """BASELINE config: [8192, 4096] fp32, gamma ~ U(0.5, 1.5), eps 1e-6."""
    x = synth.normal(2001, (8192, 4096))
    g = synth.uniform_f32(2002, (4096,), 0.5, 1.5)
    y = ops.rmsnorm(to_dev(x, cuda), to_dev(g, cuda), 1e-6).cpu().numpy()
    assert rel_err(y, orc.rmsnorm(x, g, 1e-6)) <= F32_TOL


def test_rmsnorm_config_bf16(cuda):
    x = synth.round_bf16(synth.normal(2001, (8192, 4096)))
    g = synth.round_bf16(synth.uniform_f32(2002, (4096,), 0.5, 1.5))
    y = ops.rmsnorm(to_dev(x, cuda, torch.bfloat16), to_dev(g, cuda, torch.bfloat16), 1e-6)
    assert bf16_ulps(y, orc.rmsnorm(x, g, 1e-6)) <= 1


def test_layernorm_config_f32(cuda):
    x = synth.normal(2001, (8192, 4096))
    g = synth.uniform_f32(2002, (4096,), 0.5, 1.5)
    b = synth.normal(2003, (4096,), std=0.1)
    y = ops.layernorm(to_dev(x, cuda), to_dev(g, cuda), to_dev(b, cuda), 1e-5).cpu().numpy()
    assert rel_err(y, orc.layernorm(x, g, b, 1e-5)) <= F32_TOL


def test_layernorm_config_bf16(cuda):
    x = synth.round_bf16(synth.normal(2001, (8192, 4096)))
    g = synth.round_bf16(synth.uniform_f32(2002, (4096,), 0.5, 1.5))
    b = synth.round_bf16(synth.normal(2003, (4096,), std=0.1))
    y = ops.layernorm(to_dev(x, cuda, torch.bfloat16), to_dev(g, cuda, torch.bfloat16),
                      to_dev(b, cuda, torch.bfloat16), 1e-5)
    # x - mean (and beta) put outputs arbitrarily close to zero, where a ulp count is
    # ill-conditioned: bound the RMS-floored relative error by one bf16 rounding.
    assert rel_err(y.float().cpu().numpy(), orc.layernorm(x, g, b, 1e-5)) <= BF16_TOL


def test_layernorm_known_answers(known, cuda):
    c = known["layernorm_basic"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    y = ops.layernorm(to_dev(x, cuda), eps=c["eps"]).cpu().numpy()
    assert np.max(np.abs(y.reshape(-1) - np.array(c["expected"]))) <= c["tol"]
    c = known["layernorm_gamma_beta"]
    x = np.array(c["x"], np.float32).reshape(c["shape"])
    g = np.array(c["gamma"], np.float32)
    b = np.array(c["beta"], np.float32)
    y = ops.layernorm(to_dev(x, cuda), to_dev(g, cuda), to_dev(b, cuda), c["eps"]).cpu().numpy()
    assert np.max(np.abs(y[0] - np.array(c["expected_first_row"]))) <= c["tol"]


@pytest.mark.parametrize("n", [1, 5, 64, 768, 1000, 4096, 8192, 10000, 16384, 40000])
def test_norms_shapes_f32(cuda, n):
    x = synth.normal(2100 + n, (13, n), std=2.0, mean=0.5)
    g = synth.uniform_f32(2200 + n, (n,), 0.5, 1.5)
    b = synth.normal(2300 + n, (n,), std=0.1)
    xd, gd, bd = to_dev(x, cuda), to_dev(g, cuda), to_dev(b, cuda)
    assert rel_err(ops.rmsnorm(xd, gd, 1e-6).cpu().numpy(), orc.rmsnorm(x, g, 1e-6)) <= F32_TOL
    assert rel_err(ops.rmsnorm(xd, None, 1e-6).cpu().numpy(), orc.rmsnorm(x, None, 1e-6)) <= F32_TOL
    assert rel_err(ops.layernorm(xd, gd, bd, 1e-5).cpu().numpy(),
                   orc.layernorm(x, g, b, 1e-5)) <= F32_TOL
    assert rel_err(ops.layernorm(xd, None, None, 1e-5).cpu().numpy(),
                   orc.layernorm(x, None, None, 1e-5)) <= F32_TOL


def test_norm_invariants_full_size(cuda):
    """Size-independent properties at a full config shape: RMSNorm output has
    mean(y^2) = 1 with gamma = 1 and eps = 0; LayerNorm output mean 0, var 1."""
    x = torch.randn((8192, 4096), device=cuda, generator=torch.Generator(cuda).manual_seed(7)) * 3 + 1
    y = ops.rmsnorm(x, None, 0.0).double()
    assert torch.max(torch.abs((y * y).mean(-1) - 1)).item() < 1e-5
    y = ops.layernorm(x, None, None, 0.0).double()
    assert torch.max(torch.abs(y.mean(-1))).item() < 1e-5
    assert torch.max(torch.abs(y.var(-1, unbiased=False) - 1)).item() < 1e-5


# ---------------------------------------------------------------- float16 (declared by the reference)
@pytest.mark.parametrize("n", [1024, 4096, 20000])
def test_softmax_and_log_softmax_f16(cuda, n):
    x = synth.normal(1600 + n, (4096 if n == 1024 else 33, n), std=2.0).astype(np.float16).astype(np.float32)
    xd = to_dev(x, cuda, torch.float16)
    assert f16_ulps(ops.softmax(xd), orc.softmax(x)) <= 1
    # log-softmax values reach |y| ~ 20 where an f16 ulp is 2^-6: one rounding of
    # the fp32 result, RMS-floored
    y = ops.softmax(xd, log=True).float().cpu().numpy()
    assert rel_err(y, orc.log_softmax(x)) <= 2.0 ** -11 + 1e-5


def test_norms_config_f16(cuda):
    """configs[1] shape in float16: RMSNorm within one f16 ulp of the rounded truth,
    LayerNorm within one f16 rounding (RMS-floored)."""
    x = synth.normal(2001, (8192, 4096)).astype(np.float16).astype(np.float32)
    g = synth.uniform_f32(2002, (4096,), 0.5, 1.5).astype(np.float16).astype(np.float32)
    b = synth.normal(2003, (4096,), std=0.1).astype(np.float16).astype(np.float32)
    xd, gd, bd = (to_dev(a, cuda, torch.float16) for a in (x, g, b))
    assert f16_ulps(ops.rmsnorm(xd, gd, 1e-6), orc.rmsnorm(x, g, 1e-6)) <= 1
    y = ops.layernorm(xd, gd, bd, 1e-5).float().cpu().numpy()
    assert rel_err(y, orc.layernorm(x, g, b, 1e-5)) <= 2.0 ** -11 + 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [4096, 32768])
def test_norms_16bit_odd_rows(cuda, dtype, n):
    """Row counts that leave the last workgroup partly empty, at widths that take
    2 waves per row (n 4096) and 16 vectors per lane over 4 waves (n 32768)."""
    rows = 13
    x = synth.normal(2400 + n, (rows, n), std=1.5, mean=0.25)
    g = synth.uniform_f32(2500 + n, (n,), 0.5, 1.5)
    b = synth.normal(2600 + n, (n,), std=0.1)
    if dtype == torch.bfloat16:
        x, g, b = synth.round_bf16(x), synth.round_bf16(g), synth.round_bf16(b)
        ulps, tol = bf16_ulps, BF16_TOL
    else:
        x, g, b = (a.astype(np.float16).astype(np.float32) for a in (x, g, b))
        ulps, tol = f16_ulps, 2.0 ** -11 + 1e-5
    xd, gd, bd = (to_dev(a, cuda, dtype) for a in (x, g, b))
    assert ulps(ops.rmsnorm(xd, gd, 1e-6), orc.rmsnorm(x, g, 1e-6)) <= 1
    y = ops.layernorm(xd, gd, bd, 1e-5).float().cpu().numpy()
    assert rel_err(y, orc.layernorm(x, g, b, 1e-5)) <= tol


@pytest.mark.parametrize("dtype,n,rows", [
    (torch.float32, 4096, 3001),     # 4 waves per row, one row per workgroup: ragged iteration counts
    (torch.bfloat16, 4096, 4099),    # 2 waves per row: the last group holds one row
    (torch.float16, 2048, 8195),     # 1 wave per row, 4 rows per group: last group holds 3 rows
    (torch.bfloat16, 1024, 8200),    # 2 vectors per lane
])
def test_norms_streaming_rows_match_single_group_kernel(cuda, dtype, n, rows):
    """Row counts large enough for the streaming RMSNorm / LayerNorm kernel (a
    grid of two workgroups per CU looping over row groups with the next group
    prefetched): every row is bit-identical to the one-group-per-workgroup kernel,
    which a launch over 64 rows takes, and within the dtype's rounding of the
    oracle; gamma / beta in every combination."""
    x = synth.normal(2700 + n, (rows, n), std=1.5, mean=0.25)
    g = synth.uniform_f32(2800 + n, (n,), 0.5, 1.5)
    b = synth.normal(2900 + n, (n,), std=0.1)
    if dtype == torch.bfloat16:
        x, g, b = synth.round_bf16(x), synth.round_bf16(g), synth.round_bf16(b)
        tol = BF16_TOL
    elif dtype == torch.float16:
        x, g, b = (a.astype(np.float16).astype(np.float32) for a in (x, g, b))
        tol = 2.0 ** -11 + 1e-5
    else:
        tol = F32_TOL
    xd, gd, bd = (to_dev(a, cuda, dtype) for a in (x, g, b))
    picks = np.array([0, 1, 2, 3, 511, 512, 1023, 2047, rows // 2, rows - 3, rows - 2, rows - 1])
    sub = xd[torch.from_numpy(picks).to(cuda)].contiguous()
    for gg, bb in [(gd, bd), (gd, None), (None, bd), (None, None)]:
        ys = [ops.rmsnorm(xd, gg, 1e-6), ops.layernorm(xd, gg, bb, 1e-5)]
        small = [ops.rmsnorm(sub, gg, 1e-6), ops.layernorm(sub, gg, bb, 1e-5)]
        for y, s in zip(ys, small):
            assert torch.equal(y[torch.from_numpy(picks).to(cuda)].view(torch.int16 if dtype != torch.float32 else torch.int32),
                               s.view(torch.int16 if dtype != torch.float32 else torch.int32))
        gn = g if gg is not None else None
        bn = b if bb is not None else None
        assert rel_err(ys[0].float().cpu().numpy(), orc.rmsnorm(x, gn, 1e-6)) <= tol
        assert rel_err(ys[1].float().cpu().numpy(), orc.layernorm(x, gn, bn, 1e-5)) <= tol
