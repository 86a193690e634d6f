"""Parity of the batched GEMM (DotGeneral lowering target) against the oracle.

Tolerances: bf16 inputs with bf16 output <= 1e-2 relative (north star, fp32
reference); bf16 inputs with fp32 output and fp32 inputs <= 1e-4 relative
(RMS-floored max elementwise error, conftest.rel_err)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import ops, synth
from conftest import rel_err, norm_err

pytestmark = pytest.mark.gpu


def dev(a, d, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(d).to(dtype)


@pytest.mark.parametrize("name", ["dot_simple", "dot_batched", "dot_bf16"])
def test_known_answers(known, cuda, name):
    c = known[name]
    lhs = np.array(c["lhs"], np.float32).reshape(c["lhs_shape"])
    rhs = np.array(c["rhs"], np.float32).reshape(c["rhs_shape"])
    dt = torch.bfloat16 if name == "dot_bf16" else torch.float32
    got = ops.gemm(dev(lhs, cuda, dt), dev(rhs, cuda, dt)).float().cpu().numpy()
    assert np.max(np.abs(got.reshape(-1) - np.array(c["expected"]))) <= c["tol"]


SHAPES = [  # (batch, M, N, K)
    (1, 256, 256, 64),
    (2, 512, 256, 128),
    (1, 300, 200, 136),     # ragged tiles in M, N and K
    (3, 128, 136, 72),
    (1, 1024, 1024, 512),
    (4, 64, 512, 256),
    (1, 8, 8, 8),
    (2, 520, 264, 1000),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
def test_bf16_layouts(cuda, shape, a_t, b_t):
    """Every operand majorness (K- or MN-contiguous) through strided views."""
    B, M, N, K = shape
    a = synth.round_bf16(synth.normal(3000 + M, (B, M, K), std=0.125))
    b = synth.round_bf16(synth.normal(3100 + N, (B, K, N), std=0.125))
    ta = dev(a, cuda, torch.bfloat16)
    tb = dev(b, cuda, torch.bfloat16)
    if a_t:  # same values, M-contiguous storage
        ta = ta.transpose(1, 2).contiguous().transpose(1, 2)
    if b_t:  # same values, K-contiguous storage
        tb = tb.transpose(1, 2).contiguous().transpose(1, 2)
    ref = orc.dot_general(a, [2], [0], b, [1], [0])
    c32 = ops.gemm(ta, tb, out_dtype=torch.float32).cpu().numpy()
    assert rel_err(c32, ref) <= 1e-4
    c16 = ops.gemm(ta, tb).float().cpu().numpy()
    assert rel_err(c16, ref) <= 1e-2


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
def test_f32_layouts(cuda, shape, a_t, b_t):
    B, M, N, K = shape
    a = synth.normal(3200 + M, (B, M, K), std=0.125)
    b = synth.normal(3300 + N, (B, K, N), std=0.125)
    ta, tb = dev(a, cuda), dev(b, cuda)
    if a_t:
        ta = ta.transpose(1, 2).contiguous().transpose(1, 2)
    if b_t:
        tb = tb.transpose(1, 2).contiguous().transpose(1, 2)
    c = ops.gemm(ta, tb).cpu().numpy()
    assert rel_err(c, orc.dot_general(a, [2], [0], b, [1], [0])) <= 1e-4


@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
def test_f32_layouts_large_tiles(cuda, a_t, b_t):
    """Big enough for the 256 x 256 fp32 tiles (>= 128 of them), ragged M, N, K."""
    g = torch.Generator(cuda).manual_seed(3401)
    ta = torch.randn((2, 2056, 140), device=cuda, generator=g) * 0.125
    tb = torch.randn((2, 140, 2060), device=cuda, generator=g) * 0.125
    if a_t:
        ta = ta.transpose(1, 2).contiguous().transpose(1, 2)
    if b_t:
        tb = tb.transpose(1, 2).contiguous().transpose(1, 2)
    c = ops.gemm(ta, tb)
    got, ref = _sampled_check(ta, tb, c, seed=7)
    assert rel_err(got, ref) <= 1e-4


@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_16bit_large_tiles_ragged(cuda, a_t, b_t, dt):
    """>= 128 tiles of 256 x 256 (the 4-wave core) with ragged M, N and K, every
    operand majorness, bf16 and f16, 16-bit and fp32 outputs, against fp64 dot
    products of the same input bytes (4096 sampled entries)."""
    ta = synth.normal_device(3501, (2, 2056, 200), std=0.125, device=cuda, dtype=dt)
    tb = synth.normal_device(3502, (2, 200, 2060), std=0.125, device=cuda, dtype=dt)
    if a_t:
        ta = ta.transpose(1, 2).contiguous().transpose(1, 2)
    if b_t:
        tb = tb.transpose(1, 2).contiguous().transpose(1, 2)
    c16 = ops.gemm(ta, tb)
    assert c16.dtype == dt
    got, ref = _sampled_check(ta, tb, c16, seed=11)
    # one 16-bit rounding of the fp32 result (bf16 2^-8, f16 2^-11), RMS-floored
    assert rel_err(got, ref) <= (1e-2 if dt == torch.bfloat16 else 1e-3)
    c32 = ops.gemm(ta, tb, out_dtype=torch.float32)
    got, ref = _sampled_check(ta, tb, c32, seed=12)
    assert rel_err(got, ref) <= 1e-4
    # the last row / column tiles (ragged edges) in full
    e32 = c32[:, 2048:, :].cpu().numpy()
    a = ta.float().cpu().numpy()
    b = tb.float().cpu().numpy()
    assert rel_err(e32, orc.dot_general(np.ascontiguousarray(a[:, 2048:]), [2], [0], b, [1], [0])) <= 1e-4
    e32 = c32[:, :, 2048:].cpu().numpy()
    assert rel_err(e32, orc.dot_general(a, [2], [0], np.ascontiguousarray(b[:, :, 2048:]), [1], [0])) <= 1e-4


@pytest.mark.parametrize("K", [1024, 1000])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_mn_major_core_matches_k_major_core(cuda, K, dt):
    """Both operands MN-contiguous (a weight-gradient layout) run the 32-deep,
    four-stage core; the same values K-contiguous run the 64-deep core.  Same MFMA,
    same k order per accumulator: bit-identical products, for a K that fills whole
    k-tiles (steady-state loop) and one that does not, 16-bit and fp32 outputs; and
    sampled entries against fp64."""
    # [2, 2304, K] x [2, K, 2048]: 144 tiles of 256 x 256 (the 256 x 256 cores)
    ta_k = synth.normal_device(3601, (2, 2304, K), std=0.125, device=cuda, dtype=dt)
    tb_k = synth.normal_device(3602, (2, K, 2048), std=0.125, device=cuda, dtype=dt).transpose(1, 2).contiguous().transpose(1, 2)
    ta_mn = ta_k.transpose(1, 2).contiguous().transpose(1, 2)   # [2, 2304, K] with unit M stride
    tb_mn = tb_k.contiguous()                                   # [2, K, 2048] row-major: unit N stride
    assert ta_mn.stride(1) == 1 and tb_mn.stride(2) == 1 and ta_k.stride(2) == 1 and tb_k.stride(1) == 1
    for out_dtype in (dt, torch.float32):
        c_mn = ops.gemm(ta_mn, tb_mn, out_dtype=out_dtype)
        c_k = ops.gemm(ta_k, tb_k, out_dtype=out_dtype)
        assert torch.equal(c_mn, c_k)
    got, ref = _sampled_check(ta_mn, tb_mn, c_mn, seed=13)
    assert rel_err(got, ref) <= 1e-4


@pytest.mark.parametrize("shape", [(2, 2056, 2312, 200), (1, 4104, 2056, 72), (3, 1032, 2568, 520)])
@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
def test_16bit_large_grids_ragged_layouts(cuda, shape, a_t, b_t):
    """>= 128 tiles of 256 x 256 with ragged M, N and K (k-tiles of 32 and 64 cut
    short) and batches, every operand majorness: sampled entries and the whole last
    row tile and column tile against fp64, bf16 and fp32 outputs."""
    B, M, N, K = shape
    ta = synth.normal_device(3801 + M, (B, M, K), std=0.125, device=cuda, dtype=torch.bfloat16)
    tb = synth.normal_device(3802 + N, (B, K, N), std=0.125, device=cuda, dtype=torch.bfloat16)
    if a_t:
        ta = ta.transpose(1, 2).contiguous().transpose(1, 2)
    if b_t:
        tb = tb.transpose(1, 2).contiguous().transpose(1, 2)
    c16 = ops.gemm(ta, tb)
    got, ref = _sampled_check(ta, tb, c16, seed=15)
    assert rel_err(got, ref) <= 1e-2
    c32 = ops.gemm(ta, tb, out_dtype=torch.float32)
    got, ref = _sampled_check(ta, tb, c32, seed=16)
    assert rel_err(got, ref) <= 1e-4
    a = ta.float().cpu().numpy()
    b = tb.float().cpu().numpy()
    m0, n0 = (M - 1) // 256 * 256, (N - 1) // 256 * 256
    e = c32[:, m0:, :].cpu().numpy()
    assert rel_err(e, orc.dot_general(np.ascontiguousarray(a[:, m0:]), [2], [0], b, [1], [0])) <= 1e-4
    e = c32[:, :, n0:].cpu().numpy()
    assert rel_err(e, orc.dot_general(a, [2], [0], np.ascontiguousarray(b[:, :, n0:]), [1], [0])) <= 1e-4


@pytest.mark.parametrize("K", [16, 32, 1000, 1024])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_cores_bit_identical_across_layouts(cuda, K, dt):
    """The same values in all four operand layouts take three code paths at more than
    128 tiles of 256 x 256 (here 136): A K- / B N-contiguous the 4-wave 16x16x32 core,
    B K-contiguous (A either way) the 8-wave 64-deep 16x16x32 core, both MN-contiguous
    the 4-wave 32x32x16 core.  The products must agree bit for bit, for K inside one
    k-tile (16, 32: the MFMAs run straight into the epilogue), a ragged K and one that
    reaches the steady-state loop; plus sampled entries against fp64."""
    a_k = synth.normal_device(3701, (1, 2048, K), std=0.125, device=cuda, dtype=dt)       # A K-contiguous
    b_n = synth.normal_device(3702, (1, K, 4352), std=0.125, device=cuda, dtype=dt)       # B N-contiguous
    a_m = a_k.transpose(1, 2).contiguous().transpose(1, 2)
    b_k = b_n.transpose(1, 2).contiguous().transpose(1, 2)
    assert a_k.stride(2) == 1 and a_m.stride(1) == 1 and b_n.stride(2) == 1 and b_k.stride(1) == 1
    outs = [ops.gemm(a, b) for a, b in ((a_k, b_n), (a_k, b_k), (a_m, b_k), (a_m, b_n))]
    for c in outs[1:]:
        assert torch.equal(c, outs[0])
    got, ref = _sampled_check(a_k, b_n, outs[0], seed=14)
    assert rel_err(got, ref) <= (1e-2 if dt == torch.bfloat16 else 1e-3)


@pytest.mark.parametrize("K", [1000, 4096])
@pytest.mark.parametrize("layout", ["km", "kk", "mm", "mk"])
def test_small_grid_core_matches_large_grid_cores(cuda, K, layout):
    """A grid of 128 tiles of 256 x 256 ([2048, K] x [K, 4096]) runs the 128 x 128
    core (two workgroups per CU); the same product as batch 0 of a two-batch call
    (256 tiles) runs a 256 x 256 core.  Both must give the same bits, in every
    operand layout, with bf16 and fp32 outputs."""
    a2 = synth.normal_device(3801, (2, 2048, K), std=0.125, device=cuda, dtype=torch.bfloat16)
    b2 = synth.normal_device(3802, (2, K, 4096), std=0.125, device=cuda, dtype=torch.bfloat16)
    if layout[0] == "m":
        a2 = a2.transpose(1, 2).contiguous().transpose(1, 2)
    if layout[1] == "k":
        b2 = b2.transpose(1, 2).contiguous().transpose(1, 2)
    for odt in (torch.bfloat16, torch.float32):
        c2 = ops.gemm(a2, b2, out_dtype=odt)
        c1 = ops.gemm(a2[:1], b2[:1], out_dtype=odt)
        assert torch.equal(c1[0], c2[0])
    got, ref = _sampled_check(a2[:1], b2[:1], c1, seed=15)
    assert rel_err(got, ref) <= 1e-4


@pytest.mark.parametrize("shape", SHAPES)
def test_f16_layouts(cuda, shape):
    """f16 DotGeneral (the f16 MFMA) on the small-tile cores and the generic path."""
    B, M, N, K = shape
    a = synth.normal(3600 + M, (B, M, K), std=0.125).astype(np.float16).astype(np.float32)
    b = synth.normal(3700 + N, (B, K, N), std=0.125).astype(np.float16).astype(np.float32)
    ta, tb = dev(a, cuda, torch.float16), dev(b, cuda, torch.float16)
    ref = orc.dot_general(a, [2], [0], b, [1], [0])
    assert rel_err(ops.gemm(ta, tb, out_dtype=torch.float32).cpu().numpy(), ref) <= 1e-4
    assert rel_err(ops.gemm(ta, tb).float().cpu().numpy(), ref) <= 1e-3
    # a column view of odd width takes the generic kernel
    tbo = tb[:, :, : max(1, N - 1)]
    ref = orc.dot_general(a, [2], [0], np.ascontiguousarray(b[:, :, : max(1, N - 1)]), [1], [0])
    assert rel_err(ops.gemm(ta, tbo, out_dtype=torch.float32).cpu().numpy(), ref) <= 1e-4


def test_generic_path_odd_strides(cuda):
    """Shapes/strides the vector paths cannot address fall back to the generic kernel."""
    a = synth.normal(3400, (2, 33, 19))
    b = synth.normal(3401, (2, 19, 27))
    c = ops.gemm(dev(a, cuda), dev(b, cuda)).cpu().numpy()
    assert rel_err(c, orc.dot_general(a, [2], [0], b, [1], [0])) <= 1e-5
    ab = synth.round_bf16(a)
    bb = synth.round_bf16(b)
    c = ops.gemm(dev(ab, cuda, torch.bfloat16), dev(bb, cuda, torch.bfloat16),
                 out_dtype=torch.float32).cpu().numpy()
    assert rel_err(c, orc.dot_general(ab, [2], [0], bb, [1], [0])) <= 1e-5


def _sampled_check(ta, tb, c, count=4096, seed=0):
    """Size-independent check of a full-size product: `count` random entries of c
    against fp64 dot products computed on the host from the same input bytes."""
    B, M, K = ta.shape
    N = tb.shape[2]
    rng = np.random.default_rng(seed)
    bs = rng.integers(0, B, count)
    ms = rng.integers(0, M, count)
    ns = rng.integers(0, N, count)
    a = ta.float().cpu().numpy()
    b = tb.float().cpu().numpy()
    ref = orc.dot_sampled(a, b, bs, ms, ns)
    got = c.float().cpu().numpy()[bs, ms, ns]
    return got, ref


def test_dot_general_config_bf16(cuda):
    """BASELINE config: A [8,2048,4096] x B [8,4096,4096], bf16, fp32 accumulate,
    bf16 out; entries ~ N(0, 1/64) from the SplitMix64 streams 3001 / 3002."""
    ta = synth.normal_device(3001, (8, 2048, 4096), std=0.125, device=cuda, dtype=torch.bfloat16)
    tb = synth.normal_device(3002, (8, 4096, 4096), std=0.125, device=cuda, dtype=torch.bfloat16)
    c = ops.gemm(ta, tb)
    got, ref = _sampled_check(ta, tb, c)
    assert rel_err(got, ref) <= 1e-2
    assert norm_err(got, ref) <= 4e-3
    c32 = ops.gemm(ta, tb, out_dtype=torch.float32)
    got, ref = _sampled_check(ta, tb, c32, seed=1)
    assert rel_err(got, ref) <= 1e-4


def test_dot_general_config_f32(cuda):
    ta = synth.normal_device(3001, (8, 2048, 4096), std=0.125, device=cuda)
    tb = synth.normal_device(3002, (8, 4096, 4096), std=0.125, device=cuda)
    c = ops.gemm(ta, tb)
    got, ref = _sampled_check(ta, tb, c)
    assert rel_err(got, ref) <= 1e-4


def test_attention_shapes_bf16(cuda):
    """The two attention GEMMs at config shape: Q.K^T (rhs K-contiguous) and P.V."""
    g = torch.Generator(cuda).manual_seed(4001)
    q = torch.randn((64, 2048, 128), device=cuda, generator=g).to(torch.bfloat16)
    k = torch.randn((64, 2048, 128), device=cuda, generator=g).to(torch.bfloat16)
    s = ops.gemm(q, k.transpose(1, 2), out_dtype=torch.float32)
    got, ref = _sampled_check(q, k.transpose(1, 2), s)
    assert rel_err(got, ref) <= 1e-4
    p = torch.softmax(s[:, :, :], dim=-1).to(torch.bfloat16)
    v = torch.randn((64, 2048, 128), device=cuda, generator=g).to(torch.bfloat16)
    o = ops.gemm(p, v, out_dtype=torch.float32)
    got, ref = _sampled_check(p, v, o, seed=2)
    assert rel_err(got, ref) <= 1e-4


def test_empty_and_k0(cuda):
    a = torch.empty((2, 0, 16), device=cuda)
    b = torch.empty((2, 16, 8), device=cuda)
    assert ops.gemm(a, b).shape == (2, 0, 8)
    a = torch.empty((1, 4, 0), device=cuda)
    b = torch.empty((1, 0, 8), device=cuda)
    c = ops.gemm(a, b)
    assert torch.count_nonzero(c).item() == 0


@pytest.mark.parametrize("G,M,N,K", [(3, 2048, 2048, 1024), (2, 2000, 2056, 520), (4, 1032, 2312, 200),
                                     (3, 300, 264, 72), (2, 256, 256, 40)])
@pytest.mark.parametrize("dt,odt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                    (torch.bfloat16, torch.float32)])
def test_gemm_grouped_equals_separate(cuda, G, M, N, K, dt, odt):
    """ghip_gemm_grouped: G products sharing A in one launch (>= 128 tiles of 256 x
    256: the grouped 4-wave grid; fewer: one dispatch per product) equal the
    stand-alone ghip_gemm_batched results bit for bit, ragged M, N and K included;
    plus sampled entries of every product against fp64."""
    a = synth.normal_device(3901 + M, (M, K), std=0.125, device=cuda, dtype=dt)
    bs = [synth.normal_device(3902 + g, (K, N), std=0.125, device=cuda, dtype=dt) for g in range(G)]
    got = ops.gemm_grouped(a, bs, out_dtype=odt)
    torch.cuda.synchronize()
    for g in range(G):
        ref_c = ops.gemm(a, bs[g], out_dtype=odt)
        assert torch.equal(got[g], ref_c), f"product {g} differs from the stand-alone GEMM"
        s_got, s_ref = _sampled_check(a[None], bs[g][None], got[g][None], count=1024, seed=20 + g)
        assert rel_err(s_got, s_ref) <= (1e-4 if odt == torch.float32 else 1e-2)


def test_gemm_grouped_f32_and_rejects(cuda):
    """fp32 operands run product by product (equal to the batched entry); groups
    outside 1..4 are rejected."""
    a = synth.normal_device(3911, (300, 130), device=cuda)
    bs = [synth.normal_device(3912 + g, (130, 270), device=cuda) for g in range(3)]
    got = ops.gemm_grouped(a, bs)
    for g in range(3):
        assert torch.equal(got[g], ops.gemm(a, bs[g]))
    with pytest.raises(Exception):
        ops.gemm_grouped(a, bs + bs)  # 6 groups
