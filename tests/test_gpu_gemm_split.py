"""The contraction split of few-tile 16-bit products (ghip_gemm_batched_ws /
ghip_gemm_grouped_ws with a workspace): s ranges of K / s steps in one grid, fp32
partials summed in range order by a second kernel.

Parity against fp64 (the oracle's dot_general on the same input bytes: the whole
product where it is small, sampled entries otherwise) at the GEMM tolerances
(bf16 output <= 1e-2, fp32 output <= 1e-4 relative); every operand layout gives the
same bits (one core, one split); two calls give the same bits; the grouped entry
equals the stand-alone one product by product; the graph path runs the split
unfused and equals ops.gemm; workspace errors are reported."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import _lib, ops, synth
from gomlx_hip.backend import Backend, dtypes, make_shape
from conftest import rel_err

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _ab(cuda, M, N, K, dt, seed, layout="km"):
    a = synth.normal_device(seed, (M, K), std=0.125, device=cuda, dtype=dt)
    b = synth.normal_device(seed + 1, (K, N), std=0.125, device=cuda, dtype=dt)
    if layout[0] == "m":
        a = a.t().contiguous().t()        # A MN-contiguous ([K, M] storage)
    if layout[1] == "k":
        b = b.t().contiguous().t()        # B K-contiguous ([N, K] storage)
    return a, b


def _ref(a, b, rows=None):
    an = a.float().cpu().numpy()
    if rows is not None:
        an = an[rows]
    return orc.dot_general(np.ascontiguousarray(an), [1], [], np.ascontiguousarray(b.float().cpu().numpy()), [0], [])


# (M, N, K, splits): decoding-size rows, ragged M / N, 64-tile grids and a 256-tile
# one, a K that is not a power of two (14 ranges), ranges of 128 steps
SPLIT_SHAPES = [(16, 4096, 4096, 16), (1, 4096, 4096, 16), (300, 264, 4096, 16), (1024, 1024, 8192, 8),
                (2048, 2048, 8192, 2), (16, 4096, 14336, 14), (8, 4104, 11008, 4), (256, 4096, 4096, 4),
                (4, 2048, 1024, 8)]


@pytest.mark.parametrize("M,N,K,S", SPLIT_SHAPES)
@pytest.mark.parametrize("dt,odt", [(BF16, BF16), (BF16, F32), (F16, F16)])
def test_split_matches_oracle(cuda, M, N, K, S, dt, odt):
    ws = ops.gemm_workspace(dt, odt, 1, M, N, K, cuda)
    assert ws is not None and ws.numel() == S * M * N * 4, "the shape must take the split"
    print(f"split gemm M={M} N={N} K={K} s={S} {dt}->{odt}", flush=True)
    a, b = _ab(cuda, M, N, K, dt, 5101 + M)
    c = ops.gemm(a, b, out_dtype=odt, workspace=ws)
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 64 else np.random.default_rng(M).choice(M, 64, replace=False)
    ref = _ref(a, b, rows)
    got = c.float().cpu().numpy()[rows]
    tol = 1e-4 if odt == F32 else (1e-2 if dt == BF16 else 1e-3)
    assert rel_err(got, ref) <= tol


# fp32 operands (the fp32 MFMA core's ranges; a split only fills idle CUs):
# (M, N, K, splits)
F32_SHAPES = [(16, 4096, 4096, 8), (300, 264, 2048, 16), (1024, 1024, 8192, 4), (512, 4096, 4096, 2),
              (16, 4100, 14336, 7)]


@pytest.mark.parametrize("M,N,K,S", F32_SHAPES)
@pytest.mark.parametrize("odt", [F32, BF16])
def test_split_f32_matches_oracle(cuda, M, N, K, S, odt):
    ws = ops.gemm_workspace(F32, odt, 1, M, N, K, cuda)
    assert ws is not None and ws.numel() == S * M * N * 4, "the shape must take the split"
    print(f"split gemm f32 M={M} N={N} K={K} s={S} -> {odt}", flush=True)
    a, b = _ab(cuda, M, N, K, F32, 5601 + M)
    c = ops.gemm(a, b, out_dtype=odt, workspace=ws)
    c2 = ops.gemm(a, b, out_dtype=odt, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(c, c2)
    rows = np.arange(M) if M <= 64 else np.random.default_rng(M).choice(M, 64, replace=False)
    ref = _ref(a, b, rows)
    got = c.float().cpu().numpy()[rows]
    assert rel_err(got, ref) <= (1e-4 if odt == F32 else 1e-2)


@pytest.mark.parametrize("dt", [BF16, F32])
def test_split_columns_not_multiple_of_4(cuda, dt):
    """N = 1030 with B K-contiguous ([N, K] storage; an N-contiguous B needs N to be
    a multiple of the vector width): the partials' stores and the sum run their
    scalar forms; against fp64, and two calls give the same bits."""
    M, N, K = 16, 1030, 4096
    ws = ops.gemm_workspace(dt, dt, 1, M, N, K, cuda)
    assert ws is not None
    a, b = _ab(cuda, M, N, K, dt, 5701, "kk")
    c = ops.gemm(a, b, workspace=ws)
    c2 = ops.gemm(a, b, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(c, c2)
    assert rel_err(c.float().cpu().numpy(), _ref(a, b)) <= (1e-4 if dt == F32 else 1e-2)


@pytest.mark.parametrize("dt", [BF16, F32])
def test_split_32_row_tiles_match_128_row_tiles(cuda, dt):
    """At most 32 rows run the split on 32 x 128 tiles, more rows on 128 x 128 ones
    (same MFMA, same k order per accumulator): the 16-row product equals the first 16
    rows of the 33-row product that extends it, bit for bit (both split into the same
    ranges: 16 tiles of 128 x 128 either way)."""
    N, K = 2048, 4096
    a33 = synth.normal_device(5801, (33, K), std=0.125, device=cuda, dtype=dt)
    b = synth.normal_device(5802, (K, N), std=0.125, device=cuda, dtype=dt)
    w16 = ops.gemm_workspace(dt, dt, 1, 16, N, K, cuda)
    w33 = ops.gemm_workspace(dt, dt, 1, 33, N, K, cuda)
    assert w16.numel() // (16 * N * 4) == w33.numel() // (33 * N * 4) > 1
    for odt in (dt, F32):
        c16 = ops.gemm(a33[:16], b, out_dtype=odt)
        c33 = ops.gemm(a33, b, out_dtype=odt)
        assert torch.equal(c16, c33[:16])


@pytest.mark.parametrize("M,N,K", [(16, 4096, 4096), (304, 264, 4096), (1024, 1024, 8192)])
def test_split_bit_identical_across_layouts(cuda, M, N, K):
    """All four operand layouts run the 128 x 128 core over the same ranges: the
    same bits, bf16 and fp32 operands, 16-bit and fp32 outputs (M and N multiples
    of 8, which MN-contiguous operands need for the vector path; ragged against the
    128 x 128 tiles)."""
    for dt in (BF16, F32):
        outs = {}
        for layout in ("km", "kk", "mk", "mm"):
            a, b = _ab(cuda, M, N, K, dt, 5201, layout)
            outs[layout] = [ops.gemm(a, b, out_dtype=BF16), ops.gemm(a, b, out_dtype=F32)]
        for layout in ("kk", "mk", "mm"):
            for i in range(2):
                assert torch.equal(outs[layout][i], outs["km"][i]), (dt, layout)


def test_split_deterministic_and_close_to_unsplit(cuda):
    """Two calls: the same bits.  Against the unsplit product (k_split=False): equal
    up to the fp32 summation order, i.e. within a few bf16 roundings."""
    M, N, K = 64, 4096, 8192
    a, b = _ab(cuda, M, N, K, BF16, 5301)
    c1 = ops.gemm(a, b, out_dtype=F32)
    c2 = ops.gemm(a, b, out_dtype=F32)
    c0 = ops.gemm(a, b, out_dtype=F32, k_split=False)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    assert rel_err(c1.cpu().numpy(), c0.cpu().numpy()) <= 1e-5
    ref = _ref(a, b, np.arange(8))
    assert rel_err(c1[:8].cpu().numpy(), ref) <= 1e-4


@pytest.mark.parametrize("G,M,N,K", [(3, 16, 4096, 4096), (2, 1024, 2048, 8192), (4, 300, 264, 2048)])
def test_split_grouped_equals_separate(cuda, G, M, N, K):
    """ghip_gemm_grouped_ws: products that split run as the stand-alone split, one
    after another in one workspace: bit for bit the stand-alone results."""
    a = synth.normal_device(5401, (M, K), std=0.125, device=cuda, dtype=BF16)
    bs = [synth.normal_device(5402 + g, (K, N), std=0.125, device=cuda, dtype=BF16) for g in range(G)]
    assert ops.gemm_workspace(BF16, BF16, 1, M, N, K, cuda) is not None
    got = ops.gemm_grouped(a, bs)
    torch.cuda.synchronize()
    for g in range(G):
        assert torch.equal(got[g], ops.gemm(a, bs[g])), f"product {g}"


def test_split_workspace_errors(cuda):
    """A workspace smaller than the split needs, or misaligned, is an error; without
    one the product runs unsplit."""
    M, N, K = 16, 4096, 4096
    a, b = _ab(cuda, M, N, K, BF16, 5501)
    need = _lib.load().ghip_gemm_workspace_bytes(_lib.DT_BFLOAT16, _lib.DT_BFLOAT16, 1, M, N, K)
    small = torch.empty((need - 16,), dtype=torch.uint8, device=cuda)
    with pytest.raises(Exception, match="workspace"):
        ops.gemm(a, b, workspace=small)
    big = torch.empty((need + 64,), dtype=torch.uint8, device=cuda)
    with pytest.raises(Exception, match="aligned"):
        ops.gemm(a, b, workspace=big[8:])
    c = ops.gemm(a, b, k_split=False)
    assert rel_err(c[:4].float().cpu().numpy(), _ref(a, b, np.arange(4))) <= 1e-2


def test_graph_dot_bias_split(cuda):
    """DotGeneral + bias through Builder / Compile / Execute at a split shape: the
    plan runs the product with its contraction split (unfused: the bias add is an
    elementwise step), and the product equals ops.gemm's bit for bit; the sum is
    checked against fp64."""
    M, N, K = 16, 4096, 4096
    rng = np.random.default_rng(7)
    x = synth.to_bf16_bits(rng.standard_normal((M, K), dtype=np.float32) * 0.125)
    w = synth.to_bf16_bits(rng.standard_normal((K, N), dtype=np.float32) * 0.125)
    bias = synth.to_bf16_bits(rng.standard_normal((N,), dtype=np.float32))
    be = Backend("")
    try:
        b = be.Builder("split_dot")
        f = b.Main()
        px = f.Parameter("x", make_shape(dtypes.BFloat16, M, K))
        pw = f.Parameter("w", make_shape(dtypes.BFloat16, K, N))
        pb = f.Parameter("b", make_shape(dtypes.BFloat16, N))
        d = f.DotGeneral(px, [1], [], pw, [0], [])
        f.Return([d, f.Add(d, f.BroadcastInDim(pb, make_shape(dtypes.BFloat16, M, N), [1]))])
        ex = b.Compile()
        plan = ex.Plan()
        assert "contraction split in 16" in plan and "epilogue" not in plan, plan
        bufs = [be.BufferFromFlatData(0, x, make_shape(dtypes.BFloat16, M, K)),
                be.BufferFromFlatData(0, w, make_shape(dtypes.BFloat16, K, N)),
                be.BufferFromFlatData(0, bias, make_shape(dtypes.BFloat16, N))]
        prod, y = ex.Execute(bufs, None, 0)
        pn = be.BufferToFlatData(prod).reshape(M, N).copy()
        yn = be.BufferToFlatData(y).reshape(M, N).copy()
        ex.Finalize()
    finally:
        be.Finalize()
    xt = torch.from_numpy(x.view(np.int16)).to(cuda).view(BF16)
    wt = torch.from_numpy(w.view(np.int16)).to(cuda).view(BF16)
    ref_prod = ops.gemm(xt, wt).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(pn, ref_prod)
    xf = synth.bf16_bits_to_f32(x).astype(np.float64)
    wf = synth.bf16_bits_to_f32(w).astype(np.float64)
    ref = xf @ wf + synth.bf16_bits_to_f32(bias).astype(np.float64)
    assert rel_err(synth.bf16_bits_to_f32(yn), ref) <= 1e-2


@pytest.mark.parametrize("dt", [dtypes.BFloat16, dtypes.Float16])
def test_graph_split_sums_fold_into_consumers(cuda, dt):
    """A residual add after a split product, and SiLU(x.Wg) * (x.Wu) over two split
    products: the products' partials are summed by the consumers' generated
    kernels (no sum launches), bit for bit the plan compiled with
    GHIP_EPILOGUE_FUSION=0 (sum kernels, then the elementwise kernels); and
    against fp64 with the graph's rounding points."""
    import os
    M, K, N, F = 16, 4096, 2048, 4096
    rng = np.random.default_rng(11)

    # host storage: bf16 as its uint16 bit pattern, f16 as numpy float16
    def bits(a):
        return synth.to_bf16_bits(a) if dt == dtypes.BFloat16 else a.astype(np.float16)

    def val(b):
        return synth.bf16_bits_to_f32(b) if dt == dtypes.BFloat16 else b.astype(np.float32)
    x = bits(rng.standard_normal((M, K), dtype=np.float32))
    w1 = bits(rng.standard_normal((K, N), dtype=np.float32) * K ** -0.5)
    r = bits(rng.standard_normal((M, N), dtype=np.float32))
    wg = bits(rng.standard_normal((K, F), dtype=np.float32) * K ** -0.5)
    wu = bits(rng.standard_normal((K, F), dtype=np.float32) * K ** -0.5)
    shapes = [make_shape(dt, M, K), make_shape(dt, K, N), make_shape(dt, M, N), make_shape(dt, K, F),
              make_shape(dt, K, F)]
    host = [x, w1, r, wg, wu]
    be = Backend("")
    outs, plans = {}, {}
    try:
        for fuse in (True, False):
            os.environ["GHIP_EPILOGUE_FUSION"] = "1" if fuse else "0"
            try:
                b = be.Builder("split_fold")
                f = b.Main()
                px, pw1, pr, pwg, pwu = [f.Parameter(f"p{i}", s) for i, s in enumerate(shapes)]
                y1 = f.Add(f.DotGeneral(px, [1], [], pw1, [0], []), pr)
                g = f.DotGeneral(px, [1], [], pwg, [0], [])
                y2 = f.Mul(f.Mul(g, f.Logistic(g)), f.DotGeneral(px, [1], [], pwu, [0], []))
                f.Return([y1, y2])
                ex = b.Compile()
            finally:
                del os.environ["GHIP_EPILOGUE_FUSION"]
            plans[fuse] = ex.Plan()
            bufs = [be.BufferFromFlatData(0, a, s) for a, s in zip(host, shapes)]
            outs[fuse] = [be.BufferToFlatData(o).copy() for o in ex.Execute(bufs, None, 0)]
            ex.Finalize()
    finally:
        be.Finalize()
    assert plans[True].count("gemm_split_partials") == 3 and "sums the split partials of 2 products" in plans[True], \
        plans[True]
    assert "gemm_split_partials" not in plans[False] and plans[False].count("contraction split in") == 3, plans[False]
    for a, b in zip(outs[True], outs[False]):
        assert np.array_equal(a, b)
    xf, w1f, rf, wgf, wuf = (val(a).astype(np.float64) for a in host)
    rnd = (lambda a: synth.round_bf16(a.astype(np.float32)).astype(np.float64)) if dt == dtypes.BFloat16 else \
        (lambda a: a.astype(np.float16).astype(np.float64))
    ref1 = rnd(rnd(xf @ w1f) + rf)
    gq, uq = rnd(xf @ wgf), rnd(xf @ wuf)
    ref2 = rnd(rnd(gq * rnd(1 / (1 + np.exp(-gq)))) * uq)
    assert rel_err(val(outs[True][0]).reshape(M, N), ref1) <= 1e-2
    assert rel_err(val(outs[True][1]).reshape(M, F), ref2) <= 2e-2
