"""Operands whose slices span more than 4 GiB (one batch slice of a DotGeneral
operand, one (batch, kv head) slice of attention's K / V).

The MFMA kernels address their operands through buffer descriptors with 32-bit
records and offsets, based at each tile (and k step, or key tile).  Slices of
2 GiB or more run the same cores compiled with 64-bit records (the BIG
instantiations); everything else runs the 32-bit forms.  Each case here compares
the large-slice result bit for bit with the same product computed from a compact
copy of the operand (whose slice is small, so the 32-bit form runs): both forms
issue the same MFMAs in the same order, so any addressing mistake past 2 or 4 GiB
shows as a bit difference.  The large slices come either from genuinely large
tensors (a block of rows repeated past 4 GiB: every block of the result must equal
the small product) or from strided views whose row stride spreads a few thousand
rows over more than 4 GiB (only the rows in use are written).

Each case allocates ~4.5 GB of device memory and frees it before the next."""
import gc

import numpy as np
import pytest
import torch

from gomlx_hip import ops, synth
from gomlx_hip.backend import Backend, dtypes, make_shape
from conftest import norm_err

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
GiB = 1 << 30


@pytest.fixture(autouse=True)
def _free(cuda):
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _rand(cuda, shape, seed, dtype=BF16, std=0.05):
    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    return (torch.randn(shape, device=cuda, generator=g) * std).to(dtype)


def _strided_rows(cuda, rows, cols, stride, seed, dtype=BF16):
    """[rows, cols] view with row stride `stride` elements into an allocation of
    rows x stride (only the viewed elements are written)."""
    buf = torch.empty((rows, stride), device=cuda, dtype=dtype)
    v = buf[:, :cols]
    v.copy_(_rand(cuda, (rows, cols), seed, dtype))
    return v


def _span_bytes(t):
    return ((t.shape[0] - 1) * t.stride(0) + (t.shape[1] - 1) * t.stride(1) + 1) * t.element_size()


def _log(msg):
    print(msg, flush=True)


def test_gemm_rows_past_4gib(cuda):
    """A [270336, 8192] bf16 (4.4 GB, K-contiguous): 33 copies of one 8192-row block;
    every block of A.B must equal block . B (4-wave K-contiguous core, 64-bit form)."""
    reps, mb, K, N = 33, 8192, 8192, 256
    a0 = _rand(cuda, (mb, K), 1)
    b = _rand(cuda, (K, N), 2)
    a = a0.repeat(reps, 1)
    assert a.numel() * 2 > 4 * GiB
    _log(f"gemm A{tuple(a.shape)} x B{tuple(b.shape)}")
    c = ops.gemm(a, b)
    c0 = ops.gemm(a0, b, k_split=False)  # (128 tiles would split the contraction: another summation order)
    torch.cuda.synchronize()
    cv = c.view(reps, mb, N)
    for r in range(reps):
        assert torch.equal(cv[r], c0), f"row block {r} differs"
    ref = a0[:256].float() @ b.float()
    assert norm_err(c0[:256].float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2


def test_gemm_generic_fallback_past_4gib(cuda):
    """The same A with N = 64 (a grid the 256 x 256 cores do not take): the generic
    kernel; every block equal, and within bf16 tolerance of fp32."""
    reps, mb, K, N = 33, 8192, 8192, 64
    a0 = _rand(cuda, (mb, K), 3)
    b = _rand(cuda, (K, N), 4)
    a = a0.repeat(reps, 1)
    _log(f"gemm (generic) A{tuple(a.shape)} x B{tuple(b.shape)}")
    c = ops.gemm(a, b)
    torch.cuda.synchronize()
    cv = c.view(reps, mb, N)
    for r in range(1, reps):
        assert torch.equal(cv[r], cv[0]), f"row block {r} differs"
    ref = a0[:512].float() @ b.float()
    assert norm_err(cv[0, :512].float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2


# (layout, M, N, K): the operand made large by a wide row stride
#   a_km: A K-contiguous, rows 1114112 elements apart (4-wave K-contiguous core)
#   a_mn: A MN-contiguous ([K, M] storage), k rows 1114112 apart (4-wave MN core)
#   b_mn: B N-contiguous, k rows far apart (4-wave K-contiguous core, large B)
#   b_k:  B K-contiguous ([N, K] storage), n rows far apart (8-wave 64-deep core)
STRIDED = [("a_km", 2048, 8192, 2048), ("a_mn", 4096, 4096, 2048), ("b_mn", 2048, 8192, 2048),
           ("b_k", 4096, 2048, 2048)]


@pytest.mark.parametrize("layout,M,N,K", STRIDED)
def test_gemm_strided_operand_past_4gib(cuda, layout, M, N, K):
    S = 1114112
    if layout == "a_km":
        a = _strided_rows(cuda, M, K, S, 10)
        b = _rand(cuda, (K, N), 11)
        a_c, b_c = a.contiguous(), b
        big = a
    elif layout == "a_mn":
        at = _strided_rows(cuda, K, M, S, 12)
        a = at.t()
        b = _rand(cuda, (K, N), 13)
        a_c, b_c = at.contiguous().t(), b
        big = at
    elif layout == "b_mn":
        a = _rand(cuda, (M, K), 14)
        b = _strided_rows(cuda, K, N, S, 15)
        a_c, b_c = a, b.contiguous()
        big = b
    else:
        a = _rand(cuda, (M, K), 16)
        bt = _strided_rows(cuda, N, K, S, 17)
        b = bt.t()
        a_c, b_c = a, bt.contiguous().t()
        big = bt
    assert _span_bytes(big) > 4 * GiB
    _log(f"gemm strided {layout} M={M} N={N} K={K} span={_span_bytes(big)}")
    c = ops.gemm(a, b)
    c_ref = ops.gemm(a_c, b_c)
    torch.cuda.synchronize()
    assert torch.equal(c, c_ref)
    ref = a_c[:256].float() @ b_c.float()
    assert norm_err(c[:256].float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2


def test_gemm_f32_strided_past_4gib(cuda):
    """fp32 A with rows 560000 elements apart (4.6 GB span): the fp32 MFMA core's
    64-bit form, bit-identical to the compact copy."""
    M, N, K, S = 2048, 4096, 2048, 560000
    a = _strided_rows(cuda, M, K, S, 20, torch.float32)
    b = _rand(cuda, (K, N), 21, torch.float32)
    assert _span_bytes(a) > 4 * GiB
    _log(f"gemm f32 strided M={M} N={N} K={K}")
    c = ops.gemm(a, b)
    c_ref = ops.gemm(a.contiguous(), b)
    torch.cuda.synchronize()
    assert torch.equal(c, c_ref)


def test_graph_epilogue_rows_past_4gib(cuda):
    """DotGeneral + bias through Builder / Compile / Execute with x [270336, 8192]
    bf16 (a 4.4 GB parameter): the generated epilogue kernel's 64-bit form.  Every
    8192-row block of the result equals the small graph's result (N = 1024, so the
    small graph's 512 tiles of 128 x 128 run the fused epilogue too rather than a
    contraction split)."""
    reps, mb, K, N = 33, 8192, 8192, 1024
    rng = np.random.default_rng(5)
    x0 = synth.to_bf16_bits(rng.standard_normal((mb, K), dtype=np.float32) * 0.05)
    w = synth.to_bf16_bits(rng.standard_normal((K, N), dtype=np.float32) * 0.05)
    bias = synth.to_bf16_bits(rng.standard_normal((N,), dtype=np.float32))
    be = Backend("")
    try:
        def run(xbits, rows):
            b = be.Builder("big_epi")
            f = b.Main()
            px = f.Parameter("x", make_shape(dtypes.BFloat16, rows, K))
            pw = f.Parameter("w", make_shape(dtypes.BFloat16, K, N))
            pb = f.Parameter("b", make_shape(dtypes.BFloat16, N))
            d = f.DotGeneral(px, [1], [], pw, [0], [])
            f.Return([f.Add(d, f.BroadcastInDim(pb, make_shape(dtypes.BFloat16, rows, N), [1]))])
            ex = b.Compile()
            plan = ex.Plan()
            bufs = [be.BufferFromFlatData(0, xbits, make_shape(dtypes.BFloat16, rows, K)),
                    be.BufferFromFlatData(0, w, make_shape(dtypes.BFloat16, K, N)),
                    be.BufferFromFlatData(0, bias, make_shape(dtypes.BFloat16, N))]
            (r,) = ex.Execute(bufs, None, 0)
            out = be.BufferToFlatData(r).reshape(rows, N).copy()
            ex.Finalize()
            return plan, out
        plan0, y0 = run(x0, mb)
        xb = np.tile(x0, (reps, 1))
        assert xb.nbytes > 4 * GiB
        _log(f"graph DotGeneral+bias x[{reps * mb},{K}]")
        plan, y = run(xb, reps * mb)
        del xb
        assert "gemm_batched+epilogue" in plan and "gemm_batched+epilogue" in plan0, (plan, plan0)
        yv = y.reshape(reps, mb, N)
        for r in range(reps):
            assert np.array_equal(yv[r], y0), f"row block {r} differs"
    finally:
        be.Finalize()


@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_kv_past_4gib(cuda, masked):
    """K / V [1, 139264 keys, 1 head, 128] bf16 viewed with a 16384-element key
    stride (4.6 GB per slice): the 16-bit kernel's 64-bit form (split schedule
    without a mask, plain with a bool mask), bit-identical to compact K / V."""
    Sq, Sk, D, S = 256, 139264, 128, 16384
    q = _rand(cuda, (1, 1, Sq, D), 30, std=1.0)
    kb = _strided_rows(cuda, Sk, D, S, 31)
    vb = _strided_rows(cuda, Sk, D, S, 32)
    k, v = kb[None, None], vb[None, None]
    assert _span_bytes(kb) > 4 * GiB
    kc, vc = k.contiguous(), v.contiguous()
    scale = D ** -0.5
    _log(f"sdpa Sq={Sq} Sk={Sk} key stride {S} masked={masked}")
    if masked:
        g = torch.Generator(device=cuda)
        g.manual_seed(33)
        m = torch.rand((Sq, Sk), device=cuda, generator=g) > 0.25
        o = ops.sdpa_masked(q, k, v, m, scale, False)
        o_ref = ops.sdpa_masked(q, kc, vc, m, scale, False)
    else:
        o = ops.sdpa(q, k, v, scale, False)
        o_ref = ops.sdpa(q, kc, vc, scale, False)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    # and against an fp32 reference on a few queries
    s = (q[0, 0, :8].float() @ kc[0, 0].float().t()) * scale
    if masked:
        s = s.masked_fill(~m[:8], float("-inf"))
    ref = torch.softmax(s, -1) @ vc[0, 0].float()
    assert norm_err(o[0, 0, :8].float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2
