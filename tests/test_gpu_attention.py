"""Parity of the fused attention kernel (ghip_sdpa_fwd) against the oracle's
attention (fp64, oracle/oracle.c orc_sdpa following function.go:2669-2907).

Tolerances: bf16 inputs, fp32 softmax / accumulation, P rounded to bf16 before the
second product and the output rounded to bf16.  Normwise ||got - ref|| / ||ref||
<= 1e-2 (the north-star bf16 bound).  Elementwise (RMS-floored, conftest.rel_err)
<= 2.5e-2: two bf16 roundings of up to 2^-9 each (P, then the output) leave the
worst of ~10^5 outputs just above 1e-2."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import ops, synth
from gomlx_hip._lib import BackendError
from conftest import rel_err, norm_err

pytestmark = pytest.mark.gpu


def bf16(shape, seed):
    return synth.round_bf16(synth.normal(seed, shape))


CASES = [  # (B, H, Hkv, Sq, Sk, causal)
    (1, 2, 2, 128, 128, True),
    (1, 2, 2, 128, 128, False),
    (2, 4, 4, 200, 200, True),     # ragged query block and key tile
    (1, 8, 2, 320, 320, True),     # GQA 4:1
    (1, 2, 2, 130, 257, False),    # Sq != Sk, ragged
    (1, 2, 1, 64, 300, True),      # causal with Sk > Sq (top-left aligned mask)
    (1, 1, 1, 1, 1, True),
    (2, 3, 3, 1, 70, False),       # single query row
]


@pytest.mark.parametrize("case", CASES)
def test_sdpa_matches_oracle(cuda, case):
    B, H, Hkv, Sq, Sk, causal = case
    D = 128
    q = bf16((B, H, Sq, D), 4001 + Sq)
    k = bf16((B, Hkv, Sk, D), 4002 + Sk)
    v = bf16((B, Hkv, Sk, D), 4003 + Sk)
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    tq, tk, tv = (torch.from_numpy(a).to(cuda).to(torch.bfloat16) for a in (q, k, v))
    got = ops.sdpa(tq, tk, tv, scale, causal).float().cpu().numpy()
    assert norm_err(got, ref) <= 1e-2
    assert rel_err(got, ref) <= 2.5e-2


def test_sdpa_bshd_strides(cuda):
    """BSHD storage read through strides (no copy), output written as BSHD."""
    B, S, H, D = 2, 192, 4, 128
    q = bf16((B, S, H, D), 4101)
    k = bf16((B, S, H, D), 4102)
    v = bf16((B, S, H, D), 4103)
    to_bhsd = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
    ref = orc.sdpa(to_bhsd(q), to_bhsd(k), to_bhsd(v), scale=0.09, causal=True)
    tq, tk, tv = (torch.from_numpy(a).to(cuda).to(torch.bfloat16).transpose(1, 2) for a in (q, k, v))
    out = torch.empty((B, S, H, D), device=cuda, dtype=torch.bfloat16)
    ops.sdpa(tq, tk, tv, 0.09, True, out=out.transpose(1, 2))
    got = out.float().cpu().numpy().transpose(0, 2, 1, 3)
    assert norm_err(got, ref) <= 1e-2


def test_sdpa_causal_row0_is_v0(cuda):
    """Causal row 0 attends to key 0 only: out[.., 0, :] == v[.., 0, :] (function.go
    causal mask, the reference's known answer mpsgraph_test.go:2996-3015)."""
    B, H, S, D = 1, 2, 96, 128
    q, k, v = bf16((B, H, S, D), 4201), bf16((B, H, S, D), 4202), bf16((B, H, S, D), 4203)
    tq, tk, tv = (torch.from_numpy(a).to(cuda).to(torch.bfloat16) for a in (q, k, v))
    got = ops.sdpa(tq, tk, tv, 0.1, True).float().cpu().numpy()
    assert np.array_equal(got[:, :, 0, :], v[:, :, 0, :])


def test_sdpa_config_shape_rows(cuda):
    """BASELINE config shape B4 H16 S2048 D128 causal, checked on sampled rows of
    every head against the fp64 oracle on those rows."""
    B, H, S, D = 4, 16, 2048, 128
    q, k, v = bf16((B, H, S, D), 4301), bf16((B, H, S, D), 4302), bf16((B, H, S, D), 4303)
    tq, tk, tv = (torch.from_numpy(a).to(cuda).to(torch.bfloat16) for a in (q, k, v))
    got = ops.sdpa(tq, tk, tv, D ** -0.5, True).float().cpu().numpy()
    rows = np.array([0, 1, 127, 128, 1000, 2047])
    for b in (0, 3):
        ref = orc.sdpa(q[b:b + 1, :, rows], k[b:b + 1, :, : rows.max() + 1],
                       v[b:b + 1, :, : rows.max() + 1], scale=D ** -0.5, causal=False,
                       mask=np.arange(rows.max() + 1)[None, :] <= rows[:, None])
        assert norm_err(got[b:b + 1, :, rows], ref) <= 1e-2


def test_sdpa_rejects_unsupported(cuda):
    q = torch.zeros((1, 2, 16, 64), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, 1.0, False)  # head dim 64: not fused (composite path)
    q = torch.zeros((1, 3, 16, 128), device=cuda, dtype=torch.bfloat16)
    k = torch.zeros((1, 2, 16, 128), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, k, k, 1.0, False)  # 3 heads over 2 KV heads
    q = torch.zeros((1, 2, 16, 128), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, -0.5, False)  # negative scale: composite path only
