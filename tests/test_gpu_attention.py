"""Parity of the fused attention kernels (ghip_sdpa_fwd / ghip_sdpa_fwd_masked)
against the oracle's attention (fp64, oracle/oracle.c orc_sdpa following
function.go:2669-2907), for bf16 and f16 with head dims that are multiples of 8 up
to 256 (64 and 128 exactly, the others padded to 64 / 128 / 256), fp32 with head
dims that are multiples of 4 up to 128, and the reference's masks (boolean
keep-masks and additive masks of any rank broadcast to the scores,
function.go:2840-2878, 2959-2974).

Tolerances, fp32: fp32 products, sums and softmax (exponents by v_exp_f32, within
1 ulp), P unrounded: normwise <= 1e-5, elementwise <= 1e-4.
Tolerances, 16-bit: 16-bit inputs, fp32 softmax / accumulation, P rounded to the 16-bit
type before the second product and the output rounded once more.  Normwise
||got - ref|| / ||ref|| <= 1e-2 (the north-star bf16 bound).  Elementwise
(RMS-floored, conftest.rel_err) <= 2.5e-2: two bf16 roundings of up to 2^-9 each
(P, then the output) leave the worst of ~10^5 outputs just above 1e-2 (f16 rounds
8x finer, so the same bounds hold with room)."""
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


def r16(a, dt):
    """fp32 values rounded to dt (returned as fp32; fp32 unchanged)."""
    if dt == torch.float32:
        return np.asarray(a, np.float32)
    return synth.round_bf16(a) if dt == torch.bfloat16 else a.astype(np.float16).astype(np.float32)


def tols(dt):
    """(normwise, elementwise) bounds: fp32 or a 16-bit dtype (module docstring)."""
    return (1e-5, 1e-4) if dt == torch.float32 else (1e-2, 2.5e-2)


def dev(a, cuda, dt):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda).to(dt)


CASES = [  # (B, H, Hkv, Sq, Sk, causal)
    (1, 2, 2, 128, 128, True),
    (1, 2, 2, 128, 128, False),
    (2, 4, 4, 200, 200, True),     # ragged query block and key tile
    (1, 8, 2, 320, 320, True),     # GQA 4:1
    (1, 2, 2, 130, 257, False),    # Sq != Sk, ragged
    (1, 2, 1, 64, 300, True),      # causal with Sk > Sq (top-left aligned mask)
    (1, 1, 1, 1, 1, True),
    (2, 3, 3, 1, 70, False),       # single query row
    (1, 2, 2, 1100, 1100, True),   # causal with > 16 key tiles (the split K / V schedule), ragged
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kv_split", [True, False])
def test_sdpa_matches_oracle(cuda, case, D, dt, kv_split):
    """kv_split: with a workspace (ghip_sdpa_fwd_masked_ws), so the grids small
    enough split their key range; without one every case runs unsplit."""
    B, H, Hkv, Sq, Sk, causal = case
    q = r16(synth.normal(4001 + Sq, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4002 + Sk, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4003 + Sk, (B, Hkv, Sk, D)), dt)
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    tq, tk, tv = (dev(a, cuda, dt) for a in (q, k, v))
    got = ops.sdpa(tq, tk, tv, scale, causal, kv_split=kv_split).float().cpu().numpy()
    assert norm_err(got, ref) <= 1e-2
    assert rel_err(got, ref) <= 2.5e-2


# Grids of few (batch, head, query block) workgroups with long key ranges: the key
# range splits over several workgroups (ghip_sdpa_workspace_bytes > 0) and a second
# kernel merges them by log-sum-exp.
SPLIT_CASES = [  # (B, H, Hkv, Sq, Sk, causal)
    (2, 8, 2, 1, 4096, False),     # decoding, GQA 4:1
    (1, 4, 4, 16, 2048, False),    # a few queries
    (1, 4, 1, 1, 777, False),      # ragged last split (keys 640 .. 776)
    (1, 2, 2, 4200, 4200, True),   # causal prefill of 66 key tiles: later splits of early blocks hold no keys
    (3, 2, 1, 130, 4500, False),   # two query blocks, ragged
    (1, 8, 2, 40, 4500, False),    # grouped-query rows: 4 heads x 40 queries, two row blocks
    (2, 6, 3, 5, 700, False),      # grouped-query rows: 2 heads x 5 queries, ragged keys
]


@pytest.mark.parametrize("case", [(2, 8, 2, 3, 300, False), (1, 12, 4, 50, 200, False), (1, 16, 1, 1, 64, False)])
@pytest.mark.parametrize("D,dt", [(64, torch.bfloat16), (128, torch.float16), (256, torch.bfloat16)])
@pytest.mark.parametrize("kv_split", [True, False])
def test_sdpa_grouped_query_rows_match_oracle(cuda, case, D, dt, kv_split):
    """GQA without a causal mask and Sq < 128: the (head, query) rows of each kv
    head's group share workgroups (3 heads x 50 queries span two row blocks; 16
    heads of one query), with and without a workspace."""
    B, H, Hkv, Sq, Sk, causal = case
    q = r16(synth.normal(4121 + Sq, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4122 + Sk, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4123 + Sk, (B, Hkv, Sk, D)), dt)
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    got = ops.sdpa(*(dev(a, cuda, dt) for a in (q, k, v)), scale, causal, kv_split=kv_split)
    got = got.float().cpu().numpy()
    assert norm_err(got, ref) <= 1e-2
    assert rel_err(got, ref) <= 2.5e-2


@pytest.mark.parametrize("case", SPLIT_CASES)
@pytest.mark.parametrize("D,dt", [(64, torch.bfloat16), (128, torch.bfloat16), (128, torch.float16),
                                  (256, torch.bfloat16), (96, torch.float16)])
def test_sdpa_split_key_range_matches_oracle(cuda, case, D, dt):
    B, H, Hkv, Sq, Sk, causal = case
    assert ops.sdpa_workspace(torch.empty((B, H, Sq, D), dtype=dt, device=cuda), Hkv, Sk, causal) is not None
    q = r16(synth.normal(4101 + Sq, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4102 + Sk, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4103 + Sk, (B, Hkv, Sk, D)), dt)
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    tq, tk, tv = (dev(a, cuda, dt) for a in (q, k, v))
    got = ops.sdpa(tq, tk, tv, scale, causal)
    again = ops.sdpa(tq, tk, tv, scale, causal)
    assert torch.equal(got, again)  # the merge is in a fixed order
    got = got.float().cpu().numpy()
    assert norm_err(got, ref) <= 1e-2
    assert rel_err(got, ref) <= 2.5e-2
    unsplit = ops.sdpa(tq, tk, tv, scale, causal, kv_split=False).float().cpu().numpy()
    assert norm_err(got, unsplit) <= 1e-2


@pytest.mark.parametrize("kind", ["bool", "add"])
@pytest.mark.parametrize("mh", [1, 4])
def test_sdpa_split_key_range_masks(cuda, kind, mh):
    """Decoding shapes (grouped-query rows, split key range) with a bool keep-mask or
    an additive mask, broadcast over heads (mh 1) or per head (mh 4), one query row
    fully masked (NaN, as unsplit)."""
    B, H, Hkv, Sq, Sk, D = 2, 4, 2, 2, 3000, 128
    dt = torch.bfloat16
    q = r16(synth.normal(4111, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4112, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4113, (B, Hkv, Sk, D)), dt)
    rng = np.random.default_rng(4114 + mh)
    keep = rng.random((B, mh, Sq, Sk)) > 0.3
    keep[1, :, 1, :] = False
    if kind == "bool":
        mask = keep
        tm = torch.from_numpy(keep).to(cuda)
    else:
        mask = r16(np.where(keep, rng.normal(0.0, 1.0, keep.shape), -np.inf).astype(np.float32), dt)
        tm = dev(mask, cuda, dt)
    scale = D ** -0.5
    if kind == "bool":
        ref = orc.sdpa(q, k, v, scale=scale, causal=False, mask=mask)
    else:
        ref = orc.sdpa(q, k, v, scale=scale, causal=False, additive=mask)
    tq, tk, tv = (dev(a, cuda, dt) for a in (q, k, v))
    got = ops.sdpa_masked(tq, tk, tv, tm, scale, False).float().cpu().numpy()
    assert np.all(np.isnan(got[1, :, 1]))
    ok = ~np.isnan(ref)
    assert np.array_equal(ok, ~np.isnan(got))
    assert norm_err(got[ok], ref[ok]) <= 1e-2
    assert rel_err(got[ok], ref[ok]) <= 2.5e-2


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3], CASES[4], CASES[5], CASES[6]])
@pytest.mark.parametrize("D,dt", [(8, torch.bfloat16), (32, torch.bfloat16), (80, torch.float16),
                                  (96, torch.bfloat16), (96, torch.float16), (160, torch.bfloat16),
                                  (256, torch.bfloat16), (256, torch.float16)])
def test_sdpa_head_dims_match_oracle(cuda, case, D, dt):
    """16-bit head dims other than 64 / 128: padded to the next of 64 / 128 / 256
    (zero chunks past D, output columns past D never written)."""
    B, H, Hkv, Sq, Sk, causal = case
    q = r16(synth.normal(4021 + D, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4022 + D, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4023 + D, (B, Hkv, Sk, D)), dt)
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    # Output in a wider buffer: columns past D must stay as they were.
    wide = torch.full((B, H, Sq, D + 8), 7.0, device=cuda, dtype=dt)
    ops.sdpa(*(dev(a, cuda, dt) for a in (q, k, v)), scale, causal, out=wide[..., :D])
    got = wide[..., :D].float().cpu().numpy()
    assert torch.all(wide[..., D:] == 7.0)
    assert norm_err(got, ref) <= 1e-2
    assert rel_err(got, ref) <= 2.5e-2


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("D", [4, 32, 64, 96, 128])
def test_sdpa_f32_matches_oracle(cuda, case, D):
    """fp32 Q / K / V / O on fp32 MFMAs: every case, head dims 4 .. 128."""
    B, H, Hkv, Sq, Sk, causal = case
    q = synth.normal(4031 + Sq, (B, H, Sq, D))
    k = synth.normal(4032 + Sk, (B, Hkv, Sk, D))
    v = synth.normal(4033 + Sk, (B, Hkv, Sk, D))
    scale = D ** -0.5
    ref = orc.sdpa(q, k, v, scale=scale, causal=causal)
    got = ops.sdpa(*(dev(a, cuda, torch.float32) for a in (q, k, v)), scale, causal).cpu().numpy()
    assert norm_err(got, ref) <= 1e-5
    assert rel_err(got, ref) <= 1e-4


def test_sdpa_f32_large_scores(cuda):
    """fp32 with scores spread over ~±300 (scale 1, |q|, |k| ~ 4): exercises the
    lazy rescale of the running max and very small weights."""
    B, H, S, D = 1, 2, 520, 64
    q = synth.normal(4041, (B, H, S, D), std=2.2)
    k = synth.normal(4042, (B, H, S, D), std=2.2)
    v = synth.normal(4043, (B, H, S, D))
    for causal in (False, True):
        ref = orc.sdpa(q, k, v, scale=1.0, causal=causal)
        got = ops.sdpa(*(dev(a, cuda, torch.float32) for a in (q, k, v)), 1.0, causal).cpu().numpy()
        assert norm_err(got, ref) <= 1e-5
        assert rel_err(got, ref) <= 1e-4


def test_sdpa_head_dim_256_long(cuda):
    """Head dim 256 (one workgroup a CU) over many key tiles: B2 H4 S1536 causal,
    GQA 2:1, sampled rows against the oracle."""
    B, H, Hkv, S, D = 2, 4, 2, 1536, 256
    dt = torch.bfloat16
    q = bf16((B, H, S, D), 4051)
    k = bf16((B, Hkv, S, D), 4052)
    v = bf16((B, Hkv, S, D), 4053)
    got = ops.sdpa(*(dev(a, cuda, dt) for a in (q, k, v)), D ** -0.5, True).float().cpu().numpy()
    rows = np.array([0, 63, 64, 700, 1535])
    kmax = rows.max() + 1
    kr, vr = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    ref = orc.sdpa(q[:, :, rows], kr[:, :, :kmax], vr[:, :, :kmax], scale=D ** -0.5,
                   mask=np.arange(kmax)[None, :] <= rows[:, None])
    assert norm_err(got[:, :, rows], ref) <= 1e-2
    assert rel_err(got[:, :, rows], ref) <= 2.5e-2


MASKS = [  # (kind, mask shape as a function of (B, H, Sq, Sk))
    ("bool", lambda B, H, Sq, Sk: (B, 1, 1, Sk)),      # key padding per batch row
    ("bool", lambda B, H, Sq, Sk: (B, H, Sq, Sk)),
    ("bool", lambda B, H, Sq, Sk: (Sq, Sk)),
    ("add", lambda B, H, Sq, Sk: (B, 1, 1, Sk)),
    ("add", lambda B, H, Sq, Sk: (B, H, Sq, Sk)),
    ("add", lambda B, H, Sq, Sk: (1, Sk)),
    ("add", lambda B, H, Sq, Sk: (1, H, Sq, 1)),       # per-row constant: no effect
]


def _mask(kind, shape, seed, dt):
    """A boolean keep-mask (key 0 always kept, so no row is empty) or an additive
    mask in the 16-bit dtype with finite values and some -inf."""
    if kind == "bool":
        m = synth.uniform(seed, int(np.prod(shape))).reshape(shape) > 0.35
        m[..., 0] = True
        return m
    a = r16(synth.normal(seed, shape, std=1.5), dt)
    drop = synth.uniform(seed + 1, int(np.prod(shape))).reshape(shape) > 0.8
    if shape[-1] > 1:
        drop[..., 0] = False
        a = np.where(drop, -np.inf, a).astype(np.float32)
    return a


@pytest.mark.parametrize("mi", range(len(MASKS)))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D,dt", [(128, torch.bfloat16), (64, torch.float16), (96, torch.bfloat16),
                                  (128, torch.float32), (64, torch.float32), (96, torch.float32)])
def test_sdpa_masks_match_oracle(cuda, mi, causal, D, dt):
    """Every mask shape and kind, GQA, ragged query and key tiles."""
    B, H, Hkv, Sq, Sk = 2, 4, 2, 200, 264
    kind, fshape = MASKS[mi]
    q = r16(synth.normal(4401, (B, H, Sq, D)), dt)
    k = r16(synth.normal(4402, (B, Hkv, Sk, D)), dt)
    v = r16(synth.normal(4403, (B, Hkv, Sk, D)), dt)
    m = _mask(kind, fshape(B, H, Sq, Sk), 4404 + mi, dt)
    scale = D ** -0.5
    if kind == "bool":
        ref = orc.sdpa(q, k, v, mask=m, scale=scale, causal=causal)
        tm = torch.from_numpy(np.ascontiguousarray(m)).to(cuda)
    else:
        ref = orc.sdpa(q, k, v, additive=m, scale=scale, causal=causal)
        tm = dev(m, cuda, dt)
    got = ops.sdpa_masked(*(dev(a, cuda, dt) for a in (q, k, v)), tm, scale, causal).float().cpu().numpy()
    nt, et = tols(dt)
    assert norm_err(got, ref) <= nt
    assert rel_err(got, ref) <= et


@pytest.mark.parametrize("kind,mshape", [("bool", "b11k"), ("bool", "bhqk"), ("add", "b11k")])
def test_sdpa_masks_config_shape_rows(cuda, kind, mshape):
    """BASELINE attention shape B4 H16 S2048 D128 bf16, causal, with a key-padding
    mask [B,1,1,Sk], a full boolean mask [B,H,Sq,Sk], or an additive float mask
    [B,1,1,Sk]; sampled rows of every head of two batch rows against the oracle."""
    B, H, S, D = 4, 16, 2048, 128
    dt = torch.bfloat16
    tq = synth.normal_device(4501, (B, H, S, D), device=cuda, dtype=dt)
    tk = synth.normal_device(4502, (B, H, S, D), device=cuda, dtype=dt)
    tv = synth.normal_device(4503, (B, H, S, D), device=cuda, dtype=dt)
    shape = (B, 1, 1, S) if mshape == "b11k" else (B, H, S, S)
    if kind == "bool":
        u = synth.normal_device(4504, shape, device=cuda)
        tm = u > -1.0                                     # keeps ~84%
        tm[..., 0] = True
    else:
        tm = (synth.normal_device(4504, shape, device=cuda) * 2.0).to(dt)
    got = ops.sdpa_masked(tq, tk, tv, tm, D ** -0.5, True).float().cpu().numpy()
    rows = np.array([0, 1, 127, 128, 1000, 2047])
    kmax = rows.max() + 1
    q, k, v = (t.float().cpu().numpy() for t in (tq, tk, tv))
    m = (tm if kind == "bool" else tm.float()).cpu().numpy()
    causal = np.arange(kmax)[None, :] <= rows[:, None]
    for b in (0, 3):
        mb = m[b:b + 1, :, :, :kmax] if mshape == "b11k" else m[b:b + 1, :, rows, :kmax]
        if kind == "bool":
            ref = orc.sdpa(q[b:b + 1, :, rows], k[b:b + 1, :, :kmax], v[b:b + 1, :, :kmax], scale=D ** -0.5,
                           mask=mb & causal)
        else:
            add = np.where(causal, mb, -np.inf).astype(np.float32)
            ref = orc.sdpa(q[b:b + 1, :, rows], k[b:b + 1, :, :kmax], v[b:b + 1, :, :kmax], scale=D ** -0.5,
                           additive=add)
        assert norm_err(got[b:b + 1, :, rows], ref) <= 1e-2


@pytest.mark.parametrize("D,dt", [(128, torch.bfloat16), (96, torch.float16), (128, torch.float32),
                                  (40, torch.float32)])
def test_sdpa_fully_masked_row_is_nan(cuda, D, dt):
    """A query whose keys are all masked: NaN, like the reference's softmax of -inf
    (the oracle gives the same)."""
    B, H, S = 1, 2, 128
    q, k, v = bf16((B, H, S, D), 4601), bf16((B, H, S, D), 4602), bf16((B, H, S, D), 4603)
    m = np.ones((S, S), bool)
    m[5] = False
    got = ops.sdpa_masked(*(dev(a, cuda, dt) for a in (q, k, v)),
                          torch.from_numpy(m).to(cuda), 0.1, False).float().cpu().numpy()
    assert np.all(np.isnan(got[:, :, 5])) and np.all(np.isfinite(np.delete(got, 5, axis=2)))
    assert np.all(np.isnan(orc.sdpa(q, k, v, mask=m, scale=0.1)[:, :, 5]))


@pytest.mark.parametrize("kind", ["bool", "add"])
def test_composite_masked_softmax_general_masks(cuda, kind):
    """The composite's row kernel (ghip_scale_mask_softmax_rows_ex) with broadcast
    masks of both kinds, fp32 scores, against numpy."""
    B, H, Sq, Sk = 2, 3, 40, 70
    x = synth.normal(4701, (B, H, Sq, Sk))
    for shape in ((B, 1, 1, Sk), (B, H, Sq, Sk), (Sq, Sk)):
        m = _mask(kind, shape, 4702, torch.float32)
        for causal in (False, True):
            s = x.astype(np.float64) * 0.3
            s = np.where(m, s, -np.inf) if kind == "bool" else s + m
            if causal:
                s = np.where(np.tril(np.ones((Sq, Sk), bool)), s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            ref = p / p.sum(-1, keepdims=True)
            tm = torch.from_numpy(np.ascontiguousarray(m)).to(cuda)
            got = ops.scale_mask_softmax_ex(torch.from_numpy(x).to(cuda), 0.3, causal, tm).cpu().numpy()
            assert rel_err(got, ref) <= 1e-5


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


@pytest.mark.parametrize("D,dt", [(96, torch.bfloat16), (96, torch.float32), (64, torch.float32)])
def test_sdpa_bshd_strides_other_dims(cuda, D, dt):
    """BSHD storage through strides for a padded 16-bit head dim and for fp32."""
    B, S, H = 2, 160, 4
    q, k, v = (r16(synth.normal(4111 + i, (B, S, H, D)), dt) for i in range(3))
    to_bhsd = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
    ref = orc.sdpa(to_bhsd(q), to_bhsd(k), to_bhsd(v), scale=0.09, causal=True)
    tq, tk, tv = (torch.from_numpy(a).to(cuda).to(dt).transpose(1, 2) for a in (q, k, v))
    out = torch.empty((B, S, H, D), device=cuda, dtype=dt)
    ops.sdpa(tq, tk, tv, 0.09, True, out=out.transpose(1, 2))
    got = out.float().cpu().numpy().transpose(0, 2, 1, 3)
    assert norm_err(got, ref) <= tols(dt)[0]


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
    # 24 query rows per batch row (every 128-query block's first and last rows among
    # them, and the rows of the first and last 64-key tiles), every head, all 4
    # batch rows: 1536 rows of 128 outputs.
    rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, 255, 1000, 1023, 1024, 1983, 2047],
                                     np.random.default_rng(4304).integers(0, S, 12)]))
    kmax = rows.max() + 1
    for b in range(B):
        ref = orc.sdpa(q[b:b + 1, :, rows], k[b:b + 1, :, :kmax], v[b:b + 1, :, :kmax], scale=D ** -0.5,
                       causal=False, mask=np.arange(kmax)[None, :] <= rows[:, None])
        assert norm_err(got[b:b + 1, :, rows], ref) <= 1e-2
        assert rel_err(got[b:b + 1, :, rows], ref) <= 2.5e-2


def test_sdpa_rejects_unsupported(cuda):
    q = torch.zeros((1, 2, 16, 100), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, 1.0, False)  # 16-bit head dim not a multiple of 8: composite path
    q = torch.zeros((1, 2, 16, 264), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, 1.0, False)  # 16-bit head dim above 256
    q = torch.zeros((1, 2, 16, 256), device=cuda, dtype=torch.float32)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, 1.0, False)  # fp32 head dim above 128
    q = torch.zeros((1, 2, 16, 6), device=cuda, dtype=torch.float32)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, 1.0, False)  # fp32 head dim not a multiple of 4
    q = torch.zeros((1, 3, 16, 128), device=cuda, dtype=torch.bfloat16)
    k = torch.zeros((1, 2, 16, 128), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, k, k, 1.0, False)  # 3 heads over 2 KV heads
    q = torch.zeros((1, 2, 16, 128), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(BackendError):
        ops.sdpa(q, q, q, -0.5, False)  # negative scale: composite path only
