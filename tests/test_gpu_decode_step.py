"""One decoding step of a decoder block through Builder / Compile / Execute
(gomlx_hip.graphs.decode_step): every product has B rows, so the projections run
as contraction splits, and the attention of the B queries over their K / V caches
as grouped-query rows with a split key range.  Outputs (x', and the new K / V
columns of the QKV projection) against the fp64 composition of the same step
(oracle.decode_step) on the same parameter bytes, normwise <= 1e-2 (bf16 rounding
at every op of the graph, as in the block test); two Executes give the same bits."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import graphs, synth
from gomlx_hip.backend import Backend
from conftest import norm_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be(cuda):
    b = Backend("")
    yield b
    b.Finalize()


def _params(cfg, seed, cuda):
    """bf16 values as fp32 host arrays: x and the caches ~ N(0, 1), weights
    ~ N(0, 1/fan_in) (the SplitMix64 streams, generated on the device), gammas
    ~ U(0.5, 1.5)."""
    P = {}
    for i, (name, shape) in enumerate(cfg.param_shapes()):
        if name.startswith("g_"):
            P[name] = synth.round_bf16(synth.uniform_f32(seed + i, shape.dims, 0.5, 1.5))
        else:
            std = 1.0 if name in ("x", "k_cache", "v_cache") else shape.dims[0] ** -0.5
            t = synth.normal_device(seed + i, shape.dims, std=std, device=cuda, dtype=torch.bfloat16)
            P[name] = t.float().cpu().numpy()
    return P


CONFIGS = [
    dict(batch=4, cache=1500, d_model=1024, heads=8, kv_heads=2, head_dim=128, ffn=2048),
    dict(batch=16, cache=4096, d_model=2048, heads=16, kv_heads=4, head_dim=128, ffn=8192),
]


@pytest.mark.parametrize("kw", CONFIGS, ids=["small", "b16"])
def test_decode_step_matches_oracle(be, cuda, kw):
    cfg = graphs.DecodeStepConfig(**kw)
    ex = graphs.decode_step(be, cfg)
    plan = ex.Plan()
    assert "contraction split" in plan and "key range split" in plan, plan
    P = _params(cfg, 9100, cuda)
    bufs = [be.BufferFromFlatData(0, P[name], shape) for name, shape in cfg.param_shapes()]
    print(f"decode step {kw}", flush=True)
    outs = [be.BufferToFlatData(o).copy() for o in ex.Execute(bufs, None, 0)]
    again = [be.BufferToFlatData(o).copy() for o in ex.Execute(bufs, None, 0)]
    ex.Finalize()
    for a, b in zip(outs, again):
        assert np.array_equal(a, b)
    B, d, q, kv = cfg.batch, cfg.d_model, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    x2 = synth.bf16_bits_to_f32(outs[0]).reshape(B, d)
    qkv = synth.bf16_bits_to_f32(outs[1]).reshape(B, q + 2 * kv)
    rows = np.arange(B) if B <= 4 else np.array([0, 5, B - 1])
    ref = orc.decode_step(P, rows, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps)
    got = [x2[rows], qkv[rows, q:q + kv], qkv[rows, q + kv:]]
    for g, r, name in zip(got, ref, ["x'", "k_new", "v_new"]):
        assert norm_err(g, r) <= 1e-2, name
