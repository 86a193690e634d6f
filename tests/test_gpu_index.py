"""Bit-exact parity of the integer / indexing kernels: embedding gather,
argmin/argmax, iota."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from gomlx_hip import ops, synth

pytestmark = pytest.mark.gpu


def test_gather_known_answer(known, cuda):
    c = known["gather_embedding"]
    t = torch.tensor(c["table"], dtype=torch.float32, device=cuda).view(*c["table_shape"])
    ids = torch.tensor(c["ids"], dtype=torch.int32, device=cuda)
    assert ops.gather_rows(t, ids).view(-1).tolist() == c["expected"]


def test_gather_config_bf16(cuda):
    """Transformer-block embedding: table [32000, 2048] bf16, ids [8, 1024] int32."""
    table = synth.to_bf16_bits(synth.normal(5002, (32000, 2048), std=0.02))
    ids = synth.uniform_int(5001, (8, 1024), 0, 32000)
    tt = torch.from_numpy(table.view(np.int16)).to(cuda)
    out = ops.gather_rows(tt, torch.from_numpy(ids).to(cuda))
    ref = orc.gather_rows(table, ids.reshape(-1)).reshape(8, 1024, 2048)
    assert out.shape == (8, 1024, 2048)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("row_bytes_dtype", [(3, torch.float32), (5, torch.int8), (7, torch.int16)])
def test_gather_odd_rows_and_clamp(cuda, row_bytes_dtype):
    width, dt = row_bytes_dtype
    table = (torch.arange(50 * width, device=cuda) % 97).to(dt).view(50, width)
    ids_np = np.array([0, 49, -3, 50, 1000, 7, 7], np.int32)
    out = ops.gather_rows(table, torch.from_numpy(ids_np).to(cuda)).cpu().numpy()
    ref = orc.gather_rows(table.cpu().numpy(), ids_np)
    assert np.array_equal(out, ref)


def test_gather_empty(cuda):
    t = torch.ones((4, 8), device=cuda)
    assert ops.gather_rows(t, torch.empty((0,), dtype=torch.int32, device=cuda)).shape == (0, 8)


def test_argmax_known_answer(known, cuda):
    c = known["argmax"]
    x = torch.tensor(c["x"], dtype=torch.float32, device=cuda).view(*c["shape"])
    assert ops.argminmax(x, c["axis"]).tolist() == c["expected"]


@pytest.mark.parametrize("shape_axis", [((64, 1000), 1), ((64, 1000), 0), ((3, 200, 7), 1),
                                        ((5, 4, 3), 2), ((1, 70000), 1)])
@pytest.mark.parametrize("is_min", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argminmax_random_with_ties_nans(cuda, shape_axis, is_min, dtype):
    shape, axis = shape_axis
    x = synth.normal(6000 + sum(shape), shape)
    x = np.round(x * 4) / 4                         # many ties
    flat = x.reshape(-1)
    flat[::97] = np.nan                             # some NaNs
    flat[5::89] = np.inf
    flat[7::83] = -np.inf
    x = synth.round_bf16(x.astype(np.float32))
    t = torch.from_numpy(x).to(cuda).to(dtype)
    for odt in (torch.int32, torch.int64):
        got = ops.argminmax(t, axis, is_min, odt).cpu().numpy()
        assert np.array_equal(got, orc.argminmax(x, axis, is_min))


@pytest.mark.parametrize("dtype", [torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8,
                                   torch.float16, "uint16", "uint32", "uint64"])
def test_argminmax_integers_and_f16(cuda, dtype):
    """The reference passes any dtype to the arg-reduction (function.go:1204-1242):
    integers compare exactly (int64 / uint64, the type's extremes included, ties to
    the lowest index), float16 like the other floats."""
    if isinstance(dtype, str):
        if not hasattr(torch, dtype):
            pytest.skip(f"torch has no {dtype}")
        npdt, dtype = np.dtype(dtype), getattr(torch, dtype)
    else:
        npdt = np.dtype({torch.int8: np.int8, torch.int16: np.int16, torch.int32: np.int32, torch.int64: np.int64,
                         torch.uint8: np.uint8, torch.float16: np.float16}[dtype])
    rng = np.random.default_rng(23)
    for shape, axis in [((64, 1000), 1), ((64, 1000), 0), ((3, 200, 7), 1), ((1, 70000), 1)]:
        if npdt.kind in "iu":
            info = np.iinfo(npdt)
            pool = np.array([info.min, info.max, 0, 1, info.max - 1, info.min + 1, 7], dtype=npdt)
            x = pool[rng.integers(0, len(pool), size=shape)]
        else:
            x = (np.round(rng.standard_normal(shape) * 4) / 4).astype(npdt)
        signed = {1: np.int8, 2: np.int16, 4: np.int32, 8: np.int64}[npdt.itemsize]
        t = torch.from_numpy(np.ascontiguousarray(x).view(signed)).to(cuda).view(dtype)
        for is_min in (False, True):
            got = ops.argminmax(t, axis, is_min, torch.int64).cpu().numpy()
            assert np.array_equal(got, orc.argminmax(x, axis, is_min))


def test_iota_known_answer_and_dtypes(known, cuda):
    c = known["iota"]
    assert ops.iota(c["shape"], c["axis"], torch.float32, cuda).view(-1).tolist() == c["expected"]
    for dt in (torch.int32, torch.int64, torch.float32, torch.bfloat16):
        for shape, axis in (((2048, 2048), 0), ((2048, 2048), 1), ((3, 5, 7), 1)):
            got = ops.iota(shape, axis, dt, cuda).float().cpu().numpy()
            assert np.array_equal(got, orc.iota(shape, axis).astype(np.float32)
                                  if dt != torch.bfloat16 else
                                  synth.round_bf16(orc.iota(shape, axis).astype(np.float32)))
