"""ghip_copy_strided, the copy that materialises views and writes outputs: dense
copies (16-byte nontemporal fast path, with and without a vector-aligned size or
base), transposed and broadcast (zero-stride) sources and mergeable axes, bit for
bit against numpy on the same bytes."""
import numpy as np
import pytest
import torch

from gomlx_hip import ops, synth

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("shape,dtype", [((4096, 1024), np.float32), ((3, 5, 7), np.float32),
                                         ((1000003,), np.uint8), ((257, 33), np.int16),
                                         ((64, 64), np.int64), ((1,), np.float32)])
def test_dense_copy(cuda, shape, dtype):
    a = (synth.normal(9101, shape) * 100).astype(dtype)
    src = _dev(a)
    out = torch.empty_like(src)
    ops.copy(src, out)
    assert np.array_equal(out.cpu().numpy(), a)
    # misaligned base (one element in): the element-wise path
    if a.size > 2:
        flat = _dev(a.reshape(-1))
        o2 = torch.zeros_like(flat)
        ops.copy(flat[1:], o2[1:])
        assert np.array_equal(o2[1:].cpu().numpy(), a.reshape(-1)[1:]) and int(o2[0].cpu()) == 0


def test_strided_copies(cuda):
    a = synth.normal(9102, (64, 48, 40))
    src = _dev(a)
    t = src.permute(2, 0, 1)                          # transposed source
    out = torch.empty(t.shape, device="cuda")
    ops.copy(t, out)
    assert np.array_equal(out.cpu().numpy(), a.transpose(2, 0, 1))
    b = src[:, :1, :].expand(64, 48, 40)              # broadcast: zero stride on axis 1
    out = torch.empty(b.shape, device="cuda")
    ops.copy(b, out)
    assert np.array_equal(out.cpu().numpy(), np.broadcast_to(a[:, :1, :], (64, 48, 40)))
    s = src[:, 8:40, :]                               # slice: axes 1 and 2 merge, axis 0 strided
    out = torch.empty(s.shape, device="cuda")
    ops.copy(s, out)
    assert np.array_equal(out.cpu().numpy(), a[:, 8:40, :])
    o = torch.zeros((64, 96, 40), device="cuda")      # into a strided destination
    ops.copy(src, o[:, ::2, :])
    want = np.zeros((64, 96, 40), np.float32)
    want[:, ::2, :] = a
    assert np.array_equal(o.cpu().numpy(), want)
