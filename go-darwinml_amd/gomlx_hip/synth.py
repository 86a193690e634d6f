"""Seeded synthetic inputs (host side, numpy).

Counter-based generator, identical bytes on every machine:
  u_i  = SplitMix64 output i of state `seed` (Steele/Lea/Flood 2014: state +=
         0x9E3779B97F4A7C15, then the 30/27/31 xor-shift-multiply mix)
         -> top 53 bits / 2^53                                   (uniform in [0, 1))
  N(0,1) pairs by Box-Muller in fp64 (textbook: sqrt(-2 ln u1) cos/sin(2 pi u2)),
  cast to fp32 (round to nearest even) and, where asked, to bf16 (RNE).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """The n SplitMix64 outputs for counters offset+1 .. offset+n of stream `seed`."""
    with np.errstate(over="ignore"):
        ctr = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + ctr * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    u = (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * u


def normal(seed: int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """fp32 N(mean, std^2) array of `shape`."""
    n = int(np.prod(shape, dtype=np.int64))
    m = (n + 1) // 2
    u = (splitmix64(seed, 2 * m) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1 = 1.0 - u[0::2]          # (0, 1]: log is finite
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def uniform_f32(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    return uniform(seed, n, lo, hi).astype(np.float32).reshape(shape)


def uniform_int(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    """int32 uniform in [lo, hi)."""
    n = int(np.prod(shape, dtype=np.int64))
    v = splitmix64(seed, n) % np.uint64(hi - lo)
    return (v.astype(np.int64) + lo).astype(np.int32).reshape(shape)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (RNE) as uint16 patterns."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 (returned as fp32)."""
    return bf16_bits_to_f32(to_bf16_bits(x))


def normal_device(seed: int, shape, std: float = 1.0, mean: float = 0.0, device="cuda", dtype=None):
    """normal() computed with torch on `device` (the same SplitMix64 counters and
    Box-Muller pairs, in fp64 then cast to fp32 and optionally to `dtype`), for
    inputs too large to generate on the host in a test's time.  The integer stream
    is identical; the fp64 log / cos / sin may differ from numpy's in the last
    bit, so the fp32 values agree with normal() except, rarely, by one ulp."""
    import torch
    n = int(np.prod(shape, dtype=np.int64))
    m = (n + 1) // 2
    out = torch.empty(2 * m, dtype=torch.float32, device=device)
    golden, m1, m2 = (int(v.astype(np.int64)) for v in (_GOLDEN, _M1, _M2))
    mask30, mask27, mask31, mask11 = ((1 << (64 - k)) - 1 for k in (30, 27, 31, 11))
    chunk = 1 << 24
    for p0 in range(0, m, chunk):
        p1 = min(m, p0 + chunk)
        ctr = torch.arange(2 * p0 + 1, 2 * p1 + 1, dtype=torch.int64, device=device)
        z = seed + ctr * golden                       # wraps modulo 2^64 like uint64
        z = (z ^ ((z >> 30) & mask30)) * m1
        z = (z ^ ((z >> 27) & mask27)) * m2
        z = z ^ ((z >> 31) & mask31)
        u = ((z >> 11) & mask11).to(torch.float64) * (1.0 / 9007199254740992.0)
        u1 = 1.0 - u[0::2]
        u2 = u[1::2]
        r = torch.sqrt(-2.0 * torch.log(u1))
        zz = torch.empty(2 * (p1 - p0), dtype=torch.float64, device=device)
        zz[0::2] = r * torch.cos(2.0 * np.pi * u2)
        zz[1::2] = r * torch.sin(2.0 * np.pi * u2)
        out[2 * p0:2 * p1] = (mean + std * zz).to(torch.float32)
    out = out[:n].reshape(shape)
    return out if dtype is None else out.to(dtype)
