"""Seeded synthetic inputs for the benchmark configurations.

Counter-based, so every element is a pure function of (seed, tensor id,
flat index) and any slice can be regenerated independently:
    key   = seed * 0x9E3779B97F4A7C15 + tensor_id            (mod 2^64)
    z(i)  = splitmix64_mix(key + (i + 1) * 0x9E3779B97F4A7C15)
    U(lo, hi): float32(lo + (hi - lo) * (z >> 40) * 2^-24)   (double, one rounding)
    N(0, s):   Box-Muller on z(2i), z(2i+1) in double, one rounding to float32
Tensor ids follow declaration order in the program. Generated on the host
and copied to HBM; there is no device RNG.
"""
import numpy as np

SEED = 0x7CA0C0DE
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _mix(x):
    x = x.copy()
    x ^= x >> np.uint64(30)
    x *= np.uint64(0xBF58476D1CE4E5B9)
    x ^= x >> np.uint64(27)
    x *= np.uint64(0x94D049BB133111EB)
    x ^= x >> np.uint64(31)
    return x


def _bits(n, seed, tensor_id, start=0):
    with np.errstate(over="ignore"):
        key = np.uint64(seed) * _GOLDEN + np.uint64(tensor_id)
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(key + i * _GOLDEN)


def uniform(shape, lo, hi, tensor_id, seed=SEED, chunk=1 << 24):
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        z = _bits(e - s, seed, tensor_id, s)
        u = (z >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)
        out[s:e] = (lo + (hi - lo) * u).astype(np.float32)
    return out.reshape(shape)


def normal(shape, sigma, tensor_id, seed=SEED, chunk=1 << 23):
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        z = _bits(2 * (e - s), seed, tensor_id, 2 * s)
        u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
        u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        r = np.sqrt(-2.0 * np.log(u1))
        out[s:e] = (sigma * r * np.cos(2.0 * np.pi * u2)).astype(np.float32)
    return out.reshape(shape)


def elem(n):
    """The reference suite's input formula (testing/runners/common.cuh:19-21):
    elem(i) = float32((i * 2654435761 mod 2^32) mod 1000) / 1000, i < 2^32."""
    i = np.arange(n, dtype=np.uint64)
    v = ((i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)) % np.uint64(1000)
    return v.astype(np.float32) / np.float32(1000.0)
