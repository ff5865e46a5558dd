"""Seeded synthetic workloads of the MXFP4 path (numpy, host side).

The generator is splitmix64 (crates/kern-test/src/workload.rs:11-26), used counter-style: draw i of the
stream seeded with s is mix(s + (i+1)*0x9E3779B97F4A7C15), so any slice can be drawn independently and
the device fill (kern_fill_random_u8) produces the same bytes. Normals use Box-Muller on draws 2i, 2i+1:
u = (d >> 11) * 2^-53, z = sqrt(-2 ln(1-u1)) cos(2 pi u2).

Every tensor gets its own stream seed: tensor_seed(seed, tag).
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def draws(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Draws start .. start+n-1 of the splitmix64 stream seeded with `seed` (uint64)."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed & (2**64 - 1)) + i * GOLDEN)


def tensor_seed(seed: int, tag: int) -> int:
    """Stream seed of tensor `tag` of a workload seeded with `seed` (draw `tag` of the base stream)."""
    return int(draws(seed, 1, tag)[0])


def uniform_bytes(seed: int, n: int, lo: int = 0, span: int = 256) -> np.ndarray:
    return (lo + (draws(seed, n) % np.uint64(span))).astype(np.uint8)


def normal(seed: int, n: int) -> np.ndarray:
    d = draws(seed, 2 * n)
    u1 = (d[0::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    return np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16); NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def activations_bf16(seed: int, T: int, K: int, outlier_frac: float = 0.0, outlier_mul: float = 20.0) -> np.ndarray:
    """bf16 bits [T, K] ~ N(0,1); a fraction of elements (chosen by their own stream) multiplied."""
    x = normal(tensor_seed(seed, 1), T * K)
    if outlier_frac > 0:
        pick = draws(tensor_seed(seed, 2), T * K) % np.uint64(1_000_000) < np.uint64(int(outlier_frac * 1_000_000))
        x = np.where(pick, x * outlier_mul, x)
    return f32_to_bf16_bits(x.astype(np.float32)).reshape(T, K)


def mxfp4_weights(seed: int, E: int, N: int, K: int, exp_lo: int, exp_hi: int):
    """Raw MXFP4 weights: nibbles uniform over all 16 codes (bytes uniform), e8m0 uniform in [exp_lo, exp_hi]."""
    w = uniform_bytes(tensor_seed(seed, 3), E * N * K // 2).reshape(E, N, K // 2)
    sf = uniform_bytes(tensor_seed(seed, 4), E * N * K // 32, exp_lo, exp_hi - exp_lo + 1).reshape(E, N, K // 32)
    return w, sf


def topk_ids(seed: int, T: int, E: int, k: int) -> np.ndarray:
    """Per token, k expert ids uniform without replacement (partial Fisher-Yates on the token's draws)."""
    d = draws(tensor_seed(seed, 5), T * k).reshape(T, k)
    out = np.empty((T, k), np.int32)
    perm = np.arange(E, dtype=np.int64)
    for t in range(T):
        p = perm.copy()
        for j in range(k):
            r = j + int(d[t, j] % np.uint64(E - j))
            p[j], p[r] = p[r], p[j]
        out[t] = p[:k]
    return out


def topk_weights(seed: int, T: int, k: int) -> np.ndarray:
    """Per token, k positive routing weights summing to one (uniform draws in [0.1, 1.1), normalised), f32."""
    d = draws(tensor_seed(seed, 6), T * k).reshape(T, k)
    w = (d >> np.uint64(11)).astype(np.float64) * 2.0**-53 + 0.1
    return (w / w.sum(1, keepdims=True)).astype(np.float32)
