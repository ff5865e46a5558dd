"""Oracle pins for the MoE glue: the finalize combine (tools/trtllm-bmm/probe.py:100-110) and its norm
(op moe_finalize_rms). The combine is pinned by closed forms (one-hot weights return the routed row
exactly, skipped rows add nothing, a permutation of j with the same pairs changes only rounding) and by
a float64 restatement; the norm by a constant row, whose result is gamma * c / sqrt(c^2 + eps), and by
float64. The norm's own convention (eps, plain gamma) is this build's choice: parity unpinned against
the reference kernel, whose source is not in the reference tree."""
import numpy as np
import pytest

from kern_amd import workload as wl


@pytest.fixture(scope="module")
def oracle():
    from oracle import mxoracle
    mxoracle.lib()
    return mxoracle


def bf16_to_f64(b):
    return wl.bf16_bits_to_f32(b).astype(np.float64)


def f64_to_bf16(x):
    return wl.f32_to_bf16_bits(np.asarray(x, np.float32))


def ulp_diff(a, b):
    ai, bi = a.astype(np.int32), b.astype(np.int32)
    # bf16 bit patterns as ordered integers (sign-magnitude -> two's complement order)
    oa = np.where(ai & 0x8000, -(ai & 0x7FFF), ai)
    ob = np.where(bi & 0x8000, -(bi & 0x7FFF), bi)
    return np.abs(oa - ob)


def _case(seed, T, H, topk, rows):
    rng = np.random.default_rng(seed)
    fc2 = wl.f32_to_bf16_bits(rng.standard_normal((rows, H)).astype(np.float32))
    e2p = rng.permutation(rows)[: T * topk].astype(np.int32)
    w = rng.random((T, topk)).astype(np.float32) + 0.05
    w /= w.sum(1, keepdims=True)
    return fc2, e2p, w


def test_one_hot_returns_row(oracle):
    T, H, k, rows = 5, 64, 4, 40
    fc2, e2p, _ = _case(1, T, H, k, rows)
    w = np.zeros((T, k), np.float32)
    w[np.arange(T), np.arange(T) % k] = 1.0
    out = oracle.moe_finalize(fc2, e2p, w, None, T, H, k)
    for t in range(T):
        np.testing.assert_array_equal(out[t], fc2[e2p[t * k + t % k]])


def test_skipped_rows_add_nothing(oracle):
    T, H, k, rows = 6, 32, 3, 30
    fc2, e2p, w = _case(2, T, H, k, rows)
    ref = oracle.moe_finalize(fc2, e2p, w, None, T, H, k)
    e2 = e2p.copy()
    e2[1::k] = -1  # every token loses its second routed row
    w2 = w.copy()
    w2[:, 1] = 0.0
    a = oracle.moe_finalize(fc2, e2, w, None, T, H, k)
    b = oracle.moe_finalize(fc2, e2p, w2, None, T, H, k)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, ref)


def test_combine_against_float64(oracle):
    T, H, k, rows = 16, 256, 8, 200
    fc2, e2p, w = _case(3, T, H, k, rows)
    out = oracle.moe_finalize(fc2, e2p, w, None, T, H, k)
    x = bf16_to_f64(fc2)
    ref = np.einsum("tj,tjh->th", w.astype(np.float64), x[e2p.reshape(T, k)])
    assert ulp_diff(out, f64_to_bf16(ref)).max() <= 1
    # a wrong pairing of weights and rows (j reversed on one side) is caught
    bad = np.einsum("tj,tjh->th", w[:, ::-1].astype(np.float64), x[e2p.reshape(T, k)])
    assert ulp_diff(out, f64_to_bf16(bad)).max() > 1


@pytest.mark.parametrize("c", [0.75, -3.0, 1e-3, 40.0])
def test_norm_constant_row(oracle, c):
    H, k, eps = 128, 2, 1e-6
    fc2 = np.tile(f64_to_bf16([c]), (4, H)).astype(np.uint16)
    e2p = np.array([0, -1], np.int32)
    w = np.array([[1.0, 0.3]], np.float32)
    gamma = wl.f32_to_bf16_bits(np.linspace(-2, 2, H).astype(np.float32))
    out = oracle.moe_finalize(fc2, e2p, w, gamma, 1, H, k, eps)
    cb = bf16_to_f64(fc2[0, 0])
    want = bf16_to_f64(gamma) * cb / np.sqrt(cb * cb + eps)
    assert ulp_diff(out[0], f64_to_bf16(want)).max() <= 1


def test_norm_against_float64(oracle):
    T, H, k, rows, eps = 8, 512, 4, 64, 1e-6
    fc2, e2p, w = _case(4, T, H, k, rows)
    gamma = wl.f32_to_bf16_bits((np.random.default_rng(5).random(H) + 0.5).astype(np.float32))
    out = oracle.moe_finalize(fc2, e2p, w, gamma, T, H, k, eps)
    x = bf16_to_f64(fc2)
    y = np.einsum("tj,tjh->th", w.astype(np.float64), x[e2p.reshape(T, k)])
    ref = y / np.sqrt((y * y).mean(1, keepdims=True) + eps) * bf16_to_f64(gamma)
    assert ulp_diff(out, f64_to_bf16(ref)).max() <= 1


# ---------------------------------------------------------------- weight_prep: the RoPE cache

def test_rope_closed_forms(oracle):
    rows, half, base = 64, 32, 10000.0
    c, s = oracle.rope_table(rows, half, half, base)
    c, s = c.reshape(rows, half), s.reshape(rows, half)
    # row 0: angle 0 -> cos 1, sin 0; column 0: inv = 1 -> angle = r
    np.testing.assert_array_equal(c[0], f64_to_bf16(np.ones(half)))
    np.testing.assert_array_equal(s[0], f64_to_bf16(np.zeros(half)))
    r = np.arange(rows, dtype=np.float64)
    assert ulp_diff(c[:, 0], f64_to_bf16(np.cos(r))).max() <= 1
    assert ulp_diff(s[:, 0], f64_to_bf16(np.sin(r))).max() <= 1


def test_rope_against_float64(oracle):
    rows, half, stride, base = 300, 64, 128, 500000.0
    c, s = oracle.rope_table(rows, half, stride, base)
    c, s = c.reshape(rows, stride), s.reshape(rows, stride)
    j = np.arange(half, dtype=np.float64)
    inv = (1.0 / np.float32(base) ** (np.float32(2 * j) / np.float32(2 * half))).astype(np.float32)
    ang = (np.arange(rows, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    # value space: one bf16 ulp relative, plus an absolute floor for values near a zero crossing, where
    # an ulp of the f32 angle (numpy's power here, libm's powf in the oracle) moves several bf16 ulps
    for got, want in [(c[:, :half], np.cos(ang)), (s[:, :half], np.sin(ang))]:
        g = bf16_to_f64(got)
        assert (np.abs(g - want) <= 2.0**-8 * np.abs(want) + 1e-5).all()
    # the stride's gap stays untouched, and cos/sin are not swapped
    assert not c[:, half:].any() and not s[:, half:].any()
    assert ulp_diff(c[:, :half], f64_to_bf16(np.sin(ang))).max() > 1
