"""The FC1 epilogue's SiTU-GLU approximation (kern_amd/csrc/mx_device.h: situ_coef, tanh_pq_clamped, situ_fast),
emulated step by step in f32 with the coefficients read from that source file, against the float64 formula
alpha*tanh(g/alpha)*sigmoid(g)*beta*tanh(u/beta) (tools/trtllm-bmm/probe.py:23, :46-47). The GPU tests bound the
device's values at 2e-5 relative on every routed row; this pins the approximation's own error well inside that,
for alpha, beta and inputs beyond the bench's. (The device's exponential and reciprocal are approximate
instructions; here they are exact, so their error is the GPU tests' to bound.)"""
import os
import re

import numpy as np

SRC = os.path.join(os.path.dirname(__file__), "..", "kern_amd", "csrc", "mx_device.h")
f = np.float32


def _coefficients():
    src = open(SRC).read()
    coef = src[src.index("KERN_DEV SituCoef situ_coef("):src.index("KERN_DEV void tanh_pq_clamped(")]
    lit = lambda name: f(re.search(rf"C\.{name} = uniform_f32\(([0-9.e+-]+)f \* sc\)", coef).group(1))
    clamp = f(re.search(r"C\.c = uniform_f32\(([0-9.e+-]+)f \* alpha\)", coef).group(1))
    body = src[src.index("KERN_DEV void tanh_pq_clamped("):src.index("KERN_DEV float situ_fast(")]
    p0 = f(re.search(r"p = __builtin_fmaf\(p, s, ([0-9.e+-]+)f\);\n  float q", body).group(1))
    return [p0, lit("p1"), lit("p2"), lit("p3")], [f(1), lit("q1"), lit("q2"), lit("q3"), lit("q4")], clamp


def _fma(a, b, c):  # one rounding, as the device's FMA (values past the f32 range become inf, as there)
    with np.errstate(over="ignore"):
        return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def _situ_f32(g, u, al, be):
    P, Q, C = _coefficients()

    def coef(alpha):  # situ_coef: the y^2k coefficient times alpha^-2k, in the device's order of rounding
        ia = f(f(1) / f(alpha))
        i2 = f(ia * ia)
        pk, qk, sc = [P[0]], [Q[0]], i2
        for k in range(1, 5):
            if k < 4:
                pk.append(f(P[k] * sc))
            qk.append(f(Q[k] * sc))
            sc = f(sc * i2)
        return pk, qk, f(C * f(alpha))

    def half(x, pk, qk, c, gate):  # tanh_pq: alpha*tanh(x/alpha) = num/den
        if gate:  # the gate's clamp is V_MED3_F32, which gives the lower bound for a NaN (the exp keeps it)
            a = np.where(np.isnan(x), -c, np.clip(x, -c, c)).astype(np.float32)
        else:  # the up projection's clamp keeps a NaN
            a = np.minimum(np.maximum(x, -c), c).astype(np.float32)
        s = (a * a).astype(np.float32)
        p = _fma(_fma(_fma(s, pk[3], pk[2]), s, pk[1]), s, pk[0])
        q = _fma(_fma(_fma(_fma(s, qk[4], qk[3]), s, qk[2]), s, qk[1]), s, qk[0])
        return (a * p).astype(np.float32), q

    na, da = half(g, *coef(al), True)
    nb, db = half(u, *coef(be), False)
    d = (da * db).astype(np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    den = _fma(d, e, d)
    with np.errstate(divide="ignore"):
        r = (1.0 / den.astype(np.float64)).astype(np.float32)
    return ((na * nb).astype(np.float32) * r).astype(np.float32)


def test_situ_rational_error():
    rng = np.random.default_rng(1)
    worst = 0.0
    for al, be in [(4.0, 25.0), (1.0, 1.0), (7.0, 3.0), (0.5, 100.0)]:
        for scale in (0.01, 1, 5, 30, 200):
            g = (rng.standard_normal(200_000) * scale).astype(np.float32)
            u = (rng.standard_normal(200_000) * scale).astype(np.float32)
            got = _situ_f32(g, u, al, be).astype(np.float64)
            gd, ud = g.astype(np.float64), u.astype(np.float64)
            with np.errstate(over="ignore"):
                ref = al * np.tanh(gd / al) / (1 + np.exp(-gd)) * be * np.tanh(ud / be)
            live = np.abs(ref) > 1e-20
            worst = max(worst, float((np.abs(got - ref)[live] / np.abs(ref)[live]).max()))
            assert np.all(np.abs(got - ref) <= 2e-5 * np.abs(ref) + 1e-6)
    assert worst < 1.5e-6, worst


def test_situ_special_values():
    g = np.array([np.nan, 0.0, -0.0, 1e30, -1e30, 100.0, -100.0, np.inf, -np.inf], np.float32)
    h = _situ_f32(g, np.ones_like(g), 4.0, 25.0)
    assert np.isnan(h[0]) and np.isnan(_situ_f32(np.ones(1, np.float32), np.full(1, np.nan, np.float32), 4.0, 25.0)[0])
    assert h[1] == 0 and h[2] == 0 and h[4] == 0 and h[6] == 0 and h[8] == 0  # sigmoid's underflow gives 0
    ref = 4.0 * 25.0 * np.tanh(1.0 / 25.0)  # tanh(g/4) -> 1 and sigmoid(g) -> 1
    for v in (h[3], h[5], h[7]):
        assert abs(v - ref) <= 2e-6 * ref
