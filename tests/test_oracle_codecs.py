"""Pins the oracle's element codecs and generator (CPU only).

Each check is independent of the oracle's own formula: the e2m1 table of the reference against the
textbook E2M1 (bias 1) formula; the reference's codec tests (crates/kern-manifest/tests/values.rs:7-54,
kept as data in tests/golden/values_rs_kats.json); torch's own float8_e4m3fn and bfloat16 conversions;
a brute-force nearest-value search for the RNE encoder; and the published splitmix64 test vector.
"""
import json
import os

import numpy as np
import pytest

from kern_amd import workload as wl

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def e4m3_table():
    """All 256 e4m3fn values from the OCP FP8 definition (bias 7, no inf, S.1111.111 = NaN)."""
    vals = np.empty(256, np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * m * 2.0**-9
        else:
            vals[c] = s * (8 + m) * 2.0 ** (e - 10)
    return vals


def test_e2m1_all_codes(oracle):
    # tools/trtllm-bmm/probe.py:24-31 table vs the E2M1 formula: (-1)^s 2^(E-1) (1 + M/2), E=0 -> M/2
    for n in range(16):
        s, e, m = n >> 3, (n >> 1) & 3, n & 1
        want = (m / 2.0 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2.0)) * (-1) ** s
        assert oracle.e2m1_decode(n) == want, n


def test_e8m0_all_codes(oracle):
    # values.rs:38-48: codes 0..254 decode to 2^(c-127) and re-encode to themselves; 255 is NaN
    for c in range(255):
        assert oracle.e8m0_decode(c) == np.float32(2.0 ** (c - 127)), c
        assert oracle.e8m0_encode(2.0 ** (c - 127)) == c
    assert np.isnan(oracle.e8m0_decode(255))
    # values.rs:115-135: nearest power of two, ties to the even code; zero saturates; NaN/negative -> 255
    assert oracle.e8m0_encode(0.0) == 0
    assert oracle.e8m0_encode(-1.0) == 255 and oracle.e8m0_encode(float("nan")) == 255
    assert oracle.e8m0_encode(1.5) == 128      # midpoint of 2^0, 2^1: code 127 is odd -> 128
    assert oracle.e8m0_encode(3.0) == 128      # midpoint of 2^1, 2^2: code 128 is even -> stays
    assert oracle.e8m0_encode(1.49) == 127 and oracle.e8m0_encode(1.51) == 128
    assert oracle.e8m0_encode(2.0**130) == 254


def test_e4m3_decode_matches_torch_and_definition(oracle):
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    t = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    d = np.array([oracle.e4m3_decode(c) for c in range(256)], np.float64)
    ref = e4m3_table()
    np.testing.assert_array_equal(np.isnan(d), np.isnan(ref))
    np.testing.assert_array_equal(np.isnan(t), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(d[ok], ref[ok])
    np.testing.assert_array_equal(t[ok], ref[ok])


def test_values_rs_golden(oracle):
    """The reference's own codec test cases (crates/kern-manifest/tests/values.rs:7-54)."""
    with open(os.path.join(GOLDEN, "values_rs_kats.json")) as f:
        kat = json.load(f)
    for v in kat["e4m3_roundtrip_within_sixteenth"]:
        back = oracle.e4m3_decode(oracle.e4m3_encode_values_rs(v))
        assert abs(back - v) <= abs(v) * 0.0625 + 1e-9
        # our RNE encoder agrees on these samples
        back2 = oracle.e4m3_decode(oracle.e4m3_encode_rne(int(np.float32(v).view(np.uint32)), 0))
        assert abs(back2 - v) <= abs(v) * 0.0625 + 1e-9
    assert np.isnan(oracle.e4m3_decode(kat["e4m3_nan_code"]))
    for c, v in kat["e8m0_decode"].items():
        assert oracle.e8m0_decode(int(c)) == v
    assert np.isnan(oracle.e8m0_decode(kat["e8m0_nan_code"]))


def _nearest_even(v, table):
    """Brute-force RNE onto the finite e4m3 values, saturating to +-448: nearest value, ties to the code
    with an even mantissa."""
    fin = [(c, table[c]) for c in range(128) if not np.isnan(table[c])]
    a = abs(v)
    if a >= 448.0:
        code = 0x7E
    else:
        best = min(fin, key=lambda cv: (abs(cv[1] - a), cv[0] & 1))
        code = best[0]
    return code | (0x80 if np.signbit(v) else 0)


def test_e4m3_rne_encoder_bruteforce(oracle):
    table = e4m3_table()
    rng = np.random.default_rng(0)
    vals = list(rng.normal(0, 1, 3000) * np.exp2(rng.integers(-12, 10, 3000)))
    vals += [float(table[c]) for c in range(127)]                         # every representable value
    vals += [(table[c] + table[c + 1]) / 2 for c in range(126)]           # every midpoint (ties)
    vals += [2.0**-10, 2.0**-10 * 1.0001, 3 * 2.0**-10, 464.0, 463.9, 500.0, -0.0, 1e-30]
    for v in vals:
        bits = int(np.float32(v).view(np.uint32))
        got = oracle.e4m3_encode_rne(bits, 0)
        want = _nearest_even(float(np.float32(v)), table)
        if float(np.float32(v)) == 0.0:
            want = 0x80 if np.signbit(np.float32(v)) else 0
        assert got == want, (v, hex(got), hex(want))


def test_e4m3_rne_matches_torch_on_all_bf16(oracle):
    """Every finite bf16 below the saturation point, at several block shifts, against torch's RNE cast."""
    torch = pytest.importorskip("torch")
    bits = np.arange(65536, dtype=np.uint32)
    f = ((bits << 16).view(np.float32)).astype(np.float32)
    for shift in (0, -3, 5):
        with np.errstate(invalid="ignore", over="ignore"):
            scaled = f.astype(np.float64) * 2.0**shift
        ok = np.isfinite(scaled) & (np.abs(scaled) < 464.0)
        t = torch.from_numpy(scaled[ok].astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got = np.array([oracle.e4m3_encode_rne(int(b), shift) for b in (bits << 16)[ok][::7]], np.uint8)
        np.testing.assert_array_equal(got, t[::7])


def test_e4m3_saturation_and_specials(oracle):
    enc = lambda v, s=0: oracle.e4m3_encode_rne(int(np.float32(v).view(np.uint32)), s)
    assert enc(448.0) == 0x7E and enc(464.0) == 0x7E and enc(1e30) == 0x7E and enc(-1e30) == 0xFE
    assert enc(np.inf) == 0x7E and enc(-np.inf) == 0xFE
    assert enc(np.nan) & 0x7F == 0x7F
    assert enc(2.0**-9) == 0x01 and enc(2.0**-10) == 0x00 and enc(1.5 * 2.0**-10) == 0x01
    assert enc(1.0, 8) == 0x78  # 256


def test_bf16_rne_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = (rng.normal(0, 1, 20000) * np.exp2(rng.integers(-60, 60, 20000))).astype(np.float32)
    x[:4] = [np.float32(1.0 + 2.0**-8), np.float32(1.0 + 3 * 2.0**-8), np.float32(-(1.0 + 2.0**-8)), 0.0]
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(wl.f32_to_bf16_bits(x), t)
    got = np.array([oracle.f32_to_bf16(float(v)) for v in x[:2000]], np.uint16)
    np.testing.assert_array_equal(got, t[:2000])


def test_splitmix64_published_vector(oracle):
    # splitmix64 reference test vector (seed 1234567), the generator of crates/kern-test/src/workload.rs:11-26
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    assert [int(v) for v in wl.draws(1234567, 5)] == want
    assert [oracle.splitmix64_at(1234567, i) for i in range(5)] == want
    # the reference's sequential Rng::draw (workload.rs:18-24) is the same stream
    s, seq = 1234567, []
    for _ in range(5):
        s = (s + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        seq.append(z ^ (z >> 31))
    assert seq == want


def test_normals_match_between_numpy_and_c(oracle):
    z = wl.normal(99, 64)
    zc = np.array([oracle.normal_at(99, i) for i in range(64)])
    np.testing.assert_allclose(z, zc, rtol=1e-12, atol=1e-12)
    big = wl.normal(5, 200000)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01
