"""Pins the oracle's bf16 -> MXFP8 quantizer (op moe_quant) on the CPU.

The rule (tools/trtllm-bmm/probe.py:38-43, also the OCP MX v1.0 scale rule for E4M3): per block of 32,
scale = 2^(floor(log2 amax) - 8); elements are x / scale rounded to nearest-even e4m3, saturating to
+-448 (probe.py casts without saturating, which would turn the top of any block whose amax mantissa is
>= 1.8125 into NaN; saturating is the OCP choice and ours). The numpy restatement below computes the
scale with frexp and each code by a nearest-value search over the e4m3 value table, so it shares no
arithmetic with the oracle's integer encoder.
"""
import os

import numpy as np

from kern_amd import workload as wl
from tests.test_oracle_codecs import e4m3_table

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def numpy_quant(x_bf16):
    x = wl.bf16_bits_to_f32(x_bf16).astype(np.float64)
    T, K = x.shape
    blocks = x.reshape(T, K // 32, 32)
    amax = np.abs(blocks).max(-1)
    _, e = np.frexp(amax)                     # amax = f * 2^e, f in [0.5, 1) -> floor(log2 amax) = e - 1
    code = np.where(amax > 0, np.clip(e - 1 - 8 + 127, 0, 254), 0).astype(np.int64)
    scaled = blocks / np.exp2(code - 127.0)[..., None]
    table = e4m3_table()
    pos = np.array([c for c in range(127)])           # finite non-negative codes, ascending values
    vals = table[pos]
    a = np.minimum(np.abs(scaled), 448.0)
    hi = np.clip(np.searchsorted(vals, a), 1, len(vals) - 1)
    lo = hi - 1
    dlo, dhi = a - vals[lo], vals[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (pos[hi] % 2 == 0))
    c = np.where(pick_hi, pos[hi], pos[lo])
    c = np.where(a == 0, 0, c)
    c = c | np.where(np.signbit(scaled), 0x80, 0)
    return c.reshape(T, K).astype(np.uint8), code.astype(np.uint8)


def test_quant_matches_numpy_restatement(oracle):
    x = wl.activations_bf16(5, 64, 1024, outlier_frac=0.01)
    # blocks at every scale: multiply rows by powers of two from 2^-140 to 2^120
    f = wl.bf16_bits_to_f32(x).astype(np.float64)
    f *= np.exp2(np.linspace(-140, 120, 64))[:, None]
    with np.errstate(over="ignore"):
        x = wl.f32_to_bf16_bits(f.astype(np.float32))
    q, s = oracle.quant_mxfp8(x)
    qn, sn = numpy_quant(x)
    np.testing.assert_array_equal(s, sn)
    np.testing.assert_array_equal(q, qn)


def test_quant_closed_form_cases(oracle):
    K = 32
    rows = []
    rows.append(np.zeros(K))                                           # 0: all zero -> scale 0, codes 0
    r = np.zeros(K); r[0] = 1.0; r[1] = -0.5; rows.append(r)           # 1: amax 1 -> scale 2^-8; 1 -> 256
    r = np.zeros(K); r[0] = 1.875; rows.append(r)                      # 2: 1.875*256 = 480 saturates to 448
    r = np.zeros(K); r[0] = 1.75; r[1] = 2.0**-6; rows.append(r)       # 3: 448 exactly; 2^-6 -> 4
    r = np.full(K, 2.0**-130); rows.append(r)                          # 4: bf16 subnormals -> scale code 0
    r = np.zeros(K); r[0] = 3.0e38; rows.append(r)                     # 5: 1.76*2^127 -> 127-8+127
    x = wl.f32_to_bf16_bits(np.array(rows, np.float32))
    q, s = oracle.quant_mxfp8(x)
    assert s[:, 0].tolist() == [0, 127 - 8, 127 - 8, 127 - 8, 0, 246]
    assert q[0].tolist() == [0] * 32
    assert q[1, 0] == 0x78 and q[1, 1] == 0xF0                         # 256 = 2^8, -128 = -2^7
    assert q[2, 0] == 0x7E
    assert q[3, 0] == 0x7E and q[3, 1] == 0x48                         # 2^-6 * 2^8 = 4: exponent field 9
    # 2^-130 / 2^-127 = 2^-3 -> exponent field -3+7 = 4 -> 0x20
    assert q[4].tolist() == [0x20] * 32


def test_quant_nonfinite_blocks(oracle):
    f = np.ones((1, 64), np.float32)
    f[0, 3] = np.inf
    f[0, 40] = np.nan
    q, s = oracle.quant_mxfp8(wl.f32_to_bf16_bits(f))
    assert s.tolist() == [[255, 255]]
    assert set(q[0].tolist()) == {0x7F}


def test_quant_golden_fixture(oracle):
    """Committed fixture (tests/golden/mxfp8_quant.npz, written by tests/golden/make_golden.py with the
    numpy restatement above): inputs and expected codes/scales."""
    d = np.load(os.path.join(GOLDEN, "mxfp8_quant.npz"))
    q, s = oracle.quant_mxfp8(d["x_bf16"])
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(s, d["sf"])
