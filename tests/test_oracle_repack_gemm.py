"""Pins the oracle's repack (derive ops k3_moe_w_shuffle / k3_moe_sf_shuffle), its GEMM references and
the SiTU-GLU / silu_mul activations on the CPU.

Repack: bijection and inverse round trip, the gated row order, hand-computed byte offsets, and
GEMM(repacked) == GEMM(raw). GEMMs: the closed-form permutation KAT of
crates/kern-runtime/tests/mxfp8_gemm.rs:40-95 (exact in bf16), and float64 numpy matmuls of the
dequantised operands (tools/trtllm-bmm/probe.py:27-35, :100-112).
"""
import numpy as np
import pytest

from kern_amd import workload as wl
from tests._util import assert_gemm_close, r128c4_offsets, mxfp8_kat


@pytest.mark.parametrize("gated", [0, 1])
def test_repack_roundtrip_and_bijection(oracle, gated):
    E, rows, K = 2, 32, 1024
    w, sf = wl.mxfp4_weights(3, E, rows, K, 110, 140)
    ws = oracle.w_shuffle(w, E, rows, K // 2, gated)
    ss = oracle.sf_shuffle(sf, E, rows, K // 32, gated)
    np.testing.assert_array_equal(oracle.w_unshuffle(ws, E, rows, K // 2, gated), w)
    np.testing.assert_array_equal(oracle.sf_unshuffle(ss, E, rows, K // 32, gated), sf)
    # every destination byte is written exactly once: offsets form a permutation
    offs = sorted(oracle.lib().mxo_w_offset(R, kb, rows, K // 2) for R in range(rows) for kb in range(K // 2))
    assert offs == list(range(rows * K // 2))
    soffs = sorted(oracle.lib().mxo_sf_offset(R, b, rows, K // 32) for R in range(rows) for b in range(K // 32))
    assert soffs == list(range(rows * K // 32))
    src = sorted(oracle.w_src_row(R, rows, gated) for R in range(rows))
    assert src == list(range(rows))


def test_repack_hand_offsets(oracle):
    L = oracle.lib()
    # K = 512 (row_bytes 256): byte 70 of row 3 holds k = 140, 141 -> k-tile 1, k-group 0, lane 3, byte 6
    assert L.mxo_w_offset(3, 70, 16, 256) == 1 * 1024 + 3 * 16 + 6
    # row 21 (group 1, lane row 5), byte 100 = k 200: k-tile 1, group (200 % 128) / 32 = 2, byte 100 % 16 = 4
    assert L.mxo_w_offset(21, 100, 32, 256) == (1 * 4 + 1) * 1024 + (16 * 2 + 5) * 16 + 4
    # scale of row 5, k-block 9 (K = 512: one 16-block group): dword of lane 16*(9%4) + 5, byte (9%16)/4
    assert L.mxo_sf_offset(5, 9, 16, 16) == (16 * 1 + 5) * 4 + 2
    # gated quads: group 0 -> gate 0, gate 1, up 0, up 1, gate 2, gate 3, up 2, ... (gate = rows [m/2, m))
    rows = 32
    got = [oracle.w_src_row(R, rows, 1) for R in range(8)]
    assert got == [16, 17, 0, 1, 18, 19, 2, 3]
    assert [oracle.w_src_row(R, rows, 1) for R in range(16, 20)] == [24, 25, 8, 9]


def test_r128c4_matches_cublas_prose(oracle):
    # crates/kern-runtime/src/cublas.rs:396-400: 128-row x 4-block tiles of 512 bytes
    assert oracle.r128c4_offset(0, 0, 8) == 0
    assert oracle.r128c4_offset(1, 0, 8) == 16
    assert oracle.r128c4_offset(32, 0, 8) == 4
    assert oracle.r128c4_offset(0, 3, 8) == 3
    assert oracle.r128c4_offset(0, 4, 8) == 512
    assert oracle.r128c4_offset(128, 0, 8) == 1024
    offs = r128c4_offsets(256, 8).reshape(-1)
    assert sorted(offs.tolist()) == list(range(256 * 8))
    assert oracle.r128c4_size(130, 5) == 2 * 512 * 2


def test_gemm_repacked_equals_raw(oracle):
    m, K, T = 64, 1024, 40
    w, sf = wl.mxfp4_weights(4, 1, m, K, 118, 134)
    x = wl.activations_bf16(6, T, K)
    q, qs = oracle.quant_mxfp8(x)
    ws = oracle.w_shuffle(w, 1, m, K // 2, 0)
    ss = oracle.sf_shuffle(sf, 1, m, K // 32, 0)
    _, acc = oracle.gemm_e4m3_pt(ws, ss, q, qs, m, K, 1.0)
    ref = oracle.gemm_f32(oracle.deq_fp8(q, qs, T, K), oracle.deq_fp4(w[0], sf[0], m, K))
    np.testing.assert_array_equal(acc, ref)          # same products, same ascending-k order
    ref64 = oracle.deq_fp8(q, qs, T, K).astype(np.float64) @ oracle.deq_fp4(w[0], sf[0], m, K).astype(np.float64).T
    assert_gemm_close(acc, ref64, "oracle vs float64")


def test_deq_fp4_matches_probe_formula(oracle):
    # probe.py:27-31: nibble 2j low, 2j+1 high; value = E2M1[n & 7] * (-1 if n & 8) * 2^(sf - 127)
    rng = np.random.default_rng(2)
    w = rng.integers(0, 256, (4, 64), dtype=np.uint8)
    sf = rng.integers(120, 135, (4, 4), dtype=np.uint8)
    nib = np.stack([w & 15, w >> 4], -1).reshape(4, 128)
    tab = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    ref = tab[nib & 7] * np.where(nib & 8, -1.0, 1.0) * np.exp2(sf.astype(np.float64) - 127).repeat(32, 1)
    np.testing.assert_array_equal(oracle.deq_fp4(w, sf, 4, 128), ref.astype(np.float32))


def _kat_operands(M, N, K):
    """mxfp8_gemm.rs:40-95 design: A rows are one-hot e4m3 1.0, W in {-2..2}, power-of-two scales."""
    col = (np.arange(M) * 7) % K
    a = np.zeros((M, K), np.uint8)
    a[np.arange(M), col] = 0x38
    wv = ((np.arange(N)[:, None] + np.arange(K)[None, :]) % 5) - 2
    code = {-2: 0xC, -1: 0xA, 0: 0x0, 1: 0x2, 2: 0x4}
    nib = np.vectorize(code.get)(wv).astype(np.uint8)
    w = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    rr, bb = np.meshgrid(np.arange(M), np.arange(K // 32), indexing="ij")
    sa = (127 + ((rr + bb) % 3) - 1).astype(np.uint8)
    rn, bn = np.meshgrid(np.arange(N), np.arange(K // 32), indexing="ij")
    sw = (127 + ((3 * rn + 2 * bn) % 5) - 2).astype(np.uint8)
    b = col // 32
    ea = ((np.arange(M) + b) % 3) - 1
    ew = ((3 * np.arange(N)[None, :] + 2 * b[:, None]) % 5) - 2
    expect = wv[:, col].T * np.exp2(ea[:, None] + ew)
    return a, sa, w, sw, expect


def test_gemm_closed_form_kat_oracle(oracle):
    M, N, K = 64, 128, 512
    a, sa, w, sw, expect = _kat_operands(M, N, K)
    ws = oracle.w_shuffle(w[None], 1, N, K // 2, 0)
    ss = oracle.sf_shuffle(sw[None], 1, N, K // 32, 0)
    _, acc = oracle.gemm_e4m3_pt(ws, ss, a, sa, N, K, 1.0)
    np.testing.assert_array_equal(acc, expect.astype(np.float32))
    tabs = {"num_non_exiting": np.array([1], np.int32), "cta_batch": np.array([0], np.int32),
            "cta_limit": np.array([M], np.int32)}
    a_pad = np.zeros((128, K), np.uint8)
    a_pad[:M] = a
    sa_pad = np.zeros((128, K // 32), np.uint8)
    sa_pad[:M] = sa
    c, acc2 = oracle.fc2(ws, ss, a_pad, sa_pad, False, tabs, N, K)
    np.testing.assert_array_equal(acc2[:M], expect.astype(np.float32))
    np.testing.assert_array_equal(wl.bf16_bits_to_f32(c[:M]), expect.astype(np.float32))


def test_situ_formula(oracle):
    # probe.py:23, :46-47: situ(g, u) = alpha tanh(g/alpha) sigmoid(g) * beta tanh(u/beta)
    rng = np.random.default_rng(3)
    for g, u in rng.normal(0, 8, (200, 2)):
        a, b = 4.0, 25.0
        ref = a * np.tanh(g / a) / (1 + np.exp(-g)) * b * np.tanh(u / b)
        assert oracle.situ(g, u, a, b) == pytest.approx(ref, rel=2e-6, abs=1e-7)
    assert oracle.situ(0.0, 5.0, 4.0, 25.0) == 0.0
    assert oracle.situ(100.0, 1000.0, 4.0, 25.0) == pytest.approx(4.0 * 25.0, rel=1e-6)


def test_silu_mul_formula(oracle):
    # tools/kernels-src/silu_mul.cu:1-5: out = bf16(bf16(silu(g)) * u)
    T, d = 4, 64
    x = wl.activations_bf16(8, T, 2 * d)
    out = wl.bf16_bits_to_f32(oracle.silu_mul_bf16(x, d))
    f = wl.bf16_bits_to_f32(x).astype(np.float64)
    g, u = f[:, :d], f[:, d:]
    s = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits((g / (1 + np.exp(-g))).astype(np.float32)))
    ref = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits((s * u).astype(np.float32)))
    np.testing.assert_allclose(out, ref, rtol=2**-7, atol=0)


def test_gemv_oracle_vs_float64(oracle):
    M, N, K = 3, 96, 1024
    x = wl.activations_bf16(9, M, K)
    w, sf = wl.mxfp4_weights(10, 1, N, K, 120, 130)
    y, yf = oracle.gemv_w4a16(x, w[0], sf[0])
    ref = wl.bf16_bits_to_f32(x).astype(np.float64) @ oracle.deq_fp4(w[0], sf[0], N, K).astype(np.float64).T
    assert_gemm_close(yf, ref, "gemv oracle")
    np.testing.assert_array_equal(y, wl.f32_to_bf16_bits(yf))


def test_fc1_oracle_gated_pairs(oracle):
    """FC1's gate/up accumulators are the plain products with raw gate rows [m/2, m) and up rows [0, m/2)."""
    T, E, k, m, K = 16, 4, 2, 64, 512
    ids = wl.topk_ids(11, T, E, k)
    tabs = oracle.routing(ids, 0, E)
    S = int(tabs["num_non_exiting"][0])
    x = wl.activations_bf16(12, T, K)
    q, qs = oracle.quant_mxfp8(x)
    w, sf = wl.mxfp4_weights(13, E, m, K, 120, 126)
    ws = oracle.w_shuffle(w, E, m, K // 2, 1)
    ss = oracle.sf_shuffle(sf, E, m, K // 32, 1)
    alpha = np.full(E, 4.0, np.float32)
    beta = np.full(E, 25.0, np.float32)
    c, sf_c, dbg = oracle.fc1(ws, ss, q, qs, tabs, alpha, beta, m, K, S * 128)
    xd = oracle.deq_fp8(q, qs, T, K).astype(np.float64)
    half = m // 2
    for s in range(S):
        e = tabs["cta_batch"][s]
        wd = oracle.deq_fp4(w[e], sf[e], m, K).astype(np.float64)
        for p in range(s * 128, tabs["cta_limit"][s]):
            tok = tabs["route_map"][p]
            gate = xd[tok] @ wd[half:].T
            up = xd[tok] @ wd[:half].T
            np.testing.assert_allclose(dbg[p, 0], gate, rtol=1e-5, atol=1e-3)
            np.testing.assert_allclose(dbg[p, 1], up, rtol=1e-5, atol=1e-3)
            qq, sref = oracle.quant_blocks(dbg[p, 2][None])
            np.testing.assert_array_equal(c[p], qq[0])
            for b in range(half // 32):
                assert sf_c[oracle.r128c4_offset(p, b, half // 32)] == sref[0, b]


# ---------------------------------------------------------------- MXFP8 x MXFP8 (extern:cublaslt_mxfp8_tn)

@pytest.mark.parametrize("shift", [0, -1])
def test_mxfp8_gemm_oracle_kat(oracle, shift):
    c = mxfp8_kat(shift)
    got = oracle.mxfp8_gemm(c["a"], c["w"], c["a_sf"], c["w_sf"], c["M"], c["N"], c["K"])
    np.testing.assert_array_equal(got, c["want"])
