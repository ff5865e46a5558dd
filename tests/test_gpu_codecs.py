"""Exhaustive GPU checks of the element codecs, through the C ABI, against the CPU oracle.

* The bf16 -> MXFP8 quantizer (moe_quant, the hardware e4m3 conversion of mx_pack4) on every finite bf16
  pattern under every block scale code the floor rule can produce (0..246: a bf16 or f32 block's largest
  magnitude is below 2^128, so floor(log2 amax) - 8 + 127 <= 246), plus every non-finite pattern (code 255).
  Each block holds one anchor, the largest value of its binade, and 31 patterns no larger than it, so the
  block's scale is the anchor's and every pattern is encoded under it. Bit-exact.
* The f32 -> MXFP8 quantizer (kern_mxfp8_quant_f32), whose codec is the FC1 epilogue's (mx_scale_code then
  mx_code2): the same blocks as f32, each pattern once exactly and once with random low mantissa bits
  (values between bf16 neighbours, and f32 subnormals). Bit-exact.
* Weight scale codes at the ends of the e8m0 range (0 = the subnormal 2^-127, 1, 2, 252..254, and 255 = NaN)
  through the decode GEMV's V_CVT_SCALEF32_PK_BF16_FP4, the MXFP4 GEMM's and the MXFP8 GEMM's scaled MFMA
  operands, against float64 sums over exactly dequantized operands (the dequantized weight 6 * 2^126 is not
  an f32, so the f32 oracle cannot stand in here): each extreme code sits alone in one k block of its rows,
  whose other blocks are zero, so each row's result is that block's contribution alone and the row
  tolerance (north star) measures it. A NaN scale makes its rows NaN.
"""
import numpy as np
import pytest

from kern_amd import workload as wl
from tests._util import assert_gemm_close, bf16_to_f32, r128c4_offsets, to_dev, to_np

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    return ops


# ------------------------------------------------------------------------------------ block construction

def _anchor_mags():
    """bf16 magnitude bits of the largest value of each binade 2^e, e = -133 .. 127 (subnormals first)."""
    sub = [(1 << (j + 1)) - 1 for j in range(7)]                    # m * 2^-133, floor(log2 m) = j
    norm = [((e + 127) << 7) | 0x7F for e in range(-126, 128)]
    return np.array(sub + norm, np.uint16)


def exhaustive_blocks(seed=1):
    """uint16 bf16 bits [nblocks, 32]: for every binade anchor, every finite pattern of magnitude <= the
    anchor (both signs, +-0 included), 31 to a block with the anchor (random sign, at a varying position);
    then one block per non-finite pattern (+-Inf, every NaN) padded with random finite values."""
    rng = np.random.default_rng(seed)
    blocks = []
    for a in _anchor_mags():
        mags = np.arange(int(a) + 1, dtype=np.uint16)
        pats = np.concatenate([mags, mags | np.uint16(0x8000)])
        pats = pats[rng.permutation(pats.size)]
        nb = -(-pats.size // 31)
        body = np.zeros(nb * 31, np.uint16)
        body[: pats.size] = pats
        body = body.reshape(nb, 31)
        anchor = np.where(rng.random(nb) < 0.5, a, a | np.uint16(0x8000)).astype(np.uint16)
        blk = np.concatenate([anchor[:, None], body], axis=1)
        pos = np.arange(nb) % 32  # the anchor moves through every position of the block
        idx = np.arange(32)[None, :].repeat(nb, 0)
        idx[np.arange(nb), 0], idx[np.arange(nb), pos] = pos, 0
        blocks.append(np.take_along_axis(blk, idx, axis=1))
    nonfinite = np.array([0x7F80, 0xFF80] + [s | 0x7F80 | m for s in (0, 0x8000) for m in range(1, 128)], np.uint16)
    fin = rng.integers(0, 0x7F00, size=(nonfinite.size, 32), dtype=np.uint16) | (
        rng.integers(0, 2, size=(nonfinite.size, 32), dtype=np.uint16) << 15)
    fin[np.arange(nonfinite.size), np.arange(nonfinite.size) % 32] = nonfinite
    blocks.append(fin)
    return np.concatenate(blocks)


def _as_rows(blocks, K=7168):
    """[nblocks, 32] -> [T, K] (zero blocks pad the last row)."""
    per = K // 32
    T = -(-blocks.shape[0] // per)
    out = np.zeros((T * per, 32), blocks.dtype)
    out[: blocks.shape[0]] = blocks
    return out.reshape(T, K)


def test_exhaustive_blocks_cover_every_code():
    """The construction itself (no GPU): every finite bf16 pattern occurs, and the oracle's scales span
    0..246 and 255."""
    from oracle import mxoracle as mo

    mo.lib()
    b = exhaustive_blocks()
    finite = b[(b & 0x7F80) != 0x7F80]
    assert np.unique(finite).size == 65536 - 256
    _, sf = mo.quant_mxfp8(_as_rows(b))
    assert set(np.unique(sf).tolist()) == set(range(247)) | {255}


@pytest.mark.gpu
def test_quant_bf16_exhaustive(ops, oracle):
    x = _as_rows(exhaustive_blocks())
    print(f"[quant bf16 exhaustive] {x.shape}", flush=True)
    q, sf = ops.quantize_mxfp8(to_dev(x))
    torch.cuda.synchronize()
    q_ref, sf_ref = oracle.quant_mxfp8(x)
    np.testing.assert_array_equal(to_np(sf), sf_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)


@pytest.mark.gpu
def test_quant_f32_exhaustive(ops, oracle):
    """kern_mxfp8_quant_f32 (the FC1 epilogue's mx_scale_code + mx_code2) over the same blocks as f32: each
    block once exactly and once with random low mantissa bits under an anchor whose low bits are all ones."""
    b = exhaustive_blocks(2).astype(np.uint32) << 16
    rng = np.random.default_rng(3)
    low = rng.integers(0, 1 << 16, size=b.shape, dtype=np.uint32)
    finite = (b & 0x7F800000) != 0x7F800000
    ext = np.where(finite, b | low, b)
    # the anchor of a finite block keeps the block maximum: its low bits all ones
    mag = ext & 0x7FFFFFFF
    top = mag.argmax(axis=1)
    rows = np.arange(b.shape[0])
    fin_blk = finite.all(axis=1)
    ext[rows[fin_blk], top[fin_blk]] |= 0xFFFF
    v = np.concatenate([b, ext]).view(np.float32)
    x = _as_rows(v)
    print(f"[quant f32 exhaustive] {x.shape}", flush=True)
    T, K = x.shape
    xd = to_dev(x)
    q = torch.empty((T, K), dtype=torch.uint8, device="cuda")
    sf = torch.empty((T, K // 32), dtype=torch.uint8, device="cuda")
    ops.mxfp8_quant_f32(xd, q, sf, T, K=K)
    torch.cuda.synchronize()
    q_ref, sf_ref = oracle.quant_blocks(x)
    np.testing.assert_array_equal(to_np(sf), sf_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)


# ------------------------------------------------------------------------------------ extreme scale codes

CODES = [0, 1, 2, 100, 126, 127, 128, 200, 252, 253, 254, 255]
E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)


def _extreme_weights(rng, N, K):
    """Raw nibbles [N, K/2] and e8m0 scales [N, K/32]: 16-row group j < len(CODES) has only k block j
    non-zero, under scale code CODES[j], with nibbles whose dequantized value is finite in bf16 (|w| <= 3
    at 253, 1.5 at 254); the other groups are ordinary. Returns (w, sf, nibbles [N, K])."""
    KB = K // 32
    nib = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    sf = rng.integers(122, 133, size=(N, KB), dtype=np.uint8)
    for j, c in enumerate(CODES):
        r = slice(16 * j, 16 * j + 16)
        nib[r] = 0
        sf[r] = 127
        lim = 8 if c <= 252 else (6 if c == 253 else 4)  # magnitude codes < lim: |w| <= 6, 3, 1.5
        blk = rng.integers(0, lim, size=(16, 32), dtype=np.uint8) | (rng.integers(0, 2, size=(16, 32), dtype=np.uint8) << 3)
        nib[r, 32 * j: 32 * j + 32] = blk
        sf[r, j] = c
    # the ordinary rows use only the ordinary k blocks: the extreme blocks' activations reach 2^127 * 448
    nib[16 * len(CODES):, : 32 * len(CODES)] = 0
    w = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return w, sf, nib


def _deq_w(nib, sf):
    v = E2M1[nib & 7] * np.where(nib & 8, -1.0, 1.0)
    s = np.where(sf == 255, np.nan, np.exp2(sf.astype(np.float64) - 127))
    return v * np.repeat(s, 32, axis=1)


def _x_exp(c):
    """Activation magnitude exponent for the k block of code c: products land near 1 (x stays a normal bf16)."""
    return int(np.clip(127 - c, -100, 100)) if c != 255 else 0


def _compare_with_nans(got, ref, ref_abs, what):
    """NaN exactly where the float64 reference has NaN; elsewhere the north-star tolerance over each row
    (a row mixes groups whose magnitudes differ by up to 2^54), and element by element the rounding of a
    bf16 result: |got - ref| <= 2^-8 |ref| (half a bf16 ulp) + 2^-14 sum_k |x_k w_k| (the worst-case error of
    f32 accumulation over K = 1024 terms). ref_abs holds sum_k |x_k w_k|."""
    nan_ref = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan_ref, err_msg=f"{what}: NaN pattern")
    g, r = np.where(nan_ref, 0.0, got), np.where(nan_ref, 0.0, ref)
    live = np.abs(r).max(axis=1) > 0
    assert_gemm_close(g[live], r[live], what)
    ra = np.where(nan_ref, 0.0, ref_abs)
    err = np.abs(g - r)
    bound = 2.0 ** -8 * np.abs(r) + 2.0 ** -14 * ra
    for j, c in enumerate(CODES):
        sl = slice(16 * j, 16 * j + 16)
        bad = err[:, sl] > bound[:, sl]
        assert not bad.any(), f"{what}: scale code {c}: {bad.sum()} results off by more than rounding " \
                              f"(worst {(err[:, sl] / np.maximum(bound[:, sl], 1e-300)).max():.3g}x the bound)"


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4])
def test_gemv_extreme_weight_scales(ops, M):
    rng = np.random.default_rng(40 + M)
    N, K = 256, 1024
    w, sf, nib = _extreme_weights(rng, N, K)
    xf = rng.standard_normal((M, K)).clip(-1.9, 1.9)
    for j, c in enumerate(CODES):
        xf[:, 32 * j: 32 * j + 32] *= 2.0 ** _x_exp(c)
    x = wl.f32_to_bf16_bits(xf.astype(np.float32))
    wp, sfp = ops.repack_weights(to_dev(w), to_dev(sf))
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ops.mxfp4_gemv_bf16(to_dev(x), wp[0], sfp[0], y, M, N=N, K=K)
    torch.cuda.synchronize()
    xd, wd = bf16_to_f32(x).astype(np.float64), _deq_w(nib, sf)
    _compare_with_nans(bf16_to_f32(to_np(y)).astype(np.float64), xd @ wd.T, np.abs(xd) @ np.abs(wd).T,
                       f"gemv M={M}")


def _extreme_activations(rng, M, K):
    """e4m3 codes [M, K] (finite) and scales [M, K/32]: k block j carries code 254 - CODES[j] (clamped), so
    that its products with block j of the extreme weights are near 1; row M-1 has a NaN scale in the last
    block."""
    KB = K // 32
    q = rng.integers(0, 0x7F, size=(M, K), dtype=np.uint8) | (rng.integers(0, 2, size=(M, K), dtype=np.uint8) << 7)
    sa = rng.integers(122, 133, size=(M, KB), dtype=np.uint8)
    for j, c in enumerate(CODES):
        sa[:, j] = 127 if c == 255 else min(254, max(0, 254 - c))
    sa[M - 1, KB - 1] = 255
    return q, sa


def _deq_x(q, sa):
    from oracle import mxoracle as mo

    mo.lib()
    v = np.vectorize(mo.e4m3_decode, otypes=[np.float64])(np.arange(256))[q]
    s = np.where(sa == 255, np.nan, np.exp2(sa.astype(np.float64) - 127))
    return v * np.repeat(s, 32, axis=1)


@pytest.mark.gpu
def test_gemm_extreme_scales(ops):
    """kern_mxfp4_gemm_bf16 (the scaled MFMA of every GEMM mode) with extreme weight and activation codes."""
    rng = np.random.default_rng(50)
    M, N, K = 32, 256, 1024
    w, sf, nib = _extreme_weights(rng, N, K)
    q, sa = _extreme_activations(rng, M, K)
    wp, sfp = ops.repack_weights(to_dev(w), to_dev(sf))
    c = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ops.mxfp4_gemm_bf16(wp[0], sfp[0], to_dev(q), to_dev(sa), c, M=M, m=N, k=K)
    torch.cuda.synchronize()
    xd, wd = _deq_x(q, sa), _deq_w(nib, sf)
    _compare_with_nans(bf16_to_f32(to_np(c)).astype(np.float64), xd @ wd.T, np.abs(xd) @ np.abs(wd).T, "mxfp4 gemm")


@pytest.mark.gpu
def test_mxfp8_gemm_extreme_scales(ops):
    """kern_mxfp8_gemm_bf16 with e8m0 codes 0..255 on both operands (128x4 tiled scales)."""
    rng = np.random.default_rng(60)
    M, N, K = 32, 256, 1024
    KB = K // 32
    qa, sa = _extreme_activations(rng, M, K)
    qw = rng.integers(0, 0x7F, size=(N, K), dtype=np.uint8) | (rng.integers(0, 2, size=(N, K), dtype=np.uint8) << 7)
    sw = np.full((N, KB), 127, np.uint8)
    for j, cc in enumerate(CODES):
        r = slice(16 * j, 16 * j + 16)
        qw[r] = 0
        qw[r, 32 * j: 32 * j + 32] = rng.integers(0, 0x7F, size=(16, 32), dtype=np.uint8)
        sw[r, j] = cc
    qw[16 * len(CODES):, : 32 * len(CODES)] = 0  # ordinary rows: ordinary k blocks only
    # e4m3 448 * 2^127 is not an f32: keep the code-254 (and 253) blocks' weights small
    for j, cc in enumerate(CODES):
        if cc >= 253:
            qw[16 * j: 16 * j + 16, 32 * j: 32 * j + 32] &= 0x3F  # |w| < 2

    def tiled(s, rows):
        t = np.full(ops.r128c4_bytes(rows, KB), 127, np.uint8)
        t[r128c4_offsets(rows, KB)] = s
        return t

    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ops.cublaslt_mxfp8_tn(to_dev(qa), to_dev(qw), out, to_dev(tiled(sa, M)), to_dev(tiled(sw, N)), M, N, K)
    torch.cuda.synchronize()
    xd, wd = _deq_x(qa, sa), _deq_x(qw, sw)
    _compare_with_nans(bf16_to_f32(to_np(out)).astype(np.float64), xd @ wd.T, np.abs(xd) @ np.abs(wd).T,
                       "mxfp8 gemm")


# ------------------------------------------------------------------------------------ bf16 rounding

@pytest.mark.gpu
def test_bf16_hw_packing_exhaustive(ops):
    """The GEMM epilogues round to bf16 through V_CVT_PK_BF16_F32 (bf16x2_hw in mx_device.h). On every f32 bit
    pattern (u in [0, 2^31) and u with its sign bit set) it gives the bits of the device's software
    round-to-nearest-even f32_to_bf16_bits, the rule of the oracle's bf16 rounding (pinned against torch's cast
    in tests/test_oracle_codecs.py): ties, subnormals, overflow to infinity, NaN payloads. The probe
    (kern_peaks.hsaco) counts mismatches on the device."""
    from kern_amd import build as kb

    mod = ops.Module(kb.PEAKS, kb.pinned_sha256("kern_peaks"))
    out = torch.zeros(4, dtype=torch.int32, device="cuda")
    mod.launch("kern_probe_bf16_cvt", (4096,), (256,), 0, 1 << 31, out)
    torch.cuda.synchronize()
    got = to_np(out)
    mod.close()
    assert got[0] == 0, f"{got[0]} mismatches, e.g. f32 bits {int(got[1]) & 0xffffffff:#010x}"


@pytest.mark.gpu
def test_fp4_conversion_scale_is_the_exponent_field(ops):
    """The decode GEMVs hand V_CVT_SCALEF32_PK_BF16_FP4 the bare e8m0 field (code << 23, fp4_cvt_scale in
    mx_device.h) instead of the f32 value 2^(code - 127) (e8m0_to_f32: the subnormal 2^-127 for code 0, NaN for
    255). The instruction reads only the exponent field, so the two give the same bf16 pairs: every code, every
    fp4 byte in every byte position, all four selects (kern_probe_fp4_scale in kern_peaks.hsaco counts
    mismatches)."""
    from kern_amd import build as kb

    mod = ops.Module(kb.PEAKS, kb.pinned_sha256("kern_peaks"))
    out = torch.zeros(4, dtype=torch.int32, device="cuda")
    mod.launch("kern_probe_fp4_scale", (256,), (256,), out)
    torch.cuda.synchronize()
    got = to_np(out)
    mod.close()
    assert got[0] == 0, f"{got[0]} mismatches, e.g. code {int(got[1]) >> 8} byte {int(got[1]) & 255}"
