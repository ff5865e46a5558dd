"""GPU parity of every op of the path against the CPU oracle, through the C ABI.

Bit-exact: quantizer, repack, routing tables, the fill generator, e4m3/ue8m0 epilogue codes (given the
kernel's own pre-quantisation values). Tolerance (north star): GEMM outputs within max-abs
1e-2*||row||_inf and relative Frobenius 2e-3 of the fp32-accumulate oracle on exactly dequantised
operands.
"""
import numpy as np
import pytest

from kern_amd import workload as wl
from tests._util import assert_gemm_close, bf16_to_f32, r128c4_offsets, to_dev, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    return ops


def _sync():
    torch.cuda.synchronize()


# --------------------------------------------------------------------------------------- fills

def test_fill_random_matches_host_stream(ops):
    n = (1 << 20) + 7
    for seed, lo, span in [(1, 0, 256), (12345, 122, 11), (2**63 + 5, 124, 7)]:
        out = torch.empty(n, dtype=torch.uint8, device="cuda")
        ops.fill_random_u8(out, seed, lo, span)
        _sync()
        np.testing.assert_array_equal(to_np(out), wl.uniform_bytes(seed, n, lo, span))


# --------------------------------------------------------------------------------------- quantizer

def _special_rows(K):
    rows = []
    f = np.zeros((8, K), np.float32)
    f[0] = 0.0                                   # all-zero blocks -> scale code 0
    f[1] = 1.0                                   # power-of-two amax
    f[2, ::32] = 1.875                           # amax mantissa 1.875 -> 480 before saturation
    f[2, 1::32] = 1.75 / 2**6                    # tiny next to it
    f[3] = np.float32(2.0**-130)                 # bf16 subnormals
    f[4] = np.linspace(-3e38, 3e38, K).astype(np.float32)  # extreme magnitudes
    f[5] = np.float32(448.0)
    f[5, 1::32] = 464.0                          # the RNE midpoint above 448
    f[6] = np.tile(np.float32([1.0, 1.0625, 1.125, 1.1875, 1.03125, 1.09375]), K)[:K]  # ties
    f[7, 0] = np.inf
    f[7, 40] = np.nan
    f[7, 64:96] = -np.inf
    rows.append(wl.f32_to_bf16_bits(f))
    return np.concatenate(rows)


@pytest.mark.parametrize("T,K", [(64, 1024), (4096, 7168)])
def test_quant_bitexact(ops, oracle, T, K):
    x = wl.activations_bf16(7 + T, T, K, outlier_frac=0.01)
    x[:8] = _special_rows(K)
    xd = to_dev(x)
    q, sf = ops.quantize_mxfp8(xd)
    _sync()
    q_ref, sf_ref = oracle.quant_mxfp8(x)
    np.testing.assert_array_equal(to_np(sf), sf_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)


# --------------------------------------------------------------------------------------- repack

# weight_prep repacks, bit for bit against the oracle: small experts, gated (FC1) and plain (FC2); the
# smallest shapes the ops take (one 16-row group, K = 512; three row groups, K = 1536); and the real shapes,
# several experts each: K3's FC1 (6144 gate/up rows, K = 3584) and FC2 (3584 rows, K = 3072), config 4's FC1
# (4096 rows, K = 7168) and FC2 (7168 rows, K = 2048), and config 2's dense weights (18432 rows, K = 7168)
@pytest.mark.parametrize("E,rows,K,gated", [(3, 64, 1024, 0), (3, 64, 1024, 1), (1, 16, 512, 1), (2, 48, 1536, 0),
                                            (4, 6144, 3584, 1), (4, 3584, 3072, 0), (2, 4096, 7168, 1),
                                            (2, 7168, 2048, 0), (1, 18432, 7168, 0)])
def test_repack_bitexact(ops, oracle, E, rows, K, gated):
    print(f"[repack] E={E} rows={rows} K={K} gated={gated}", flush=True)
    w, sf = wl.mxfp4_weights(11 + gated + rows, E, rows, K, 118, 136)
    wd, sfd = ops.repack_weights(to_dev(w), to_dev(sf), gated=bool(gated))
    _sync()
    np.testing.assert_array_equal(to_np(wd).reshape(-1), oracle.w_shuffle(w, E, rows, K // 2, gated).reshape(-1))
    np.testing.assert_array_equal(to_np(sfd).reshape(-1), oracle.sf_shuffle(sf, E, rows, K // 32, gated).reshape(-1))


# --------------------------------------------------------------------------------------- decode GEMV

# kern_mxfp4_gemv_bf16 picks a kernel by shape; the cases cover each:
#   K = 512 * {2, 4, 8, 14, 16} with 2*M*K <= 144 KiB and M <= 3 or N <= 8192 ->
#   kern_mx_gemv_bf16_r{2,4,8,14,16} (unrolled; M = 8 at N = 512, 16 at N = 4096, 9 at the LDS bound);
#   M <= 2, other K -> kern_mx_gemv_bf16_rg (k groups split four ways: KG = 1, 3, 7, 32);
#   otherwise K = 1024 * {1, 2, 4, 7, 8} -> kern_mx_gemv_bf16_p{1,2,4,7,8} (half-group shares of 1, 4,
#   5, 6, 8 and 9, ragged last workgroups at N = 8336, 9216 and 18448, M = 10 just past the LDS bound);
#   anything else -> kern_mx_gemv_bf16 (K = 1536, 3072).
@pytest.mark.parametrize("M,N,K,lo,hi", [(8, 512, 1024, 124, 130), (1, 18432, 7168, 122, 132),
                                         (4, 18432, 7168, 122, 132), (16, 18432, 7168, 122, 132),
                                         (3, 1024, 2048, 100, 150),
                                         (1, 16, 512, 118, 136), (2, 48, 1536, 122, 132), (2, 32, 3584, 122, 132),
                                         (2, 9216, 7168, 122, 132), (1, 64, 16384, 122, 132),
                                         (5, 4096, 4096, 122, 132), (16, 7168, 8192, 122, 132),
                                         (7, 18448, 7168, 122, 132), (12, 1040, 7168, 122, 132),
                                         (5, 256, 1536, 122, 132), (16, 512, 3072, 122, 132),
                                         (1, 512, 1024, 122, 132), (2, 1024, 2048, 122, 132),
                                         (1, 2048, 4096, 122, 132), (1, 7168, 8192, 122, 132),
                                         (2, 112, 8192, 118, 136), (1, 9216, 7168, 122, 132),
                                         (1, 16384, 2048, 122, 132), (2, 16384, 4096, 122, 132),
                                         (1, 16384, 8192, 122, 132), (4, 512, 512, 122, 132),
                                         (16, 48, 512, 118, 136), (3, 64, 1536, 122, 132),
                                         (3, 18432, 7168, 122, 132), (3, 7168, 8192, 122, 132),
                                         (16, 4096, 4096, 122, 132), (9, 7168, 8192, 122, 132),
                                         (10, 7168, 8192, 122, 132), (4, 8336, 1024, 122, 132),
                                         (6, 16384, 2048, 122, 132), (5, 12288, 4096, 122, 132),
                                         (4, 9216, 7168, 122, 132)])
def test_gemv_w4a16(ops, oracle, M, N, K, lo, hi):
    x = wl.activations_bf16(100 + M, M, K)
    w, sf = wl.mxfp4_weights(200 + M, 1, N, K, lo, hi)
    wp, sfp = ops.repack_weights(to_dev(w[0]), to_dev(sf[0]))
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")  # rows never stored stay NaN
    ops.mxfp4_gemv_bf16(to_dev(x), wp, sfp, y, M, N=N, K=K)
    _sync()
    _, yf = oracle.gemv_w4a16(x, w[0], sf[0])
    assert_gemm_close(bf16_to_f32(to_np(y)), yf, f"gemv M={M}")


# --------------------------------------------------------------------------------------- closed-form KAT

def test_gemm_closed_form_kat(ops):
    """Row i of the e4m3 activations is one 1.0 at column 7i mod K; weights are in {-2..2}; scales are powers
    of two per (row, block) — so out[i, n] = w[n, col(i)] * 2^(ea(i,b) + ew(n,b)) exactly
    (the design of crates/kern-runtime/tests/mxfp8_gemm.rs:40-95)."""
    M, N, K = 256, 512, 1024
    col = (np.arange(M) * 7) % K
    a = np.zeros((M, K), np.uint8)
    a[np.arange(M), col] = 0x38                     # e4m3 1.0
    wv = ((np.arange(N)[:, None] + np.arange(K)[None, :]) % 5) - 2
    code = {-2: 0xC, -1: 0xA, 0: 0x0, 1: 0x2, 2: 0x4}  # e2m1 nibbles
    nib = np.vectorize(code.get)(wv).astype(np.uint8)
    w = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    ea = lambda r, b: ((r + b) % 3) - 1
    ew = lambda r, b: ((3 * r + 2 * b) % 5) - 2
    rr, bb = np.meshgrid(np.arange(M), np.arange(K // 32), indexing="ij")
    sa = (127 + ea(rr, bb)).astype(np.uint8)
    rn, bn = np.meshgrid(np.arange(N), np.arange(K // 32), indexing="ij")
    sw = (127 + ew(rn, bn)).astype(np.uint8)
    wp, swp = ops.repack_weights(to_dev(w), to_dev(sw))
    c = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ops.mxfp4_gemm_bf16(wp, swp, to_dev(a), to_dev(sa), c, M=M, m=N, k=K)
    _sync()
    b = col // 32
    expect = wv[:, col].T * np.exp2(ea(np.arange(M), b)[:, None] + ew(np.arange(N)[None, :], b[:, None]))
    np.testing.assert_array_equal(bf16_to_f32(to_np(c)), expect.astype(np.float32))


# --------------------------------------------------------------------------------------- dense e4m3 (config 3 mode)

# small M (one live 16-row subtile, or one and a row), ragged M, K not a multiple of 1024; the last 128-row
# tile of 20, 40, 70, 90, 100 and 120 rows: the activation loader's six (live subtiles, live 32-row
# request blocks) cases, (0, 1) (0, 2) (1, 3) (2, 3) (3, 4) (4, 4) for its rows 64-127
@pytest.mark.parametrize("M,m,k", [(300, 512, 1024), (4096, 2048, 7168), (5, 512, 1024), (16, 2048, 7168),
                                   (17, 512, 1536), (148, 512, 1024), (168, 512, 1024), (198, 512, 1024),
                                   (218, 512, 1024), (228, 512, 1024), (248, 512, 1024)])
def test_gemm_e4m3_per_tensor(ops, oracle, M, m, k):
    x = wl.activations_bf16(31, M, k, outlier_frac=0.01)
    w, sf = wl.mxfp4_weights(32, 1, m, k, 122, 132)
    xd = to_dev(x)
    q, qs = ops.quantize_mxfp8(xd)
    wp, sfp = ops.repack_weights(to_dev(w[0]), to_dev(sf[0]))
    d_scale = 1.0 / 64.0
    ds = torch.tensor([d_scale], dtype=torch.float32, device="cuda")
    # the production launch (no debug output), then the same with the debug accumulators: the codes must be
    # bit-identical (the debug stores make the ring's hand-counted waits stricter), and the production codes
    # are the ones checked against the oracle below
    c = torch.full((M, m), 0x5A, dtype=torch.uint8, device="cuda")
    ops.mxfp4_gemm_e4m3(wp, sfp, q, qs, c, ds, M=M, m=m, k=k)
    c_d = torch.empty((M, m), dtype=torch.uint8, device="cuda")
    dbg = torch.empty((M, m), dtype=torch.float32, device="cuda")
    ops.mxfp4_gemm_e4m3(wp, sfp, q, qs, c_d, ds, M=M, m=m, k=k, dbg=dbg)
    _sync()
    assert torch.equal(c, c_d), "e4m3 codes with and without the debug output differ"
    acc = to_np(dbg)
    qn, qsn = to_np(q), to_np(qs)
    # every row (config 3: 4096 x 2048 x 7168 takes the threaded oracle a few seconds)
    ref_c, ref_acc = oracle.gemm_e4m3_pt(to_np(wp), to_np(sfp), qn, qsn, m, k, d_scale)
    assert_gemm_close(acc, ref_acc, "prefill acc")
    # the epilogue cast is bit-exact given the kernel's own accumulator
    np.testing.assert_array_equal(to_np(c), oracle.e4m3_from_f32(acc * np.float32(d_scale)))


# --------------------------------------------------------------------------------------- routing

# One workgroup (T*k < 16384): uniform ids; every token on the same k experts (slots of 128 rows, several per
# expert); the 512-expert maximum; a segment per wave of several 64-index rounds (T*k = 12288, and 16376, one
# round below the chunked launches); decode sizes: 64 indices (one wave's round), with non-local experts,
# with every token on the same experts, and 65 (a second round). Chunked (count / scan / rank): 16384
# indices (4 chunks), a ragged last chunk with 512 experts (16392 = 4 x 3264 + 3336), a K3 rank (16384
# tokens x 16 over 224 experts, 56 local: 64 chunks), 64 chunks of 8192 indices, every token on the same
# experts, non-local experts, a single local expert.
@pytest.mark.parametrize("T,E,k,start,local,skew", [(512, 256, 8, 0, 256, 0), (37, 16, 4, 4, 8, 0),
                                                    (1, 8, 2, 0, 8, 0), (300, 224, 16, 56, 56, 0),
                                                    (2048, 64, 6, 0, 64, 0), (1000, 64, 4, 0, 64, 1),
                                                    (100, 512, 8, 0, 512, 0), (2047, 256, 8, 0, 256, 0),
                                                    (8, 256, 8, 0, 256, 0), (4, 224, 16, 56, 56, 0),
                                                    (8, 64, 8, 0, 64, 1), (13, 16, 5, 2, 8, 0),
                                                    (2048, 256, 8, 0, 256, 0), (2049, 512, 8, 0, 512, 0),
                                                    (16384, 224, 16, 56, 56, 0), (65536, 256, 8, 0, 256, 0),
                                                    (4096, 64, 4, 0, 64, 1), (3000, 256, 8, 128, 64, 0),
                                                    (4096, 8, 4, 3, 1, 0), (0, 256, 8, 0, 256, 0)])
def test_routing_bitexact(ops, oracle, T, E, k, start, local, skew):
    ids = wl.topk_ids(T * 31 + E, T, E, k)
    if skew:
        ids[:] = np.arange(k, dtype=ids.dtype)[None, ::-1] * 3
    ctas = ops.ctas_bound(T, k, local)
    ref = oracle.routing(ids, start, local, ctas_cap=ctas)
    dev = {n: torch.full((s,), -7, dtype=torch.int32, device="cuda") for n, s in
           [("counts", 2 * local), ("cta_batch", ctas), ("cta_limit", ctas), ("num_non_exiting", 1),
            ("total_padded", 1), ("route_map", ctas * 128), ("exp2perm", T * k)]}
    ops.moe_routing(to_dev(ids), dev["counts"], dev["cta_batch"], dev["cta_limit"], dev["num_non_exiting"],
                    dev["total_padded"], dev["route_map"], dev["exp2perm"], tokens=T, topk=k, local_start=start,
                    local_experts=local)
    _sync()
    S = int(ref["num_non_exiting"][0])
    assert int(to_np(dev["num_non_exiting"])[0]) == S
    assert int(to_np(dev["total_padded"])[0]) == S * 128
    np.testing.assert_array_equal(to_np(dev["counts"]), ref["counts"])
    np.testing.assert_array_equal(to_np(dev["cta_batch"])[:S], ref["cta_batch"][:S])
    np.testing.assert_array_equal(to_np(dev["cta_limit"])[:S], ref["cta_limit"][:S])
    np.testing.assert_array_equal(to_np(dev["route_map"])[:S * 128], ref["route_map"][:S * 128])
    np.testing.assert_array_equal(to_np(dev["exp2perm"]), ref["exp2perm"].reshape(-1))


# moe_quant + moe_routing in one call: decode sizes and config 4 in one launch; a K3 rank's local experts
# (ids outside the range); T*K past one launch's quantizer workgroups, which takes the two launches, with
# one-workgroup routing (T = 600) and with the chunked routing (T = 2048, 16384 expanded ids)
@pytest.mark.parametrize("T,E,k,start,local,K", [(1, 256, 8, 0, 256, 7168), (4, 256, 8, 0, 256, 7168),
                                                 (64, 256, 8, 0, 256, 7168), (512, 256, 8, 0, 256, 7168),
                                                 (300, 224, 16, 56, 56, 3584), (600, 256, 8, 0, 256, 7168),
                                                 (2048, 256, 8, 0, 256, 7168), (3, 8, 2, 0, 8, 96),
                                                 (0, 256, 8, 0, 256, 7168)])
def test_quant_routing_fused(ops, oracle, T, E, k, start, local, K):
    x = wl.activations_bf16(11 + T, T, K, outlier_frac=0.01)
    x[:min(T, 8)] = _special_rows(K)[:min(T, 8)]
    ids = wl.topk_ids(T * 7 + E, T, E, k)
    ctas = ops.ctas_bound(T, k, local)
    ref = oracle.routing(ids, start, local, ctas_cap=ctas)
    q_ref, sf_ref = oracle.quant_mxfp8(x)
    dev = {n: torch.full((s,), -7, dtype=torch.int32, device="cuda") for n, s in
           [("counts", 2 * local), ("cta_batch", ctas), ("cta_limit", ctas), ("num_non_exiting", 1),
            ("total_padded", 1), ("route_map", ctas * 128), ("exp2perm", T * k)]}
    q = torch.full((T, K), 0x5A, dtype=torch.uint8, device="cuda")
    sf = torch.full((T, K // 32), 0x5A, dtype=torch.uint8, device="cuda")
    ops.moe_quant_routing(to_dev(x), q, sf, to_dev(ids), dev["counts"], dev["cta_batch"],
                          dev["cta_limit"], dev["num_non_exiting"], dev["total_padded"], dev["route_map"],
                          dev["exp2perm"], tokens=T, K=K, topk=k, local_start=start, local_experts=local)
    _sync()
    np.testing.assert_array_equal(to_np(sf), sf_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)
    S = int(ref["num_non_exiting"][0])
    assert int(to_np(dev["num_non_exiting"])[0]) == S
    assert int(to_np(dev["total_padded"])[0]) == S * 128
    np.testing.assert_array_equal(to_np(dev["counts"]), ref["counts"])
    np.testing.assert_array_equal(to_np(dev["cta_batch"])[:S], ref["cta_batch"][:S])
    np.testing.assert_array_equal(to_np(dev["cta_limit"])[:S], ref["cta_limit"][:S])
    np.testing.assert_array_equal(to_np(dev["route_map"])[:S * 128], ref["route_map"][:S * 128])
    np.testing.assert_array_equal(to_np(dev["exp2perm"]), ref["exp2perm"].reshape(-1))


# --------------------------------------------------------------------------------------- grouped FC1 / FC2

def _route(ops, oracle, ids, local_start, local):
    T, k = ids.shape
    ctas = ops.ctas_bound(T, k, local)
    tabs = oracle.routing(ids, local_start, local, ctas_cap=ctas)
    dev = {n: to_dev(v.reshape(-1)) for n, v in tabs.items()}
    return ctas, tabs, dev


# one persistent launch: slots of at most 16 routed rows (FC1; 8 for FC2) take the skinny path, the others
# the LDS ring; decode-sized batches (all skinny), mixed ones and large ones (ring, ragged tails)
# T = 1: eight single-row slots, every tile small, its quarters dealt out over all workgroups
@pytest.mark.parametrize("T,E,k,m,K", [(64, 8, 2, 512, 1024), (512, 256, 8, 4096, 7168), (4, 256, 8, 4096, 7168),
                                       (300, 8, 2, 512, 1024), (1, 256, 8, 4096, 7168), (64, 8, 2, 512, 1536),
                                       (3, 8, 2, 512, 3584)])
def test_fc1_gated_situ(ops, oracle, T, E, k, m, K):
    _check_fc1(ops, oracle, wl.topk_ids(5 + T, T, E, k), E, m, K)


# the reference's own op shapes (moe_fc1 m=6144 k=3584, head.json:25459; moe_fc2 m=3584 k=3072, :25683): 224
# experts, top-16, this rank's 56 (ids 56..111), T = 300 (tools/trtllm-bmm/probe.py:22). K = 3584 runs the
# skinny tail (K % 1024 == 512) and the ring's odd count of 512-wide k groups; a decode-sized T = 4 too
@pytest.mark.parametrize("T", [300, 4])
def test_fc1_k3_shape(ops, oracle, T):
    _check_fc1(ops, oracle, wl.topk_ids(70 + T, T, 224, 16), 224, 6144, 3584, local_start=56, local=56)


@pytest.mark.parametrize("T", [300, 4])
def test_fc2_k3_shape(ops, oracle, T):
    _check_fc2(ops, oracle, wl.topk_ids(71 + T, T, 224, 16), 224, 3584, 3072, local_start=56, local=56)


def _split_ids():
    """64 tokens, top-2 over 64 experts: each expert takes one or two rows, except expert 5 with 41: a
    decode-like batch whose small slots take the skinny path while slot 5 takes the LDS ring, in the same
    launch."""
    ids = np.zeros((64, 2), np.int32)
    for t in range(64):
        ids[t, 0] = t
        ids[t, 1] = (6 if t == 5 else 5) if t < 41 else (t + 1) % 64
    return ids


def test_fc_split_batch(ops, oracle):
    ids = _split_ids()
    print("[fc split] 64 experts, one slot of 41 rows", flush=True)
    _check_fc1(ops, oracle, ids, 64, 512, 1024)
    _check_fc2(ops, oracle, ids, 64, 512, 1024)


def _ring_row_ids():
    """440 tokens, top-2 over 8 experts: experts 0-5 take 20, 40, 70, 90, 100 and 120 rows (first choice), expert
    6 every token's second choice (three full 128-row slots and one of 56); expert 7 none. Every slot takes the
    LDS ring, and each of its activation loader's (live subtiles, live 32-row blocks) cases occurs."""
    sizes = [20, 40, 70, 90, 100, 120]
    first = np.repeat(np.arange(len(sizes), dtype=np.int32), sizes)
    ids = np.stack([first, np.full_like(first, 6)], axis=1)
    return ids[np.random.default_rng(3).permutation(len(first))]


def test_fc_ring_row_counts(ops, oracle):
    ids = _ring_row_ids()
    print("[fc ring rows] slots of 20..128 rows", flush=True)
    _check_fc1(ops, oracle, ids, 8, 512, 1024)
    _check_fc2(ops, oracle, ids, 8, 512, 1024)


def test_fc_most_experts(ops, oracle):
    """512 local experts (the routing tables' maximum), about four rows each: every slot skinny."""
    ids = wl.topk_ids(90, 256, 512, 8)
    print("[fc max experts] E=512, T=256, top-8", flush=True)
    _check_fc1(ops, oracle, ids, 512, 512, 1024)
    _check_fc2(ops, oracle, ids, 512, 512, 1024)


def test_fc_widest_weights(ops, oracle):
    """m = 131072 weight rows (the largest the C ABI takes): 512 weight tiles per slot, so the walk's tile codes
    reach nx = 511, on a skinny slot (4 rows) and a ring slot (20 rows)."""
    ids = np.concatenate([np.zeros((4, 1), np.int32), np.ones((20, 1), np.int32)])
    print("[fc widest] m=131072, K=512, slots of 4 and 20 rows", flush=True)
    _check_fc1(ops, oracle, ids, 2, 131072, 512)
    _check_fc2(ops, oracle, ids, 2, 131072, 512)


def test_fc2_live_count_is_capped_by_the_tables(ops, oracle):
    """num_non_exiting larger than the slot tables (a corrupt count): the persistent kernel walks no slot past
    the tables' capacity; the live slots' rows come out as with the true count (the tables past the routed
    slots hold -7, which no slot takes as rows)."""
    T, E, k, m, K = 64, 8, 2, 512, 1024
    ids = wl.topk_ids(21, T, E, k)
    ctas, tabs, dev = _route(ops, oracle, ids, 0, E)
    S = int(tabs["num_non_exiting"][0])
    for n in ("cta_batch", "cta_limit"):
        dev[n][S:] = -7
    rows = ctas * 128
    q, qs = oracle.quant_mxfp8(wl.activations_bf16(22, rows, K))
    qs_r = np.zeros(oracle.r128c4_size(rows, K // 32), np.uint8)
    qs_r[r128c4_offsets(rows, K // 32)] = qs
    w, sf = wl.mxfp4_weights(23, E, m, K, 118, 126)
    wp, sfp = ops.repack_weights(to_dev(w), to_dev(sf))
    outs = []
    for nne in (S, 1 << 30):
        dev["num_non_exiting"][0] = nne
        c = torch.zeros((rows, m), dtype=torch.bfloat16, device="cuda")
        ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(wp, sfp, to_dev(q), to_dev(qs_r), c, dev["num_non_exiting"],
                                          dev["total_padded"], dev["cta_batch"], dev["cta_limit"], m=m, k=K,
                                          ctas=ctas, sf_b_r128c4=True)
        _sync()
        outs.append(to_np(c.view(torch.int16)))
    np.testing.assert_array_equal(outs[0], outs[1])


def test_empty_batch_chain(ops):
    """An empty batch through the MoE chain: zero tokens routed (the tables say no live slots), then FC1, FC2
    and the finalize on those tables write nothing (every output keeps its sentinel bytes)."""
    E, k, H, I = 8, 2, 1024, 512
    ctas = ops.ctas_bound(0, k, E)
    rows = ctas * 128
    i32 = torch.int32
    tab = {n: torch.full((sz,), -7, dtype=i32, device="cuda") for n, sz in
           [("counts", 2 * E), ("cb", ctas), ("cl", ctas), ("nne", 1), ("tp", 1), ("rm", rows)]}
    ops.moe_routing(torch.empty((0, k), dtype=i32, device="cuda"), tab["counts"], tab["cb"], tab["cl"], tab["nne"],
                    tab["tp"], tab["rm"], torch.empty(0, dtype=i32, device="cuda"), tokens=0, topk=k, local_start=0,
                    local_experts=E)
    _sync()
    assert (int(tab["nne"][0]), int(tab["tp"][0])) == (0, 0) and not tab["counts"].any()
    w1, s1 = wl.mxfp4_weights(31, E, 2 * I, H, 118, 126)
    w2, s2 = wl.mxfp4_weights(32, E, H, I, 118, 126)
    w1p, s1p = ops.repack_weights(to_dev(w1), to_dev(s1), gated=True)
    w2p, s2p = ops.repack_weights(to_dev(w2), to_dev(s2))
    q = torch.zeros((1, H), dtype=torch.uint8, device="cuda")  # a token row the launches must not read
    qs = torch.zeros((1, H // 32), dtype=torch.uint8, device="cuda")
    c1 = torch.full((rows, I), 0x5A, dtype=torch.uint8, device="cuda")
    sf1 = torch.full((ops.r128c4_bytes(rows, I // 32),), 0x5A, dtype=torch.uint8, device="cuda")
    c2 = torch.full((rows, H), 0x5A5A, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    alpha = torch.full((E,), 4.0, device="cuda")
    beta = torch.full((E,), 25.0, device="cuda")
    ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w1p, s1p, q, qs, c1, sf1, tab["rm"], alpha, beta, tab["nne"], tab["tp"],
                                        tab["cb"], tab["cl"], m=2 * I, k=H, ctas=ctas)
    ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2p, s2p, c1, sf1, c2, tab["nne"], tab["tp"], tab["cb"], tab["cl"], m=H, k=I,
                                      ctas=ctas, sf_b_r128c4=True)
    y = torch.full((1, H), 0x5A5A, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    gamma = torch.ones(H, dtype=torch.bfloat16, device="cuda")
    tw = torch.ones((1, k), dtype=torch.float32, device="cuda")
    ops.moe_finalize_rms(c2, torch.zeros(k, dtype=i32, device="cuda"), tw, gamma, y, 0, H=H, topk=k, eps=1e-6)
    _sync()
    assert bool((c1 == 0x5A).all()) and bool((sf1 == 0x5A).all()), "fc1 wrote rows of an empty batch"
    assert bool((c2.view(torch.int16) == 0x5A5A).all()), "fc2 wrote rows of an empty batch"
    assert bool((y.view(torch.int16) == 0x5A5A).all()), "the finalize wrote a token of an empty batch"


def _check_fc1(ops, oracle, ids, E, m, K, local_start=0, local=None):
    """FC1 through the C ABI over a routed batch, every live slot checked against the oracle (tests/_moe.py)."""
    from tests import _moe

    T = ids.shape[0]
    local = E if local is None else local
    ctas, tabs, dev = _route(ops, oracle, ids, local_start, local)
    x = wl.activations_bf16(6 + T, T, K)
    w, sf = _moe.gpu_raw_weights(ops, torch, 8 + T, local, m, K, 119, 6)
    q, qs = ops.quantize_mxfp8(to_dev(x))
    wp, sfp = ops.repack_weights(w, sf, gated=True)
    del w, sf
    alpha = np.full(local, 4.0, np.float32) + np.arange(local, dtype=np.float32) * 0.01
    beta = np.full(local, 25.0, np.float32)
    rows = ctas * 128
    half = m // 2
    c = torch.zeros((rows, half), dtype=torch.uint8, device="cuda")
    sf_c = torch.zeros(oracle.r128c4_size(rows, half // 32), dtype=torch.uint8, device="cuda")
    al_d, be_d = to_dev(alpha), to_dev(beta)

    def launch(c_, sf_, dbg_):
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(wp, sfp, q, qs, c_, sf_, dev["route_map"], al_d, be_d,
                                            dev["num_non_exiting"], dev["total_padded"], dev["cta_batch"],
                                            dev["cta_limit"], m=m, k=K, ctas=ctas, dbg=dbg_)

    launch(c, sf_c, None)  # the production launch (no debug output)
    _sync()
    dbg = _moe.fc1_debug_twin(torch, launch, c, sf_c, f"fc1 T={T} K={K}")
    print(f"[fc1] T={T} E={local} m={m} K={K}: {int(tabs['num_non_exiting'][0])} live slots", flush=True)
    _moe.check_fc1(torch, oracle, wp, sfp, q, qs, tabs, alpha, beta, m, K, c, sf_c, dbg, f"fc1 T={T} K={K}")


@pytest.mark.parametrize("T,E,k,m,K", [(64, 8, 2, 512, 1024), (512, 256, 8, 7168, 2048), (4, 256, 8, 7168, 2048),
                                       (300, 8, 2, 512, 1024), (1, 256, 8, 7168, 2048), (64, 8, 2, 512, 1536),
                                       (300, 8, 2, 512, 3584), (3, 8, 2, 512, 3584)])
def test_fc2_bf16(ops, oracle, T, E, k, m, K):
    _check_fc2(ops, oracle, wl.topk_ids(9 + T, T, E, k), E, m, K)


def _check_fc2(ops, oracle, ids, E, m, K, local_start=0, local=None):
    """FC2 through the C ABI over a routed batch, every live slot checked against the oracle (tests/_moe.py)."""
    from tests import _moe

    T = ids.shape[0]
    local = E if local is None else local
    ctas, tabs, dev = _route(ops, oracle, ids, local_start, local)
    rows = ctas * 128
    # activations in permuted row order (what FC1 writes): e4m3 codes and R128c4 scales
    xb = wl.activations_bf16(10 + T, rows, K)
    q_lin, qs_lin = oracle.quant_mxfp8(xb)
    qs_r = np.zeros(oracle.r128c4_size(rows, K // 32), np.uint8)
    qs_r[r128c4_offsets(rows, K // 32)] = qs_lin
    w, sf = _moe.gpu_raw_weights(ops, torch, 12 + T, local, m, K, 118, 9)
    wp, sfp = ops.repack_weights(w, sf)
    del w, sf
    c = torch.zeros((rows, m), dtype=torch.bfloat16, device="cuda")
    qd, qsd = to_dev(q_lin), to_dev(qs_r)
    ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(wp, sfp, qd, qsd, c, dev["num_non_exiting"], dev["total_padded"],
                                      dev["cta_batch"], dev["cta_limit"], m=m, k=K, ctas=ctas, sf_b_r128c4=True)
    _sync()
    print(f"[fc2] T={T} E={local} m={m} K={K}: {int(tabs['num_non_exiting'][0])} live slots", flush=True)
    _moe.check_fc2(torch, oracle, wp, sfp, qd, qsd, tabs, m, K, c, f"fc2 T={T} K={K}")


# --------------------------------------------------------------------------------------- MoE glue

def _ulp(a, b):
    ai, bi = a.astype(np.int32), b.astype(np.int32)
    oa = np.where(ai & 0x8000, -(ai & 0x7FFF), ai)
    ob = np.where(bi & 0x8000, -(bi & 0x7FFF), bi)
    return np.abs(oa - ob)


@pytest.fixture(scope="module")
def oracle():
    from oracle import mxoracle
    mxoracle.lib()
    return mxoracle


@pytest.mark.parametrize("T,d", [(7, 2056), (64, 2048), (3, 8), (512, 7168)])
def test_silu_mul(ops, oracle, T, d):
    x = wl.activations_bf16(300 + d, T, 2 * d)
    if T == 7:  # special values in the gate half
        f = wl.bf16_bits_to_f32(x).copy()
        f[0, :6] = [np.inf, -np.inf, np.nan, 0.0, -100.0, 100.0]
        f[1, :4] = [88.0, -88.0, 1e-30, -1e-30]
        x = wl.f32_to_bf16_bits(f)
    out = torch.zeros((T, d), dtype=torch.bfloat16, device="cuda")
    ops.silu_mul(out, to_dev(x), T, d)
    _sync()
    got = to_np(out).view(np.uint16)
    ref = oracle.silu_mul_bf16(x, d)
    nan_g, nan_r = np.isnan(wl.bf16_bits_to_f32(got)), np.isnan(wl.bf16_bits_to_f32(ref))
    np.testing.assert_array_equal(nan_g, nan_r)
    fin = ~nan_r
    # exp is the platform's (ocml on the GPU, libm here): results agree to one bf16 ulp, almost all exactly
    d_ulp = _ulp(got[fin], ref[fin])
    assert d_ulp.max() <= 1
    assert (d_ulp == 0).mean() > 0.999


def _finalize_case(T, H, k, rows, seed):
    rng = np.random.default_rng(seed)
    fc2 = wl.f32_to_bf16_bits(rng.standard_normal((rows, H)).astype(np.float32))
    e2p = rng.permutation(rows)[: T * k].astype(np.int32)
    e2p[5 % e2p.size] = -1  # a non-local expert
    w = rng.random((T, k)).astype(np.float32) + 0.05
    w /= w.sum(1, keepdims=True)
    return fc2, e2p, w


@pytest.mark.parametrize("T,H,k", [(512, 7168, 8), (9, 3584, 16), (3, 64, 2)])
def test_moe_finalize_bitexact(ops, oracle, T, H, k):
    rows = ((T * k + 127) // 128 + 4) * 128
    fc2, e2p, w = _finalize_case(T, H, k, rows, 40 + H)
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_finalize(to_dev(fc2), to_dev(e2p), to_dev(w), out, T, H=H, topk=k)
    _sync()
    np.testing.assert_array_equal(to_np(out).view(np.uint16), oracle.moe_finalize(fc2, e2p, w, None, T, H, k))


@pytest.mark.parametrize("T,H,k", [(512, 7168, 8), (9, 3584, 16), (3, 8192, 2), (5, 520, 4), (2, 8, 1)])
def test_moe_finalize_rms(ops, oracle, T, H, k):
    rows = ((T * k + 127) // 128 + 4) * 128
    fc2, e2p, w = _finalize_case(T, H, k, rows, 50 + H)
    gamma = wl.f32_to_bf16_bits((np.random.default_rng(H).random(H) + 0.5).astype(np.float32))
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_finalize_rms(to_dev(fc2), to_dev(e2p), to_dev(w), to_dev(gamma), out, T, H=H, topk=k, eps=1e-6)
    _sync()
    ref = oracle.moe_finalize(fc2, e2p, w, gamma, T, H, k, 1e-6)
    # the combine is exact; the row's sum of squares is reduced in another order: one bf16 ulp at most
    assert _ulp(to_np(out).view(np.uint16), ref).max() <= 1


@pytest.mark.parametrize("T,H,k,block", [(9, 7168, 8, 256), (5, 3584, 16, 64), (4, 8192, 2, 512), (3, 512, 4, 1024)])
def test_moe_finalize_rms_any_block(ops, oracle, T, H, k, block):
    """A manifest may launch the kernel with another whole-wave block than the C ABI's (H/8 threads rounded up
    to 64): with fewer threads than chunks each thread takes several, with more the extra ones idle."""
    from kern_amd import manifest as mf
    print(f"[finalize_rms] T={T} H={H} k={k} block {block}", flush=True)
    rows = ((T * k + 127) // 128 + 4) * 128
    fc2, e2p, w = _finalize_case(T, H, k, rows, 60 + H)
    gamma = wl.f32_to_bf16_bits((np.random.default_rng(H + 1).random(H) + 0.5).astype(np.float32))
    op = mf.moe_finalize_rms(H, k)
    op["impl"]["launches"][0]["block"] = [block, 1, 1]
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    ops.ManifestOp(op)(to_dev(fc2), to_dev(e2p), to_dev(w), to_dev(gamma), out, T, vars={"tokens": T})
    _sync()
    ref = oracle.moe_finalize(fc2, e2p, w, gamma, T, H, k, 1e-6)
    assert _ulp(to_np(out).view(np.uint16), ref).max() <= 1


# --------------------------------------------------------------------------------------- weight_prep

def test_weight_p1_and_cast(ops):
    n = 100003
    w = wl.activations_bf16(401, 1, n).reshape(-1)
    out = torch.zeros(n, dtype=torch.float32, device="cuda")
    ops.weight_p1_bf16_f32(to_dev(w), out)
    _sync()
    np.testing.assert_array_equal(to_np(out), wl.bf16_bits_to_f32(w) + np.float32(1.0))
    ops.cast_bf16_f32(to_dev(w), out)
    _sync()
    np.testing.assert_array_equal(to_np(out), wl.bf16_bits_to_f32(w))


@pytest.mark.parametrize("n", [1, 224, 100003])
def test_fills(ops, n):
    for dtype, v, want in [(torch.float32, -2.5, np.float32(-2.5)), (torch.int32, -7, np.int32(-7)),
                           (torch.int64, 2**40 + 3, np.int64(2**40 + 3)), (torch.uint8, 201, np.uint8(201)),
                           (torch.bfloat16, 0.1, wl.f32_to_bf16_bits(np.float32([0.1]))[0])]:
        p = torch.zeros(n + 5, dtype=dtype, device="cuda")
        ops.fill(p[:n], v)
        _sync()
        got = to_np(p)
        assert (got[:n] == want).all(), dtype
        assert not got[n:].any(), dtype  # nothing past n


def test_iota(ops):
    n, start, step, stride = 1000, -5, 3, 4
    p = torch.full(((n - 1) * stride + 1 + 8,), -1, dtype=torch.int32, device="cuda")
    ops.iota_i32(p, n, start, step, stride)
    _sync()
    got = to_np(p)
    np.testing.assert_array_equal(got[: (n - 1) * stride + 1: stride], start + np.arange(n) * step)
    mask = np.ones(got.size, bool)
    mask[: (n - 1) * stride + 1: stride] = False
    assert (got[mask] == -1).all()


@pytest.mark.parametrize("rows,half,stride,base", [(4096, 64, 64, 10000.0), (300, 96, 192, 500000.0)])
def test_rope_table(ops, oracle, rows, half, stride, base):
    c = torch.zeros(rows * stride, dtype=torch.bfloat16, device="cuda")
    s = torch.zeros(rows * stride, dtype=torch.bfloat16, device="cuda")
    ops.rope_table_bf16(c, s, rows, half, stride, base)
    _sync()
    rc, rs = oracle.rope_table(rows, half, stride, base)
    # powf, cos and sin are the platform's: a one-ulp difference in powf moves the f32 angle r*inv by
    # about an ulp of the angle, which |d cos| <= |d angle| carries into the result; beyond that, one
    # bf16 ulp of the result
    j = np.arange(stride) % stride
    inv = np.where(j < half, 1.0 / base ** (2.0 * np.minimum(j, half - 1) / (2 * half)), 0.0)
    ang = (np.arange(rows)[:, None] * inv[None, :]).reshape(-1)
    for got, ref in [(to_np(c), rc), (to_np(s), rs)]:
        g, r = wl.bf16_bits_to_f32(got).astype(np.float64), wl.bf16_bits_to_f32(ref).astype(np.float64)
        assert (np.abs(g - r) <= 2.0**-7 * np.abs(r) + 4 * 2.0**-23 * ang + 1e-6).all()  # ulp <= 2^-7 |x|
        assert (got == ref).mean() > 0.99


# --------------------------------------------------------------------------------------- MXFP8 x MXFP8

def test_mxfp8_gemm_kat(ops):
    from tests._util import mxfp8_kat
    c = mxfp8_kat(0)
    M, N, K = c["M"], c["N"], c["K"]
    a, w, a_sf, w_sf = (to_dev(c[x]) for x in ("a", "w", "a_sf", "w_sf"))
    out = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    ops.cublaslt_mxfp8_tn(a, w, out, a_sf, w_sf, M, N, K)
    _sync()
    np.testing.assert_array_equal(to_np(out), wl.f32_to_bf16_bits(c["want"]))
    # captured once, replayed after the scales change on the device: they are read at run time
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with ops.Graph() as g:
            ops.cublaslt_mxfp8_tn(a, w, out, a_sf, w_sf, M, N, K)
        w_sf.copy_(to_dev(mxfp8_kat(-1)["w_sf"]))
        out.zero_()
        g.launch()
    _sync()
    np.testing.assert_array_equal(to_np(out), wl.f32_to_bf16_bits(mxfp8_kat(-1)["want"]))


# ragged m, n and k; and the benchmark's shape, config 3's 4096 x 2048 x 7168
@pytest.mark.parametrize("m,n,k", [(300, 520, 1024), (64, 1000, 2080), (200, 256, 96), (2048, 2048, 7168),
                                   (4096, 2048, 7168)])
def test_mxfp8_gemm_random(ops, oracle, m, n, k):
    from kern_amd import ops as o
    rng = np.random.default_rng(m + n + k)
    xa = wl.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    xw = wl.f32_to_bf16_bits(rng.standard_normal((n, k)).astype(np.float32))
    qa, sa = oracle.quant_mxfp8(xa)
    qw, sw = oracle.quant_mxfp8(xw)

    def tiled(sf, rows):
        t = np.full(o.r128c4_bytes(rows, k // 32), 127, np.uint8)
        t[r128c4_offsets(rows, k // 32)] = sf
        return t

    ta, tw = tiled(sa, m), tiled(sw, n)
    out = torch.zeros((m, n + 8), dtype=torch.bfloat16, device="cuda")  # ldc = n + 8: the gap stays zero
    ops.cublaslt_mxfp8_tn(to_dev(qa), to_dev(qw), out, to_dev(ta), to_dev(tw), m, n, k, ldc=n + 8)
    _sync()
    got = bf16_to_f32(to_np(out))
    assert not got[:, n:].any()
    ref = oracle.mxfp8_gemm(qa, qw, ta, tw, m, n, k)
    assert_gemm_close(got[:, :n], ref, f"mxfp8 {m}x{n}x{k}")


# --------------------------------------------------------------------------------------- high operand addresses

class _HighArena:
    """Device views whose addresses all have bit 31 of their low 32 bits set. The LDS ring's requests build a
    wave-uniform 64-bit base in an SGPR pair from two readfirstlane halves, and a form that sign-extended the
    low half into the high one sent an illegal address exactly when that bit was set. Views are 4 KiB
    aligned, one after another from the first such address past the buffer's start."""

    def __init__(self, nbytes):
        self.buf = torch.empty(nbytes + (1 << 32) + 8192, dtype=torch.uint8, device="cuda")
        base = self.buf.data_ptr()
        lo = base & 0xFFFFFFFF
        if lo >= (1 << 31) and lo + nbytes + 8192 <= (1 << 32):
            start = base
        elif lo < (1 << 31):
            start = base - lo + (1 << 31)
        else:
            start = base - lo + (1 << 32) + (1 << 31)
        self.cur, self.end = start - base, start - base + nbytes + 8192

    def put(self, t):
        n = t.numel() * t.element_size()
        self.cur = (self.cur + 4095) & ~4095
        assert self.cur + n <= self.end
        v = self.buf[self.cur:self.cur + n].view(t.dtype).view(t.shape)
        v.copy_(t)
        a = v.data_ptr()
        assert (a & 0xFFFFFFFF) >= (1 << 31) and ((a + max(n, 1) - 1) & 0xFFFFFFFF) >= (1 << 31), hex(a)
        self.cur += n
        return v


def test_ring_operands_above_bit31(ops, oracle):
    """The LDS-ring GEMMs with every operand and output at an address whose bit 31 is set: the config-3 mode
    GEMM, FC1 and FC2 (slots of 20..128 rows, all on the ring) each equal the same launch on ordinary buffers
    bit for bit; those are checked against the oracle here too (the GEMM's accumulators, FC1's codes through
    its debug twin, FC2's rows)."""
    from tests import _moe

    arena = _HighArena(64 << 20)
    hi = arena.put
    # config-3 mode, dense
    M, m, k = 300, 512, 1024
    x = wl.activations_bf16(41, M, k, outlier_frac=0.01)
    w, sf = wl.mxfp4_weights(42, 1, m, k, 122, 132)
    q, qs = ops.quantize_mxfp8(to_dev(x))
    wp, sfp = ops.repack_weights(to_dev(w[0]), to_dev(sf[0]))
    ds = torch.tensor([1.0 / 64.0], dtype=torch.float32, device="cuda")
    c = torch.empty((M, m), dtype=torch.uint8, device="cuda")
    dbg = torch.empty((M, m), dtype=torch.float32, device="cuda")
    ops.mxfp4_gemm_e4m3(wp, sfp, q, qs, c, ds, M=M, m=m, k=k, dbg=dbg)
    c_hi = hi(torch.zeros_like(c))
    ops.mxfp4_gemm_e4m3(hi(wp), hi(sfp), hi(q), hi(qs), c_hi, hi(ds), M=M, m=m, k=k)
    _sync()
    print("[bit 31] e4m3 GEMM", flush=True)
    _, ref_acc = oracle.gemm_e4m3_pt(to_np(wp), to_np(sfp), to_np(q), to_np(qs), m, k, 1.0 / 64.0)
    assert_gemm_close(to_np(dbg), ref_acc, "bit 31: e4m3 acc")
    np.testing.assert_array_equal(to_np(c), oracle.e4m3_from_f32(to_np(dbg) * np.float32(1.0 / 64.0)))
    assert torch.equal(c_hi, c), "bit 31: e4m3 GEMM output differs"

    # FC1 then FC2 on its output: every slot on the ring
    ids = _ring_row_ids()
    E, m1, K1, m2 = 8, 2048, 1024, 512
    T = ids.shape[0]
    ctas, tabs, dev = _route(ops, oracle, ids, 0, E)
    rows = ctas * 128
    xq, xqs = ops.quantize_mxfp8(to_dev(wl.activations_bf16(43, T, K1)))
    w1, s1 = _moe.gpu_raw_weights(ops, torch, 44, E, m1, K1, 119, 6)
    w1p, s1p = ops.repack_weights(w1, s1, gated=True)
    w2, s2 = _moe.gpu_raw_weights(ops, torch, 45, E, m2, m1 // 2, 118, 9)
    w2p, s2p = ops.repack_weights(w2, s2)
    alpha = np.full(E, 4.0, np.float32)
    beta = np.full(E, 25.0, np.float32)
    al, be = to_dev(alpha), to_dev(beta)
    tab_hi = {n: hi(v) for n, v in dev.items()}

    def fc1(args, c_, sf_, dbg_=None):
        wa, sa, b, sb, rm, a_, b_, t = args
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(wa, sa, b, sb, c_, sf_, rm, a_, b_, t["num_non_exiting"],
                                            t["total_padded"], t["cta_batch"], t["cta_limit"], m=m1, k=K1, ctas=ctas,
                                            dbg=dbg_)

    lo_args = (w1p, s1p, xq, xqs, dev["route_map"], al, be, dev)
    hi_args = (hi(w1p), hi(s1p), hi(xq), hi(xqs), tab_hi["route_map"], hi(al), hi(be), tab_hi)
    c1 = torch.zeros((rows, m1 // 2), dtype=torch.uint8, device="cuda")
    sf1 = torch.zeros(oracle.r128c4_size(rows, m1 // 64), dtype=torch.uint8, device="cuda")
    fc1(lo_args, c1, sf1)
    c1_hi, sf1_hi = hi(torch.zeros_like(c1)), hi(torch.zeros_like(sf1))
    fc1(hi_args, c1_hi, sf1_hi)
    _sync()
    print("[bit 31] FC1", flush=True)
    assert torch.equal(c1_hi, c1) and torch.equal(sf1_hi, sf1), "bit 31: FC1 output differs"
    dbg1 = _moe.fc1_debug_twin(torch, lambda c_, s_, d_: fc1(lo_args, c_, s_, d_), c1, sf1, "bit 31 fc1")
    _moe.check_fc1(torch, oracle, w1p, s1p, xq, xqs, tabs, alpha, beta, m1, K1, c1, sf1, dbg1, "bit 31 fc1")

    def fc2(wa, sa, b, sb, c_, t):
        ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(wa, sa, b, sb, c_, t["num_non_exiting"], t["total_padded"],
                                          t["cta_batch"], t["cta_limit"], m=m2, k=m1 // 2, ctas=ctas,
                                          sf_b_r128c4=True)

    c2 = torch.zeros((rows, m2), dtype=torch.bfloat16, device="cuda")
    fc2(w2p, s2p, c1, sf1, c2, dev)
    c2_hi = hi(torch.zeros_like(c2))
    fc2(hi(w2p), hi(s2p), c1_hi, sf1_hi, c2_hi, tab_hi)
    _sync()
    print("[bit 31] FC2", flush=True)
    assert torch.equal(c2_hi.view(torch.int16), c2.view(torch.int16)), "bit 31: FC2 output differs"
    _moe.check_fc2(torch, oracle, w2p, s2p, c1, sf1, tabs, m2, m1 // 2, c2, "bit 31 fc2")
