"""Stage checks of the MoE ops against the CPU oracle, over every live slot (shared by the GPU tests).

Each check takes the GPU's own inputs to the stage (so the oracle and the kernel see the same bytes) and
runs the oracle once over all live slots, on only the experts the slots use (gathered on the device and
renumbered), so full checks at config-4/5 and K3 sizes take seconds on the host.
"""
import numpy as np

from kern_amd import workload as wl
from tests._util import assert_gemm_close, bf16_to_f32, to_dev, to_np


def gpu_raw_weights(ops, torch, seed, E, rows, K, lo=119, span=6):
    """Raw MXFP4 nibbles u8 [E, rows, K/2] and e8m0 scales u8 [E, rows, K/32] filled on the device with
    the workload streams (the bytes wl.mxfp4_weights(seed, ...) makes on the host)."""
    w = torch.empty((E, rows, K // 2), dtype=torch.uint8, device="cuda")
    s = torch.empty((E, rows, K // 32), dtype=torch.uint8, device="cuda")
    ops.fill_random_u8(w, wl.tensor_seed(seed, 3))
    ops.fill_random_u8(s, wl.tensor_seed(seed, 4), lo, span)
    return w, s


def route(ops, oracle, ids, local_start, local):
    """Routing tables from the oracle (bit-exact with kern_moe_routing, checked elsewhere), on the device."""
    T, k = ids.shape
    ctas = ops.ctas_bound(T, k, local)
    tabs = oracle.routing(ids, local_start, local, ctas_cap=ctas)
    dev = {n: to_dev(v.reshape(-1)) for n, v in tabs.items()}
    return ctas, tabs, dev


def live_rows(tabs, rows):
    """Mask [rows] of the routed rows of the live slots."""
    S = int(tabs["num_non_exiting"][0])
    pr = np.arange(rows)
    s = pr // 128
    lim = np.where(s < S, tabs["cta_limit"][np.minimum(s, len(tabs["cta_limit"]) - 1)], 0)
    return (s < S) & (pr < lim)


def compact_experts(torch, wp, sfp, tabs, *per_expert):
    """The live slots' experts gathered from device weights [E, ...] to the host, and the tables with
    cta_batch renumbered to match; per_expert arrays (alpha, beta, ...) gathered alike."""
    S = int(tabs["num_non_exiting"][0])
    used = np.unique(tabs["cta_batch"][:S])
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    a = to_np(wp.index_select(0, idx))
    sa = to_np(sfp.index_select(0, idx))
    remap = np.full(max(int(used.max()) + 1, 1), -1, np.int32)
    remap[used] = np.arange(used.size, dtype=np.int32)
    sub = dict(tabs)
    cb = tabs["cta_batch"].copy()
    cb[:S] = remap[cb[:S]]
    sub["cta_batch"] = cb
    return (a, sa, sub) + tuple(np.asarray(p)[used] for p in per_expert)


def check_fc1(torch, oracle, wp, sfp, xq, xqs, tabs, alpha, beta, m, K, c, sf_c, dbg, what):
    """FC1 over every live slot: gate and up accumulators within the north-star tolerance of the oracle
    (gathered activation rows, gated weight rows); SiTU-GLU on the kernel's accumulators within f32
    rounding of the formula (probe.py:46-47); e4m3 codes and ue8m0 sf_c (R128c4) bit-exact against the
    oracle quantizer on the kernel's own SiTU values. c / sf_c are a production launch's (no debug
    output), dbg the values of its debug twin (fc1_debug_twin)."""
    rows = c.shape[0]
    half = m // 2
    a, sa, sub, al, be = compact_experts(torch, wp, sfp, tabs, alpha, beta)
    _, _, ref_dbg = oracle.fc1(a, sa, to_np(xq), to_np(xqs), sub, al, be, m, K, rows)
    valid = live_rows(tabs, rows)
    g = to_np(dbg)
    assert_gemm_close(g[valid, 0], ref_dbg[valid, 0], f"{what}: fc1 gate acc")
    assert_gemm_close(g[valid, 1], ref_dbg[valid, 1], f"{what}: fc1 up acc")
    S = int(tabs["num_non_exiting"][0])
    slot_e = np.repeat(tabs["cta_batch"][:S], 128)[valid[: S * 128]]
    gg, uu = g[valid, 0].astype(np.float64), g[valid, 1].astype(np.float64)
    al_r = np.asarray(alpha, np.float64)[slot_e][:, None]
    be_r = np.asarray(beta, np.float64)[slot_e][:, None]
    with np.errstate(over="ignore"):
        h_ref = al_r * np.tanh(gg / al_r) / (1.0 + np.exp(-gg)) * be_r * np.tanh(uu / be_r)
    np.testing.assert_allclose(g[valid, 2], h_ref, rtol=2e-5, atol=1e-6, err_msg=f"{what}: situ")
    qref, sref = oracle.quant_blocks(g[valid, 2])
    np.testing.assert_array_equal(to_np(c)[valid], qref, err_msg=f"{what}: fc1 codes")
    pv = np.nonzero(valid)[0]
    kb = half // 32
    kb4 = -(-kb // 4)
    b = np.arange(kb)[None, :]
    offs = 512 * ((pv[:, None] // 128) * kb4 + b // 4) + (pv[:, None] % 32) * 16 + ((pv[:, None] % 128) // 32) * 4 + b % 4
    np.testing.assert_array_equal(to_np(sf_c)[offs], sref, err_msg=f"{what}: fc1 sf_c")


def fc1_debug_twin(torch, launch, c, sf_c, what):
    """FC1 as production launches it (no debug output) has written c / sf_c. Launch it again on the same
    inputs with the debug output into fresh buffers and require its codes and scales to be bit-identical to
    the production ones over the whole buffers: the debug stores are extra vector-memory operations, which
    make the ring's hand-counted waits stricter, so a production wait one short would show here. Returns
    the debug launch's [rows, 3, m/2] gate / up / SiTU values for check_fc1, which then compares the
    production codes with the oracle."""
    rows, half = c.shape
    c_d, sf_d = torch.zeros_like(c), torch.zeros_like(sf_c)
    dbg = torch.zeros((rows, 3, half), dtype=torch.float32, device=c.device)
    launch(c_d, sf_d, dbg)
    torch.cuda.synchronize()
    assert torch.equal(c_d, c), f"{what}: fc1 codes with and without the debug output differ"
    assert torch.equal(sf_d, sf_c), f"{what}: fc1 sf_c with and without the debug output differ"
    return dbg


def check_fc2(torch, oracle, wp, sfp, b, sfb_r128c4, tabs, m, K, c, what):
    """FC2 over every live slot: the bf16 output within the north-star tolerance of the oracle's f32
    accumulators on the same e4m3 rows and R128c4 scales."""
    rows = c.shape[0]
    a, sa, sub = compact_experts(torch, wp, sfp, tabs)
    _, acc = oracle.fc2(a, sa, to_np(b), to_np(sfb_r128c4), True, sub, m, K)
    valid = live_rows(tabs, rows)
    assert_gemm_close(bf16_to_f32(to_np(c))[valid], acc[valid], f"{what}: fc2")


def ulp_bf16(a, b):
    ai, bi = a.astype(np.int32), b.astype(np.int32)
    oa = np.where(ai & 0x8000, -(ai & 0x7FFF), ai)
    ob = np.where(bi & 0x8000, -(bi & 0x7FFF), bi)
    return np.abs(oa - ob)


def check_finalize(oracle, c2, exp2perm, tw, gamma, y, T, H, k, eps, what):
    """The combine is exact; with the norm the row's sum of squares is reduced in another order: at most
    one bf16 ulp apart."""
    ref = oracle.moe_finalize(to_np(c2), to_np(exp2perm), to_np(tw), None if gamma is None else to_np(gamma),
                              T, H, k, eps)
    got = to_np(y)
    if gamma is None:
        np.testing.assert_array_equal(got, ref, err_msg=f"{what}: finalize")
    else:
        assert ulp_bf16(got, ref).max() <= 1, f"{what}: finalize_rms"
