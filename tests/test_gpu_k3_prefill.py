"""One EP4 rank's share of K3 prefill at its full size, on the GPU: 16384 tokens x top-16 over 224 experts,
this rank's 56 (ids 56..111), H = 3584, I = 3072 (the reference's K3 shapes, docs/roadmap.md:63). That is
65,443 routed rows in 540 CTA slots, so the persistent FC1 / FC2 walks cover every CU of every XCD with
many chained tiles per workgroup, and routing takes its chunked launches (262,144 expanded ids).

The chain runs as production launches it (no debug output): moe_quant -> moe_routing -> FC1 -> FC2. The
routing tables are checked bit for bit against the oracle. FC1 and FC2 are checked on 16 whole slots: the
first, the last, and the two slots on either side of each XCD's range boundary (slot S*x/8). The oracle
recomputes those slots alone, on tables renumbered to them.
* FC1 (gated SiTU-GLU, MXFP8 out): launched again with the debug output (about 10 GB of f32 values), whose
  codes and sf_c must equal the production launch's over the whole buffers. On the sampled slots the
  debug launch's gate and up accumulators are within the north-star GEMM tolerance of the oracle's, its
  SiTU values within 2e-5 of the float64 formula on them (tools/trtllm-bmm/probe.py:46-47), and the codes
  and sf_c are the oracle quantizer's on those values, bit for bit.
* FC2 (bf16 out): the kernel's rows against the oracle's f32 accumulators over the kernel's own FC1 rows and
  R128c4 scales, within the north-star GEMM tolerance.
"""
import numpy as np
import pytest
import torch

from kern_amd import workload as wl

from tests._moe import fc1_debug_twin, gpu_raw_weights
from tests._util import assert_gemm_close, bf16_to_f32, to_np

pytestmark = pytest.mark.gpu

T, E, TOPK, START, LOCAL, H, I = 16384, 224, 16, 56, 56, 3584, 3072


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops as o
    o.lib()
    return o


def _sample_slots(S):
    pick = {0, S - 1}
    for x in range(1, 8):
        b = (S * x) >> 3
        pick.update({b - 1, b})
    return np.array(sorted(s for s in pick if 0 <= s < S), np.int64)


def _sub_tables(tabs, slots, remap):
    """Tables of the sampled slots alone: sub-slot j is slot slots[j], rows j*128 .. j*128 + valid, its expert
    renumbered by remap, its route_map rows copied."""
    n = len(slots)
    valid = tabs["cta_limit"][slots] - slots * 128
    sub = {
        "num_non_exiting": np.array([n], np.int32),
        "total_padded": np.array([n * 128], np.int32),
        "cta_batch": remap[tabs["cta_batch"][slots]].astype(np.int32),
        "cta_limit": (np.arange(n) * 128 + valid).astype(np.int32),
        "route_map": tabs["route_map"].reshape(-1, 128)[slots].reshape(-1).astype(np.int32),
    }
    return sub, valid


def test_k3_prefill_full_size(ops, oracle):
    print(f"[k3 full] T={T} E={E} top-{TOPK} local {START}+{LOCAL} H={H} I={I}", flush=True)
    u8, i32 = torch.uint8, torch.int32
    x = torch.from_numpy(wl.activations_bf16(905, T, H).view(np.int16)).cuda().view(torch.bfloat16)
    ids_np = wl.topk_ids(906, T, E, TOPK)
    ids = torch.from_numpy(ids_np).cuda()
    w1r, s1r = gpu_raw_weights(ops, torch, 907, LOCAL, 2 * I, H)
    w2r, s2r = gpu_raw_weights(ops, torch, 908, LOCAL, H, I)
    w1, s1 = ops.repack_weights(w1r, s1r, gated=True)
    w2, s2 = ops.repack_weights(w2r, s2r, gated=False)
    del w1r, s1r, w2r, s2r
    alpha = torch.full((LOCAL,), 4.0, dtype=torch.float32, device="cuda")
    beta = torch.full((LOCAL,), 25.0, dtype=torch.float32, device="cuda")
    ctas = ops.ctas_bound(T, TOPK, LOCAL)
    rows = ctas * 128
    dev = {n: torch.full((sz,), -7, dtype=i32, device="cuda") for n, sz in
           [("counts", 2 * LOCAL), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("tp", 1),
            ("route_map", rows), ("exp2perm", T * TOPK)]}
    q = torch.empty((T, H), dtype=u8, device="cuda")
    qs = torch.empty((T, H // 32), dtype=u8, device="cuda")
    c1 = torch.zeros((rows, I), dtype=u8, device="cuda")
    sf1 = torch.zeros(ops.r128c4_bytes(rows, I // 32), dtype=u8, device="cuda")
    c2 = torch.zeros((rows, H), dtype=torch.bfloat16, device="cuda")

    ops.moe_quant(x, q, qs, T, K=H)
    ops.moe_routing(ids, dev["counts"], dev["cta_batch"], dev["cta_limit"], dev["nne"], dev["tp"],
                    dev["route_map"], dev["exp2perm"], tokens=T, topk=TOPK, local_start=START, local_experts=LOCAL)

    def fc1(c_, sf_, dbg_):
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w1, s1, q, qs, c_, sf_, dev["route_map"], alpha, beta, dev["nne"],
                                            dev["tp"], dev["cta_batch"], dev["cta_limit"], m=2 * I, k=H, ctas=ctas,
                                            dbg=dbg_)

    fc1(c1, sf1, None)  # the production launch (no debug output)
    ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, dev["nne"], dev["tp"], dev["cta_batch"],
                                      dev["cta_limit"], m=H, k=I, ctas=ctas, sf_b_r128c4=True)
    torch.cuda.synchronize()

    # routing, bit for bit
    ref = oracle.routing(ids_np, START, LOCAL, ctas_cap=ctas)
    S = int(ref["num_non_exiting"][0])
    tabs = {"num_non_exiting": to_np(dev["nne"]), "cta_batch": to_np(dev["cta_batch"]),
            "cta_limit": to_np(dev["cta_limit"]), "route_map": to_np(dev["route_map"])}
    assert int(tabs["num_non_exiting"][0]) == S and int(to_np(dev["tp"])[0]) == S * 128
    np.testing.assert_array_equal(to_np(dev["counts"]), ref["counts"])
    for n in ("cta_batch", "cta_limit"):
        np.testing.assert_array_equal(tabs[n][:S], ref[n][:S], err_msg=n)
    np.testing.assert_array_equal(tabs["route_map"][:S * 128], ref["route_map"][:S * 128])
    np.testing.assert_array_equal(to_np(dev["exp2perm"]), ref["exp2perm"].reshape(-1))
    assert S >= 500 and int(np.sum(tabs["cta_limit"][:S] - np.arange(S) * 128)) == int(np.sum(ref["counts"][:LOCAL]))

    slots = _sample_slots(S)
    used = np.unique(tabs["cta_batch"][slots])
    remap = np.full(LOCAL, -1, np.int32)
    remap[used] = np.arange(used.size, dtype=np.int32)
    sub, valid = _sub_tables(tabs, slots, remap)
    idx = torch.from_numpy(used).cuda()
    a1, sa1 = to_np(w1.index_select(0, idx)), to_np(s1.index_select(0, idx))
    a2, sa2 = to_np(w2.index_select(0, idx)), to_np(s2.index_select(0, idx))
    n = len(slots)
    live = np.arange(n * 128) % 128 < np.repeat(valid, 128)
    gpu_rows = torch.from_numpy((slots[:, None] * 128 + np.arange(128)[None, :]).reshape(-1)).cuda()

    # FC1 on the sampled slots: the debug twin's values against the oracle, the production codes against the
    # oracle quantizer on them
    dbg = fc1_debug_twin(torch, fc1, c1, sf1, "k3 full: fc1")
    g = to_np(dbg.index_select(0, gpu_rows))  # [n*128, 3, I]: gate acc, up acc, SiTU
    del dbg
    torch.cuda.empty_cache()
    _, _, rdbg = oracle.fc1(a1, sa1, to_np(q), to_np(qs), sub, to_np(alpha)[used], to_np(beta)[used], 2 * I, H,
                            n * 128)
    assert_gemm_close(g[live, 0], rdbg[live, 0], "k3 full: fc1 gate acc")
    assert_gemm_close(g[live, 1], rdbg[live, 1], "k3 full: fc1 up acc")
    gg, uu = g[live, 0].astype(np.float64), g[live, 1].astype(np.float64)
    with np.errstate(over="ignore"):
        h_ref = 4.0 * np.tanh(gg / 4.0) / (1.0 + np.exp(-gg)) * 25.0 * np.tanh(uu / 25.0)
    np.testing.assert_allclose(g[live, 2], h_ref, rtol=2e-5, atol=1e-6, err_msg="k3 full: fc1 situ")
    qref, sref = oracle.quant_blocks(g[live, 2])
    gc = to_np(c1.index_select(0, gpu_rows))
    np.testing.assert_array_equal(gc[live], qref, err_msg="k3 full: fc1 codes")
    sf1_h = to_np(sf1)
    kb, kb4 = I // 32, -(-(I // 32) // 4)
    pr = (slots[:, None] * 128 + np.arange(128)[None, :]).reshape(-1)[live]
    b = np.arange(kb)[None, :]
    offs = 512 * ((pr[:, None] // 128) * kb4 + b // 4) + (pr[:, None] % 32) * 16 + ((pr[:, None] % 128) // 32) * 4 + b % 4
    np.testing.assert_array_equal(sf1_h[offs], sref, err_msg="k3 full: fc1 sf_c")
    print(f"[k3 full] {S} slots; fc1 checked on slots {slots.tolist()} ({int(live.sum())} rows)", flush=True)

    # FC2 on the sampled slots, from the kernel's own FC1 rows and scales (each slot's 128-row R128c4 block)
    blk = np.concatenate([sf1_h[512 * kb4 * s: 512 * kb4 * (s + 1)] for s in slots])
    _, acc = oracle.fc2(a2, sa2, gc, blk, True, sub, H, I)
    g2 = bf16_to_f32(to_np(c2.index_select(0, gpu_rows).view(torch.int16)).view(np.uint16))
    assert_gemm_close(g2[live], acc[live], "k3 full: fc2")
