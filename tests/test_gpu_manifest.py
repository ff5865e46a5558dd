"""Manifest-op layer on the GPU: the path's ops, run from their manifest JSON through kern_op_create /
kern_op_launch with impl pointed at kern_mx, give bit-identical results to the direct C-ABI entry
points (same kernels, same arguments); create-time checks against the code object reject mismatches."""
import numpy as np
import pytest
import torch

from kern_amd import manifest as mf
from kern_amd import workload as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops as o
    o.lib()
    return o


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def _r128c4_bytes(rows, blocks):
    return (rows // 128) * 512 * -(-blocks // 4)


def test_moe_layer_through_manifest_ops(ops):
    T, E, k, H, I = 64, 8, 2, 1024, 512
    print(f"[manifest] MoE layer T={T} E={E} k={k} H={H} I={I}", flush=True)
    man = {n: ops.ManifestOp(o) for n, o in mf.moe_ops(H, I, E, k).items()}
    v = {"tokens": T}
    x = _dev(wl.activations_bf16(71, T, H))
    ids = _dev(wl.topk_ids(72, T, E, k))
    w13, s13 = (_dev(a) for a in wl.mxfp4_weights(73, E, 2 * I, H, 119, 124))
    w2, s2 = (_dev(a) for a in wl.mxfp4_weights(74, E, H, I, 119, 124))
    tw = torch.rand((T, k), device="cuda") + 0.1
    gamma = _dev(wl.f32_to_bf16_bits(np.linspace(0.5, 1.5, H).astype(np.float32)))
    alpha = torch.full((E,), 4.0, device="cuda")
    beta = torch.full((E,), 25.0, device="cuda")
    ctas = ops.ctas_bound(T, k, E)
    rows = ctas * 128
    u8, i32 = torch.uint8, torch.int32

    def run(manifest: bool):
        out = {"q": torch.zeros((T, H), dtype=u8, device="cuda"), "qs": torch.zeros((T, H // 32), dtype=u8, device="cuda"),
               "w13": torch.zeros_like(w13), "s13": torch.zeros_like(s13), "w2": torch.zeros_like(w2),
               "s2": torch.zeros_like(s2)}
        tabs = [torch.full((n,), -7, dtype=i32, device="cuda") for n in (2 * E, ctas, ctas, 1, 1, rows, T * k)]
        c1 = torch.zeros((rows, I), dtype=u8, device="cuda")
        sf1 = torch.zeros(_r128c4_bytes(rows, I // 32), dtype=u8, device="cuda")
        c2 = torch.zeros((rows, H), dtype=torch.bfloat16, device="cuda")
        fin = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
        counts, cb, cl, nne, tp, rmap, e2p = tabs
        if manifest:
            man["moe_quant"](x, out["q"], out["qs"], T, vars=v)
            man["k3_moe_w_shuffle"](w13, out["w13"], 2 * I, H // 2, 1, vars=v)
            man["k3_moe_sf_shuffle"](s13, out["s13"], 2 * I, H // 32, 1, vars=v)
            man["k3_moe_w_shuffle"](w2, out["w2"], H, I // 2, 0, vars=v)
            man["k3_moe_sf_shuffle"](s2, out["s2"], H, I // 32, 0, vars=v)
            man["moe_routing"](ids, counts, cb, cl, nne, tp, rmap, e2p, vars=v)
            man["moe_fc1"](out["w13"], out["s13"], out["q"], out["qs"], c1, sf1, rmap, alpha, beta, nne, tp, cb, cl,
                           vars=v)
            man["moe_fc2"](out["w2"], out["s2"], c1, sf1, c2, nne, tp, cb, cl, vars=v)
            man["moe_finalize_rms"](c2, e2p, tw, gamma, fin, T, vars=v)
        else:
            ops.moe_quant(x, out["q"], out["qs"], T, K=H)
            ops.k3_moe_w_shuffle(w13, out["w13"], 2 * I, H // 2, True, experts=E)
            ops.k3_moe_sf_shuffle(s13, out["s13"], 2 * I, H // 32, True, experts=E)
            ops.k3_moe_w_shuffle(w2, out["w2"], H, I // 2, False, experts=E)
            ops.k3_moe_sf_shuffle(s2, out["s2"], H, I // 32, False, experts=E)
            ops.moe_routing(ids, counts, cb, cl, nne, tp, rmap, e2p, tokens=T, topk=k, local_start=0, local_experts=E)
            ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(out["w13"], out["s13"], out["q"], out["qs"], c1, sf1, rmap, alpha, beta,
                                                nne, tp, cb, cl, m=2 * I, k=H, ctas=ctas)
            ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(out["w2"], out["s2"], c1, sf1, c2, nne, tp, cb, cl, m=H, k=I, ctas=ctas)
            ops.moe_finalize_rms(c2, e2p, tw, gamma, fin, T, H=H, topk=k, eps=1e-6)
        torch.cuda.synchronize()
        out.update({f"tab{i}": t for i, t in enumerate(tabs)})
        out.update({"c1": c1, "sf1": sf1, "c2": c2, "fin": fin})
        return out

    a, b = run(False), run(True)
    assert int(a["tab3"][0]) > 0
    for name in a:
        assert torch.equal(a[name].view(torch.uint8) if a[name].dtype == torch.bfloat16 else a[name],
                           b[name].view(torch.uint8) if b[name].dtype == torch.bfloat16 else b[name]), name


# moe_routing through its manifest op on both sides of the switch to the chunked launches (`when` on tokens):
# 16376 expanded ids (one workgroup), 16384 (count / scan / rank over 4 chunks) and a K3 rank's 262144 (64
# chunks, non-local experts); every table bit for bit against the oracle
@pytest.mark.parametrize("T,E,k,start,local", [(2047, 256, 8, 0, 256), (2048, 256, 8, 0, 256),
                                               (16384, 224, 16, 56, 56)])
def test_routing_op_on_both_paths(ops, T, E, k, start, local):
    from oracle import mxoracle as oracle
    print(f"[manifest] moe_routing T={T} E={E} k={k} local {start}+{local}", flush=True)
    op = ops.ManifestOp(mf.moe_routing(k, start, local))
    ids = wl.topk_ids(T * 3 + E, T, E, k)
    ctas = ops.ctas_bound(T, k, local)
    ref = oracle.routing(ids, start, local, ctas_cap=ctas)
    tabs = [torch.full((n,), -7, dtype=torch.int32, device="cuda")
            for n in (2 * local, ctas, ctas, 1, 1, ctas * 128, T * k)]
    op(_dev(ids), *tabs, vars={"tokens": T})
    torch.cuda.synchronize()
    counts, cb, cl, nne, tp, rmap, e2p = (t.cpu().numpy() for t in tabs)
    S = int(ref["num_non_exiting"][0])
    assert (int(nne[0]), int(tp[0])) == (S, S * 128)
    np.testing.assert_array_equal(counts, ref["counts"])
    np.testing.assert_array_equal(cb[:S], ref["cta_batch"][:S])
    np.testing.assert_array_equal(cl[:S], ref["cta_limit"][:S])
    np.testing.assert_array_equal(rmap[:S * 128], ref["route_map"][:S * 128])
    np.testing.assert_array_equal(e2p, ref["exp2perm"].reshape(-1))


def test_create_checks_against_code_object(ops):
    o = mf.moe_fc2(1024, 512, 8, 2)
    with pytest.raises(ops.KernError) as e:  # the manifest names another module
        ops.ManifestOp(o, module_name="other")
    assert e.value.code == 1
    bad = mf.moe_fc2(1024, 512, 8, 2)
    launch = bad["impl"]["launches"][0]
    launch["params"] = launch["params"][:-2] + ["i64"]  # drop one i32: the code object disagrees
    launch["args"] = launch["args"][:-2] + [{"i64": 0}]
    with pytest.raises(ops.KernError) as e:
        ops.ManifestOp(bad)
    assert e.value.code == 2 and "code object has" in str(e.value)
    bad = mf.moe_fc2(1024, 512, 8, 2)
    bad["impl"]["launches"][0]["entry"] = "kern_mx_no_such_entry"
    with pytest.raises(ops.KernError) as e:
        ops.ManifestOp(bad)
    assert e.value.code == 2


def test_launch_errors_carry_context(ops):
    m = ops.ManifestOp(mf.moe_quant(1024))
    x = torch.zeros((4, 1024), dtype=torch.bfloat16, device="cuda")
    q = torch.zeros((4, 1024), dtype=torch.uint8, device="cuda")
    s = torch.zeros((4, 32), dtype=torch.uint8, device="cuda")
    with pytest.raises(ops.KernError) as e:
        m(x, q, s, 4)  # no `tokens` bound
    assert e.value.code == 7 and "launch #0" in str(e.value)
    with pytest.raises(ops.KernError) as e:
        m(x, q, 0, 4, vars={"tokens": 4})  # a null buffer
    assert e.value.code == 4


def test_k3_fills_through_manifest_ops(ops):
    p_i = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    p_f = torch.zeros(230, dtype=torch.float32, device="cuda")
    p_b = torch.zeros(4, dtype=torch.bfloat16, device="cuda")
    ops.ManifestOp(mf.fill_i32(1))(p_i, 42)
    ops.ManifestOp(mf.fill_f32(224))(p_f, -0.75)
    ops.ManifestOp(mf.fill_bf16(1, 1.0))(p_b)
    torch.cuda.synchronize()
    assert p_i.tolist() == [42] + [-1] * 7
    assert (p_f[:224] == -0.75).all() and (p_f[224:] == 0).all()
    assert p_b.float().tolist() == [1.0, 0.0, 0.0, 0.0]


def test_mxfp8_kat_through_manifest_op(ops):
    from tests._util import mxfp8_kat
    c = mxfp8_kat(0)
    M, N, K = c["M"], c["N"], c["K"]
    out = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    op = ops.ManifestOp(mf.cublaslt_mxfp8_tn(N))
    op(*(_dev(c[x]) for x in ("a", "w")), out, *(_dev(c[x]) for x in ("a_sf", "w_sf")), M, N, K, vars={"tokens": M})
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), wl.f32_to_bf16_bits(c["want"]))


# The dense ops whose C-ABI entries choose a kernel by row count: their manifest ops (launches conditioned on
# `tokens` by `when`) against the C ABI, bit for bit, at row counts on either side of every switch.

@pytest.mark.parametrize("N,K,Ms", [(18432, 7168, [1, 3, 4, 16]), (7168, 8192, [9, 10]), (2048, 3584, [1, 2, 3, 7, 16]),
                                    (512, 1024, [1, 16])])
def test_gemv_op_takes_the_c_abi_kernels(ops, N, K, Ms):
    op = ops.ManifestOp(mf.mxfp4_gemv_bf16(N, K))
    w, sf = wl.mxfp4_weights(300 + K, 1, N, K, 122, 132)
    wp, sfp = ops.repack_weights(_dev(w[0]), _dev(sf[0]))
    for M in Ms:
        print(f"[manifest] mxfp4_gemv_bf16 N={N} K={K} M={M}", flush=True)
        x = _dev(wl.activations_bf16(310 + M, M, K))
        y0 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        y1 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        ops.mxfp4_gemv_bf16(x, wp, sfp, y0, M, N=N, K=K)
        op(x, wp, sfp, y1, vars={"tokens": M})
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), M


@pytest.mark.parametrize("N,K,Ms", [(9216, 7168, [17, 64, 65, 200]), (2048, 3584, [5, 130])])
def test_dense_gemm_op_takes_the_c_abi_kernels(ops, N, K, Ms):
    op = ops.ManifestOp(mf.mxfp4_gemm_bf16(N, K))
    w, sf = wl.mxfp4_weights(320 + K, 1, N, K, 122, 132)
    wp, sfp = ops.repack_weights(_dev(w[0]), _dev(sf[0]))
    for M in Ms:
        print(f"[manifest] mxfp4_gemm_bf16 N={N} K={K} M={M}", flush=True)
        x = _dev(wl.activations_bf16(330 + M, M, K))
        q = torch.zeros((M, K), dtype=torch.uint8, device="cuda")
        qs = torch.zeros((M, K // 32), dtype=torch.uint8, device="cuda")
        ops.moe_quant(x, q, qs, M, K=K)
        c0 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        c1 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        ops.mxfp4_gemm_bf16(wp, sfp, q, qs, c0, M=M, m=N, k=K)
        op(wp, sfp, q, qs, c1, vars={"tokens": M})
        torch.cuda.synchronize()
        assert torch.equal(c0.view(torch.int16), c1.view(torch.int16)), M


@pytest.mark.parametrize("K,k,E,Ts", [(7168, 8, 256, [1, 582, 583, 2048]), (512, 16, 64, [8160, 8161])])
def test_quant_routing_op_takes_the_c_abi_launches(ops, K, k, E, Ts):
    op = ops.ManifestOp(mf.moe_quant_routing(K, k, 0, E))
    for T in Ts:
        print(f"[manifest] moe_quant_routing K={K} top-{k} E={E} T={T}", flush=True)
        x = _dev(wl.activations_bf16(340 + T, T, K))
        ids = _dev(wl.topk_ids(341 + T, T, E, k))
        ctas = ops.ctas_bound(T, k, E)
        outs = []
        for path in ("c_abi", "manifest"):
            q = torch.full((T, K), 0x5A, dtype=torch.uint8, device="cuda")
            qs = torch.full((T, K // 32), 0x5A, dtype=torch.uint8, device="cuda")
            tabs = [torch.full((n,), -7, dtype=torch.int32, device="cuda")
                    for n in (2 * E, ctas, ctas, 1, 1, ctas * 128, T * k)]
            if path == "c_abi":
                ops.moe_quant_routing(x, q, qs, ids, *tabs, tokens=T, K=K, topk=k, local_start=0, local_experts=E)
            else:
                op(x, q, qs, ids, *tabs, vars={"tokens": T})
            torch.cuda.synchronize()
            outs.append([q, qs] + tabs)
        for a, b in zip(*outs):
            assert torch.equal(a, b), T


@pytest.mark.parametrize("N,K,M", [(2048, 7168, 4096), (512, 1024, 37)])
def test_e4m3_gemm_op_matches_the_c_abi(ops, N, K, M):
    """Config 3's prefill GEMM (per-tensor e4m3 out) as a manifest op, at its full shape and a ragged one."""
    print(f"[manifest] mxfp4_gemm_e4m3 N={N} K={K} M={M}", flush=True)
    op = ops.ManifestOp(mf.mxfp4_gemm_e4m3(N, K))
    w, sf = wl.mxfp4_weights(350 + K, 1, N, K, 122, 132)
    wp, sfp = ops.repack_weights(_dev(w[0]), _dev(sf[0]))
    x = _dev(wl.activations_bf16(351, M, K))
    q = torch.zeros((M, K), dtype=torch.uint8, device="cuda")
    qs = torch.zeros((M, K // 32), dtype=torch.uint8, device="cuda")
    ops.moe_quant(x, q, qs, M, K=K)
    ds = torch.tensor([0.05], dtype=torch.float32, device="cuda")
    c0 = torch.full((M, N), 0x5A, dtype=torch.uint8, device="cuda")
    c1 = torch.full((M, N), 0x5A, dtype=torch.uint8, device="cuda")
    ops.mxfp4_gemm_e4m3(wp, sfp, q, qs, c0, ds, M=M, m=N, k=K)
    op(wp, sfp, q, qs, c1, ds, vars={"tokens": M})
    torch.cuda.synchronize()
    assert torch.equal(c0, c1)
