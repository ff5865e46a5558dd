"""Config 5 (the quantized layer stack) on the GPU, through the C ABI, against the CPU oracle.

* The dense bf16-output GEMM (kern_mxfp4_gemm_bf16) at the stack's shapes: QKV [M, 7168] x [9216, 7168] and
  O [M, 8192] x [7168, 8192] at M = 64 and 2048, every row: the f32 accumulators within the north-star
  tolerance of the oracle over exactly dequantized raw (un-repacked) weights, and the bf16 output the RNE
  rounding of the kernel's own accumulators, bit for bit.
* Layers of the stack (quantize -> QKV -> O -> quantize + routing -> MoE of 256 experts, top-8, H = 7168,
  I = 2048 -> RMS finalize), chained as the bench's step chains them, at M = 1 (decode GEMV for QKV and O;
  two layers), M = 64 (quantizer + dense walk; two layers) and M = 2048 (quantizer + tiled GEMM, 16,384
  routed rows; one layer), captured once through the library's own hipGraph C ABI (kern_graph_begin / end)
  and replayed: every replay equals the eager run bit for bit, and every stage of every layer is checked
  against the oracle on the GPU's own inputs to that stage (quantizers and routing tables bit-exact, GEMV /
  GEMM / FC1 / FC2 within tolerance, the production FC1's codes and scales bit-exact on the kernel's own
  SiTU values, the finalize within one bf16 ulp).
"""
import numpy as np
import pytest

from kern_amd import workload as wl
from tests import _moe
from tests._util import assert_gemm_close, bf16_to_f32, to_dev, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H, I, E, TOPK, QKV, OIN = 7168, 2048, 256, 8, 9216, 8192


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    return ops


# kern_mxfp4_gemm_bf16 takes the persistent walk (kern_mx_gemm_bf16_s{k/1024}) at M <= 64 with k = 1024 *
# {1, 2, 4, 7, 8} (config 5's M = 64), else the tiled GEMM (config 5's M = 2048). The cases reach every
# persistent instance with ragged token groups (M = 1, 17, 33, 50), half-group shares of 1, 2, 3 and 9
# with a ragged last workgroup (m = 4352: 544 half groups in shares of 3), and the tiled side of both
# bounds (M = 65; k = 3072).
@pytest.mark.parametrize("M,m,k", [(64, QKV, H), (64, H, OIN), (2048, QKV, H), (2048, H, OIN),
                                   (17, 256, 1024), (33, 4352, 2048), (50, 2304, 4096), (1, 512, 8192),
                                   (64, 18432, 7168), (65, 2304, 4096), (40, 768, 3072)])
def test_gemm_bf16_config5_shapes(ops, oracle, M, m, k):
    print(f"[gemm bf16] M={M} m={m} k={k}", flush=True)
    w_raw, s_raw = _moe.gpu_raw_weights(ops, torch, 700 + m + k, 1, m, k, 119, 6)
    wp, sp = ops.repack_weights(w_raw, s_raw)
    x = wl.activations_bf16(701 + M, M, k, outlier_frac=0.01)
    q, qs = ops.quantize_mxfp8(to_dev(x))
    # the production launch (no debug output), then its debug twin: bit-identical outputs
    c = torch.empty((M, m), dtype=torch.bfloat16, device="cuda")
    ops.mxfp4_gemm_bf16(wp[0], sp[0], q, qs, c, M=M, m=m, k=k)
    c_d = torch.empty((M, m), dtype=torch.bfloat16, device="cuda")
    dbg = torch.empty((M, m), dtype=torch.float32, device="cuda")
    ops.mxfp4_gemm_bf16(wp[0], sp[0], q, qs, c_d, M=M, m=m, k=k, dbg=dbg)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), c_d.view(torch.int16)), "bf16 output with and without the debug output differ"
    acc = to_np(dbg)
    np.testing.assert_array_equal(to_np(c), wl.f32_to_bf16_bits(acc))
    W = oracle.deq_fp4(to_np(w_raw[0]), to_np(s_raw[0]), m, k)
    X = oracle.deq_fp8(to_np(q), to_np(qs), M, k)
    assert_gemm_close(acc, oracle.gemm_f32(X, W), f"gemm bf16 M={M} m={m} k={k}")


# Layers chained as bench.py's config-5 step runs them: layer l's QKV input is layer l-1's finalize output;
# the O input stands in for attention; O's output goes through moe_quant_routing (the quantizer and the
# routing tables in one call) into production FC1 (no debug output), FC2 and the RMS finalize. M = 1 takes
# the decode GEMV for QKV and O, M = 64 the dense walk, M = 2048 the tiled GEMM and a MoE of 16,384 routed
# rows (64 per expert: every slot on the LDS ring with its second wave group idle).
@pytest.mark.parametrize("M,NL", [(1, 2), (64, 2), (2048, 1)])
def test_config5_layers_graph(ops, oracle, M, NL):
    print(f"[config 5] M={M}, {NL} layer(s): weights", flush=True)
    u8, i32, bf16 = torch.uint8, torch.int32, torch.bfloat16
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        layers = []
        for l in range(NL):
            L = {}
            L["wq_raw"], L["sq_raw"] = _moe.gpu_raw_weights(ops, torch, 600 + 10 * l, 1, QKV, H)
            L["wo_raw"], L["so_raw"] = _moe.gpu_raw_weights(ops, torch, 601 + 10 * l, 1, H, OIN)
            L["wq"], L["sq"] = (t[0] for t in ops.repack_weights(L["wq_raw"], L["sq_raw"]))
            L["wo"], L["so"] = (t[0] for t in ops.repack_weights(L["wo_raw"], L["so_raw"]))
            r13, s13r = _moe.gpu_raw_weights(ops, torch, 602 + 10 * l, E, 2 * I, H)
            L["w13"], L["s13"] = ops.repack_weights(r13, s13r, gated=True)
            del r13, s13r
            r2, s2r = _moe.gpu_raw_weights(ops, torch, 603 + 10 * l, E, H, I)
            L["w2"], L["s2"] = ops.repack_weights(r2, s2r)
            del r2, s2r
            L["ids_np"] = wl.topk_ids(612 + M + 10 * l, M, E, TOPK)
            L["ids"] = to_dev(L["ids_np"])
            layers.append(L)
        x0 = to_dev(wl.activations_bf16(610 + M, M, H))
        attn = to_dev(wl.activations_bf16(611 + M, M, OIN))
        tw = to_dev(wl.topk_weights(613 + M, M, TOPK))
        gamma = to_dev(wl.activations_bf16(614, 1, H).reshape(-1))
        alpha_np = np.full(E, 4.0, np.float32) + np.arange(E, dtype=np.float32) * 0.01
        beta_np = np.full(E, 25.0, np.float32)
        alpha, beta = to_dev(alpha_np), to_dev(beta_np)
        ctas = ops.ctas_bound(M, TOPK, E)
        rows = ctas * 128

        def buffers():
            out = []
            for _ in range(NL):
                b = {"qkv": torch.empty((M, QKV), dtype=bf16, device="cuda"),
                     "o": torch.empty((M, H), dtype=bf16, device="cuda"),
                     "xq": torch.empty((M, H), dtype=u8, device="cuda"),
                     "xqs": torch.empty((M, H // 32), dtype=u8, device="cuda"),
                     "aq": torch.empty((M, OIN), dtype=u8, device="cuda"),
                     "aqs": torch.empty((M, OIN // 32), dtype=u8, device="cuda"),
                     "oq": torch.empty((M, H), dtype=u8, device="cuda"),
                     "oqs": torch.empty((M, H // 32), dtype=u8, device="cuda"),
                     "c1": torch.empty((rows, I), dtype=u8, device="cuda"),
                     "sf1": torch.empty(ops.r128c4_bytes(rows, I // 32), dtype=u8, device="cuda"),
                     "c2": torch.empty((rows, H), dtype=bf16, device="cuda"),
                     "y": torch.empty((M, H), dtype=bf16, device="cuda")}
                for n, sz in [("counts", 2 * E), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("tp", 1),
                              ("route_map", rows), ("exp2perm", M * TOPK)]:
                    b[n] = torch.empty(sz, dtype=i32, device="cuda")
                out.append(b)
            return out

        def fc1(L, b, c1, sf1, dbg=None):
            ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(L["w13"], L["s13"], b["oq"], b["oqs"], c1, sf1, b["route_map"], alpha,
                                                beta, b["nne"], b["tp"], b["cta_batch"], b["cta_limit"], m=2 * I, k=H,
                                                ctas=ctas, dbg=dbg)

        def step(bs):
            x = x0
            for L, b in zip(layers, bs):
                if M <= 16:  # decode: W4A16 GEMV straight from bf16
                    ops.mxfp4_gemv_bf16(x, L["wq"], L["sq"], b["qkv"], M, N=QKV, K=H)
                    ops.mxfp4_gemv_bf16(attn, L["wo"], L["so"], b["o"], M, N=H, K=OIN)
                else:
                    ops.moe_quant(x, b["xq"], b["xqs"], M, K=H)
                    ops.mxfp4_gemm_bf16(L["wq"], L["sq"], b["xq"], b["xqs"], b["qkv"], M=M, m=QKV, k=H)
                    ops.moe_quant(attn, b["aq"], b["aqs"], M, K=OIN)
                    ops.mxfp4_gemm_bf16(L["wo"], L["so"], b["aq"], b["aqs"], b["o"], M=M, m=H, k=OIN)
                ops.moe_quant_routing(b["o"], b["oq"], b["oqs"], L["ids"], b["counts"], b["cta_batch"],
                                      b["cta_limit"], b["nne"], b["tp"], b["route_map"], b["exp2perm"], tokens=M,
                                      K=H, topk=TOPK, local_start=0, local_experts=E)
                fc1(L, b, b["c1"], b["sf1"])
                ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(L["w2"], L["s2"], b["c1"], b["sf1"], b["c2"], b["nne"], b["tp"],
                                                  b["cta_batch"], b["cta_limit"], m=H, k=I, ctas=ctas)
                ops.moe_finalize_rms(b["c2"], b["exp2perm"], tw, gamma, b["y"], M, H=H, topk=TOPK, eps=1e-6)
                x = b["y"]

        # rows the kernels never write (padding rows, slots past the live ones) stay zero in both runs
        keys = ["qkv", "o", "oq", "oqs", "c1", "sf1", "c2", "y", "counts", "cta_batch", "cta_limit", "nne",
                "route_map", "exp2perm"]
        eager, cap = buffers(), buffers()
        for b in eager:
            for n in keys:
                b[n].zero_()
        step(eager)
        torch.cuda.synchronize()
        print(f"[config 5] M={M}: capture and replay", flush=True)
        with ops.Graph() as g:
            step(cap)
        for r in range(3):
            for b in cap:
                for n in keys:
                    b[n].zero_()
            torch.cuda.synchronize()
            g.launch()
            torch.cuda.synchronize()
            for l, (bc, be) in enumerate(zip(cap, eager)):
                for n in keys:
                    assert torch.equal(bc[n].view(u8), be[n].view(u8)), f"replay {r}: layer {l}: {n}"
        g.close()
        del cap
        # the debug twin of each layer's production FC1, on that layer's own inputs
        dbgs = [_moe.fc1_debug_twin(torch, lambda c_, s_, d_, L=L, b=b: fc1(L, b, c_, s_, d_), b["c1"], b["sf1"],
                                    f"config 5 M={M} layer {l}") for l, (L, b) in enumerate(zip(layers, eager))]

    an = to_np(attn)
    x_in = to_np(x0)
    for l, (L, b) in enumerate(zip(layers, eager)):
        what = f"config 5 M={M} layer {l}"
        print(f"[config 5] M={M}: layer {l} against the oracle", flush=True)
        if M <= 16:
            _, yq = oracle.gemv_w4a16(x_in, to_np(L["wq_raw"][0]), to_np(L["sq_raw"][0]))
            _, yo = oracle.gemv_w4a16(an, to_np(L["wo_raw"][0]), to_np(L["so_raw"][0]))
        else:
            for qn, sn, src in [("xq", "xqs", x_in), ("aq", "aqs", an)]:
                q_ref, s_ref = oracle.quant_mxfp8(src)
                np.testing.assert_array_equal(to_np(b[qn]), q_ref)
                np.testing.assert_array_equal(to_np(b[sn]), s_ref)
            yq = oracle.gemm_f32(oracle.deq_fp8(to_np(b["xq"]), to_np(b["xqs"]), M, H),
                                 oracle.deq_fp4(to_np(L["wq_raw"][0]), to_np(L["sq_raw"][0]), QKV, H))
            yo = oracle.gemm_f32(oracle.deq_fp8(to_np(b["aq"]), to_np(b["aqs"]), M, OIN),
                                 oracle.deq_fp4(to_np(L["wo_raw"][0]), to_np(L["so_raw"][0]), H, OIN))
        assert_gemm_close(bf16_to_f32(to_np(b["qkv"])), yq, f"{what}: qkv")
        assert_gemm_close(bf16_to_f32(to_np(b["o"])), yo, f"{what}: o")
        del yq, yo
        q_ref, s_ref = oracle.quant_mxfp8(to_np(b["o"]))
        np.testing.assert_array_equal(to_np(b["oq"]), q_ref)
        np.testing.assert_array_equal(to_np(b["oqs"]), s_ref)
        tabs = oracle.routing(L["ids_np"], 0, E, ctas_cap=ctas)
        S = int(tabs["num_non_exiting"][0])
        assert int(to_np(b["nne"])[0]) == S and int(to_np(b["tp"])[0]) == S * 128
        np.testing.assert_array_equal(to_np(b["counts"]), tabs["counts"])
        np.testing.assert_array_equal(to_np(b["cta_batch"])[:S], tabs["cta_batch"][:S])
        np.testing.assert_array_equal(to_np(b["cta_limit"])[:S], tabs["cta_limit"][:S])
        np.testing.assert_array_equal(to_np(b["route_map"])[: S * 128], tabs["route_map"][: S * 128])
        np.testing.assert_array_equal(to_np(b["exp2perm"]), tabs["exp2perm"].reshape(-1))
        _moe.check_fc1(torch, oracle, L["w13"], L["s13"], b["oq"], b["oqs"], tabs, alpha_np, beta_np, 2 * I, H,
                       b["c1"], b["sf1"], dbgs[l], what)
        _moe.check_fc2(torch, oracle, L["w2"], L["s2"], b["c1"], b["sf1"], tabs, H, I, b["c2"], what)
        _moe.check_finalize(oracle, b["c2"], b["exp2perm"], tw, gamma, b["y"], M, H, TOPK, 1e-6, what)
        x_in = to_np(b["y"])
