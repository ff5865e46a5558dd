"""Program runtime (kern_rt_*) on the GPU: a whole MoE-layer manifest loaded from JSON (module by file
and sha256, buffers at their var maxima), weights repacked by its derive program, and the layer run by
program name, launch by launch and as a hipGraph, gives bit-identical outputs to the direct op calls;
graphs are keyed by var values and replay new inputs; misuse is reported as the reference's Api errors."""
import numpy as np
import pytest
import torch

from kern_amd import manifest as mf
from kern_amd import workload as wl

pytestmark = pytest.mark.gpu

H, I, E, K, TMAX = 1024, 512, 8, 2, 64


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


@pytest.fixture(scope="module")
def weights():
    w13, s13 = wl.mxfp4_weights(173, E, 2 * I, H, 119, 124)
    w2, s2 = wl.mxfp4_weights(174, E, H, I, 119, 124)
    gamma = wl.f32_to_bf16_bits(np.linspace(0.5, 1.5, H).astype(np.float32))
    alpha = (np.full(E, 4.0, np.float32) + np.arange(E, dtype=np.float32) * 0.01)
    beta = np.full(E, 25.0, np.float32)
    return dict(w13_raw=w13, s13_raw=s13, w2_raw=w2, s2_raw=s2, gamma=gamma, alpha=alpha, beta=beta)


def _inputs(seed, T):
    x = wl.activations_bf16(seed, T, H)
    ids = wl.topk_ids(seed + 1, T, E, K)
    tw = (np.random.default_rng(seed).random((T, K)) + 0.1).astype(np.float32)
    return x, ids, tw


def _direct(ops, weights, x, ids, tw):
    """The same layer through the direct op entry points."""
    T = x.shape[0]
    w13, s13 = ops.repack_weights(_dev(weights["w13_raw"]), _dev(weights["s13_raw"]), gated=True)
    w2, s2 = ops.repack_weights(_dev(weights["w2_raw"]), _dev(weights["s2_raw"]))
    q = torch.zeros((T, H), dtype=torch.uint8, device="cuda")
    qs = torch.zeros((T, H // 32), dtype=torch.uint8, device="cuda")
    ctas = ops.ctas_bound(T, K, E)
    tabs = [torch.zeros(n, dtype=torch.int32, device="cuda") for n in (2 * E, ctas, ctas, 1, 1, ctas * 128, T * K)]
    counts, cb, cl, nne, tp, rmap, e2p = tabs
    c1 = torch.zeros((ctas * 128, I), dtype=torch.uint8, device="cuda")
    sf1 = torch.zeros(ops.r128c4_bytes(ctas * 128, I // 32), dtype=torch.uint8, device="cuda")
    c2 = torch.zeros((ctas * 128, H), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_quant(_dev(x), q, qs, T, K=H)
    ops.moe_routing(_dev(ids), counts, cb, cl, nne, tp, rmap, e2p, tokens=T, topk=K, local_start=0, local_experts=E)
    ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w13, s13, q, qs, c1, sf1, rmap, _dev(weights["alpha"]), _dev(weights["beta"]),
                                        nne, tp, cb, cl, m=2 * I, k=H, ctas=ctas)
    ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, nne, tp, cb, cl, m=H, k=I, ctas=ctas)
    ops.moe_finalize_rms(c2, e2p, _dev(tw), _dev(weights["gamma"]), y, T, H=H, topk=K, eps=1e-6)
    torch.cuda.synchronize()
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def rt(ops, weights):
    r = ops.Runtime(mf.moe_layer_manifest(H, I, E, K, TMAX, ops.code_object_sha256()))
    for name, data in weights.items():
        r.load_weight(name, data)
    r.derive()
    yield r
    r.close()


def _run(rt, program, x, ids, tw):
    T = x.shape[0]
    rt.write_input("x", x)
    rt.write_input("topk_ids", ids)
    rt.write_input("topk_weight", tw)
    rt.run(program, {"tokens": T})
    return rt.read_output("y", T * H * 2).view(np.uint16).reshape(T, H)


@pytest.mark.parametrize("T", [64, 37, 1])
def test_layer_program_matches_direct_ops(ops, weights, rt, T):
    print(f"[runtime] moe_layer T={T}", flush=True)
    x, ids, tw = _inputs(300 + T, T)
    got = _run(rt, "moe_layer", x, ids, tw)
    np.testing.assert_array_equal(got, _direct(ops, weights, x, ids, tw))


def test_graph_program_replays_new_inputs(ops, weights, rt):
    print("[runtime] moe_layer_graph", flush=True)
    for seed in (401, 402, 403):  # captured at tokens=48 on the first run, replayed after
        x, ids, tw = _inputs(seed, 48)
        np.testing.assert_array_equal(_run(rt, "moe_layer_graph", x, ids, tw), _direct(ops, weights, x, ids, tw))
    x, ids, tw = _inputs(404, 20)  # another var value: another graph
    np.testing.assert_array_equal(_run(rt, "moe_layer_graph", x, ids, tw), _direct(ops, weights, x, ids, tw))
    rt.run_captured("moe_layer_graph", {"tokens": 20})
    assert rt.time_captured("moe_layer_graph", {"tokens": 48}, iters=5) > 0
    with pytest.raises(ops.KernError) as e:
        rt.run_captured("moe_layer_graph", {"tokens": 30})
    assert e.value.code == 4 and "captured at" in str(e.value)


def test_programs_at_chunked_routing_sizes(ops, weights):
    """From mf.ROUTE_CHUNKED_MIN expanded ids on, moe_routing's manifest launches are the chunked count / scan /
    rank, whose grid is a clamp of the token count: the runtime picks them by `when` and sizes them per call,
    launch by launch and inside graphs replayed with new inputs, and the layer stays bit-identical to the
    direct op calls (which choose the same launches in the C ABI)."""
    first = mf.ROUTE_CHUNKED_MIN // K
    r = ops.Runtime(mf.moe_layer_manifest(H, I, E, K, first + 320, ops.code_object_sha256()))
    try:
        for name, data in weights.items():
            r.load_weight(name, data)
        r.derive()
        for T, seed, program in [(first - 1, 501, "moe_layer"), (first, 503, "moe_layer"),
                                 (first + 301, 505, "moe_layer"), (first + 301, 507, "moe_layer_graph"),
                                 (first + 301, 509, "moe_layer_graph"), (first, 511, "moe_layer_graph")]:
            print(f"[runtime] {program} T={T} (chunked routing from T={first})", flush=True)
            x, ids, tw = _inputs(seed, T)
            np.testing.assert_array_equal(_run(r, program, x, ids, tw), _direct(ops, weights, x, ids, tw),
                                          err_msg=f"{program} T={T}")
    finally:
        r.close()


def test_misuse(ops, rt):
    for call, code in [
        (lambda: rt.run("moe_layer", {"tokens": TMAX + 1}), 4),     # above the var's max
        (lambda: rt.run("nope", {"tokens": 1}), 4),                 # unknown program
        (lambda: rt.run("derive_weights"), 4),                      # derive programs run only through derive
        (lambda: rt.read_output("q", 16), 4),                       # a workspace is not an output
        (lambda: rt.write_input("y", b"\0" * 16), 4),               # an output is not an input
        (lambda: rt.load_weight("w13_raw", b"\0"), 4),              # sources are freed after derive
        (lambda: rt.derive(), 4),                                   # derive runs once
        (lambda: rt.run("moe_layer", {}), 7),                       # a call needs `tokens`: call context
    ]:
        with pytest.raises(ops.KernError) as e:
            call()
        assert e.value.code == code, str(e.value)


def test_programs_need_derive(ops, weights):
    r = ops.Runtime(mf.moe_layer_manifest(H, I, E, K, 8, ops.code_object_sha256()))
    try:
        with pytest.raises(ops.KernError) as e:
            r.run("moe_layer", {"tokens": 1})
        assert e.value.code == 4 and "derive" in str(e.value)
        ptr, n = r.buffer("c2")
        assert ptr and n == (E + 1) * 128 * H * 2
    finally:
        r.close()
