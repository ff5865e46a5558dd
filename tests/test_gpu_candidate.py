"""One MoE layer of the reference's own K3 manifest, run on gfx950 after splicing in this build's candidate.

The manifest is tests/golden/k3_moe_layer_manifest.json (cut from crates/kern-manifest/tests/fixtures/k3/
head.json: the layer's prefill calls l1.moe_quant .. l1.finalize, its derive repacks and its load fills, with
the reference's buffers at their K3 sizes), spliced with kernel_index/k3_moe_candidate.json. The program
runtime loads it, takes the raw expert weights by buffer name, runs `derive` and the `load` once-program,
then `prefill` at two token counts; the output equals, bit for bit, the same ops called directly through
the C ABI on the same inputs. time_range (harness.rs:209-250) times the prefill calls one by one."""
import json
import os

import numpy as np
import pytest

from kern_amd import workload as wl
from tests._util import to_dev, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
H, I, E, K = 3584, 3072, 224, 16


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    return ops


def test_spliced_k3_layer_runs(ops):
    with open(os.path.join(ROOT, "tests", "golden", "k3_moe_layer_manifest.json")) as f:
        m = json.load(f)
    with open(os.path.join(ROOT, "kernel_index", "k3_moe_candidate.json")) as f:
        cand = json.load(f)
    spliced = ops.splice(m, cand)
    print("[k3 candidate] loading the spliced layer", flush=True)
    rt = ops.Runtime(spliced, os.path.dirname(ops.HSACO_PATH))
    rng = np.random.default_rng(11)
    raw = {"layers.1.moe.w13.raw": rng.integers(0, 256, E * 2 * I * H // 2, dtype=np.uint8),
           "layers.1.moe.w13_sf.raw": rng.integers(119, 125, E * 2 * I * H // 32, dtype=np.uint8),
           "layers.1.moe.w2.raw": rng.integers(0, 256, E * H * I // 2, dtype=np.uint8),
           "layers.1.moe.w2_sf.raw": rng.integers(118, 127, E * H * I // 32, dtype=np.uint8)}
    gamma = wl.f32_to_bf16_bits((rng.random(H) + 0.5).astype(np.float32))
    for name, a in raw.items():
        rt.load_weight(name, a)
    rt.load_weight("layers.1.gamma_lat", gamma)
    rt.derive()
    rt.run("load")

    # the same weights through the direct C-ABI ops
    w13, s13 = ops.repack_weights(to_dev(raw["layers.1.moe.w13.raw"]).view(E, 2 * I, H // 2),
                                  to_dev(raw["layers.1.moe.w13_sf.raw"]).view(E, 2 * I, H // 32), gated=True)
    w2, s2 = ops.repack_weights(to_dev(raw["layers.1.moe.w2.raw"]).view(E, H, I // 2),
                                to_dev(raw["layers.1.moe.w2_sf.raw"]).view(E, H, I // 32))
    del raw
    alpha = torch.full((E,), 4.0, dtype=torch.float32, device="cuda")
    beta = torch.full((E,), 25.0, dtype=torch.float32, device="cuda")
    gd = to_dev(gamma)

    for T in (300, 4):
        print(f"[k3 candidate] prefill at tokens={T}", flush=True)
        x = wl.activations_bf16(900 + T, T, H)
        ids = wl.topk_ids(901 + T, T, E, K)
        tw = wl.topk_weights(902 + T, T, K)
        rt.write_buffer("latent", x)
        rt.write_buffer("topk_idx", ids)
        rt.write_buffer("topk_weight", tw)
        rt.run("prefill", {"tokens": T})
        got = rt.read_buffer("routed_latent_norm", T * H * 2).view(np.uint16).reshape(T, H)

        ctas = ops.ctas_bound(T, K, E)
        rows = ctas * 128
        i32, u8 = torch.int32, torch.uint8
        tab = {n: torch.zeros(sz, dtype=i32, device="cuda") for n, sz in
               [("counts", 2 * E), ("cb", ctas), ("cl", ctas), ("nne", 1), ("tp", 1), ("rm", rows), ("e2p", T * K)]}
        q, qs = ops.quantize_mxfp8(to_dev(x))
        c1 = torch.zeros((rows, I), dtype=u8, device="cuda")
        sf1 = torch.zeros(ops.r128c4_bytes(rows, I // 32), dtype=u8, device="cuda")
        c2 = torch.zeros((rows, H), dtype=torch.bfloat16, device="cuda")
        y = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
        twd = to_dev(tw)
        ops.moe_routing(to_dev(ids), tab["counts"], tab["cb"], tab["cl"], tab["nne"], tab["tp"], tab["rm"], tab["e2p"],
                        tokens=T, topk=K, local_start=0, local_experts=E)
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w13, s13, q, qs, c1, sf1, tab["rm"], alpha, beta, tab["nne"], tab["tp"],
                                            tab["cb"], tab["cl"], m=2 * I, k=H, ctas=ctas)
        ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, tab["nne"], tab["tp"], tab["cb"], tab["cl"], m=H, k=I,
                                          ctas=ctas)
        ops.moe_finalize_rms(c2, tab["e2p"], twd, gd, y, T, H=H, topk=K, eps=1e-6)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, to_np(y))
        assert np.isfinite(wl.bf16_bits_to_f32(got)).all()

    # per-call times of the prefill program (eager, event-bracketed, minimum over runs), and a sub-range
    ms = rt.time_range("prefill", 0, 5, {"tokens": 300}, iters=3)
    print("[k3 candidate] time_range prefill (ms):", [round(t, 4) for t in ms], flush=True)
    assert len(ms) == 5 and all(t > 0 for t in ms)
    assert len(rt.time_range("prefill", 2, 4, {"tokens": 300}, iters=2)) == 2
    rt.run_range("prefill", 0, 2, {"tokens": 300})
    for lo, hi in [(-1, 2), (3, 2), (0, 6)]:
        with pytest.raises(ops.KernError):
            rt.time_range("prefill", lo, hi, {"tokens": 300})
        with pytest.raises(ops.KernError):
            rt.run_range("prefill", lo, hi, {"tokens": 300})
    rt.close()
