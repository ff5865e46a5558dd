"""hipGraph capture and replay through the C ABI (kern_graph_begin / end / launch, the analog of
crates/kern-runtime/src/exec.rs:489-548 and :644-654): a captured quantizer + GEMM + decode GEMV,
replayed several times with the inputs changed eagerly in between, matches the eager launches bit for
bit on every replay."""
import numpy as np
import pytest
import torch

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


def test_graph_replays_match_eager(ops):
    M, N, K = 256, 512, 1024      # GEMM
    DM, DN, DK = 4, 1024, 7168   # decode GEMV
    print(f"[graph] GEMM {M}x{N}x{K} + GEMV M={DM} N={DN} K={DK}", flush=True)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        w, s = (_dev(a) for a in wl.mxfp4_weights(81, 1, N, K, 120, 126))
        wp, sp = ops.repack_weights(w[0], s[0])
        dw, ds = (_dev(a) for a in wl.mxfp4_weights(82, 1, DN, DK, 120, 126))
        dwp, dsp = ops.repack_weights(dw[0], ds[0])
        x = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
        dx = torch.empty((DM, DK), dtype=torch.bfloat16, device="cuda")
        q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
        qs = torch.empty((M, K // 32), dtype=torch.uint8, device="cuda")
        c = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        y = torch.empty((DM, DN), dtype=torch.bfloat16, device="cuda")
        # eager references go to their own buffers
        q_e, qs_e = torch.empty_like(q), torch.empty_like(qs)
        c_e, y_e = torch.empty_like(c), torch.empty_like(y)

        def chain(q, qs, c, y):
            ops.moe_quant(x, q, qs, M, K=K)
            ops.mxfp4_gemm_bf16(wp, sp, q, qs, c, M=M, m=N, k=K)
            ops.mxfp4_gemv_bf16(dx, dwp, dsp, y, DM, N=DN, K=DK)

        x.copy_(_dev(wl.activations_bf16(83, M, K)))
        dx.copy_(_dev(wl.activations_bf16(84, DM, DK)))
        chain(q, qs, c, y)  # warm-up: modules and functions resolved before capture
        torch.cuda.synchronize()
        with ops.Graph() as g:
            chain(q, qs, c, y)
        for r in range(4):
            # new inputs, written eagerly between replays
            x.copy_(_dev(wl.activations_bf16(90 + r, M, K, outlier_frac=0.01)))
            dx.copy_(_dev(wl.activations_bf16(95 + r, DM, DK)))
            c.zero_(), y.zero_()
            g.launch()
            torch.cuda.synchronize()
            chain(q_e, qs_e, c_e, y_e)
            torch.cuda.synchronize()
            for name, a, b in [("q", q, q_e), ("qs", qs, qs_e), ("c", c, c_e), ("y", y, y_e)]:
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"replay {r}: {name}"
        g.close()


def test_graph_errors(ops):
    with pytest.raises(ops.KernError):
        ops.Graph().launch()  # never captured
