"""Seeded random shapes through the two shape-dispatching entries, against the CPU oracle.

* kern_mxfp4_gemv_bf16 (W4A16 decode): M in 1..16, N a multiple of 16 from 16 to 19200 (ragged shares of
  the persistent kernel's half groups), K from 512 to 16384 (every kernel the entry picks: the row-group
  instances, the k-group loop, the persistent instances and the sliced kernel).
* kern_mxfp4_gemm_bf16 (dense bf16 out): M in 1..80 (the persistent walk up to 64, tiled above), m a
  multiple of 256, k in {1024, 2048, 3072, 4096, 7168, 8192}; the bf16 output is the RNE rounding of the
  kernel's own f32 sums, and those sums are within the north-star tolerance of the oracle.

The shapes come from a fixed seed, so each run sends the same sequence of launches; kernels that read
LDS or registers before their data has landed would show up here as mismatches on some shapes.
"""
import random

import numpy as np
import pytest

from kern_amd import workload as wl
from tests import _moe
from tests._util import assert_gemm_close, bf16_to_f32, to_dev, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _gemv_cases():
    rng = random.Random(7)
    out = []
    for M in range(1, 17):
        for _ in range(2):
            K = rng.choice([1024, 2048, 4096, 7168, 8192, 1536, 3072, 512, 16384, 6144])
            N = 16 * rng.choice([1, 3, 64, 257, 500, 513, 576, 1040, 1152, 1200])
            out.append((M, N, K))
    return out + [(M, 8192, K) for M in (4, 9, 16) for K in (4096, 8192)] + [(15, 16640, 2048), (16, 8208, 4096)]


def _gemm_cases():
    rng = random.Random(11)
    return [(rng.choice(list(range(1, 65)) + [65, 80]), 256 * rng.choice([1, 3, 9, 17, 28, 36, 52, 72]),
             rng.choice([1024, 2048, 4096, 7168, 8192, 3072])) for _ in range(24)]


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    return ops


@pytest.mark.parametrize("i,M,N,K", [(i,) + c for i, c in enumerate(_gemv_cases())])
def test_gemv_sweep(ops, oracle, i, M, N, K):
    print(f"[gemv sweep] M={M} N={N} K={K}", flush=True)
    x = wl.activations_bf16(1000 + i, M, K)
    w, sf = wl.mxfp4_weights(2000 + i, 1, N, K, 122, 132)
    wp, sfp = ops.repack_weights(to_dev(w[0]), to_dev(sf[0]))
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.mxfp4_gemv_bf16(to_dev(x), wp, sfp, y, M, N=N, K=K)
    torch.cuda.synchronize()
    _, yf = oracle.gemv_w4a16(x, w[0], sf[0])
    assert_gemm_close(bf16_to_f32(to_np(y)), yf, f"gemv M={M} N={N} K={K}")


@pytest.mark.parametrize("i,M,m,k", [(i,) + c for i, c in enumerate(_gemm_cases())])
def test_gemm_bf16_sweep(ops, oracle, i, M, m, k):
    print(f"[gemm bf16 sweep] M={M} m={m} k={k}", flush=True)
    w_raw, s_raw = _moe.gpu_raw_weights(ops, torch, 900 + i, 1, m, k, 119, 6)
    wp, sp = ops.repack_weights(w_raw, s_raw)
    x = wl.activations_bf16(950 + i, M, k, outlier_frac=0.01)
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
