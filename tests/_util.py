"""Shared helpers of the parity tests (numpy <-> torch, tolerance of the north star)."""
import numpy as np


def to_dev(a, dtype=None):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    t = torch.from_numpy(a).cuda()
    return t if dtype is None else t.to(dtype)


def to_np(t):
    import torch

    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_gemm_close(got, ref, what=""):
    """max|err| <= 1e-2 * ||ref row||_inf per row, and ||err||_F / ||ref||_F <= 2e-3."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    rowmax = np.abs(ref).max(axis=-1, keepdims=True)
    bad = err > 1e-2 * rowmax + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} elements over 1e-2*||row||inf (max err {err.max():.4g})"
    rel = np.sqrt((err**2).sum()) / max(np.sqrt((ref**2).sum()), 1e-30)
    assert rel <= 2e-3, f"{what}: relative Frobenius error {rel:.3g} > 2e-3"
    return rel


def r128c4_offsets(rows, kblocks):
    """Offsets [rows, kblocks] of the R128c4 scale layout (crates/kern-runtime/src/cublas.rs:396-400)."""
    r = np.arange(rows)[:, None]
    b = np.arange(kblocks)[None, :]
    kb4 = (kblocks + 3) // 4
    return 512 * ((r // 128) * kb4 + b // 4) + (r % 32) * 16 + ((r % 128) // 32) * 4 + b % 4


def mxfp8_kat(shift=0):
    """The closed-form case of crates/kern-runtime/tests/mxfp8_gemm.rs:9-95: A row i holds one 1.0 at column
    7i mod K, W[n][k] = ((n + k) % 5) - 2, e8m0 exponents ea(r, b), ew(r, b) (+ shift on W), tiled 128x4;
    out[i][n] = W[n][col(i)] * 2^(ea(i, b) + ew(n, b) + shift), exact in bf16."""
    M, N, K = 256, 160, 320
    KB = K // 32
    code = {0.0: 0x00, 1.0: 0x38, 2.0: 0x40, -1.0: 0xB8, -2.0: 0xC0}
    col = lambda i: i * 7 % K
    a = np.zeros((M, K), np.uint8)
    for i in range(M):
        a[i, col(i)] = code[1.0]
    wv = lambda n, k: float((n + k) % 5 - 2)
    w = np.array([[code[wv(n, k)] for k in range(K)] for n in range(N)], np.uint8)
    ea = lambda r, b: (r + b) % 3 - 1
    ew = lambda r, b: (3 * r + 2 * b) % 5 - 2 + shift

    def tiled(rows, e):
        kb4, sf = -(-KB // 4), np.full(-(-rows // 128) * -(-KB // 4) * 512, 127, np.uint8)
        for r in range(rows):
            for b in range(KB):
                sf[(r // 128 * kb4 + b // 4) * 512 + r % 32 * 16 + r % 128 // 32 * 4 + b % 4] = 127 + e(r, b)
        return sf

    want = np.array([[wv(n, col(i)) * 2.0 ** (ea(i, col(i) // 32) + ew(n, col(i) // 32)) for n in range(N)]
                     for i in range(M)], np.float32)
    return dict(M=M, N=N, K=K, a=a, w=w, a_sf=tiled(M, ea), w_sf=tiled(N, ew), want=want)
