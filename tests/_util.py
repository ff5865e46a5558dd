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
