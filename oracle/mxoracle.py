"""ctypes view of the C oracle (oracle/libmxoracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as
the checker. The product (kern_amd/) never imports it. Each wrapper names the C function it calls;
the C header (oracle/mxoracle.h) names the reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmxoracle.so")


def build() -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int


def _declare(L):
    L.mxo_splitmix64_at.restype = ctypes.c_uint64
    L.mxo_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    L.mxo_normal_at.restype = ctypes.c_double
    L.mxo_normal_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    L.mxo_e2m1_decode.restype = ctypes.c_float
    L.mxo_e2m1_decode.argtypes = [ctypes.c_uint8]
    L.mxo_e8m0_decode.restype = ctypes.c_float
    L.mxo_e8m0_decode.argtypes = [ctypes.c_uint8]
    L.mxo_e8m0_encode.restype = ctypes.c_uint8
    L.mxo_e8m0_encode.argtypes = [ctypes.c_double]
    L.mxo_e4m3_decode.restype = ctypes.c_float
    L.mxo_e4m3_decode.argtypes = [ctypes.c_uint8]
    L.mxo_e4m3_encode_values_rs.restype = ctypes.c_uint8
    L.mxo_e4m3_encode_values_rs.argtypes = [ctypes.c_double]
    L.mxo_e4m3_encode_rne.restype = ctypes.c_uint8
    L.mxo_e4m3_encode_rne.argtypes = [ctypes.c_uint32, ctypes.c_int]
    L.mxo_f32_to_bf16.restype = ctypes.c_uint16
    L.mxo_f32_to_bf16.argtypes = [ctypes.c_float]
    L.mxo_situ.restype = ctypes.c_float
    L.mxo_situ.argtypes = [ctypes.c_float] * 4
    L.mxo_quant_mxfp8.argtypes = [P, I64, I64, P, P]
    L.mxo_quant_block32_f32.restype = ctypes.c_uint8
    L.mxo_quant_block32_f32.argtypes = [P, P]
    for f in ("mxo_w_shuffle", "mxo_w_unshuffle", "mxo_sf_shuffle", "mxo_sf_unshuffle"):
        getattr(L, f).argtypes = [P, P, I64, I64, I64, I32]
    L.mxo_w_src_row.restype = I64
    L.mxo_w_src_row.argtypes = [I64, I64, I32]
    L.mxo_w_offset.restype = I64
    L.mxo_w_offset.argtypes = [I64, I64, I64, I64]
    L.mxo_sf_offset.restype = I64
    L.mxo_sf_offset.argtypes = [I64, I64, I64, I64]
    L.mxo_r128c4_offset.restype = I64
    L.mxo_r128c4_offset.argtypes = [I64, I64, I64]
    L.mxo_r128c4_size.restype = I64
    L.mxo_r128c4_size.argtypes = [I64, I64]
    L.mxo_deq_fp4.argtypes = [P, P, I64, I64, P]
    L.mxo_deq_fp8.argtypes = [P, P, I64, I64, P]
    L.mxo_gemm_f32.argtypes = [P, P, I64, I64, I64, P, I32]
    L.mxo_gemv_w4a16.argtypes = [P, P, P, I64, I64, I64, P, P, I32]
    L.mxo_silu_mul_bf16.argtypes = [P, I64, I64, P]
    L.mxo_moe_finalize.argtypes = [P, P, P, P, I64, I64, I32, ctypes.c_float, P]
    L.mxo_rope_table.argtypes = [P, P, I64, I64, I64, ctypes.c_float]
    L.mxo_r128c4_gather.argtypes = [P, I64, I64, P]
    L.mxo_routing.argtypes = [P, I64, I32, I32, I32, I32, P, P, P, P, P, P, P]
    L.mxo_max_ctas.restype = I64
    L.mxo_max_ctas.argtypes = [I64, I32, I32, I32]
    L.mxo_fc2.argtypes = [P, P, P, P, I32, I64, P, P, P, P, P, I64, I64, I32, I32]
    L.mxo_fc1.argtypes = [P, P, P, P, P, P, I64, P, P, P, P, P, P, P, I64, I64, I32, I32]
    L.mxo_e4m3_from_f32_array.argtypes = [P, I64, P]
    L.mxo_quant_blocks_f32.argtypes = [P, I64, P, P]
    L.mxo_gemm_e4m3_pt.argtypes = [P, P, P, P, I64, I64, I64, ctypes.c_float, P, P, I32]


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def nthreads_default() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


# ---------------------------------------------------------------- scalar codecs

def e2m1_decode(n):
    return lib().mxo_e2m1_decode(n)


def e8m0_decode(c):
    return lib().mxo_e8m0_decode(c)


def e8m0_encode(v):
    return lib().mxo_e8m0_encode(v)


def e4m3_decode(c):
    return lib().mxo_e4m3_decode(c)


def e4m3_encode_values_rs(v):
    return lib().mxo_e4m3_encode_values_rs(v)


def e4m3_encode_rne(bits, shift=0):
    return lib().mxo_e4m3_encode_rne(bits, shift)


def f32_to_bf16(f):
    return lib().mxo_f32_to_bf16(f)


def situ(g, u, alpha, beta):
    return lib().mxo_situ(g, u, alpha, beta)


def splitmix64_at(seed, i):
    return lib().mxo_splitmix64_at(seed, i)


def normal_at(seed, i):
    return lib().mxo_normal_at(seed, i)


# ---------------------------------------------------------------- array ops

def quant_mxfp8(x_bf16: np.ndarray):
    """bf16 bits [T, K] (uint16) -> (q u8 [T, K], sf u8 [T, K/32])."""
    x = _c(x_bf16, np.uint16)
    T, K = x.shape
    q = np.empty((T, K), np.uint8)
    sf = np.empty((T, K // 32), np.uint8)
    lib().mxo_quant_mxfp8(_p(x), T, K, _p(q), _p(sf))
    return q, sf


def quant_block32(v: np.ndarray):
    v = _c(v, np.float32)
    q = np.empty(32, np.uint8)
    s = lib().mxo_quant_block32_f32(_p(v), _p(q))
    return q, s


def e4m3_from_f32(v):
    """RNE-saturating e4m3 codes of an f32 array (any shape)."""
    v = _c(v, np.float32)
    out = np.empty(v.shape, np.uint8)
    lib().mxo_e4m3_from_f32_array(_p(v), v.size, _p(out))
    return out


def quant_blocks(v):
    """Quantise an f32 array whose last dim is a multiple of 32 block by block -> (codes, scales)."""
    v = _c(v, np.float32)
    q = np.empty(v.shape, np.uint8)
    sf = np.empty(v.shape[:-1] + (v.shape[-1] // 32,), np.uint8)
    lib().mxo_quant_blocks_f32(_p(v), v.size // 32, _p(q), _p(sf))
    return q, sf


def w_shuffle(raw, E, rows, row_bytes, gated):
    raw = _c(raw, np.uint8)
    out = np.empty_like(raw)
    lib().mxo_w_shuffle(_p(raw), _p(out), E, rows, row_bytes, int(gated))
    return out


def w_unshuffle(x, E, rows, row_bytes, gated):
    x = _c(x, np.uint8)
    out = np.empty_like(x)
    lib().mxo_w_unshuffle(_p(x), _p(out), E, rows, row_bytes, int(gated))
    return out


def sf_shuffle(raw, E, rows, sf_cols, gated):
    raw = _c(raw, np.uint8)
    out = np.empty_like(raw)
    lib().mxo_sf_shuffle(_p(raw), _p(out), E, rows, sf_cols, int(gated))
    return out


def sf_unshuffle(x, E, rows, sf_cols, gated):
    x = _c(x, np.uint8)
    out = np.empty_like(x)
    lib().mxo_sf_unshuffle(_p(x), _p(out), E, rows, sf_cols, int(gated))
    return out


def w_src_row(R, rows, gated):
    return lib().mxo_w_src_row(R, rows, int(gated))


def r128c4_offset(r, b, kblocks):
    return lib().mxo_r128c4_offset(r, b, kblocks)


def r128c4_size(rows, kblocks):
    return lib().mxo_r128c4_size(rows, kblocks)


def deq_fp4(w, sf, N, K):
    w = _c(w, np.uint8)
    sf = _c(sf, np.uint8)
    out = np.empty((N, K), np.float32)
    lib().mxo_deq_fp4(_p(w), _p(sf), N, K, _p(out))
    return out


def deq_fp8(q, sf, T, K):
    q = _c(q, np.uint8)
    sf = _c(sf, np.uint8)
    out = np.empty((T, K), np.float32)
    lib().mxo_deq_fp8(_p(q), _p(sf), T, K, _p(out))
    return out


def gemm_f32(X, W, nthreads=None):
    X = _c(X, np.float32)
    W = _c(W, np.float32)
    T, K = X.shape
    N = W.shape[0]
    C = np.empty((T, N), np.float32)
    lib().mxo_gemm_f32(_p(X), _p(W), T, N, K, _p(C), nthreads or nthreads_default())
    return C


def r128c4_gather(tiled, rows, kblocks):
    """Linear [rows, kblocks] scales from the 128x4 tiled layout."""
    t = _c(tiled, np.uint8)
    out = np.empty((rows, kblocks), np.uint8)
    lib().mxo_r128c4_gather(_p(t), rows, kblocks, _p(out))
    return out


def mxfp8_gemm(a, w, a_sf_tiled, w_sf_tiled, m, n, k, nthreads=None):
    """extern:cublaslt_mxfp8_tn on the CPU: f32 C [m, n] = deq(a) [m, k] x deq(w) [n, k]^T, f32 accumulation
    over exactly dequantised operands (scales in the 128x4 tiled layout)."""
    A = deq_fp8(a, r128c4_gather(a_sf_tiled, m, k // 32), m, k)
    W = deq_fp8(w, r128c4_gather(w_sf_tiled, n, k // 32), n, k)
    return gemm_f32(A, W, nthreads)


def gemv_w4a16(x_bf16, w_raw, sf_raw, nthreads=None):
    """x bf16 bits [M, K], raw (unrepacked) w [N, K/2], sf [N, K/32] -> (y bf16 bits, y f32)."""
    x = _c(x_bf16, np.uint16)
    w = _c(w_raw, np.uint8)
    sf = _c(sf_raw, np.uint8)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.uint16)
    yf = np.empty((M, N), np.float32)
    lib().mxo_gemv_w4a16(_p(x), _p(w), _p(sf), M, N, K, _p(y), _p(yf), nthreads or nthreads_default())
    return y, yf


def silu_mul_bf16(x_bf16, d):
    x = _c(x_bf16, np.uint16)
    T = x.shape[0]
    out = np.empty((T, d), np.uint16)
    lib().mxo_silu_mul_bf16(_p(x), T, d, _p(out))
    return out


def moe_finalize(fc2_bf16, exp2perm, topk_weight, gamma_bf16, T, H, topk, eps=0.0):
    """MoE finalize (mxo_moe_finalize): fc2 bf16 bits [rows][H], exp2perm i32 [T*topk], topk_weight f32
    [T][topk], gamma bf16 bits [H] or None -> bf16 bits [T][H]."""
    fc2 = _c(fc2_bf16, np.uint16)
    e2p = _c(exp2perm, np.int32)
    w = _c(topk_weight, np.float32)
    g = None if gamma_bf16 is None else _c(gamma_bf16, np.uint16)
    out = np.empty((T, H), np.uint16)
    lib().mxo_moe_finalize(_p(fc2), _p(e2p), _p(w), None if g is None else _p(g), T, H, topk, float(eps), _p(out))
    return out


def rope_table(rows, half, stride, base):
    """weight_prep's RoPE cache -> (cos, sin) bf16 bits, each [rows * stride] (unwritten columns zero)."""
    c = np.zeros(rows * stride, np.uint16)
    s_ = np.zeros(rows * stride, np.uint16)
    lib().mxo_rope_table(_p(c), _p(s_), rows, half, stride, float(base))
    return c, s_


def max_ctas(tokens, topk, experts, tile=128):
    return lib().mxo_max_ctas(tokens, topk, experts, tile)


def routing(topk_idx, local_start, E_local, tile=128, ctas_cap=None):
    idx = _c(topk_idx, np.int32)
    T, topk = idx.shape
    cap = ctas_cap or (E_local + -(-T * topk // tile))
    counts = np.zeros(2 * E_local, np.int32)
    cta_batch = np.full(cap, -7, np.int32)
    cta_limit = np.full(cap, -7, np.int32)
    nne = np.zeros(1, np.int32)
    tp = np.zeros(1, np.int32)
    route_map = np.full(cap * tile, -7, np.int32)
    exp2perm = np.empty(T * topk, np.int32)
    lib().mxo_routing(_p(idx), T, topk, local_start, E_local, tile, _p(counts), _p(cta_batch), _p(cta_limit),
                      _p(nne), _p(tp), _p(route_map), _p(exp2perm))
    return dict(counts=counts, cta_batch=cta_batch, cta_limit=cta_limit, num_non_exiting=nne, total_padded=tp,
                route_map=route_map, exp2perm=exp2perm.reshape(T, topk))


def fc2(a, sf_a, b, sf_b, sf_b_r128c4, tables, m, k, tile=128, nthreads=None):
    b = _c(b, np.uint8)
    rows_b = b.shape[0]
    c = np.zeros((rows_b, m), np.uint16)
    acc = np.zeros((rows_b, m), np.float32)
    lib().mxo_fc2(_p(_c(a, np.uint8)), _p(_c(sf_a, np.uint8)), _p(b), _p(_c(sf_b, np.uint8)), int(sf_b_r128c4),
                  rows_b, _p(c), _p(acc), _p(tables["num_non_exiting"]), _p(tables["cta_batch"]),
                  _p(tables["cta_limit"]), m, k, tile, nthreads or nthreads_default())
    return c, acc


def fc1(a, sf_a, b, sf_b, tables, alpha, beta, m, k, padded_rows, tile=128, nthreads=None):
    half = m // 2
    c = np.zeros((padded_rows, half), np.uint8)
    sf_c = np.zeros(r128c4_size(padded_rows, half // 32), np.uint8)
    dbg = np.zeros((padded_rows, 3, half), np.float32)
    lib().mxo_fc1(_p(_c(a, np.uint8)), _p(_c(sf_a, np.uint8)), _p(_c(b, np.uint8)), _p(_c(sf_b, np.uint8)), _p(c),
                  _p(sf_c), padded_rows, _p(tables["route_map"]), _p(_c(alpha, np.float32)),
                  _p(_c(beta, np.float32)), _p(dbg), _p(tables["num_non_exiting"]), _p(tables["cta_batch"]),
                  _p(tables["cta_limit"]), m, k, tile, nthreads or nthreads_default())
    return c, sf_c, dbg


def gemm_e4m3_pt(a, sf_a, b, sf_b, m, k, d_scale, nthreads=None):
    b = _c(b, np.uint8)
    T = b.shape[0]
    c = np.empty((T, m), np.uint8)
    acc = np.empty((T, m), np.float32)
    lib().mxo_gemm_e4m3_pt(_p(_c(a, np.uint8)), _p(_c(sf_a, np.uint8)), _p(b), _p(_c(sf_b, np.uint8)), T, m, k,
                           float(d_scale), _p(c), _p(acc), nthreads or nthreads_default())
    return c, acc
