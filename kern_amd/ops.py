"""Python mirror of the path's manifest ops over the C ABI (include/kern_amd.h).

Each function has the name, parameter order and meaning of a manifest op of kern's MXFP4 matmul
path (fixtures/k3/head.json ops `moe_quant`, `k3_moe_w_shuffle`, `k3_moe_sf_shuffle`, `moe_routing`,
`moe_fc1` = trtllm_bmm_mxe4m3_mxe2m1_mxe4m3, `moe_fc2` = trtllm_bmm_bf16_mxe2m1_mxe4m3), followed by the
scalars the op's launch supplies as keywords. Buffers are torch tensors on a HIP device; the call is
enqueued on torch's current stream. A contract violation raises KernError with the library's message,
as the reference runtime returns Error::Api (crates/kern-runtime/src/error.rs:25-30). There is no CPU
fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libkern_amd.so")
HSACO_PATH = os.path.join(HERE, "lib", "kern_mx.hsaco")

STATUS = {0: "ok", 1: "manifest", 2: "kernel artifact", 3: "weight artifact", 4: "caller contract", 6: "domain",
          7: "call", 8: "hip"}


class KernError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64

_SIGS = {
    "kern_moe_quant": [P, P, P, I32, I32, P],
    "kern_mxfp8_quant_f32": [P, P, P, I32, I32, P],
    "kern_moe_w_shuffle": [P, P, I32, I32, I32, I32, P],
    "kern_moe_sf_shuffle": [P, P, I32, I32, I32, I32, P],
    "kern_moe_routing": [P] * 8 + [I32] * 4 + [P],
    "kern_moe_quant_routing": [P, P, P, I32, I32] + [P] * 8 + [I32] * 3 + [P],
    "kern_trtllm_bmm_bf16_mxe2m1_mxe4m3": [P] * 9 + [I32, I32, I32, I32, P, P],
    "kern_trtllm_bmm_mxe4m3_mxe2m1_mxe4m3": [P] * 13 + [I32, I32, I32, P, P],
    "kern_mxfp4_gemm_e4m3": [P] * 6 + [I32, I32, I32, P, P],
    "kern_mxfp4_gemm_bf16": [P] * 5 + [I32, I32, I32, P, P],
    "kern_mxfp4_gemv_bf16": [P] * 4 + [I32, I32, I32, P],
    "kern_fill_random_u8": [P, I64, ctypes.c_uint64, I32, I32, P],
    "kern_silu_mul": [P, P, I32, I32, P],
    "kern_mxfp8_gemm_bf16": [P] * 5 + [I32, I32, I32, I32, P],
    "kern_weight_p1_bf16_f32": [P, P, I32, P],
    "kern_cast_bf16_f32": [P, P, I32, P],
    "kern_rope_table_bf16": [P, P, I32, I32, I32, ctypes.c_float, P],
    "kern_fill_f32": [P, I32, ctypes.c_float, P],
    "kern_fill_i32": [P, I32, I32, P],
    "kern_fill_i64": [P, I32, I64, P],
    "kern_fill_u8": [P, I32, I32, P],
    "kern_fill_bf16": [P, I32, ctypes.c_float, P],
    "kern_iota_i32": [P, I32, I32, I32, I32, P],
    "kern_moe_finalize_rms": [P] * 5 + [I32, I32, I32, ctypes.c_float, P],
    "kern_moe_finalize": [P] * 4 + [I32, I32, I32, P],
    "kern_init": [ctypes.c_char_p],
    "kern_sha256_hex": [P, ctypes.c_size_t, ctypes.c_char_p],
    "kern_code_object_param_sizes": [P, ctypes.c_size_t, ctypes.c_char_p, P, ctypes.c_int, P],
    "kern_module_load": [P, ctypes.c_size_t, ctypes.c_char_p, P],
    "kern_module_unload": [P],
    "kern_module_function": [P, ctypes.c_char_p, P],
    "kern_function_param_sizes": [P, P, ctypes.c_int, P],
    "kern_function_check_params": [P, P, ctypes.c_int],
    "kern_launch": [P, P, P, ctypes.c_uint32, P, P, ctypes.c_size_t],
    "kern_graph_begin": [P],
    "kern_graph_end": [P, P],
    "kern_graph_launch": [P, P],
    "kern_graph_destroy": [P],
    "kern_function_release": [P],
    "kern_function_param_offsets": [P, P, ctypes.c_int, P],
    "kern_mx_module": [P],
    "kern_op_create": [ctypes.c_char_p, ctypes.c_char_p, P, P],
    "kern_op_destroy": [P],
    "kern_op_num_params": [P],
    "kern_op_num_launches": [P],
    "kern_op_launch": [P, P, ctypes.c_int, P, P, ctypes.c_int, P],
    "kern_op_plan": [ctypes.c_char_p, ctypes.c_int, P, ctypes.c_int, P, P, ctypes.c_int, P, P, P, P, ctypes.c_size_t,
                     P, P],
    "kern_op_verify": [ctypes.c_char_p],
    "kern_rt_load": [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, P],
    "kern_rt_destroy": [P],
    "kern_rt_check": [ctypes.c_char_p, ctypes.c_char_p],
    "kern_rt_write_input": [P, ctypes.c_char_p, P, ctypes.c_size_t],
    "kern_rt_read_output": [P, ctypes.c_char_p, P, ctypes.c_size_t],
    "kern_rt_write_buffer": [P, ctypes.c_char_p, ctypes.c_size_t, P, ctypes.c_size_t],
    "kern_rt_read_buffer": [P, ctypes.c_char_p, ctypes.c_size_t, P, ctypes.c_size_t],
    "kern_rt_load_weight": [P, ctypes.c_char_p, P, ctypes.c_size_t],
    "kern_rt_derive": [P],
    "kern_rt_run": [P, ctypes.c_char_p, P, P, ctypes.c_int],
    "kern_rt_capture": [P, ctypes.c_char_p, P, P, ctypes.c_int],
    "kern_rt_run_captured": [P, ctypes.c_char_p, P, P, ctypes.c_int],
    "kern_rt_time_captured": [P, ctypes.c_char_p, P, P, ctypes.c_int, ctypes.c_int, P],
    "kern_rt_run_range": [P, ctypes.c_char_p, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int],
    "kern_rt_time_range": [P, ctypes.c_char_p, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P],
    "kern_rt_synchronize": [P],
    "kern_candidate_splice": [ctypes.c_char_p, ctypes.c_char_p, P, ctypes.c_size_t, P],
    "kern_candidate_of": [ctypes.c_char_p, P, ctypes.c_int, P, ctypes.c_size_t, P],
    "kern_candidate_only": [ctypes.c_char_p, P, ctypes.c_int, P, ctypes.c_size_t, P],
    "kern_candidate_join": [P, ctypes.c_int, P, ctypes.c_size_t, P],
    "kern_candidate_tile": [ctypes.c_char_p, ctypes.c_char_p, P, ctypes.c_int, P, ctypes.c_size_t, P],
    "kern_rt_buffer": [P, ctypes.c_char_p, P, P],
}


def lib() -> ctypes.CDLL:
    """The C-ABI library; raises if it has not been built (python -m kern_amd.build)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KernError(2, f"{LIB_PATH} is missing: build it with `python -m kern_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.kern_last_error.restype = ctypes.c_char_p
        L.kern_last_error.argtypes = []
        L.kern_code_object_sha256.restype = ctypes.c_char_p
        L.kern_code_object_sha256.argtypes = []
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise KernError(rc, lib().kern_last_error().decode())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t, name, dtype=None, numel=None):
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise KernError(4, f"{name}: expected a torch.Tensor")
    if not t.is_cuda:
        raise KernError(4, f"{name}: must be a device tensor")
    if not t.is_contiguous():
        raise KernError(4, f"{name}: must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise KernError(4, f"{name}: dtype {t.dtype}, expected {dtype}")
    if numel is not None and t.numel() < numel:
        raise KernError(4, f"{name}: {t.numel()} elements, need at least {numel}")
    return ctypes.c_void_p(t.data_ptr())


u8, i32, f32, bf16 = torch.uint8, torch.int32, torch.float32, torch.bfloat16


def code_object_sha256() -> str:
    return lib().kern_code_object_sha256().decode()


# ------------------------------------------------------------------------------------------- ops

def moe_quant(x, q, sf, tokens, *, K):
    """moe_quant(in bf16 x[T,K], out u8 q[T,K], out u8 sf[T,K/32], i32 tokens) — head.json:25057."""
    check(lib().kern_moe_quant(_ptr(x, "x", bf16, tokens * K), _ptr(q, "q", u8, tokens * K),
                               _ptr(sf, "sf", u8, tokens * K // 32), tokens, K, _stream()))


def mxfp8_quant_f32(x, q, sf, tokens, *, K):
    """f32 [T,K] -> MXFP8 codes u8 [T,K] and ue8m0 scales u8 [T,K/32] with the FC1 epilogue's codec."""
    check(lib().kern_mxfp8_quant_f32(_ptr(x, "x", f32, tokens * K), _ptr(q, "q", u8, tokens * K),
                                     _ptr(sf, "sf", u8, tokens * K // 32), tokens, K, _stream()))


def k3_moe_w_shuffle(raw, out, rows, row_bytes, gated, *, experts):
    """k3_moe_w_shuffle(in u8 raw, out u8 shuffled, i32 rows, i32 row_bytes, i32 gated) — head.json:26358."""
    n = experts * rows * row_bytes
    check(lib().kern_moe_w_shuffle(_ptr(raw, "raw", u8, n), _ptr(out, "out", u8, n), experts, rows, row_bytes,
                                   int(gated), _stream()))


def k3_moe_sf_shuffle(raw, out, rows, sf_cols, gated, *, experts):
    """k3_moe_sf_shuffle(in u8 raw, out u8 shuffled, i32 rows, i32 sf_cols, i32 gated) — head.json:26413."""
    n = experts * rows * sf_cols
    check(lib().kern_moe_sf_shuffle(_ptr(raw, "raw", u8, n), _ptr(out, "out", u8, n), experts, rows, sf_cols,
                                    int(gated), _stream()))


def ctas_bound(tokens, topk, experts, tile=128):
    """The op's grid.y: experts + ceil(tokens*topk/tile) (tools/kernels/abi/trtllm_bmm.py:58-60)."""
    return experts + -(-tokens * topk // tile)


def moe_routing(topk_idx, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map, exp2perm, *,
                tokens, topk, local_start, local_experts):
    """moe_routing(in i32 topk_idx, out counts, cta_batch, cta_limit, num_non_exiting, total_padded,
    route_map, exp2perm) — head.json:25117."""
    ctas = ctas_bound(tokens, topk, local_experts)
    check(lib().kern_moe_routing(
        _ptr(topk_idx, "topk_idx", i32, tokens * topk), _ptr(counts, "counts", i32, 2 * local_experts),
        _ptr(cta_batch, "cta_batch", i32, ctas), _ptr(cta_limit, "cta_limit", i32, ctas),
        _ptr(num_non_exiting, "num_non_exiting", i32, 1), _ptr(total_padded, "total_padded", i32, 1),
        _ptr(route_map, "route_map", i32, ctas * 128), _ptr(exp2perm, "exp2perm", i32, tokens * topk),
        tokens, topk, local_start, local_experts, _stream()))


def moe_quant_routing(x, q, sf, topk_idx, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map,
                      exp2perm, *, tokens, K, topk, local_start, local_experts):
    """moe_quant and moe_routing in one call (one launch for decode-sized batches): the outputs of
    moe_quant(x, q, sf, tokens, K=K) and moe_routing(topk_idx, ..., tokens=tokens, topk=topk, ...)."""
    ctas = ctas_bound(tokens, topk, local_experts)
    check(lib().kern_moe_quant_routing(
        _ptr(x, "x", bf16, tokens * K), _ptr(q, "q", u8, tokens * K), _ptr(sf, "sf", u8, tokens * K // 32), tokens, K,
        _ptr(topk_idx, "topk_idx", i32, tokens * topk), _ptr(counts, "counts", i32, 2 * local_experts),
        _ptr(cta_batch, "cta_batch", i32, ctas), _ptr(cta_limit, "cta_limit", i32, ctas),
        _ptr(num_non_exiting, "num_non_exiting", i32, 1), _ptr(total_padded, "total_padded", i32, 1),
        _ptr(route_map, "route_map", i32, ctas * 128), _ptr(exp2perm, "exp2perm", i32, tokens * topk),
        topk, local_start, local_experts, _stream()))


def trtllm_bmm_bf16_mxe2m1_mxe4m3(a, sf_a, b, sf_b, c, num_non_exiting, total_padded, cta_batch, cta_limit, *, m, k,
                                  ctas, sf_b_r128c4=True, dbg=None):
    """moe_fc2 (head.json:25683): bf16 c[rows, m] = MXFP8 b[rows, k] x MXFP4 a[e, m, k]^T per CTA slot."""
    rows = ctas * 128
    check(lib().kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(
        _ptr(a, "a", u8), _ptr(sf_a, "sf_a", u8), _ptr(b, "b", u8, rows * k), _ptr(sf_b, "sf_b", u8),
        _ptr(c, "c", bf16, rows * m), _ptr(num_non_exiting, "num_non_exiting", i32, 1),
        _ptr(total_padded, "total_padded", i32, 1), _ptr(cta_batch, "cta_batch", i32, ctas),
        _ptr(cta_limit, "cta_limit", i32, ctas), m, k, ctas, int(bool(sf_b_r128c4)),
        _ptr(dbg, "dbg", f32, rows * m), _stream()))


def trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(a, sf_a, b, sf_b, c, sf_c, route_map, alpha, beta, num_non_exiting,
                                    total_padded, cta_batch, cta_limit, *, m, k, ctas, dbg=None):
    """moe_fc1 (head.json:25459): e4m3 c[rows, m/2] + ue8m0 sf_c = MXFP8(SiTU-GLU(b[route_map] x a^T))."""
    rows = ctas * 128
    check(lib().kern_trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(
        _ptr(a, "a", u8), _ptr(sf_a, "sf_a", u8), _ptr(b, "b", u8), _ptr(sf_b, "sf_b", u8),
        _ptr(c, "c", u8, rows * m // 2), _ptr(sf_c, "sf_c", u8), _ptr(route_map, "route_map", i32, rows),
        _ptr(alpha, "alpha", f32), _ptr(beta, "beta", f32), _ptr(num_non_exiting, "num_non_exiting", i32, 1),
        _ptr(total_padded, "total_padded", i32, 1), _ptr(cta_batch, "cta_batch", i32, ctas),
        _ptr(cta_limit, "cta_limit", i32, ctas), m, k, ctas, _ptr(dbg, "dbg", f32, rows * 3 * (m // 2)),
        _stream()))


def mxfp4_gemm_e4m3(a, sf_a, b, sf_b, c, d_scale, *, M, m, k, dbg=None):
    """Dense e4m3-output mode: c[M, m] = e4m3(MXFP8 b[M, k] x MXFP4 a[m, k]^T * d_scale)."""
    check(lib().kern_mxfp4_gemm_e4m3(
        _ptr(a, "a", u8, m * k // 2), _ptr(sf_a, "sf_a", u8, m * k // 32), _ptr(b, "b", u8, M * k),
        _ptr(sf_b, "sf_b", u8, M * k // 32), _ptr(c, "c", u8, M * m), _ptr(d_scale, "d_scale", f32, 1), M, m, k,
        _ptr(dbg, "dbg", f32, M * m), _stream()))


def mxfp4_gemm_bf16(a, sf_a, b, sf_b, c, *, M, m, k, dbg=None):
    """Dense bf16-output mode: c[M, m] = bf16(MXFP8 b[M, k] x MXFP4 a[m, k]^T)."""
    check(lib().kern_mxfp4_gemm_bf16(
        _ptr(a, "a", u8, m * k // 2), _ptr(sf_a, "sf_a", u8, m * k // 32), _ptr(b, "b", u8, M * k),
        _ptr(sf_b, "sf_b", u8, M * k // 32), _ptr(c, "c", bf16, M * m), M, m, k, _ptr(dbg, "dbg", f32, M * m),
        _stream()))


def mxfp4_gemv_bf16(x, w, w_sf, y, M, *, N, K):
    """W4A16 decode: y[M, N] = bf16(x[M, K] x deq(w)[N, K]^T), 1 <= M <= 16."""
    check(lib().kern_mxfp4_gemv_bf16(
        _ptr(x, "x", bf16, M * K), _ptr(w, "w", u8, N * K // 2), _ptr(w_sf, "w_sf", u8, N * K // 32),
        _ptr(y, "y", bf16, M * N), M, N, K, _stream()))


def r128c4_bytes(rows, kblocks):
    """Bytes of the 128x4 tiled scale layout: rows padded to 128, k blocks to 4 (cublas.rs:396-400)."""
    return -(-rows // 128) * 512 * -(-kblocks // 4)


def cublaslt_mxfp8_tn(a, w, c, a_sf, w_sf, m, n, k, ldc=None):
    """extern:cublaslt_mxfp8_tn: c bf16 [m, ldc] = MXFP8 a [m, k] x MXFP8 w [n, k]^T, scales 128x4-tiled."""
    ldc = n if ldc is None else ldc
    check(lib().kern_mxfp8_gemm_bf16(
        _ptr(a, "a", u8, m * k), _ptr(w, "w", u8, n * k), _ptr(c, "c", bf16, (m - 1) * ldc + n if m else 0),
        _ptr(a_sf, "a_sf", u8, r128c4_bytes(m, k // 32)), _ptr(w_sf, "w_sf", u8, r128c4_bytes(n, k // 32)),
        m, n, k, ldc, _stream()))


def silu_mul(out, x, tokens, d):
    """silu_mul (tools/kernels-src/silu_mul.cu): out bf16 [tokens, d] = bf16(bf16(silu(g)) * u) over
    x bf16 [tokens, 2d] = [g | u]."""
    check(lib().kern_silu_mul(_ptr(out, "out", bf16, tokens * d), _ptr(x, "x", bf16, tokens * 2 * d), tokens, d,
                              _stream()))


def moe_finalize_rms(fc2_out, exp2perm, topk_weight, gamma, out, tokens, *, H, topk, eps=1e-6):
    """moe_finalize_rms (fixtures/k3/head.json): out[t] = bf16(rms_norm(sum_j w[t,j] * fc2_out[exp2perm[t,j]]) * gamma)."""
    check(lib().kern_moe_finalize_rms(
        _ptr(fc2_out, "fc2_out", bf16), _ptr(exp2perm, "exp2perm", i32, tokens * topk),
        _ptr(topk_weight, "topk_weight", f32, tokens * topk), _ptr(gamma, "gamma", bf16, H),
        _ptr(out, "out", bf16, tokens * H), tokens, H, topk, float(eps), _stream()))


def moe_finalize(fc2_out, exp2perm, topk_weight, out, tokens, *, H, topk):
    """MoE finalize without the norm: out[t] = bf16(sum_j w[t,j] * fc2_out[exp2perm[t,j]])."""
    check(lib().kern_moe_finalize(
        _ptr(fc2_out, "fc2_out", bf16), _ptr(exp2perm, "exp2perm", i32, tokens * topk),
        _ptr(topk_weight, "topk_weight", f32, tokens * topk), _ptr(out, "out", bf16, tokens * H), tokens, H, topk,
        _stream()))


# weight_prep family (tools/kernels-src/weight_prep.cu)

def weight_p1_bf16_f32(w, out):
    check(lib().kern_weight_p1_bf16_f32(_ptr(w, "w", bf16), _ptr(out, "out", f32, w.numel()), w.numel(), _stream()))


def cast_bf16_f32(w, out):
    check(lib().kern_cast_bf16_f32(_ptr(w, "w", bf16), _ptr(out, "out", f32, w.numel()), w.numel(), _stream()))


def rope_table_bf16(cos_t, sin_t, rows, half, stride, base):
    need = (rows - 1) * stride + half if rows else 0
    check(lib().kern_rope_table_bf16(_ptr(cos_t, "cos", bf16, need), _ptr(sin_t, "sin", bf16, need), rows, half, stride,
                                     float(base), _stream()))


def fill(p, v):
    """p[:] = v, by the dtype of p: fill_f32 / fill_i32 / fill_i64 / fill_u8 / fill_bf16."""
    n = p.numel()
    fn = {torch.float32: lib().kern_fill_f32, torch.int32: lib().kern_fill_i32, torch.int64: lib().kern_fill_i64,
          torch.uint8: lib().kern_fill_u8, torch.bfloat16: lib().kern_fill_bf16}.get(p.dtype)
    if fn is None:
        raise KernError(4, f"fill: no fill for {p.dtype}")
    val = float(v) if p.dtype in (torch.float32, torch.bfloat16) else int(v)
    check(fn(_ptr(p, "p"), n, val, _stream()))


def iota_i32(p, n, start=0, step=1, stride=1):
    check(lib().kern_iota_i32(_ptr(p, "p", i32, (n - 1) * stride + 1 if n else 0), n, start, step, stride, _stream()))


def fill_random_u8(out, seed, lo=0, span=256):
    """out[i] = lo + splitmix64_i(seed) % span (crates/kern-test/src/workload.rs:11-26)."""
    check(lib().kern_fill_random_u8(_ptr(out, "out", u8), out.numel(), seed & (2**64 - 1), lo, span, _stream()))


# ------------------------------------------------------------------------------------- helpers

def quantize_mxfp8(x: torch.Tensor):
    """Allocate and run moe_quant over a bf16 [T, K] tensor -> (q u8 [T, K], sf u8 [T, K/32])."""
    T, K = x.shape
    q = torch.empty((T, K), dtype=u8, device=x.device)
    sf = torch.empty((T, K // 32), dtype=u8, device=x.device)
    moe_quant(x, q, sf, T, K=K)
    return q, sf


def repack_weights(raw_w: torch.Tensor, raw_sf: torch.Tensor, gated: bool = False):
    """Run the two derive ops over raw [E, rows, K/2] nibbles and [E, rows, K/32] scales."""
    if raw_w.dim() == 2:
        raw_w, raw_sf = raw_w.unsqueeze(0), raw_sf.unsqueeze(0)
    E, rows, rb = raw_w.shape
    w = torch.empty_like(raw_w)
    sf = torch.empty_like(raw_sf)
    k3_moe_w_shuffle(raw_w, w, rows, rb, gated, experts=E)
    k3_moe_sf_shuffle(raw_sf, sf, rows, raw_sf.shape[2], gated, experts=E)
    return w, sf


# ------------------------------------------------------------------------------- manifest ops

def _op_params(op: dict, params) -> ctypes.Array:
    """Interface params as the C ABI takes them: device addresses for buffers, scalar bits otherwise."""
    types = op["params"]
    if len(params) != len(types):
        raise KernError(4, f"the op takes {len(types)} params, got {len(params)}")
    vals = (ctypes.c_uint64 * max(1, len(types)))()
    for i, (t, v) in enumerate(zip(types, params)):
        if t is None:
            vals[i] = int(v)
        elif "buffer<" in t:
            vals[i] = v.data_ptr() if isinstance(v, torch.Tensor) else int(v)
        elif t == "f32":
            vals[i] = struct.unpack("<I", struct.pack("<f", float(v)))[0]
        elif t == "i64":
            vals[i] = int(v) & (2**64 - 1)
        elif t == "u8":
            vals[i] = int(v) & 0xFF
        else:
            vals[i] = int(v) & 0xFFFFFFFF
    return vals


def _vars(vars_: dict | None):
    vars_ = vars_ or {}
    names = (ctypes.c_char_p * max(1, len(vars_)))(*[k.encode() for k in vars_])
    values = (ctypes.c_uint64 * max(1, len(vars_)))(*[int(v) for v in vars_.values()])
    return names, values, len(vars_)


class ManifestOp:
    """One kern manifest op (an `ops` entry: params + impl.launches) run through kern_op_* with its
    launches bound to this library's own module, which the manifest names `module_name`
    (crates/kern-manifest/src/candidate.rs:1-26 swaps an op's impl the same way)."""

    def __init__(self, op: dict | str, module_name: str = "kern_mx"):
        self.op = json.loads(op) if isinstance(op, str) else op
        mod = ctypes.c_void_p()
        check(lib().kern_mx_module(ctypes.byref(mod)))
        h = ctypes.c_void_p()
        check(lib().kern_op_create(json.dumps(self.op).encode(), module_name.encode(), mod, ctypes.byref(h)))
        self._h = h
        self.num_launches = lib().kern_op_num_launches(h)

    def __call__(self, *params, vars: dict | None = None):
        """Run the op's launches on torch's current stream; `vars` binds the manifest vars (e.g. tokens)."""
        vals = _op_params(self.op, params)
        names, values, n = _vars(vars)
        check(lib().kern_op_launch(self._h, ctypes.cast(vals, P), len(params), ctypes.cast(names, P),
                                   ctypes.cast(values, P), n, _stream()))

    def close(self):
        if self._h:
            lib().kern_op_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def op_plan(op: dict | str, launch: int, params, vars: dict | None = None) -> dict:
    """Host-only plan of one launch of a manifest op (no device): grid, block, dynamic LDS bytes and
    the kernel-argument image; skip is True when the launch's `when` does not hold."""
    if isinstance(op, str):
        text = op
        try:  # the param types; malformed text goes to the library as it is, which reports it
            types = {"params": json.loads(op).get("params", [])}
        except (ValueError, AttributeError):
            types = {"params": [None] * len(params)}
    else:
        text, types = json.dumps(op), op
    vals = _op_params(types, params)
    names, values, n = _vars(vars)
    grid, block = (ctypes.c_uint32 * 3)(), (ctypes.c_uint32 * 3)()
    shared, size, skip = ctypes.c_uint32(), ctypes.c_size_t(), ctypes.c_int()
    buf = (ctypes.c_uint8 * 4096)()
    check(lib().kern_op_plan(text.encode(), launch, ctypes.cast(vals, P), len(params),
                             ctypes.cast(names, P), ctypes.cast(values, P), n, ctypes.cast(grid, P),
                             ctypes.cast(block, P), ctypes.byref(shared), ctypes.cast(buf, P), 4096,
                             ctypes.byref(size), ctypes.byref(skip)))
    return {"grid": tuple(grid), "block": tuple(block), "shared": shared.value,
            "args": bytes(buf[:size.value]) if not skip.value else b"", "skip": bool(skip.value)}


# ----------------------------------------------------------------------------------- graphs

class Graph:
    """hipGraph of everything enqueued on torch's current stream inside the `with` block, captured
    through kern_graph_begin / kern_graph_end (exec.rs:489-548) and replayed by launch()
    (exec.rs:644-654). The stream must not be the null stream, and nothing inside the block may
    allocate device memory (allocate first, as the reference runtime owns its buffers at var max)."""

    def __init__(self):
        self._g = None
        self._stream = None

    def __enter__(self):
        self._stream = _stream()
        check(lib().kern_graph_begin(self._stream))
        return self

    def __exit__(self, et, ev, tb):
        g = ctypes.c_void_p()
        rc = lib().kern_graph_end(self._stream, ctypes.byref(g))
        if et is None:
            check(rc)
            self._g = g
        return False

    def launch(self):
        if not self._g:
            raise KernError(4, "graph was not captured")
        check(lib().kern_graph_launch(self._g, _stream()))

    def close(self):
        if self._g:
            lib().kern_graph_destroy(self._g)
            self._g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Runtime:
    """A kern manifest's buffers, modules, ops and programs on one device (kern_rt_*, the analog of
    crates/kern-runtime's Runtime, src/lib.rs:137-236): load, write inputs and weights by buffer name,
    derive, run programs by name with var values, read outputs. Host bytes are numpy arrays or bytes."""

    def __init__(self, manifest: dict | str, kernels_dir: str | None = None, gpu: int = 0):
        text = manifest if isinstance(manifest, str) else json.dumps(manifest)
        h = P()
        check(lib().kern_rt_load(text.encode(), (kernels_dir or os.path.dirname(HSACO_PATH)).encode(), gpu,
                                 ctypes.byref(h)))
        self._h = h

    @staticmethod
    def check(manifest: dict | str, kernels_dir: str | None = None) -> None:
        """Host-only parse and verification (kern_rt_check): module files read and sha-checked, ops verified."""
        text = manifest if isinstance(manifest, str) else json.dumps(manifest)
        check(lib().kern_rt_check(text.encode(), (kernels_dir or os.path.dirname(HSACO_PATH)).encode()))

    def close(self) -> None:
        if self._h:
            check(lib().kern_rt_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _bytes(data):
        import numpy as np
        a = np.ascontiguousarray(data) if not isinstance(data, (bytes, bytearray)) else np.frombuffer(data, np.uint8)
        return a, a.ctypes.data, a.nbytes

    def write_input(self, name: str, data) -> None:
        a, ptr, n = self._bytes(data)
        check(lib().kern_rt_write_input(self._h, name.encode(), ptr, n))

    def read_output(self, name: str, nbytes: int):
        import numpy as np
        out = np.empty(nbytes, np.uint8)
        check(lib().kern_rt_read_output(self._h, name.encode(), out.ctypes.data, nbytes))
        return out

    def write_buffer(self, name: str, data, offset: int = 0) -> None:
        a, ptr, n = self._bytes(data)
        check(lib().kern_rt_write_buffer(self._h, name.encode(), offset, ptr, n))

    def read_buffer(self, name: str, nbytes: int, offset: int = 0):
        import numpy as np
        out = np.empty(nbytes, np.uint8)
        check(lib().kern_rt_read_buffer(self._h, name.encode(), offset, out.ctypes.data, nbytes))
        return out

    def load_weight(self, name: str, data) -> None:
        a, ptr, n = self._bytes(data)
        check(lib().kern_rt_load_weight(self._h, name.encode(), ptr, n))

    def derive(self) -> None:
        check(lib().kern_rt_derive(self._h))

    @staticmethod
    def _vars(vars_: dict | None):
        names = list((vars_ or {}).keys())
        arr_n = (ctypes.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
        arr_v = (ctypes.c_uint64 * max(1, len(names)))(*[int(vars_[n]) for n in names])
        return arr_n, arr_v, len(names)

    def run(self, program: str, vars: dict | None = None) -> None:
        n, v, k = self._vars(vars)
        check(lib().kern_rt_run(self._h, program.encode(), n, v, k))

    def capture(self, program: str, vars: dict | None = None) -> None:
        n, v, k = self._vars(vars)
        check(lib().kern_rt_capture(self._h, program.encode(), n, v, k))

    def run_captured(self, program: str, vars: dict | None = None) -> None:
        n, v, k = self._vars(vars)
        check(lib().kern_rt_run_captured(self._h, program.encode(), n, v, k))

    def run_range(self, program: str, lo: int, hi: int, vars: dict | None = None) -> None:
        n, v, k = self._vars(vars)
        check(lib().kern_rt_run_range(self._h, program.encode(), n, v, k, lo, hi))

    def time_range(self, program: str, lo: int, hi: int, vars: dict | None = None, iters: int = 5) -> list:
        """Per-call GPU ms of calls [lo, hi), each the minimum over iters eager runs (harness.rs:209-250)."""
        n, v, k = self._vars(vars)
        out = (ctypes.c_float * max(1, hi - lo))()
        check(lib().kern_rt_time_range(self._h, program.encode(), n, v, k, lo, hi, iters, out))
        return [float(out[i]) for i in range(hi - lo)]

    def time_captured(self, program: str, vars: dict | None = None, iters: int = 10) -> float:
        n, v, k = self._vars(vars)
        ms = ctypes.c_float()
        check(lib().kern_rt_time_captured(self._h, program.encode(), n, v, k, iters, ctypes.byref(ms)))
        return ms.value

    def buffer(self, name: str) -> tuple[int, int]:
        ptr, n = P(), ctypes.c_size_t()
        check(lib().kern_rt_buffer(self._h, name.encode(), ctypes.byref(ptr), ctypes.byref(n)))
        return ptr.value or 0, n.value



def splice(manifest: dict | str, candidate: dict | str) -> dict:
    """candidate::splice (crates/kern-manifest/src/candidate.rs:152-185) through kern_candidate_splice: the
    manifest with the candidate's ops and modules in; KernError(KERN_ERR_MANIFEST) lists every misfit."""
    mt = manifest if isinstance(manifest, str) else json.dumps(manifest)
    ct = candidate if isinstance(candidate, str) else json.dumps(candidate)
    n = ctypes.c_size_t()
    check(lib().kern_candidate_splice(mt.encode(), ct.encode(), None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(lib().kern_candidate_splice(mt.encode(), ct.encode(), buf, n.value + 1, ctypes.byref(n)))
    return json.loads(buf.value.decode())


def _json_text(x) -> str:
    return x if isinstance(x, str) else json.dumps(x)


def _strings(xs) -> tuple:
    """A C array of NUL-terminated strings (and the encoded bytes it points into, to keep alive)."""
    enc = [x.encode() for x in xs]
    return (ctypes.c_char_p * max(1, len(enc)))(*enc), enc


def _candidate_call(fn, *args) -> dict:
    # size query, then the text
    n = ctypes.c_size_t()
    check(fn(*args, None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(fn(*args, buf, n.value + 1, ctypes.byref(n)))
    return json.loads(buf.value.decode())


def candidate_of(manifest: dict | str, ops: list) -> dict:
    """Candidate::of (crates/kern-manifest/src/candidate.rs:84-87) through kern_candidate_of: the manifest's
    own implementation of `ops`, with the modules they launch; an op the manifest lacks is left out."""
    arr, keep = _strings(ops)
    return _candidate_call(lib().kern_candidate_of, _json_text(manifest).encode(), ctypes.cast(arr, P), len(ops))


def candidate_only(candidate: dict | str, ops: list) -> dict:
    """Candidate::only (candidate.rs:89-97) through kern_candidate_only: the candidate cut down to `ops`."""
    arr, keep = _strings(ops)
    return _candidate_call(lib().kern_candidate_only, _json_text(candidate).encode(), ctypes.cast(arr, P), len(ops))


def candidate_join(candidates: list) -> dict:
    """Candidate::join (candidate.rs:99-113) through kern_candidate_join: the candidates as one;
    KernError(KERN_ERR_MANIFEST) when two implement the same op."""
    arr, keep = _strings([_json_text(c) for c in candidates])
    return _candidate_call(lib().kern_candidate_join, ctypes.cast(arr, P), len(candidates))


class _Piece(ctypes.Structure):
    _fields_ = [("candidate_json", ctypes.c_char_p), ("has_min", ctypes.c_int32), ("has_max", ctypes.c_int32),
                ("min", ctypes.c_uint64), ("max", ctypes.c_uint64)]


def candidate_tile(op: str, var: str, pieces: list) -> dict:
    """candidate::tile (candidate.rs:231-300) through kern_candidate_tile: one implementation of `op` from
    pieces (candidate, min, max), each running its candidate's implementation while `var` is in [min, max]
    (None = open end)."""
    texts = [_json_text(c).encode() for c, _, _ in pieces]
    arr = (_Piece * max(1, len(pieces)))()
    for i, ((_, lo, hi), t) in enumerate(zip(pieces, texts)):
        arr[i] = _Piece(t, lo is not None, hi is not None, lo or 0, hi or 0)
    return _candidate_call(lib().kern_candidate_tile, op.encode(), var.encode(), ctypes.cast(arr, P), len(pieces))


class Module:
    """A code object loaded through the module layer (kern_module_load: SHA-256 check, then hipModuleLoadData,
    the analog of crates/kern-runtime/src/cubin.rs:62-109), with its entries launched by kern_launch: the
    kernel-argument image is laid out at the offsets the code object's own metadata gives
    (kern_function_param_offsets / _sizes). Arguments: device tensors (8-byte addresses), ints (as the
    entry's 4- or 8-byte integer) and floats (f32)."""

    def __init__(self, path: str, sha256: str | None = None):
        with open(path, "rb") as f:
            self._img = f.read()
        h = P()
        check(lib().kern_module_load(self._img, len(self._img), None if sha256 is None else sha256.encode(),
                                     ctypes.byref(h)))
        self._h = h
        self._fns = {}

    def _fn(self, entry: str):
        if entry not in self._fns:
            f = P()
            check(lib().kern_module_function(self._h, entry.encode(), ctypes.byref(f)))
            sizes, offs, n = (ctypes.c_uint32 * 64)(), (ctypes.c_uint32 * 64)(), ctypes.c_int()
            check(lib().kern_function_param_sizes(f, sizes, 64, ctypes.byref(n)))
            check(lib().kern_function_param_offsets(f, offs, 64, ctypes.byref(n)))
            self._fns[entry] = (f, list(sizes[: n.value]), list(offs[: n.value]))
        return self._fns[entry]

    def launch(self, entry: str, grid, block, *args, shared: int = 0) -> None:
        import struct

        f, sizes, offs = self._fn(entry)
        if len(args) != len(sizes):
            raise KernError(4, f"{entry}: {len(args)} arguments, the code object declares {len(sizes)}")
        img = bytearray(max([o + s for o, s in zip(offs, sizes)] + [8]))
        for a, s, o in zip(args, sizes, offs):
            if isinstance(a, torch.Tensor):
                v = struct.pack("<Q", _ptr(a, entry).value)
            elif isinstance(a, float):
                v = struct.pack("<f", a)
            else:
                v = int(a).to_bytes(s, "little", signed=int(a) < 0)
            if len(v) != s:
                raise KernError(4, f"{entry}: argument of {len(v)} bytes where the code object has {s}")
            img[o: o + s] = v
        g = (ctypes.c_uint32 * 3)(*(list(grid) + [1, 1])[:3])
        b = (ctypes.c_uint32 * 3)(*(list(block) + [1, 1])[:3])
        buf = (ctypes.c_char * len(img)).from_buffer(img)
        check(lib().kern_launch(f, g, b, shared, _stream(), buf, len(img)))

    def close(self) -> None:
        for f, _, _ in self._fns.values():
            lib().kern_function_release(f)
        self._fns = {}
        if self._h:
            lib().kern_module_unload(self._h)
            self._h = None
