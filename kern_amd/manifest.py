"""Manifest ops of the MXFP4 matmul path with their `impl` pointed at this build's gfx950 module.

Each function returns one `ops` entry of a kern manifest (crates/kern-manifest/src/types.rs:970-1040):
the op's interface `params`, kept exactly as the reference declares them
(crates/kern-manifest/tests/fixtures/k3/head.json: moe_quant :25057, k3_moe_w_shuffle :26358,
k3_moe_sf_shuffle :26413, moe_routing :25117, moe_fc1 :25459, moe_fc2 :25683), and an `impl` whose
launches name module `kern_mx` (kernel_index/kern_mx.toml). Swapping a manifest's `impl` for these is
the module swap of candidate::splice (crates/kern-manifest/src/candidate.rs:1-26): calls and params do
not change. Shape constants a launch needs (hidden size, expert count, top-k) are literals of the launch,
as in the reference's own launches; `tokens` is the manifest var the grids read.

The grammar is the reference's: grids are Expr trees (types.rs:1517-1576), args LaunchArg
(types.rs:1174-1191). A launch arg cannot name a var directly, so the kernel arguments that are the var
`tokens` (moe_routing's token count, the dense ops' row count) travel as 4-byte packs, the form the
reference uses for struct-taking kernels (types.rs:1193-1260).
"""
from __future__ import annotations

import json

MODULE = "kern_mx"
BMM_THREADS = 512  # threads of one GEMM workgroup (8 waves)
MOE_WORKGROUPS = 256  # the MoE GEMMs are persistent: one workgroup per CU


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


def moe_quant(K: int) -> dict:
    """moe_quant(in bf16 x[T][K], out u8 q[T][K], out u8 sf[T][K/32], i32 T); launch adds i32 K.
    A 256-thread workgroup covers 4096 elements (16 per lane): grid ceil(T*K/8 / 512) = ceil(T*K / 4096)."""
    assert K % 32 == 0
    return {
        "params": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "i32"],
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_quant_bf16",
            "params": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "i32", "i32"],
            "block": [256, 1, 1],
            "grid": [{"ceil_div": [{"mul": ["tokens", K // 8]}, 512]}, 1, 1],
            "args": [{"param": 0}, {"param": 1}, {"param": 2}, {"param": 3}, {"i32": K}],
        }]},
    }


def k3_moe_w_shuffle(E: int, max_bytes: int) -> dict:
    """k3_moe_w_shuffle(in u8 raw, out u8 repacked, i32 rows, i32 row_bytes, i32 gated); launch prepends
    i32 E after the buffers. The grid covers the largest call, max_bytes = rows*row_bytes per expert (the
    kernel bounds-checks smaller ones), as the reference's fixed grid does."""
    return {
        "params": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32"],
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_w_shuffle",
            "params": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32", "i32"],
            "block": [256, 1, 1],
            "grid": [_ceil(E * max_bytes // 16, 256), 1, 1],
            "args": [{"param": 0}, {"param": 1}, {"i32": E}, {"param": 2}, {"param": 3}, {"param": 4}],
        }]},
    }


def k3_moe_sf_shuffle(E: int, max_bytes: int) -> dict:
    """k3_moe_sf_shuffle(in u8 raw, out u8 repacked, i32 rows, i32 sf_cols, i32 gated); launch prepends i32 E.
    The grid covers the largest call, max_bytes = rows*sf_cols per expert."""
    return {
        "params": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32"],
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_sf_shuffle",
            "params": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32", "i32"],
            "block": [256, 1, 1],
            "grid": [_ceil(E * max_bytes // 4, 256), 1, 1],
            "args": [{"param": 0}, {"param": 1}, {"i32": E}, {"param": 2}, {"param": 3}, {"param": 4}],
        }]},
    }


# moe_routing's chunked launches (kern_mx_routing_count/_scan/_rank) from this many expanded indices, over
# min(ROUTE_MAX_CHUNKS, ceil(tokens*topk / ROUTE_CHUNK)) workgroups; the C ABI's kern_moe_routing switches at
# the same point
ROUTE_CHUNKED_MIN, ROUTE_CHUNK, ROUTE_MAX_CHUNKS = 16384, 4096, 64


def moe_routing(topk: int, local_start: int, local_experts: int) -> dict:
    """moe_routing(in i32 topk_idx, out i32 counts, cta_batch, cta_limit, num_non_exiting, total_padded,
    route_map, exp2perm); launch adds the token count (var `tokens`), top-k and the local expert range.
    One workgroup below ROUTE_CHUNKED_MIN expanded indices, else count -> scan -> rank over chunks (the same
    tables bit for bit); `when` on `tokens` picks the launches."""
    bufs = ["in buffer<i32>"] + ["out buffer<i32>"] * 7
    first = _ceil(ROUTE_CHUNKED_MIN, topk)  # the least token count with tokens*topk >= ROUTE_CHUNKED_MIN
    args = [{"param": i} for i in range(8)] + [{"pack": {"size": 4, "fields": [{"at": 0, "var": "tokens"}]}},
                                               {"i32": topk}, {"i32": local_start}, {"i32": local_experts}]
    chunks = {"clamp": [{"ceil_div": [{"mul": ["tokens", topk]}, ROUTE_CHUNK]}, 0, ROUTE_MAX_CHUNKS]}

    def launch(entry, grid, when):
        return {"module": MODULE, "entry": entry, "params": bufs + ["bytes<4>", "i32", "i32", "i32"],
                "block": [1024, 1, 1], "grid": [grid, 1, 1], "when": {"var": "tokens", **when}, "args": args}

    return {
        "params": bufs,
        "impl": {"launches": [launch("kern_mx_routing", 1, {"max": first - 1}),
                              launch("kern_mx_routing_count", chunks, {"min": first}),
                              launch("kern_mx_routing_scan", 1, {"min": first}),
                              launch("kern_mx_routing_rank", chunks, {"min": first})]},
    }


def slot_bound(topk: int, experts: int) -> dict:
    """The reference's CTA-slot bound E + ceil(tokens*topk/128) (tools/kernels/abi/trtllm_bmm.py:58-60): the
    size of the cta_batch / cta_limit tables."""
    return {"add": [{"ceil_div": [{"mul": ["tokens", topk]}, 128]}, experts]}


def _slot_capacity(topk: int, experts: int) -> dict:
    # the capacity of the slot tables, the slot bound at the call's token count, as a 4-byte pack (a launch
    # arg cannot be an expression)
    return {"pack": {"size": 4, "fields": [{"at": 0, "expr": slot_bound(topk, experts)}]}}


def moe_fc1(m: int, k: int, experts: int, topk: int) -> dict:
    """moe_fc1 = trtllm_bmm_mxe4m3_mxe2m1_mxe4m3 (13 params); launch adds i32 m (= 2I), i32 k (= H), the slot
    tables' capacity E + ceil(tokens*topk/128) and a null f32 debug pointer (an i64 zero). The kernel is
    persistent: grid [256, 1, 1], and each workgroup loops over the live slots' tiles (num_non_exiting is
    read on the device), so the grid needs no var."""
    assert m % 256 == 0 and m <= 131072 and k % 512 == 0  # the kernels' tile lists hold m/256 < 512
    p = ["in buffer<u8>"] * 4 + ["out buffer<u8>"] * 2 + ["in buffer<i32>", "in buffer<f32>", "in buffer<f32>"] \
        + ["in buffer<i32>"] * 4
    return {
        "params": p,
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_bmm_fc1",
            "params": p + ["i32", "i32", "bytes<4>", "i64"],
            "block": [BMM_THREADS, 1, 1],
            "grid": [MOE_WORKGROUPS, 1, 1],
            "args": [{"param": i} for i in range(13)] + [{"i32": m}, {"i32": k}, _slot_capacity(topk, experts),
                                                         {"i64": 0}],
        }]},
    }


def moe_fc2(m: int, k: int, experts: int, topk: int) -> dict:
    """moe_fc2 = trtllm_bmm_bf16_mxe2m1_mxe4m3 (9 params); launch adds i32 m (= H), i32 k (= I), the slot
    tables' capacity, i32 sf_b_r128c4 = 1 (FC1 writes its scales R128c4) and a null f32 debug pointer.
    Persistent grid as moe_fc1."""
    assert m % 256 == 0 and m <= 131072 and k % 512 == 0  # the kernels' tile lists hold m/256 < 512
    p = ["in buffer<u8>"] * 4 + ["out buffer<bf16>"] + ["in buffer<i32>"] * 4
    return {
        "params": p,
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_bmm_fc2",
            "params": p + ["i32", "i32", "bytes<4>", "i32", "i64"],
            "block": [BMM_THREADS, 1, 1],
            "grid": [MOE_WORKGROUPS, 1, 1],
            "args": [{"param": i} for i in range(9)] + [{"i32": m}, {"i32": k}, _slot_capacity(topk, experts),
                                                        {"i32": 1}, {"i64": 0}],
        }]},
    }


def moe_finalize_rms(H: int, topk: int, eps: float = 1e-6) -> dict:
    """moe_finalize_rms(in bf16 fc2_out, in i32 exp2perm, in f32 topk_weight, in bf16 gamma, out bf16 out,
    i32 T); launch adds i32 H, i32 topk and f32 eps. One workgroup per token (grid.x = tokens) of one thread
    per 8-column chunk of the row, in whole waves (the block kern_moe_finalize_rms launches)."""
    assert H % 8 == 0 and H <= 8192
    p = ["in buffer<bf16>", "in buffer<i32>", "in buffer<f32>", "in buffer<bf16>", "out buffer<bf16>", "i32"]
    return {
        "params": p,
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_moe_finalize_rms",
            "params": p + ["i32", "i32", "f32"],
            "block": [_ceil(H // 8, 64) * 64, 1, 1],
            "grid": [{"mul": ["tokens", 1]}, 1, 1],
            "args": [{"param": i} for i in range(6)] + [{"i32": H}, {"i32": topk}, {"f32": eps}],
        }]},
    }


def cublaslt_mxfp8_tn(n: int, rows_var: str = "tokens") -> dict:
    """The op of crates/kern-runtime/tests/mxfp8_gemm.rs:46-50 (params a, w, c, a_scale, w_scale, m, n, k),
    whose reference impl is the runtime built-in `extern:cublaslt_mxfp8_tn`, as a kernel launch of
    kern_mx: grid [ceil(n/256), ceil(m/128)] of 512-thread workgroups with n a literal and m the var
    `rows_var` (a launch grid reads vars, not params); c's row stride is n."""
    p = ["in buffer<fp8e4m3>", "in buffer<fp8e4m3>", "out buffer<bf16>", "in buffer<u8>", "in buffer<u8>",
         "i32", "i32", "i32"]
    return {
        "params": p,
        "impl": {"launches": [{
            "module": MODULE, "entry": "kern_mx_gemm_mxfp8",
            "params": p + ["i32"],
            "block": [512, 1, 1],
            "grid": [_ceil(n, 256), {"ceil_div": [rows_var, 128]}, 1],
            "args": [{"param": i} for i in range(8)] + [{"i32": n}],
        }]},
    }


# The dense ops beside the MoE path, whose entry points choose a kernel by row count in host code
# (kern_mxfp4_gemv_bf16, kern_mxfp4_gemm_bf16, kern_moe_quant_routing), as manifest ops: the same choices as
# launches conditioned on the rows var by `when`, so that a manifest, and candidate tiling, sees them. The
# rows (M, tokens) reach the kernels from the var, as a 4-byte pack, so that the dynamic LDS sized from the
# var always matches the kernel's own count. The reference has no such ops (its dense MX GEMM is the
# runtime's built-in `extern:cublaslt_mxfp8_tn`).
GEMV_FIXED_NKT = (2, 4, 8, 14, 16)  # K / 512 with an unrolled kern_mx_gemv_bf16_r{K/512}
WALK_KTW = (1, 2, 4, 7, 8)          # K / 1024 with a persistent kern_mx_gemv_bf16_p* / kern_mx_gemm_bf16_s*
GEMV_MAX_ROWS = 16


def _rows(rows_var: str) -> dict:
    return {"pack": {"size": 4, "fields": [{"at": 0, "var": rows_var}]}}


def _gemv_launch(N: int, K: int, M: int, rows_var: str) -> dict:
    """The launch kern_mxfp4_gemv_bf16 makes for M rows of x [M][K] against weights [N][K/2] (capi.cpp)."""
    kg = K // 512
    params = ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>", "bytes<4>", "i32", "i32"]
    args = [{"param": i} for i in range(4)] + [_rows(rows_var), {"i32": N}, {"i32": K}]
    row_groups = [N // 16, 1, 1]
    if kg in GEMV_FIXED_NKT and 2 * M * K <= 144 * 1024 and (M <= 3 or N <= 8192):
        # one workgroup per 16-row group, each wave's x slice (2 * M * K bytes in all) in LDS
        return {"entry": f"kern_mx_gemv_bf16_r{kg}", "params": params, "block": [256, 1, 1], "grid": row_groups,
                "shared_mem": {"mul": [rows_var, 2 * K]}, "args": args}
    if M <= 2:
        gmax = _ceil(kg, 4)
        return {"entry": "kern_mx_gemv_bf16_rg", "params": params + ["i32"], "block": [256, 1, 1],
                "grid": row_groups, "shared_mem": {"mul": [rows_var, 4 * gmax * 1024]},
                "args": args + [{"i32": gmax}]}
    if K % 1024 == 0 and K // 1024 in WALK_KTW:
        H = N // 8
        hb = min(9, _ceil(H, 256))
        return {"entry": f"kern_mx_gemv_bf16_p{K // 1024}", "params": params + ["i32"], "block": [512, 1, 1],
                "grid": [_ceil(H, hb), 1, 1], "args": args + [{"i32": hb}]}
    # any other shape: x staged in slices of sb k-tiles per wave, nb k-tiles of weights in flight together
    sb = next(c for c in range(min(kg, GEMV_MAX_ROWS // M), 0, -1) if kg % c == 0)
    nb = next((c for c in (7, 4, 2) if sb % c == 0), 1)
    return {"entry": "kern_mx_gemv_bf16", "params": params + ["i32", "i32"], "block": [256, 1, 1],
            "grid": row_groups, "shared_mem": M * (sb * 1024 + 16) + kg * 256, "args": args + [{"i32": nb}, {"i32": sb}]}


def _by_rows(launch_at, rows_var: str, lo: int, hi: int) -> list:
    """Launches for rows lo..hi: launch_at(M) at each M, each run of equal launches merged into one launch whose
    `when` covers the run (min and max both given, so nothing runs outside lo..hi)."""
    out = []
    for M in range(lo, hi + 1):
        L = {"module": MODULE, **launch_at(M)}
        if out and json.dumps({k: v for k, v in out[-1].items() if k != "when"}, sort_keys=True) == \
                json.dumps(L, sort_keys=True):
            out[-1]["when"]["max"] = M
        else:
            out.append({**L, "when": {"var": rows_var, "min": M, "max": M}})
    return out


def mxfp4_gemv_bf16(N: int, K: int, rows_var: str = "tokens") -> dict:
    """The W4A16 decode GEMV (C ABI kern_mxfp4_gemv_bf16): in bf16 x [M][K], in u8 w [N][K/2] and w_sf
    (repacked), out bf16 y [M][N]; M = the value of `rows_var`, 1..16 (no launch runs past 16). One launch
    per run of M that takes the same kernel: the unrolled row-group kernel while its x slices fit, the
    persistent walk above, as the C ABI chooses."""
    assert N % 16 == 0 and K % 512 == 0 and K <= 16384
    return {"params": ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>"],
            "impl": {"launches": _by_rows(lambda M: _gemv_launch(N, K, M, rows_var), rows_var, 1, GEMV_MAX_ROWS)}}


def mxfp4_gemm_bf16(N: int, K: int, rows_var: str = "tokens") -> dict:
    """The dense MXFP4 x MXFP8 GEMM with bf16 out (C ABI kern_mxfp4_gemm_bf16): in u8 a [N][K/2], sf_a (the
    repacked weights), b [M][K] and sf_b (MXFP8 activations, linear scales), out bf16 c [M][N]; M = the value
    of `rows_var`. Up to 64 rows the persistent walk over the weights (K = 1024 * {1, 2, 4, 7, 8}), else
    the tiled GEMM, grid [N/256, ceil(M/128)]; both with a null f32 debug pointer."""
    assert N % 256 == 0 and K % 512 == 0
    p = ["in buffer<u8>"] * 4 + ["out buffer<bf16>"]
    tiled = {"module": MODULE, "entry": "kern_mx_gemm_bf16", "params": p + ["bytes<4>", "i32", "i32", "i64"],
             "block": [BMM_THREADS, 1, 1], "grid": [N // 256, {"ceil_div": [rows_var, 128]}, 1],
             "args": [{"param": i} for i in range(5)] + [_rows(rows_var), {"i32": N}, {"i32": K}, {"i64": 0}]}
    if not (K % 1024 == 0 and K // 1024 in WALK_KTW):
        return {"params": p, "impl": {"launches": [tiled]}}
    H = N // 8
    hb = min(9, _ceil(H, 256))
    walk = {"module": MODULE, "entry": f"kern_mx_gemm_bf16_s{K // 1024}",
            "params": p + ["i64", "bytes<4>", "i32", "i32", "i32"], "block": [512, 1, 1], "grid": [_ceil(H, hb), 1, 1],
            "when": {"var": rows_var, "max": 64},
            "args": [{"param": i} for i in range(5)] + [{"i64": 0}, _rows(rows_var), {"i32": N}, {"i32": K},
                                                        {"i32": hb}]}
    return {"params": p, "impl": {"launches": [walk, {**tiled, "when": {"var": rows_var, "min": 65}}]}}


def mxfp4_gemm_e4m3(N: int, K: int, rows_var: str = "tokens") -> dict:
    """The dense MXFP4 x MXFP8 GEMM with per-tensor e4m3 out (C ABI kern_mxfp4_gemm_e4m3, config 3's prefill
    GEMM): in u8 a [N][K/2], sf_a (repacked weights), b [M][K], sf_b (MXFP8 activations), out u8 c [M][N] =
    e4m3(acc * d_scale[0]), in f32 d_scale [1]; M = the value of `rows_var`. One tiled launch, grid
    [N/256, ceil(M/128)], with a null f32 debug pointer."""
    assert N % 256 == 0 and K % 512 == 0
    p = ["in buffer<u8>"] * 4 + ["out buffer<u8>", "in buffer<f32>"]
    return {"params": p, "impl": {"launches": [{
        "module": MODULE, "entry": "kern_mx_gemm_e4m3", "params": p + ["bytes<4>", "i32", "i32", "i64"],
        "block": [BMM_THREADS, 1, 1], "grid": [N // 256, {"ceil_div": [rows_var, 128]}, 1],
        "args": [{"param": i} for i in range(6)] + [_rows(rows_var), {"i32": N}, {"i32": K}, {"i64": 0}]}]}}


QUANT_ROUTING_WORKGROUPS = 255  # quantizer workgroups the fused launch holds (one round beside the routing block)


def moe_quant_routing(K: int, topk: int, local_start: int, local_experts: int) -> dict:
    """moe_quant and moe_routing in one op (C ABI kern_moe_quant_routing): in bf16 x [T][K], out u8 q, sf,
    in i32 topk_idx, out the seven routing tables; T = the var `tokens`. While the quantizer's workgroups
    (T * K/16 elements / 1024 lanes) fit in one round beside the routing workgroup, one launch does both
    (kern_mx_quant_routing); past that, moe_routing's launches and then moe_quant's, as the C ABI does.
    Bit for bit the outputs of the two ops."""
    assert K % 32 == 0
    fused_max = (QUANT_ROUTING_WORKGROUPS * 1024) // (K // 16)  # the most tokens with qwg <= 255
    qwg = {"ceil_div": [{"mul": ["tokens", K // 16]}, 1024]}
    rbufs = [{"param": i} for i in range(3, 11)]  # topk_idx and the seven tables: moe_routing's eight params
    fused = {"module": MODULE, "entry": "kern_mx_quant_routing",
             "params": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "i32", "in buffer<i32>"] +
                       ["out buffer<i32>"] * 7 + ["bytes<4>", "i32", "i32", "i32"],
             "block": [1024, 1, 1], "grid": [{"add": [qwg, 1]}, 1, 1],
             "when": {"var": "tokens", "max": fused_max},
             "args": [{"param": 0}, {"param": 1}, {"param": 2}, {"i32": K}] + rbufs +
                     [_rows("tokens"), {"i32": topk}, {"i32": local_start}, {"i32": local_experts}]}
    past = {"var": "tokens", "min": fused_max + 1}
    routing = moe_routing(topk, local_start, local_experts)["impl"]["launches"]
    quant = moe_quant(K)["impl"]["launches"][0]
    split = []
    for L in routing:  # each routing launch, its own `when` narrowed to the tokens past the fused launch
        w = dict(L.get("when", {"var": "tokens"}))
        w["min"] = max(w.get("min", 0), past["min"])
        if "max" in w and w["max"] < w["min"]:
            continue
        split.append({**L, "args": [rbufs[i] if "param" in a else a for i, a in enumerate(L["args"])], "when": w})
    q = {**quant, "when": past, "args": [{"param": 0}, {"param": 1}, {"param": 2}, _rows("tokens"), {"i32": K}],
         "params": quant["params"][:3] + ["bytes<4>", "i32"]}
    return {"params": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "in buffer<i32>"] +
                      ["out buffer<i32>"] * 7,
            "impl": {"launches": [fused] + split + [q]}}


def _fill(entry: str, params: list, launch_params: list, args: list, n: int) -> dict:
    return {"params": params, "impl": {"launches": [{
        "module": MODULE, "entry": entry, "params": launch_params, "block": [256, 1, 1],
        "grid": [_ceil(n, 256), 1, 1], "args": args}]}}


def fill_i32(n: int) -> dict:
    """fill_i32(out i32 p, i32 v): p[0..n) = v (weight_prep.cu kern_fill_i32, n a launch literal)."""
    return _fill("kern_fill_i32", ["out buffer<i32>", "i32"], ["out buffer<i32>", "i32", "i32"],
                 [{"param": 0}, {"i32": n}, {"param": 1}], n)


def fill_f32(n: int) -> dict:
    """fill_f32(out f32 p, f32 v): p[0..n) = v."""
    return _fill("kern_fill_f32", ["out buffer<f32>", "f32"], ["out buffer<f32>", "i32", "f32"],
                 [{"param": 0}, {"i32": n}, {"param": 1}], n)


def fill_bf16(n: int, v: float) -> dict:
    """fill_bf16(out bf16 p): p[0..n) = bf16(v), v a launch literal (K3's k3_weight_prep kern_fill_bf16)."""
    return _fill("kern_fill_bf16", ["out buffer<bf16>"], ["out buffer<bf16>", "i32", "f32"],
                 [{"param": 0}, {"i32": n}, {"f32": v}], n)


def moe_ops(H: int, I: int, E: int, topk: int, local_start: int = 0) -> dict:
    """The ops of one MoE layer (hidden H, intermediate I, E local experts, top-k) as `ops` entries."""
    return {
        "moe_quant": moe_quant(H),
        "k3_moe_w_shuffle": k3_moe_w_shuffle(E, max(2 * I * H // 2, H * I // 2)),
        "k3_moe_sf_shuffle": k3_moe_sf_shuffle(E, max(2 * I * H // 32, H * I // 32)),
        "moe_routing": moe_routing(topk, local_start, E),
        "moe_fc1": moe_fc1(2 * I, H, E, topk),
        "moe_fc2": moe_fc2(H, I, E, topk),
        "moe_finalize_rms": moe_finalize_rms(H, topk),
    }


# K3's MoE shapes (crates/kern-manifest/tests/fixtures/k3/head.json): hidden (latent) 3584, intermediate 3072,
# 224 experts on the one rank of its EP1 prefill stage, top-16
K3_H, K3_I, K3_E, K3_TOPK = 3584, 3072, 224, 16


def candidate(ops: dict, sha256: str, source: str = "kern_mx.hsaco") -> dict:
    """A Candidate {modules, ops} (crates/kern-manifest/src/candidate.rs:34-44): implementations of a manifest's
    ops, each under the op's name and with its params, and the module they launch (this build's code object,
    pinned by sha256; `source` is its file name under the runtime's kernels_dir)."""
    return {"modules": {MODULE: {"source": source, "sha256": sha256}}, "ops": ops}


def k3_moe_candidate(sha256: str, source: str = "kern_mx.hsaco") -> dict:
    """The candidate for one K3 MoE layer: the path's ops (moe_quant, moe_routing, moe_fc1, moe_fc2,
    moe_finalize_rms, k3_moe_w_shuffle, k3_moe_sf_shuffle) and the `fill_f32` of its load program (SiTU
    alpha / beta over the 224 experts) at K3's shapes, all on kern_mx. Spliced into a K3 manifest
    (kern_candidate_splice), every call of the manifest runs on gfx950 unchanged."""
    ops = moe_ops(K3_H, K3_I, K3_E, K3_TOPK)
    ops["fill_f32"] = fill_f32(K3_E)
    return candidate(ops, sha256, source)


def moe_layer_manifest(H: int, I: int, E: int, topk: int, max_tokens: int, sha256: str,
                       source: str = "kern_mx.hsaco", eps: float = 1e-6) -> dict:
    """A whole kern manifest (types.rs:69-97) for one MoE layer of the path on kern_mx, run by the program
    runtime (kern_rt_*): var `tokens`; raw expert weights as `source` buffers that the `derive_weights`
    program repacks into `carry` buffers (the K3 derive of head.json:28670); `moe_layer` (launch by launch)
    and `moe_layer_graph` (hipGraph) = quant -> routing -> FC1 -> FC2 -> finalize_rms, input bf16 `x`,
    `topk_ids`, `topk_weight`, output bf16 `y`. Table and activation buffers are sized for max_tokens."""
    slots = E + _ceil(max_tokens * topk, 128)
    rows = slots * 128
    T = "tokens"

    def buf(dtype, shape, kind):
        return {"dtype": dtype, "shape": shape, "kind": kind}

    sf1_bytes = (rows // 128) * 512 * _ceil(I // 32, 4)
    buffers = {
        "x": buf("bf16", [T, H], "input"),
        "topk_ids": buf("i32", [T, topk], "input"),
        "topk_weight": buf("f32", [T, topk], "input"),
        "y": buf("bf16", [T, H], "output"),
        "gamma": buf("bf16", [H], "weight"),
        "alpha": buf("f32", [E], "weight"),
        "beta": buf("f32", [E], "weight"),
        "w13_raw": buf("u8", [E, 2 * I, H // 2], "source"),
        "s13_raw": buf("u8", [E, 2 * I, H // 32], "source"),
        "w2_raw": buf("u8", [E, H, I // 2], "source"),
        "s2_raw": buf("u8", [E, H, I // 32], "source"),
        "w13": buf("u8", [E, 2 * I, H // 2], "carry"),
        "s13": buf("u8", [E, 2 * I, H // 32], "carry"),
        "w2": buf("u8", [E, H, I // 2], "carry"),
        "s2": buf("u8", [E, H, I // 32], "carry"),
        "q": buf("u8", [T, H], "workspace"),
        "qs": buf("u8", [T, H // 32], "workspace"),
        "counts": buf("i32", [2 * E], "workspace"),
        "cta_batch": buf("i32", [slots], "workspace"),
        "cta_limit": buf("i32", [slots], "workspace"),
        "num_non_exiting": buf("i32", [1], "workspace"),
        "total_padded": buf("i32", [1], "workspace"),
        "route_map": buf("i32", [rows], "workspace"),
        "exp2perm": buf("i32", [T, topk], "workspace"),
        "c1": buf("u8", [rows, I], "workspace"),
        "sf1": buf("u8", [sf1_bytes], "workspace"),
        "c2": buf("bf16", [rows, H], "workspace"),
    }
    ops = moe_ops(H, I, E, topk)
    ops["moe_finalize_rms"] = moe_finalize_rms(H, topk, eps)
    b = lambda n: {"buf": n}  # noqa: E731
    i32 = lambda v: {"i32": v}  # noqa: E731
    tables = [b(n) for n in ("counts", "cta_batch", "cta_limit", "num_non_exiting", "total_padded", "route_map",
                             "exp2perm")]
    layer = [
        {"label": "quant", "op": "moe_quant", "args": [b("x"), b("q"), b("qs"), {"var": T}]},
        {"label": "routing", "op": "moe_routing", "args": [b("topk_ids")] + tables},
        {"label": "fc1", "op": "moe_fc1",
         "args": [b("w13"), b("s13"), b("q"), b("qs"), b("c1"), b("sf1"), b("route_map"), b("alpha"), b("beta"),
                  b("num_non_exiting"), b("total_padded"), b("cta_batch"), b("cta_limit")]},
        {"label": "fc2", "op": "moe_fc2",
         "args": [b("w2"), b("s2"), b("c1"), b("sf1"), b("c2"), b("num_non_exiting"), b("total_padded"),
                  b("cta_batch"), b("cta_limit")]},
        {"label": "finalize", "op": "moe_finalize_rms",
         "args": [b("c2"), b("exp2perm"), b("topk_weight"), b("gamma"), b("y"), {"var": T}]},
    ]
    derive = [
        {"label": "w13", "op": "k3_moe_w_shuffle", "args": [b("w13_raw"), b("w13"), i32(2 * I), i32(H // 2), i32(1)]},
        {"label": "s13", "op": "k3_moe_sf_shuffle", "args": [b("s13_raw"), b("s13"), i32(2 * I), i32(H // 32), i32(1)]},
        {"label": "w2", "op": "k3_moe_w_shuffle", "args": [b("w2_raw"), b("w2"), i32(H), i32(I // 2), i32(0)]},
        {"label": "s2", "op": "k3_moe_sf_shuffle", "args": [b("s2_raw"), b("s2"), i32(H), i32(I // 32), i32(0)]},
    ]
    return {
        "schema_version": 7,
        "model": f"moe layer H={H} I={I} E={E} top-{topk}",
        "vars": {T: {"max": max_tokens, "axis": "rows"}},
        "buffers": buffers,
        "modules": {MODULE: {"source": source, "sha256": sha256}},
        "ops": ops,
        "programs": {
            "derive_weights": {"derive": True, "calls": derive},
            "moe_layer": {"calls": layer},
            "moe_layer_graph": {"graph": True, "calls": layer},
        },
    }

