"""Manifest-op layer of the C ABI (kern_op_*), host side: no device is touched.

The ops come from kern_amd.manifest (the path's six ops with their impl pointed at kern_mx). Their
interface params are pinned to the reference's K3 manifest (tests/golden/k3_op_interfaces.json, taken
from crates/kern-manifest/tests/fixtures/k3/head.json by tests/golden/make_k3_interfaces.py). Grid
expressions are checked against their closed forms (crates/kern-manifest/src/types.rs:1517-1576) and the
kernel-argument images against an independent packing of the AMDGPU layout.
"""
import json
import os
import struct

import pytest

from kern_amd import manifest as mf

HERE = os.path.dirname(os.path.abspath(__file__))
ops = pytest.importorskip("kern_amd.ops")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ops.LIB_PATH):
        pytest.skip("library not built")
    return ops.lib()


def golden():
    with open(os.path.join(HERE, "golden", "k3_op_interfaces.json")) as f:
        return json.load(f)["ops"]


def pack(fields):
    """AMDGPU kernel-argument image: (format, value) pairs, each at its natural alignment, padded to 8."""
    out = b""
    for fmt, v in fields:
        size = struct.calcsize("<" + fmt)
        out += b"\0" * (-len(out) % size)
        out += struct.pack("<" + fmt, v)
    return out + b"\0" * (-len(out) % 8)


# K3 (the reference's own shapes) and config 4 (E = 256, top-8, H = 7168, I = 2048)
SHAPES = [dict(H=3584, I=3072, E=224, k=16), dict(H=7168, I=2048, E=256, k=8)]


@pytest.mark.parametrize("shape", SHAPES)
def test_interfaces_match_reference(shape):
    g = golden()
    o = mf.moe_ops(shape["H"], shape["I"], shape["E"], shape["k"])
    for name, rec in g.items():
        if name in o:
            assert o[name]["params"] == rec["params"], name


def test_k3_fill_launches_are_the_references_with_the_module_swapped():
    # the once-program fills of K3: same entry, launch params, literal args, grid and block
    g = golden()
    for name, op in [("fill_i32", mf.fill_i32(1)), ("fill_f32", mf.fill_f32(224)), ("fill_bf16", mf.fill_bf16(1, 1.0))]:
        launch, rec = op["impl"]["launches"][0], g[name]
        assert op["params"] == rec["params"], name
        assert launch["module"] == "kern_mx"
        assert (launch["entry"], launch["params"], launch["args"], launch["grid"], launch["block"]) == \
            (rec["entry"], rec["launch_params"], rec["args"], rec["grid"], rec["block"]), name


def test_k3_grids_match_reference():
    g = golden()
    o = mf.moe_ops(3584, 3072, 224, 16)
    # the weight repack: one thread per 16-byte slot, as the reference's fixed grid
    assert o["k3_moe_w_shuffle"]["impl"]["launches"][0]["grid"] == g["k3_moe_w_shuffle"]["grid"]
    # the reference launches both GEMMs over [m/256, E + ceil(tokens*topk/128)]; ours are persistent (one
    # workgroup per CU, looping over the live slots on the device), and the slot bound sizes the tables
    for name in ("moe_fc1", "moe_fc2"):
        assert mf.slot_bound(16, 224) == g[name]["grid"][1], name
        assert o[name]["impl"]["launches"][0]["grid"] == [256, 1, 1], name
    # one workgroup per token for the finalize, as the reference launches it
    assert o["moe_finalize_rms"]["impl"]["launches"][0]["grid"] == g["moe_finalize_rms"]["grid"]


@pytest.mark.parametrize("T", [1, 37, 512, 1023, 1024, 8192])
@pytest.mark.parametrize("shape", SHAPES)
def test_plan_grids_and_kernargs(lib, shape, T):
    H, I, E, k = shape["H"], shape["I"], shape["E"], shape["k"]
    o = mf.moe_ops(H, I, E, k)
    v = {"tokens": T}
    bufs = lambda n: [0x1000 * (i + 1) for i in range(n)]

    p = ops.op_plan(o["moe_quant"], 0, bufs(3) + [T], v)
    assert p["grid"] == (-(-T * H // 8 // 512), 1, 1) and p["block"] == (256, 1, 1)
    assert p["args"] == pack([("Q", 0x1000), ("Q", 0x2000), ("Q", 0x3000), ("i", T), ("i", H)])

    # one workgroup below 16384 expanded indices, else count / scan / rank over min(64, ceil(T*k / 4096))
    chunked = T * k >= 16384
    G = min(64, -(-T * k // 4096))
    for j, grid in enumerate([1, G, 1, G]):
        p = ops.op_plan(o["moe_routing"], j, bufs(8), v)
        assert p["skip"] == ((j > 0) != chunked), (j, T * k)
        if not p["skip"]:
            assert p["grid"] == (grid, 1, 1) and p["block"] == (1024, 1, 1)
            assert p["args"] == pack([("Q", 0x1000 * (i + 1)) for i in range(8)] +
                                     [("i", T), ("i", k), ("i", 0), ("i", E)])

    p = ops.op_plan(o["moe_fc1"], 0, bufs(13), v)
    assert p["grid"] == (256, 1, 1) and p["block"] == (512, 1, 1)
    slots = E + -(-T * k // 128)  # the slot tables' capacity at this token count
    assert p["args"] == pack([("Q", 0x1000 * (i + 1)) for i in range(13)] + [("i", 2 * I), ("i", H), ("i", slots),
                                                                             ("q", 0)])

    p = ops.op_plan(o["moe_fc2"], 0, bufs(9), v)
    assert p["grid"] == (256, 1, 1)
    assert p["args"] == pack([("Q", 0x1000 * (i + 1)) for i in range(9)] + [("i", H), ("i", I), ("i", slots), ("i", 1),
                                                                            ("q", 0)])

    p = ops.op_plan(o["moe_finalize_rms"], 0, bufs(5) + [T], v)
    assert p["grid"] == (T, 1, 1) and p["block"] == (-(-H // 8 // 64) * 64, 1, 1)
    assert p["args"] == pack([("Q", 0x1000 * (i + 1)) for i in range(5)] + [("i", T), ("i", H), ("i", k), ("f", 1e-6)])

    for name, rows, rb, gated in [("k3_moe_w_shuffle", 2 * I, H // 2, 1), ("k3_moe_sf_shuffle", H, I // 32, 0)]:
        p = ops.op_plan(o[name], 0, bufs(2) + [rows, rb, gated], v)
        assert p["args"] == pack([("Q", 0x1000), ("Q", 0x2000), ("i", E), ("i", rows), ("i", rb), ("i", gated)])


def _probe(grid_x, when=None, args=None, params=None, extra=None):
    launch = {"module": "kern_mx", "entry": "e", "params": params or ["i32"], "block": [64, 1, 1],
              "grid": [grid_x, 1, 1], "args": args if args is not None else [{"i32": 7}]}
    if when:
        launch["when"] = when
    launch.update(extra or {})
    return {"params": [], "impl": {"launches": [launch]}}


@pytest.mark.parametrize("tokens", [0, 1, 127, 128, 129, 4096, 5000, 8192, 9000])
def test_expr_closed_forms(lib, tokens):
    # Expr::eval (types.rs:1560-1576): ceil_div, mul, add, clamp(e, start, len) = min(max(e - start, 0), len)
    cases = [({"ceil_div": ["tokens", 128]}, -(-tokens // 128)),
             ({"mul": ["tokens", 16]}, tokens * 16),
             ({"add": [{"ceil_div": [{"mul": ["tokens", 16]}, 128]}, 224]}, 224 + -(-tokens * 16 // 128)),
             ({"clamp": ["tokens", 4096, 4096]}, min(max(tokens - 4096, 0), 4096)),
             (5, 5)]
    for expr, want in cases:
        p = ops.op_plan(_probe(expr), 0, [], {"tokens": tokens})
        assert p["grid"][0] == want, expr


@pytest.mark.parametrize("tokens,skip", [(3, True), (4, False), (16, False), (17, True)])
def test_when_range(lib, tokens, skip):
    p = ops.op_plan(_probe(1, when={"var": "tokens", "min": 4, "max": 16}), 0, [], {"tokens": tokens})
    assert p["skip"] is skip


def test_pack_fields_and_scalars(lib):
    op = {"params": ["in buffer<f32>", "f32", "i64", "u8"],
          "impl": {"launches": [{"module": "kern_mx", "entry": "e",
                                 "params": ["bytes<24>", "f32", "i64", "u8", "f32"], "block": [64, 1, 1],
                                 "grid": [1, 1, 1],
                                 "args": [{"pack": {"size": 24, "fields": [
                                     {"at": 0, "param": 0}, {"at": 8, "var": "tokens"},
                                     {"at": 12, "expr": {"mul": ["tokens", 3]}}, {"at": 16, "i64": -2},
                                 ]}}, {"param": 1}, {"param": 2}, {"param": 3}, {"f32": 0.5}]}]}}
    p = ops.op_plan(op, 0, [0xABCDEF00, 1.25, -5, 200], {"tokens": 11})
    img = struct.pack("<QIIq", 0xABCDEF00, 11, 33, -2)  # bytes<24>, aligned to 8
    img += struct.pack("<f", 1.25) + b"\0" * 4 + struct.pack("<q", -5) + struct.pack("<B", 200)
    img += b"\0" * 3 + struct.pack("<f", 0.5)
    img += b"\0" * (-len(img) % 8)
    assert p["args"] == img


BAD = [
    ("not json", "{", 1),
    ("extern launch", {"params": [], "impl": {"launches": [{"entry": "extern:cublaslt_bf16_tn", "block": [1, 1, 1],
                                                             "grid": [1, 1, 1]}]}}, 1),
    ("cluster", _probe(1, extra={"cluster": [2, 1, 1]}), 1),
    ("pdl", _probe(1, extra={"pdl": True}), 1),
    ("unknown key", _probe(1, extra={"stream": 3}), 1),
    ("block too big", _probe(1, extra={"block": [1024, 2, 1]}), 1),
    ("arg count", _probe(1, args=[]), 1),
    ("literal kind", _probe(1, args=[{"i64": 3}]), 1),
    ("scratch", _probe(1, params=["in buffer<u8>"], args=[{"scratch": "s"}]), 1),
    ("tensormap", _probe(1, params=["bytes<128>"], args=[{"pack": {"size": 128, "fields": [
        {"at": 0, "tensormap": {"param": 0}}]}}]), 1),
    ("pack overflow", _probe(1, params=["bytes<8>"], args=[{"pack": {"size": 8, "fields": [
        {"at": 4, "i64": 1}]}}]), 1),
    ("pack size", _probe(1, params=["bytes<8>"], args=[{"pack": {"size": 16, "fields": []}}]), 1),
    ("bad expr", _probe({"div": ["tokens", 2]}), 1),
]


@pytest.mark.parametrize("name,op,code", BAD, ids=[b[0] for b in BAD])
def test_malformed_ops_rejected(lib, name, op, code):
    with pytest.raises(ops.KernError) as e:
        ops.op_plan(op, 0, [], {"tokens": 1})
    assert e.value.code == code, str(e.value)


def test_dtype_and_direction_checks(lib):
    base = {"params": ["in buffer<u8>", "out buffer<bf16>"],
            "impl": {"launches": [{"module": "kern_mx", "entry": "e", "block": [64, 1, 1], "grid": [1, 1, 1],
                                   "params": ["in buffer<u8>", "out buffer<bf16>"],
                                   "args": [{"param": 0}, {"param": 1}]}]}}
    ops.op_plan(base, 0, [1, 2], {})  # consistent
    bad_dtype = json.loads(json.dumps(base))
    bad_dtype["impl"]["launches"][0]["params"][1] = "out buffer<f32>"
    bad_write = json.loads(json.dumps(base))
    bad_write["impl"]["launches"][0]["params"][0] = "out buffer<u8>"
    bad_read = json.loads(json.dumps(base))
    bad_read["impl"]["launches"][0]["params"][1] = "in buffer<bf16>"
    for op, msg in [(bad_dtype, "does not match"), (bad_write, "writes through interface `in`"),
                    (bad_read, "read before any launch wrote it")]:
        with pytest.raises(ops.KernError) as e:
            ops.op_plan(op, 0, [1, 2], {})
        assert e.value.code == 1 and msg in str(e.value)


def test_call_errors(lib):
    o = mf.moe_ops(7168, 2048, 256, 8)
    with pytest.raises(ops.KernError) as e:  # a grid var that is not bound
        ops.op_plan(o["moe_quant"], 0, [1] * 4, {})
    assert e.value.code == 7 and "unknown var `tokens`" in str(e.value)
    with pytest.raises(ops.KernError) as e:  # wrong number of interface params
        ops.op_plan(o["moe_fc2"], 0, [1] * 8, {"tokens": 1})
    assert e.value.code == 4
    tall = mf.moe_fc2(7168, 2048, 256, 8)
    tall["impl"]["launches"][0]["grid"] = [1, mf.slot_bound(8, 256), 1]
    with pytest.raises(ops.KernError) as e:  # grid.y beyond the launch limit
        ops.op_plan(tall, 0, [1] * 9, {"tokens": 1 << 20})
    assert e.value.code == 7 and "exceeds the launch limit" in str(e.value)


def test_ring_activations_past_4gib_are_refused(lib):
    """The LDS-ring GEMMs address activations by 32-bit byte offsets: a launch whose evaluated activation
    extent (FC2: max_slots * 128 rows x k) reaches 4 GiB is refused, as the direct C-ABI entry refuses it."""
    o = mf.moe_ops(7168, 2048, 256, 8)
    params = [0x1000] * 9
    ops.op_plan(o["moe_fc2"], 0, params, {"tokens": 8192})
    # (256 + ceil(tokens * 8 / 128)) * 128 * 2048 >= 2^32 from tokens = 258048 on
    with pytest.raises(ops.KernError) as e:
        ops.op_plan(o["moe_fc2"], 0, params, {"tokens": 258048})
    assert "4 GiB" in str(e.value)
    ops.op_plan(o["moe_fc2"], 0, params, {"tokens": 258047 - 15})


def _runs(op, nparams, v):
    """(entry, plan) of each launch of op that runs at vars v."""
    out = []
    for i, L in enumerate(op["impl"]["launches"]):
        p = ops.op_plan(op, i, [0x1000 * (j + 1) for j in range(nparams)], v)
        if not p["skip"]:
            out.append((L["entry"], p))
    return out


@pytest.mark.parametrize("N,K", [(18432, 7168), (7168, 8192), (2048, 3584), (512, 1024), (1040, 16384)])
def test_gemv_op_plans_one_launch_per_row_count(lib, N, K):
    """The GEMV op's launches tile rows 1..16: at each M exactly one runs, its dynamic LDS fits gfx950's
    160 KiB, and the kernel's M (after the four buffers) is the var's value; past 16 none runs."""
    op = mf.mxfp4_gemv_bf16(N, K)
    for M in range(1, 18):
        r = _runs(op, 4, {"tokens": M})
        if M > mf.GEMV_MAX_ROWS:
            assert r == [], M
            continue
        assert len(r) == 1, (M, [e for e, _ in r])
        entry, p = r[0]
        assert entry.startswith("kern_mx_gemv_bf16") and p["shared"] <= 163840, (M, entry, p["shared"])
        assert struct.unpack_from("<i", p["args"], 32)[0] == M and struct.unpack_from("<ii", p["args"], 36) == (N, K)


def test_dense_gemm_op_plans(lib):
    op = mf.mxfp4_gemm_bf16(9216, 7168)
    for M, entry, m_at in [(1, "kern_mx_gemm_bf16_s7", 48), (64, "kern_mx_gemm_bf16_s7", 48),
                           (65, "kern_mx_gemm_bf16", 40), (4096, "kern_mx_gemm_bf16", 40)]:
        (e, p), = _runs(op, 5, {"tokens": M})
        assert e == entry and struct.unpack_from("<i", p["args"], m_at)[0] == M, M
        if e == "kern_mx_gemm_bf16":
            assert p["grid"] == (9216 // 256, -(-M // 128), 1)
    (e, _), = _runs(mf.mxfp4_gemm_bf16(2048, 3584), 5, {"tokens": 8})  # K = 3584: no walk instance
    assert e == "kern_mx_gemm_bf16"
    (e, p), = _runs(mf.mxfp4_gemm_e4m3(2048, 7168), 6, {"tokens": 4096})
    assert e == "kern_mx_gemm_e4m3" and p["grid"] == (8, 32, 1) and struct.unpack_from("<iii", p["args"], 48) == \
        (4096, 2048, 7168)


def test_quant_routing_op_plans(lib):
    """One launch while the quantizer's workgroups fit beside the routing workgroup, then moe_routing's
    launches and moe_quant's, each with its own grid at that token count."""
    K, k = 7168, 8
    op = mf.moe_quant_routing(K, k, 0, 256)
    fused_max = 255 * 1024 // (K // 16)
    (e, p), = _runs(op, 11, {"tokens": fused_max})
    assert e == "kern_mx_quant_routing" and p["grid"][0] == 1 + -(-fused_max * (K // 16) // 1024) == 256
    for T in (fused_max + 1, 2048, 8192):
        got = [e for e, _ in _runs(op, 11, {"tokens": T})]
        want = [e for e, _ in _runs(mf.moe_routing(k, 0, 256), 8, {"tokens": T})] + ["kern_mx_quant_bf16"]
        assert got == want, T


@pytest.mark.parametrize("op,block,ok", [
    (mf.moe_fc2(1024, 512, 8, 2), [256, 1, 1], False),       # the GEMM's eight waves have roles
    (mf.moe_fc2(1024, 512, 8, 2), [512, 2, 1], False),
    (mf.moe_routing(8, 0, 64), [512, 1, 1], False),
    (mf.moe_quant(1024), [128, 1, 1], False),                 # lanes index 256-lane blocks
    (mf.mxfp4_gemv_bf16(512, 1024), [512, 1, 1], False),      # kern_mx_gemv_bf16_r2
    (mf.moe_finalize_rms(7168, 8), [100, 1, 1], False),       # whole waves only
    (mf.moe_finalize_rms(7168, 8), [256, 1, 1], True),        # fewer threads than chunks: still correct
    (mf.moe_finalize_rms(7168, 8), [1024, 1, 1], True),
])
def test_blocks_the_entries_are_written_for(lib, op, block, ok):
    """A launch of a kern_mx entry with a block its thread mapping was not written for is refused when the op
    is read (here through the host-only plan), naming the block it needs."""
    import copy
    op = copy.deepcopy(op)
    op["impl"]["launches"][0]["block"] = block
    n = len(op["params"])
    if ok:
        ops.op_plan(op, 0, [0x1000] * n, {"tokens": 4})
    else:
        with pytest.raises(ops.KernError, match="is written for block"):
            ops.op_plan(op, 0, [0x1000] * n, {"tokens": 4})
