"""A whole MoE layer, chained, checked the way tools/trtllm-bmm/probe.py:100-112 checks the reference's:
x -> moe_quant -> moe_routing -> FC1 (SiTU-GLU, MXFP8 out) -> FC2 -> weighted combine (probe.py's index_add)
against a float64 reference over exactly dequantized operands, with the max |err| and relative RMS error
that probe.py prints, bounded.

The float64 chain (f64_chain) follows probe.py:100-110: per local expert, h = deq(x) deq(W13)^T, gate = the
second half of the rows (K3 binds w3 then w1, head.json:1161), SiTU-GLU (probe.py:46-47), the MXFP8 round
trip of h (probe.py:38-43's floor rule, saturating), times deq(W2)^T, weighted and added into the token's
row. Its only roundings are the two MXFP8 quantizations the layer itself defines; the kernels' f32
accumulation can move an h value across an e4m3 rounding boundary, which changes that element by one
e4m3 step. The bound is checked first on the CPU oracle's own chain (f32 accumulation like the kernels,
test_oracle_chain_within_bound, no GPU), then on the GPU chain, whose every stage is also checked against
the oracle on the GPU's own inputs to it (tests/_moe.py).

Shapes: a small layer (64 tokens, 8 experts, top-2, H = 1024, I = 512) and probe.py's own K3 shape: H = 3584,
I = 3072, 224 experts, top-16, this rank's 56 (ids 56..111), T = 300, alpha = 4, beta = 25 (probe.py:22-23).
"""
import numpy as np
import pytest

from kern_amd import workload as wl
from tests import _moe
from tests._util import bf16_to_f32, to_dev, to_np

torch = pytest.importorskip("torch")

ALPHA, BETA = 4.0, 25.0
# end-to-end bounds (probe.py prints these two figures): max |err| <= MAX_ERR * max |ref|, rel RMS <= REL_RMS
MAX_ERR, REL_RMS = 2e-2, 4e-3

SHAPES = {
    "small": dict(T=64, E=8, k=2, H=1024, I=512, start=0, local=8, seed=900),
    "k3": dict(T=300, E=224, k=16, H=3584, I=3072, start=56, local=56, seed=901),
}

E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)


_NIB = E2M1[np.arange(16) & 7] * np.where(np.arange(16) & 8, -1.0, 1.0)
_BYTE2 = np.stack([_NIB[np.arange(256) & 15], _NIB[np.arange(256) >> 4]], axis=1)  # byte -> (low, high) values


def deq_fp4_f64(w, sf):
    """[n, K/2] nibbles (element 2j low) and [n, K/32] e8m0 -> float64 [n, K] (probe.py:28-31)."""
    n = w.shape[0]
    v = np.take(_BYTE2, w.astype(np.intp), axis=0).reshape(n, -1, 32)
    return (v * np.exp2(sf.astype(np.float64) - 127)[:, :, None]).reshape(n, -1)


def deq_fp8_f64(oracle, q, sf):
    lut = np.array([oracle.e4m3_decode(c) for c in range(256)], np.float64)
    n = q.shape[0]
    v = np.take(lut, q.astype(np.intp)).reshape(n, -1, 32)
    return (v * np.exp2(sf.astype(np.float64) - 127)[:, :, None]).reshape(n, -1)


def f64_chain(oracle, xq, xqs, ids, wts, w13, s13, w2, s2, start, I):
    """The float64 reference layer (probe.py:100-110) over raw weights [local, rows, .]."""
    T = xq.shape[0]
    H = w2.shape[1]
    xd = deq_fp8_f64(oracle, xq, xqs)
    out = np.zeros((T, H), np.float64)
    for le in range(w13.shape[0]):
        t_idx, k_idx = np.nonzero(ids == start + le)
        if t_idx.size == 0:
            continue
        h = xd[t_idx] @ deq_fp4_f64(w13[le], s13[le]).T
        up, gate = h[:, :I], h[:, I:]
        with np.errstate(over="ignore"):
            act = ALPHA * np.tanh(gate / ALPHA) / (1.0 + np.exp(-gate)) * BETA * np.tanh(up / BETA)
        q, s = oracle.quant_blocks(act.astype(np.float32))
        y = deq_fp8_f64(oracle, q, s) @ deq_fp4_f64(w2[le], s2[le]).T
        np.add.at(out, t_idx, y * wts[t_idx, k_idx][:, None].astype(np.float64))
    return out


def end_to_end(got, ref):
    err = np.abs(np.asarray(got, np.float64) - ref)
    return err.max() / np.abs(ref).max(), np.sqrt((err ** 2).mean() / (ref ** 2).mean())


def _case(name):
    c = SHAPES[name]
    T, E, k, H, I = c["T"], c["E"], c["k"], c["H"], c["I"]
    x = wl.activations_bf16(c["seed"], T, H)
    ids = wl.topk_ids(c["seed"] + 1, T, E, k)
    wts = wl.topk_weights(c["seed"] + 2, T, k)
    return c, x, ids, wts


# ------------------------------------------------------------------------------------ CPU: the bound itself

def test_oracle_chain_within_bound(oracle):
    """The oracle's staged chain (f32 accumulation, as the kernels) against the float64 chain, small shape:
    the end-to-end bound holds for an implementation whose only differences are accumulation order and
    precision. A chain that pairs gate and up the other way round ("gate=first", probe.py:108) fails it."""
    c, x, ids, wts = _case("small")
    T, k, H, I, L = c["T"], c["k"], c["H"], c["I"], c["local"]
    w13, s13 = wl.mxfp4_weights(c["seed"] + 3, L, 2 * I, H, 119, 124)
    w2, s2 = wl.mxfp4_weights(c["seed"] + 4, L, H, I, 118, 126)
    xq, xqs = oracle.quant_mxfp8(x)
    ref = f64_chain(oracle, xq, xqs, ids, wts, w13, s13, w2, s2, c["start"], I)
    ctas = L + -(-T * k // 128)
    tabs = oracle.routing(ids, c["start"], L, ctas_cap=ctas)
    rows = ctas * 128
    a13 = oracle.w_shuffle(w13, L, 2 * I, H // 2, 1)
    sa13 = oracle.sf_shuffle(s13, L, 2 * I, H // 32, 1)
    al, be = np.full(L, ALPHA, np.float32), np.full(L, BETA, np.float32)
    c1, sf1, _ = oracle.fc1(a13, sa13, xq, xqs, tabs, al, be, 2 * I, H, rows)
    a2 = oracle.w_shuffle(w2, L, H, I // 2, 0)
    sa2 = oracle.sf_shuffle(s2, L, H, I // 32, 0)
    c2, _ = oracle.fc2(a2, sa2, c1, sf1, True, tabs, H, I)
    out = oracle.moe_finalize(c2, tabs["exp2perm"].reshape(-1), wts, None, T, H, k)
    mx, rms = end_to_end(bf16_to_f32(out), ref)
    print(f"oracle chain vs float64: max|err| {mx:.3g} of max|ref|, rel rms {rms:.3g}")
    assert mx <= MAX_ERR and rms <= REL_RMS
    # the wrong gate/up pairing is far outside the bound
    swapped = np.concatenate([w13[:, I:], w13[:, :I]], axis=1), np.concatenate([s13[:, I:], s13[:, :I]], axis=1)
    bad = f64_chain(oracle, xq, xqs, ids, wts, *swapped, w2, s2, c["start"], I)
    assert end_to_end(bad, ref)[1] > 10 * REL_RMS


# ------------------------------------------------------------------------------------ GPU: the chained layer

@pytest.mark.gpu
@pytest.mark.parametrize("name", ["small", "k3"])
def test_moe_layer_chain(oracle, name):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kern_amd import ops

    ops.lib()
    c, x, ids, wts = _case(name)
    T, k, H, I, L, start = c["T"], c["k"], c["H"], c["I"], c["local"], c["start"]
    print(f"[moe layer {name}] T={T} E={c['E']} local={L} top-{k} H={H} I={I}", flush=True)
    r13, rs13 = _moe.gpu_raw_weights(ops, torch, c["seed"] + 3, L, 2 * I, H, 119, 6)
    r2, rs2 = _moe.gpu_raw_weights(ops, torch, c["seed"] + 4, L, H, I, 118, 9)
    w13, s13 = ops.repack_weights(r13, rs13, gated=True)
    w2, s2 = ops.repack_weights(r2, rs2)
    ctas = ops.ctas_bound(T, k, L)
    rows = ctas * 128
    i32, u8 = torch.int32, torch.uint8
    tab = {n: torch.zeros(sz, dtype=i32, device="cuda") for n, sz in
           [("counts", 2 * L), ("cta_batch", ctas), ("cta_limit", ctas), ("nne", 1), ("tp", 1),
            ("route_map", rows), ("exp2perm", T * k)]}
    xd, idd, wd = to_dev(x), to_dev(ids), to_dev(wts)
    al, be = np.full(L, ALPHA, np.float32), np.full(L, BETA, np.float32)
    q = torch.empty((T, H), dtype=u8, device="cuda")
    qs = torch.empty((T, H // 32), dtype=u8, device="cuda")
    c1 = torch.zeros((rows, I), dtype=u8, device="cuda")
    sf1 = torch.zeros(ops.r128c4_bytes(rows, I // 32), dtype=u8, device="cuda")
    c2 = torch.zeros((rows, H), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_quant(xd, q, qs, T, K=H)
    ops.moe_routing(idd, tab["counts"], tab["cta_batch"], tab["cta_limit"], tab["nne"], tab["tp"], tab["route_map"],
                    tab["exp2perm"], tokens=T, topk=k, local_start=start, local_experts=L)
    al_d, be_d = to_dev(al), to_dev(be)

    def fc1(c_, sf_, dbg_):
        ops.trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(w13, s13, q, qs, c_, sf_, tab["route_map"], al_d, be_d, tab["nne"],
                                            tab["tp"], tab["cta_batch"], tab["cta_limit"], m=2 * I, k=H, ctas=ctas,
                                            dbg=dbg_)

    fc1(c1, sf1, None)  # production FC1 (no debug output) feeds FC2
    ops.trtllm_bmm_bf16_mxe2m1_mxe4m3(w2, s2, c1, sf1, c2, tab["nne"], tab["tp"], tab["cta_batch"], tab["cta_limit"],
                                      m=H, k=I, ctas=ctas)
    ops.moe_finalize(c2, tab["exp2perm"], wd, out, T, H=H, topk=k)
    torch.cuda.synchronize()

    # every stage against the oracle on the GPU's own inputs
    q_ref, qs_ref = oracle.quant_mxfp8(x)
    np.testing.assert_array_equal(to_np(q), q_ref)
    np.testing.assert_array_equal(to_np(qs), qs_ref)
    tabs = oracle.routing(ids, start, L, ctas_cap=ctas)
    S = int(tabs["num_non_exiting"][0])
    assert int(to_np(tab["nne"])[0]) == S
    np.testing.assert_array_equal(to_np(tab["route_map"])[: S * 128], tabs["route_map"][: S * 128])
    np.testing.assert_array_equal(to_np(tab["exp2perm"]), tabs["exp2perm"].reshape(-1))
    dbg1 = _moe.fc1_debug_twin(torch, fc1, c1, sf1, f"layer {name}")
    _moe.check_fc1(torch, oracle, w13, s13, q, qs, tabs, al, be, 2 * I, H, c1, sf1, dbg1, f"layer {name}")
    _moe.check_fc2(torch, oracle, w2, s2, c1, sf1, tabs, H, I, c2, f"layer {name}")
    _moe.check_finalize(oracle, c2, tab["exp2perm"], wd, None, out, T, H, k, 0.0, f"layer {name}")

    # end to end against the float64 chain
    ref = f64_chain(oracle, q_ref, qs_ref, ids, wts, to_np(r13), to_np(rs13), to_np(r2), to_np(rs2), start, I)
    mx, rms = end_to_end(bf16_to_f32(to_np(out)), ref)
    print(f"[moe layer {name}] max|err| {mx:.3g} of max|ref|, rel rms {rms:.3g}", flush=True)
    assert mx <= MAX_ERR and rms <= REL_RMS, (mx, rms)
