"""Building candidates through the C ABI: kern_candidate_of / _only / _join / _tile, the analogs of
Candidate::of, ::only, ::join and candidate::tile (crates/kern-manifest/src/candidate.rs:83-113, :231-300), with
the properties the reference's own tests hold them to (crates/kern-manifest/tests/candidate.rs): a manifest's
own ops splice back to the manifest, a tiling runs at every value of its var exactly what the piece covering
that value runs (randomized), a launch conditioned on another var is refused, pieces keep their own scratch,
and join refuses an op implemented twice. Host only: no device is touched."""
import json
import os
import random

import pytest

from kern_amd import manifest as mf

ops = pytest.importorskip("kern_amd.ops")

MAX = 12
PARAMS = ["in buffer<bf16>", "in buffer<bf16>", "out buffer<bf16>", "inout state", "i32"]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ops.LIB_PATH):
        pytest.skip("library not built")
    return ops.lib()


def sha(tag: int) -> str:
    return f"{tag:02x}" * 32


def manifest() -> dict:
    """A small manifest of our own with one op, `scale`, launched from module `toy`, and a program calling it."""
    return {
        "vars": {"tokens": {"max": MAX}},
        "modules": {"toy": {"source": "toy.hsaco", "sha256": sha(0x5e)}},
        "buffers": {"x": {"dtype": "bf16", "shape": ["tokens", 64]}, "g": {"dtype": "bf16", "shape": [64]},
                    "y": {"dtype": "bf16", "shape": ["tokens", 64]}},
        "ops": {"scale": {"params": PARAMS,
                          "impl": {"launches": [{"module": "toy", "entry": "scale_rows", "block": [64, 1, 1],
                                                 "grid": ["tokens", 1, 1]}]}}},
        "programs": {"step": {"calls": [{"op": "scale", "args": ["x", "g", "y", "state", 64]}]}},
    }


def launch(module, entry, when=None):
    l = {"module": module, "entry": entry, "block": [64, 1, 1], "grid": ["tokens", 1, 1]}
    if when is not None:
        lo, hi = when
        l["when"] = {"var": "tokens"}
        if lo is not None:
            l["when"]["min"] = lo
        if hi is not None:
            l["when"]["max"] = hi
    return l


def candidate(module, tag, launches):
    return {"modules": {module: {"source": f"{module}.hsaco", "sha256": sha(tag)}},
            "ops": {"scale": {"params": PARAMS, "impl": {"launches": launches}}}}


def holds(when, v):
    return when is None or ((when.get("min") is None or v >= when["min"]) and
                            (when.get("max") is None or v <= when["max"]))


def runs(c, v, op="scale"):
    """The entries of c's op that run at var value v, in order."""
    return [l["entry"] for l in c["ops"][op]["impl"]["launches"] if holds(l.get("when"), v)]


def test_a_manifests_own_ops_splice_back_to_the_manifest(lib):
    m = manifest()
    own = ops.candidate_of(m, ["scale", "absent"])
    assert (len(own["ops"]), list(own["modules"])) == (1, ["toy"])
    assert ops.splice(m, own) == m
    # only() of a candidate is the same cut
    assert ops.candidate_only(own, ["scale"]) == own
    assert ops.candidate_only(own, ["absent"]) == {"modules": {}, "ops": {}}


def test_a_splice_swaps_the_implementation_and_leaves_the_calls(lib):
    m = manifest()
    out = ops.splice(m, candidate("fast", 0xab, [launch("fast", "scale_tiled")]))
    assert out["ops"]["scale"]["impl"]["launches"][0]["entry"] == "scale_tiled"
    assert list(out["modules"]) == ["fast"]
    assert (out["programs"], out["buffers"], out["vars"]) == (m["programs"], m["buffers"], m["vars"])


@pytest.mark.parametrize("seed", range(4))
def test_a_tiling_runs_at_every_value_what_the_piece_covering_it_runs(lib, seed):
    m = manifest()
    r = random.Random(0x9E3779B97F4A7C15 + seed)
    for case in range(100):
        n = 1 + r.randrange(4)
        cands = []
        for i in range(n):
            ls = []
            for j in range(1 + r.randrange(3)):
                kind = r.randrange(3)
                if kind == 0:
                    when = None
                elif kind == 1:
                    when = (1 + r.randrange(MAX), None)
                else:
                    lo = 1 + r.randrange(MAX)
                    when = (lo, lo + r.randrange(MAX))
                ls.append(launch(f"m{i}", f"c{i}l{j}", when))
            cands.append(candidate(f"m{i}", i + 1, ls))
        # cut 1..MAX into contiguous ranges and hand each to a candidate
        cuts = [1] + [v for v in range(2, MAX + 1) if r.randrange(4) == 0]
        pieces = [(r.randrange(n), lo, cuts[k + 1] - 1 if k + 1 < len(cuts) else MAX) for k, lo in enumerate(cuts)]
        asked = [(cands[i], lo if k > 0 else None, hi if k < len(pieces) - 1 else None)
                 for k, (i, lo, hi) in enumerate(pieces)]

        def want(v):
            i = next(i for i, lo, hi in pieces if lo <= v <= hi)
            return runs(cands[i], v)

        try:
            tiled = ops.candidate_tile("scale", "tokens", asked)
        except ops.KernError as e:
            assert all(not want(v) for v in range(1, MAX + 1)), f"case {case} refused a tiling that runs: {e}"
            assert "no launch of any piece runs in its range of `tokens`" in str(e)
            continue
        for v in range(1, MAX + 1):
            assert runs(tiled, v) == want(v), f"case {case} at tokens = {v}"
        mods = [l["module"] for l in tiled["ops"]["scale"]["impl"]["launches"]]
        assert set(mods) == set(tiled["modules"]), case
        for l in tiled["ops"]["scale"]["impl"]["launches"]:
            w = l.get("when")
            assert w is None or (w["var"] == "tokens" and w.get("min", 2) > 1), case
        ops.splice(m, tiled)  # everything that runs somewhere splices


def test_a_piece_conditioned_on_another_var_cannot_be_narrowed(lib):
    c = candidate("m", 1, [launch("m", "k")])
    c["ops"]["scale"]["impl"]["launches"][0]["when"] = {"var": "seqs", "max": 2}
    with pytest.raises(ops.KernError, match="runs in a range of `seqs`, not of `tokens`"):
        ops.candidate_tile("scale", "tokens", [(c, None, None)])


def test_malformed_pieces_are_refused(lib):
    c = candidate("m", 1, [launch("m", "k")])
    c["ops"]["scale"]["impl"]["launches"][0]["when"] = {"var": "tokens", "min": -2}
    with pytest.raises(ops.KernError, match="when.min must be a non-negative integer"):
        ops.candidate_tile("scale", "tokens", [(c, None, None)])
    with pytest.raises(ops.KernError, match="unknown field `programs`"):
        ops.candidate_tile("scale", "tokens", [({"ops": {}, "programs": {}}, None, None)])
    with pytest.raises(ops.KernError, match="a launch must be an object"):
        ops.candidate_tile("scale", "tokens", [({"ops": {"scale": {"params": [], "impl": {"launches": [3]}}}},
                                                None, None)])
    with pytest.raises(ops.KernError, match="no launch of any piece runs"):
        ops.candidate_tile("scale", "tokens", [])


def test_pieces_without_the_op_or_with_other_params_are_refused(lib):
    a = candidate("m1", 1, [launch("m1", "k1")])
    b = candidate("m2", 2, [launch("m2", "k2")])
    b["ops"]["scale"]["params"] = PARAMS[:-1]
    with pytest.raises(ops.KernError) as e:
        ops.candidate_tile("scale", "tokens", [(a, None, 4), (b, 5, None), ({"ops": {}}, None, None)])
    assert "piece 1: op `scale` has other params than piece 0" in str(e.value)
    assert "piece 2: no op `scale`" in str(e.value)


def test_pieces_keep_their_own_scratch_and_candidates_join_by_op(lib):
    def with_scratch(tag, cols):
        c = candidate(f"m{tag}", tag, [])
        c["ops"]["scale"]["impl"] = {
            "scratch": {"tmp": {"dtype": "f32", "shape": ["tokens", cols]}},
            "launches": [{"module": f"m{tag}", "entry": f"k{tag}", "block": [64, 1, 1], "grid": ["tokens", 1, 1],
                          "params": ["in buffer<bf16>", "out buffer<f32>"],
                          "args": [{"param": 0}, {"scratch": "tmp"}]}]}
        return c

    a, b = with_scratch(1, 8), with_scratch(2, 16)
    tiled = ops.candidate_tile("scale", "tokens", [(a, None, 4), (b, 5, None)])
    imp = tiled["ops"]["scale"]["impl"]
    assert (list(imp["scratch"]), imp["launches"][0]["args"][1], imp["launches"][1]["args"][1]) == \
        (["tmp", "tmp@1"], {"scratch": "tmp"}, {"scratch": "tmp@1"})
    assert (imp["launches"][0]["when"], imp["launches"][1]["when"]) == \
        ({"var": "tokens", "max": 4}, {"var": "tokens", "min": 5})
    # the same scratch in both pieces is shared
    same = ops.candidate_tile("scale", "tokens", [(a, None, 4), (with_scratch(3, 8), 5, None)])
    assert list(same["ops"]["scale"]["impl"]["scratch"]) == ["tmp"]

    with pytest.raises(ops.KernError, match="op `scale` is implemented twice"):
        ops.candidate_join([a, b])
    assert ops.candidate_join([tiled]) == tiled


def test_a_module_name_given_other_bytes_is_renamed_after_its_hash(lib):
    a = candidate("m", 1, [launch("m", "k1")])
    b = candidate("m", 2, [launch("m", "k2")])
    b["ops"]["shift"] = b["ops"].pop("scale")
    joined = ops.candidate_join([a, b])
    assert sorted(joined["modules"]) == ["m", "m@02020202"]
    assert joined["ops"]["shift"]["impl"]["launches"][0]["module"] == "m@02020202"
    tiled = ops.candidate_tile("scale", "tokens", [(a, None, 4), (candidate("m", 2, [launch("m", "k2")]), 5, None)])
    assert [l["module"] for l in tiled["ops"]["scale"]["impl"]["launches"]] == ["m", "m@02020202"]


@pytest.mark.parametrize("topk", [8, 16])
def test_routing_op_is_the_tiling_of_its_two_implementations(lib, topk):
    """The path's own choice by shape, expressed as a tiling: moe_routing's one-workgroup launch below
    ROUTE_CHUNKED_MIN expanded indices and its chunked launches above, each as a candidate of its own, tile
    into an op that runs what manifest.moe_routing runs at every token count."""
    op = mf.moe_routing(topk, 0, 64)
    mod = {"kern_mx": {"source": "kern_mx.hsaco", "sha256": sha(0x11)}}

    def part(launches):
        ls = [{k: v for k, v in l.items() if k != "when"} for l in launches]
        return {"modules": mod, "ops": {"moe_routing": {"params": op["params"], "impl": {"launches": ls}}}}

    first = -(-mf.ROUTE_CHUNKED_MIN // topk)
    L = op["impl"]["launches"]
    tiled = ops.candidate_tile("moe_routing", "tokens", [(part(L[:1]), None, first - 1), (part(L[1:]), first, None)])
    got = tiled["ops"]["moe_routing"]
    assert got["params"] == op["params"]
    for t in [1, first - 1, first, first + 1, 16384]:
        assert runs(tiled, t, "moe_routing") == [l["entry"] for l in L if holds(l.get("when"), t)], t
    assert [json.dumps(l, sort_keys=True) for l in got["impl"]["launches"]] == \
        [json.dumps(l, sort_keys=True) for l in L]
