"""The drop-in in the reference's own terms: a Candidate {modules, ops} file (crates/kern-manifest/src/candidate.rs:
34-44) for the path's ops at K3's shapes, spliced (kern_candidate_splice, the analog of candidate::splice,
candidate.rs:152-185) into one MoE layer cut from the reference's K3 manifest fixture
(tests/golden/k3_moe_layer_manifest.json, made by tests/golden/make_k3_moe_manifest.py), then verified by the
program runtime on the host (kern_rt_check). No GPU: the device run of the spliced layer is
tests/test_gpu_candidate.py."""
import copy
import json
import os

import pytest

from kern_amd import build as kb
from kern_amd import manifest as mf
from kern_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "k3_moe_layer_manifest.json")
INTERFACES = os.path.join(ROOT, "tests", "golden", "k3_op_interfaces.json")
CANDIDATE = os.path.join(ROOT, "kernel_index", "k3_moe_candidate.json")
KERNELS = os.path.dirname(ops.HSACO_PATH)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ops.LIB_PATH):
        pytest.skip("library not built (python -m kern_amd.build)")
    return ops.lib()


def _load(p):
    with open(p) as f:
        return json.load(f)


def test_candidate_file_is_the_k3_interface():
    """The committed candidate is manifest.k3_moe_candidate pinned to the built code object, and every op's
    params are the reference's (head.json, via k3_op_interfaces.json)."""
    cand = _load(CANDIDATE)
    assert cand == json.loads(json.dumps(mf.k3_moe_candidate(kb.pinned_sha256())))
    assert set(cand) == {"modules", "ops"}
    assert cand["modules"] == {"kern_mx": {"source": "kern_mx.hsaco", "sha256": kb.pinned_sha256()}}
    ref = _load(INTERFACES)["ops"]
    for name, op in cand["ops"].items():
        assert op["params"] == ref[name]["params"], name
        assert {l["module"] for l in op["impl"]["launches"]} == {"kern_mx"}


def test_splice_into_the_k3_layer(lib):
    m, cand = _load(FIXTURE), _load(CANDIDATE)
    out = ops.splice(m, cand)
    # the ops are the candidate's, under the manifest's names and params
    assert set(out["ops"]) == set(m["ops"])
    for name, op in out["ops"].items():
        assert op["params"] == m["ops"][name]["params"], name
        assert op == cand["ops"][name], name
    # the reference's TRT-LLM / K3 modules are no longer launched, so they are gone; ours is in
    assert out["modules"] == cand["modules"]
    # nothing else changed: vars, every buffer, every program and call
    for key in ("schema_version", "model", "vars", "buffers", "programs"):
        assert out[key] == m[key], key


def test_spliced_k3_layer_verifies(lib):
    """The spliced layer passes the runtime's host-side load checks (modules read from kernels_dir and pinned
    by sha256, every op verified and checked against the code object's kernel-argument sizes, every call
    against its op's params)."""
    out = ops.splice(_load(FIXTURE), _load(CANDIDATE))
    ops.Runtime.check(out, KERNELS)
    # the unspliced fixture names NVIDIA cubins this runtime cannot load
    with pytest.raises(ops.KernError):
        ops.Runtime.check(_load(FIXTURE), KERNELS)


def test_splice_keeps_ops_the_candidate_leaves_alone(lib):
    m, cand = _load(FIXTURE), _load(CANDIDATE)
    part = {"modules": cand["modules"], "ops": {"moe_fc1": cand["ops"]["moe_fc1"], "moe_fc2": cand["ops"]["moe_fc2"]}}
    out = ops.splice(m, part)
    assert out["ops"]["moe_fc1"] == cand["ops"]["moe_fc1"]
    assert out["ops"]["moe_quant"] == m["ops"]["moe_quant"]
    # the modules of the FC1 / FC2 cubins are dropped (nothing launches them), the others stay
    fc_mods = {l["module"] for n in ("moe_fc1", "moe_fc2") for l in m["ops"][n]["impl"]["launches"]}
    assert set(out["modules"]) == (set(m["modules"]) - fc_mods) | {"kern_mx"}


def test_splice_reports_every_misfit(lib):
    m, cand = _load(FIXTURE), _load(CANDIDATE)
    bad = copy.deepcopy(cand)
    bad["ops"]["moe_fc9"] = bad["ops"].pop("moe_fc1")                       # an op the manifest lacks
    bad["ops"]["moe_fc2"]["params"] = bad["ops"]["moe_fc2"]["params"][:-1]  # params not the manifest's
    bad["ops"]["moe_quant"]["impl"]["launches"][0]["module"] = "nowhere"     # a module in neither
    with pytest.raises(ops.KernError) as e:
        ops.splice(m, bad)
    msg = str(e.value)
    assert e.value.code == 1 and "candidate does not fit" in msg
    assert "op `moe_fc9`: the manifest has no such op" in msg
    assert "op `moe_fc2`: params [" in msg and "are not the manifest's" in msg
    assert "op `moe_quant`: module `nowhere` is in neither the candidate nor the manifest" in msg
    for cnd, what in [({"ops": {}}, "no ops"), ({"ops": cand["ops"], "extra": 1}, "unknown field `extra`")]:
        with pytest.raises(ops.KernError) as e:
            ops.splice(m, cnd)
        assert what in str(e.value)


def test_splice_renames_a_module_the_manifest_pins_differently(lib):
    """A manifest that already names a module `kern_mx` with other bytes keeps it for its own launches; the
    candidate's is taken in as `kern_mx@<first 8 hex of its sha256>` (candidate.rs:116-131)."""
    m, cand = _load(FIXTURE), _load(CANDIDATE)
    old_sha = "0" * 64
    m["modules"]["kern_mx"] = {"source": "old.hsaco", "sha256": old_sha}
    m["ops"]["fill_f32"]["impl"]["launches"][0]["module"] = "kern_mx"
    part = {"modules": cand["modules"], "ops": {"moe_fc1": cand["ops"]["moe_fc1"]}}
    out = ops.splice(m, part)
    new_name = "kern_mx@" + kb.pinned_sha256()[:8]
    assert out["modules"]["kern_mx"]["sha256"] == old_sha          # still launched by fill_f32
    assert out["modules"][new_name] == cand["modules"]["kern_mx"]
    assert {l["module"] for l in out["ops"]["moe_fc1"]["impl"]["launches"]} == {new_name}
    assert out["ops"]["fill_f32"]["impl"]["launches"][0]["module"] == "kern_mx"
    # when the candidate replaces that op too, the old module is no longer launched and goes
    out = ops.splice(m, {"modules": cand["modules"],
                         "ops": {"moe_fc1": cand["ops"]["moe_fc1"], "fill_f32": cand["ops"]["fill_f32"]}})
    assert "kern_mx" not in out["modules"] and new_name in out["modules"]
