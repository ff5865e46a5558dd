"""Program runtime (kern_rt_*), host side: a whole MoE-layer manifest verifies (module file and sha,
ops, call bindings), and each manifest rule the runtime enforces rejects what breaks it with the error
group the reference uses (crates/kern-runtime/src/error.rs)."""
import copy
import json

import pytest

from kern_amd import manifest as mf
from kern_amd import ops


@pytest.fixture(scope="module")
def good():
    ops.lib()
    return mf.moe_layer_manifest(1024, 512, 8, 2, 64, ops.code_object_sha256())


def _code(m):
    with pytest.raises(ops.KernError) as e:
        ops.Runtime.check(m)
    return e.value.code, str(e.value)


def test_layer_manifest_verifies(good):
    ops.Runtime.check(good)
    ops.Runtime.check(json.dumps(good))  # the text form


def test_module_artifact(good):
    m = copy.deepcopy(good)
    m["modules"]["kern_mx"]["sha256"] = "0" * 64
    code, msg = _code(m)
    assert code == 2 and "sha256" in msg
    m = copy.deepcopy(good)
    m["modules"]["kern_mx"]["source"] = "no_such.hsaco"
    assert _code(m)[0] == 2


@pytest.mark.parametrize("edit,needle", [
    (lambda m: m.update(states={"kv": {"bytes_per_token": 64}}), "states"),
    (lambda m: m["buffers"]["x"].update(kind="peer"), "kind `peer`"),
    (lambda m: m["buffers"]["x"].update(dtype="bf17"), "unknown dtype"),
    (lambda m: m["buffers"]["q"].update(shape=["rows", 1024]), "neither a count nor a declared var"),
    (lambda m: m["buffers"]["x"].update(placement="host"), "placement"),
    (lambda m: m["buffers"]["q"].update(dtype="i8"), "buffer `q` is i8"),
    (lambda m: m["programs"]["moe_layer"]["calls"][0].update(op="moe_nothing"), "unknown op"),
    (lambda m: m["programs"]["moe_layer"]["calls"][0].update(lane=1), "one lane"),
    (lambda m: m["programs"]["moe_layer"]["calls"][0]["args"].pop(), "takes 4 args"),
    (lambda m: m["programs"]["moe_layer"]["calls"][0]["args"].__setitem__(3, {"f32": 1.0}), "needs {\"i32\""),
    (lambda m: m["programs"]["moe_layer"]["calls"][0]["args"].__setitem__(3, {"var": "rows"}), "unknown var"),
    # who may read and write what: sources only in derive programs, no writes to weights or inputs
    (lambda m: m["programs"]["moe_layer"]["calls"][2]["args"].__setitem__(0, {"buf": "w13_raw"}), "source buffer"),
    (lambda m: (m["buffers"]["gamma"].update(dtype="u8"),
                m["programs"]["moe_layer"]["calls"][0]["args"].__setitem__(1, {"buf": "gamma"})), "writes weight"),
    (lambda m: (m["buffers"]["y"].update(dtype="u8"),
                m["programs"]["derive_weights"]["calls"][0]["args"].__setitem__(1, {"buf": "y"})), "reads no input"),
    (lambda m: m["programs"]["derive_weights"].update(graph=True), "derive program is not a graph"),
    (lambda m: m["ops"]["moe_fc1"]["impl"]["launches"][0].update(module="other"), "module `other` is not declared"),
    (lambda m: m["ops"]["moe_fc1"]["impl"]["launches"].append(
        dict(m["ops"]["moe_fc1"]["impl"]["launches"][0], module="other")), "every launch must name"),
])
def test_manifest_rules(good, edit, needle):
    m = copy.deepcopy(good)
    edit(m)
    code, msg = _code(m)
    assert code == 1 and needle in msg, msg


def test_op_verify(good):
    assert ops.lib().kern_op_verify(json.dumps(good["ops"]["moe_fc2"]).encode()) == 0
    bad = copy.deepcopy(good["ops"]["moe_fc2"])
    bad["impl"]["launches"][0]["args"] = bad["impl"]["launches"][0]["args"][:-1]
    assert ops.lib().kern_op_verify(json.dumps(bad).encode()) == 1


def test_ring_activation_buffer_past_4gib(good):
    """FC1 gathers token rows through route_map, so no launch argument bounds its activations: the runtime
    refuses, at load, a buffer of 4 GiB or more bound as a ring GEMM's activations."""
    m = copy.deepcopy(good)
    m["buffers"]["q"].update(shape=[1 << 22, 1024])
    code, msg = _code(m)
    assert code == 1 and "below 4 GiB" in msg and "`q`" in msg, msg
    m["buffers"]["q"].update(shape=[(1 << 22) - 1, 1024])
    ops.Runtime.check(m)
