"""Cut one MoE layer of the reference's K3 manifest fixture (crates/kern-manifest/tests/fixtures/k3/head.json)
into k3_moe_layer_manifest.json: the layer-1 MoE calls of its `prefill` program (l1.moe_quant, l1.routing,
l1.fc1, l1.fc2, l1.finalize), the layer-1 calls of its `derive` program (the four repacks), the calls of its
`load` once-program that write what those read (the fills of the layer's SiTU alpha and beta), and exactly
the buffers, ops and modules those calls name, all as the fixture has them (the ops keep the reference's own
implementations, launching its TRT-LLM modules). Its vars are kept; `topology` and `states`, which no kept
call names, are dropped. This is the manifest a candidate for the path's ops is spliced into. Run in a
container that has the reference checked out:

    python tests/golden/make_k3_moe_manifest.py /root/reference
"""
import json
import os
import sys

PREFILL = ["l1.moe_quant", "l1.routing", "l1.fc1", "l1.fc2", "l1.finalize"]


def main(ref):
    path = os.path.join(ref, "crates/kern-manifest/tests/fixtures/k3/head.json")
    with open(path) as f:
        m = json.load(f)
    calls = [c for c in m["programs"]["prefill"]["calls"] if c["label"] in PREFILL]
    assert [c["label"] for c in calls] == PREFILL
    derive = [c for c in m["programs"]["derive"]["calls"]
              if any(isinstance(a, dict) and a.get("buf", "").startswith("layers.1.") for a in c["args"])]
    assert len(derive) == 4
    reads = {a["buf"] for c in calls + derive for a in c["args"] if isinstance(a, dict) and "buf" in a}
    load = [c for c in m["programs"]["load"]["calls"]
            if any(isinstance(a, dict) and a.get("buf") in reads for a in c["args"])]
    bufs = []
    for c in calls + derive + load:
        for a in c["args"]:
            if isinstance(a, dict) and "buf" in a and a["buf"] not in bufs:
                bufs.append(a["buf"])
    ops = []
    for c in calls + derive + load:
        if c["op"] not in ops:
            ops.append(c["op"])
    mods = []
    for o in ops:
        for launch in m["ops"][o]["impl"]["launches"]:
            if "module" in launch and launch["module"] not in mods:
                mods.append(launch["module"])
    prefill = {k: v for k, v in m["programs"]["prefill"].items() if k != "calls"}
    prefill["calls"] = calls
    derive_p = {k: v for k, v in m["programs"]["derive"].items() if k != "calls"}
    derive_p["calls"] = derive
    load_p = {k: v for k, v in m["programs"]["load"].items() if k != "calls"}
    load_p["calls"] = load
    out = {
        "schema_version": m["schema_version"],
        "model": m["model"],
        "vars": m["vars"],
        "buffers": {b: m["buffers"][b] for b in bufs},
        "modules": {n: m["modules"][n] for n in mods},
        "ops": {o: m["ops"][o] for o in ops},
        "programs": {"prefill": prefill, "load": load_p, "derive": derive_p},
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "k3_moe_layer_manifest.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(dst, os.path.getsize(dst), "bytes;", len(bufs), "buffers,", len(ops), "ops,", len(mods), "modules")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
