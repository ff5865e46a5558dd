"""Extract the interface params of the MXFP4 path's ops, and the fixed grids of the two repack launches,
from the reference's K3 manifest fixture (crates/kern-manifest/tests/fixtures/k3/head.json) into
k3_op_interfaces.json. Run in a container that has the reference checked out:

    python tests/golden/make_k3_interfaces.py /root/reference
"""
import json
import os
import sys

OPS = ["moe_quant", "k3_moe_w_shuffle", "k3_moe_sf_shuffle", "moe_routing", "moe_fc1", "moe_fc2", "moe_finalize_rms",
       "fill_i32", "fill_f32", "fill_bf16"]


def main(ref):
    path = os.path.join(ref, "crates/kern-manifest/tests/fixtures/k3/head.json")
    with open(path) as f:
        m = json.load(f)
    out = {"source": "crates/kern-manifest/tests/fixtures/k3/head.json", "ops": {}}
    for name in OPS:
        op = m["ops"][name]
        rec = {"params": op["params"]}
        if name in ("k3_moe_w_shuffle", "k3_moe_sf_shuffle", "moe_fc1", "moe_fc2", "moe_finalize_rms"):
            rec["grid"] = op["impl"]["launches"][0]["grid"]
        if name.startswith("fill_"):  # the kernel ABI and the literal args of the once-program launch
            launch = op["impl"]["launches"][0]
            rec.update({"entry": launch["entry"], "launch_params": launch["params"], "args": launch["args"],
                        "grid": launch["grid"], "block": launch["block"]})
        out["ops"][name] = rec
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "k3_op_interfaces.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(dst)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
