"""Build the gfx950 code object and the C-ABI library in-tree.

    python -m kern_amd.build

1. `hipcc --genco --offload-arch=gfx950` compiles kern_amd/csrc/kern_mx.hip to kern_amd/lib/kern_mx.hsaco.
2. Its SHA-256 is compiled into libkern_amd.so (the library refuses any other code object) and written
   to kernel_index/kern_mx.toml with the entries and their kernel-argument sizes, the way kern's
   kernel_index pins its modules by digest (tools/kernels/index.py:1-19).
3. The host side (capi.cpp, manifest_op.cpp, runtime.cpp, candidate.cpp; no device code) is compiled with g++
   against the HIP runtime.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HSACO = os.path.join(LIBDIR, "kern_mx.hsaco")
PEAKS = os.path.join(LIBDIR, "kern_peaks.hsaco")  # roofline probes for bench.py (not on the product path)
CLOCK = os.path.join(LIBDIR, "kern_mx_clock.hsaco")  # kern_mx.hip with its shader-clock probe (bench.py only)
LIB = os.path.join(LIBDIR, "libkern_amd.so")
ARCH = "gfx950"

# hipcc flags for device code: packed-fp32 VALU ops stay off (they have given wrong results on these boxes).
# -cuid fixes the compilation-unit id, which hipcc otherwise derives from the source and output paths: with
# it the code object, and so its pinned sha256, is the same in every checkout.
DEVICE_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-cuid=kern_mx"]

ENTRIES = {
    # entry: (launch params as the op JSON in kernel_index/ declares them)
    "kern_mx_quant_bf16": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "i32", "i32"],
    "kern_mx_quant_f32": ["in buffer<f32>", "out buffer<u8>", "out buffer<u8>", "i32", "i32"],
    "kern_mx_w_shuffle": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32", "i32"],
    "kern_mx_sf_shuffle": ["in buffer<u8>", "out buffer<u8>", "i32", "i32", "i32", "i32"],
    "kern_mx_gemv_bf16": ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>", "i32", "i32",
                          "i32", "i32", "i32"],
    "kern_mx_gemv_bf16_rg": ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>", "i32", "i32",
                             "i32", "i32"],
    **{f"kern_mx_gemv_bf16_r{nkt}": ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>", "i32",
                                     "i32", "i32"] for nkt in (2, 4, 8, 14, 16)},
    **{f"kern_mx_gemv_bf16_p{ktw}": ["in buffer<bf16>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>", "i32",
                                     "i32", "i32", "i32"] for ktw in (1, 2, 4, 7, 8)},
    "kern_mx_bmm_fc2": ["in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>",
                        "in buffer<i32>", "in buffer<i32>", "in buffer<i32>", "in buffer<i32>", "i32", "i32", "i32",
                        "i32", "out buffer<f32>"],
    "kern_mx_bmm_fc1": ["in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "out buffer<u8>",
                        "out buffer<u8>", "in buffer<i32>", "in buffer<f32>", "in buffer<f32>", "in buffer<i32>",
                        "in buffer<i32>", "in buffer<i32>", "in buffer<i32>", "i32", "i32", "i32", "out buffer<f32>"],
    "kern_mx_gemm_e4m3": ["in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "out buffer<u8>",
                          "in buffer<f32>", "i32", "i32", "i32", "out buffer<f32>"],
    "kern_mx_gemm_bf16": ["in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "out buffer<bf16>",
                          "i32", "i32", "i32", "out buffer<f32>"],
    **{f"kern_mx_gemm_bf16_s{ktw}": ["in buffer<u8>", "in buffer<u8>", "in buffer<u8>", "in buffer<u8>",
                                     "out buffer<bf16>", "out buffer<f32>", "i32", "i32", "i32", "i32"]
       for ktw in (1, 2, 4, 7, 8)},
    **{e: ["in buffer<i32>"] + ["out buffer<i32>"] * 7 + ["i32"] * 4
       for e in ("kern_mx_routing", "kern_mx_routing_count", "kern_mx_routing_scan", "kern_mx_routing_rank")},
    "kern_mx_quant_routing": ["in buffer<bf16>", "out buffer<u8>", "out buffer<u8>", "i32", "in buffer<i32>"] +
                             ["out buffer<i32>"] * 7 + ["i32"] * 4,
    "kern_mx_fill_random_u8": ["out buffer<u8>", "i64", "u64", "i32", "i32"],
    "kern_silu_mul_bf16": ["out buffer<bf16>", "in buffer<bf16>", "i32"],
    "kern_mx_moe_finalize_rms": ["in buffer<bf16>", "in buffer<i32>", "in buffer<f32>", "in buffer<bf16>",
                                 "out buffer<bf16>", "i32", "i32", "i32", "f32"],
    "kern_mx_moe_finalize": ["in buffer<bf16>", "in buffer<i32>", "in buffer<f32>", "out buffer<bf16>", "i32", "i32",
                             "i32"],
    "kern_weight_p1_bf16_f32": ["in buffer<bf16>", "out buffer<f32>", "i32"],
    "kern_cast_bf16_f32": ["in buffer<bf16>", "out buffer<f32>", "i32"],
    "kern_rope_table_bf16": ["out buffer<bf16>", "out buffer<bf16>", "i32", "i32", "i32", "f32"],
    "kern_fill_f32": ["out buffer<f32>", "i32", "f32"],
    "kern_fill_i32": ["out buffer<i32>", "i32", "i32"],
    "kern_fill_i64": ["out buffer<i64>", "i32", "i64"],
    "kern_fill_u8": ["out buffer<u8>", "i32", "i32"],
    "kern_fill_bf16": ["out buffer<bf16>", "i32", "f32"],
    "kern_iota_i32": ["out buffer<i32>", "i32", "i32", "i32", "i32"],
    "kern_mx_gemm_mxfp8": ["in buffer<fp8e4m3>", "in buffer<fp8e4m3>", "out buffer<bf16>", "in buffer<u8>",
                           "in buffer<u8>", "i32", "i32", "i32", "i32"],
}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_code_object(csrc: str = CSRC, out: str = HSACO) -> str:
    """Compile csrc/kern_mx.hip to `out`; returns its sha256 (the same for any csrc and out paths)."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "--genco", "--no-gpu-bundle-output", *DEVICE_FLAGS,
          os.path.join(csrc, "kern_mx.hip"), "-o", tmp])
    os.replace(tmp, out)
    with open(out, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def build_peaks() -> str:
    """kern_peaks.hip -> kern_peaks.hsaco, pinned in kernel_index/kern_peaks.toml (bench.py loads it through
    the module layer with that sha256)."""
    tmp = PEAKS + ".tmp"
    flags = [f if f != "-cuid=kern_mx" else "-cuid=kern_peaks" for f in DEVICE_FLAGS]
    _run([os.path.join(ROCM, "bin", "hipcc"), "--genco", "--no-gpu-bundle-output", *flags,
          os.path.join(CSRC, "kern_peaks.hip"), "-o", tmp])
    os.replace(tmp, PEAKS)
    with open(PEAKS, "rb") as f:
        sha = hashlib.sha256(f.read()).hexdigest()
    with open(os.path.join(ROOT, "kernel_index", "kern_peaks.toml"), "w") as f:
        f.write("\n".join([
            "# gfx950 roofline probes (kern_amd/csrc/kern_peaks.hip) for bench.py's peaks leg, pinned by sha256",
            "# (written by kern_amd/build.py). Not part of the MXFP4 path.",
            "[module]", 'name = "kern_peaks"', 'kind = "hsaco"', f'arch = "{ARCH}"',
            'source = "kern_amd/lib/kern_peaks.hsaco"', f'sha256 = "{sha}"', ""]))
    return sha


def build_clock_probe() -> str:
    """kern_mx.hip built with -DKERN_CLOCK_PROBE -> kern_mx_clock.hsaco, pinned in kernel_index/kern_mx_clock.toml:
    the same kernels, with the ring GEMMs' dbg argument carrying each workgroup's shader-clock and real-time
    stamps instead of debug values (bench.py's clock leg). Not part of the MXFP4 path."""
    tmp = CLOCK + ".tmp"
    flags = [f if f != "-cuid=kern_mx" else "-cuid=kern_mx_clock" for f in DEVICE_FLAGS]
    _run([os.path.join(ROCM, "bin", "hipcc"), "--genco", "--no-gpu-bundle-output", *flags, "-DKERN_CLOCK_PROBE",
          os.path.join(CSRC, "kern_mx.hip"), "-o", tmp])
    os.replace(tmp, CLOCK)
    with open(CLOCK, "rb") as f:
        sha = hashlib.sha256(f.read()).hexdigest()
    with open(os.path.join(ROOT, "kernel_index", "kern_mx_clock.toml"), "w") as f:
        f.write("\n".join([
            "# gfx950 shader-clock probe build of kern_amd/csrc/kern_mx.hip (-DKERN_CLOCK_PROBE) for bench.py's",
            "# clock leg, pinned by sha256 (written by kern_amd/build.py). Not part of the MXFP4 path.",
            "[module]", 'name = "kern_mx_clock"', 'kind = "hsaco"', f'arch = "{ARCH}"',
            'source = "kern_amd/lib/kern_mx_clock.hsaco"', f'sha256 = "{sha}"', ""]))
    return sha


def pinned_sha256(name: str = "kern_mx") -> str:
    """The sha256 kernel_index/<name>.toml pins."""
    with open(os.path.join(ROOT, "kernel_index", f"{name}.toml")) as f:
        for line in f:
            if line.startswith("sha256 = "):
                return line.split('"')[1]
    raise RuntimeError(f"kernel_index/{name}.toml has no sha256")


def build_library(sha: str) -> None:
    tmp = LIB + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-function",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f'-DKERN_MX_SHA256="{sha}"',
          os.path.join(CSRC, "capi.cpp"), os.path.join(CSRC, "manifest_op.cpp"), os.path.join(CSRC, "runtime.cpp"),
          os.path.join(CSRC, "candidate.cpp"), "-o", tmp, f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-ldl"])
    os.replace(tmp, LIB)


def write_index(sha: str) -> None:
    idx = os.path.join(ROOT, "kernel_index")
    os.makedirs(idx, exist_ok=True)
    lines = [
        "# gfx950 code object of the MXFP4 matmul path, pinned by sha256 (written by kern_amd/build.py).",
        "# Each [[entry]] lists the launch params a manifest op declares for it; the runtime checks them",
        "# against the code object's own kernel-argument metadata before the first launch.",
        "[module]",
        'name = "kern_mx"',
        'kind = "hsaco"',
        f'arch = "{ARCH}"',
        'source = "kern_amd/lib/kern_mx.hsaco"',
        f'sha256 = "{sha}"',
        "",
    ]
    for name, params in ENTRIES.items():
        lines += ["[[entry]]", f'name = "{name}"', "params = [" + ", ".join(f'"{p}"' for p in params) + "]", ""]
    with open(os.path.join(idx, "kern_mx.toml"), "w") as f:
        f.write("\n".join(lines))


def write_candidate(sha: str) -> None:
    """kernel_index/k3_moe_candidate.json: the Candidate file of the path's ops at K3's shapes (manifest.py),
    pinned to this build's code object."""
    sys.path.insert(0, ROOT)
    import json

    from kern_amd import manifest

    with open(os.path.join(ROOT, "kernel_index", "k3_moe_candidate.json"), "w") as f:
        json.dump(manifest.k3_moe_candidate(sha), f, indent=1)
        f.write("\n")


def build_oracle() -> None:
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


def build(oracle: bool = True) -> str:
    sha = build_code_object()
    build_library(sha)
    write_index(sha)
    write_candidate(sha)
    build_peaks()
    build_clock_probe()
    if oracle:
        build_oracle()
    return sha


if __name__ == "__main__":
    print(build(oracle="--no-oracle" not in sys.argv))
