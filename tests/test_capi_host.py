"""Host-side checks of the C-ABI library (no GPU needed): it loads, exports every function
include/kern_amd.h declares, pins its code object by SHA-256, reads kernel-argument sizes from the code
object's metadata, and rejects contract violations before touching a device — the host-forceable
failures of crates/kern-runtime (sha mismatch and param-layout mismatch, compile.rs:373-415; caller
contract, error.rs:25-30)."""
import ctypes
import hashlib
import os
import re
import subprocess
import sys

import pytest

from kern_amd import build as kb
from kern_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kern_amd.h")
TOML = os.path.join(ROOT, "kernel_index", "kern_mx.toml")

SIZES = {"i32": 4, "u32": 4, "f32": 4, "i64": 8, "u64": 8}


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kern_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ops.LIB_PATH):
        pytest.skip("library not built (python -m kern_amd.build)")
    return ops.lib()


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/kern_amd.h but not exported"


def test_code_object_pinned(lib):
    with open(ops.HSACO_PATH, "rb") as f:
        img = f.read()
    sha = hashlib.sha256(img).hexdigest()
    assert ops.code_object_sha256() == sha
    toml = open(TOML).read()
    assert f'sha256 = "{sha}"' in toml
    buf = ctypes.create_string_buffer(65)
    assert lib.kern_sha256_hex(img, len(img), buf) == 0
    assert buf.value.decode() == sha
    for data in [b"", b"abc", os.urandom(1000), os.urandom(64), os.urandom(55), os.urandom(56)]:
        assert lib.kern_sha256_hex(data, len(data), buf) == 0
        assert buf.value.decode() == hashlib.sha256(data).hexdigest()


def test_sha_mismatch_is_artifact_error(lib):
    with open(ops.HSACO_PATH, "rb") as f:
        img = bytearray(f.read())
    img[100] ^= 1
    out = ctypes.c_void_p()
    rc = lib.kern_module_load(bytes(img), len(img), ops.code_object_sha256().encode(), ctypes.byref(out))
    assert rc == 2
    assert "sha256 mismatch" in lib.kern_last_error().decode()


def test_kernarg_sizes_from_metadata_match_index(lib):
    """The ABI check's data (kern_code_object_param_sizes, read from our own code object's metadata)
    agrees with the launch params each entry declares in kernel_index/kern_mx.toml."""
    with open(ops.HSACO_PATH, "rb") as f:
        img = f.read()
    for entry, params in kb.ENTRIES.items():
        want = [8 if p.startswith(("in ", "out ", "inout ")) else SIZES[p] for p in params]
        sizes = (ctypes.c_uint32 * 32)()
        n = ctypes.c_int()
        assert lib.kern_code_object_param_sizes(img, len(img), entry.encode(), sizes, 32, ctypes.byref(n)) == 0, \
            lib.kern_last_error()
        assert list(sizes[: n.value]) == want, entry
    toml = open(TOML).read()
    for entry in kb.ENTRIES:
        assert f'name = "{entry}"' in toml
    n = ctypes.c_int()
    sizes = (ctypes.c_uint32 * 4)()
    assert lib.kern_code_object_param_sizes(img, len(img), b"kern_mx_nope", sizes, 4, ctypes.byref(n)) == 2


_NZ = ctypes.c_void_p(16)  # a non-null address that no call here dereferences (the checks fail first)


@pytest.mark.parametrize("call,msg", [
    (lambda L: L.kern_moe_quant(None, None, None, 4, 33, None), "K % 32"),
    (lambda L: L.kern_moe_w_shuffle(None, None, 1, 15, 256, 0, None), "rows % 16"),
    (lambda L: L.kern_moe_w_shuffle(None, None, 1, 16, 256, 2, None), "gated"),
    (lambda L: L.kern_moe_sf_shuffle(None, None, 1, 16, 8, 0, None), "sf_cols % 16"),
    (lambda L: L.kern_mxfp4_gemv_bf16(None, None, None, None, 17, 512, 1024, None), "M <= 16"),
    (lambda L: L.kern_mxfp4_gemv_bf16(None, None, None, None, 1, 512, 1000, None), "K % 512"),
    (lambda L: L.kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(*([None] * 9), 100, 512, 4, 1, None, None), "m % 256"),
    (lambda L: L.kern_trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(*([None] * 13), 256, 512, 4, None, None), "null buffer"),
    (lambda L: L.kern_mxfp4_gemm_e4m3(*([None] * 6), 16, 256, 500, None, None), "k % 512"),
    (lambda L: L.kern_mxfp4_gemm_bf16(*([None] * 5), -1, 256, 512, None, None), "m % 256"),
    (lambda L: L.kern_moe_routing(*([None] * 8), 4, 2, 0, 513, None), "local_experts <= 512"),
    (lambda L: L.kern_moe_routing(*([_NZ] * 8), 1 << 28, 16, 0, 8, None), "past the i32 tables"),
    (lambda L: L.kern_moe_routing(*([_NZ] * 8), (2**31 - 1 - 128 * 512) // 8 + 1, 8, 0, 512, None), "past the i32 tables"),
    (lambda L: L.kern_fill_random_u8(None, 16, 1, 0, 0, None), "span"),
    (lambda L: L.kern_moe_quant_routing(None, None, None, 4, 7168, *([None] * 8), 8, 0, 513, None),
     "0 < local_experts <= 512"),
    (lambda L: L.kern_moe_quant_routing(None, None, None, 4, 7000, *([None] * 8), 8, 0, 64, None), "K % 32"),
    (lambda L: L.kern_moe_finalize_rms(*([None] * 5), 4, 8200, 8, 1e-6, None), "0 < H <= 8192"),
    (lambda L: L.kern_moe_finalize_rms(*([None] * 5), 4, 7168, 8, -1.0, None), "eps >= 0"),
    (lambda L: L.kern_moe_finalize_rms(*([None] * 5), 4, 7168, 8, 1e-6, None), "null buffer"),
    (lambda L: L.kern_moe_finalize(*([None] * 4), 4, 100, 8, None), "H % 8 == 0"),
    (lambda L: L.kern_mxfp8_quant_f32(None, None, None, 4, 33, None), "K % 32"),
    (lambda L: L.kern_mxfp8_gemm_bf16(*([None] * 5), 16, 16, 48, 16, None), "k % 32 == 0"),
    (lambda L: L.kern_mxfp8_gemm_bf16(*([None] * 5), 16, 32, 64, 16, None), "ldc >= n"),
    (lambda L: L.kern_mxfp8_gemm_bf16(*([_NZ] * 5), 16, 16, 0, 16, None), "k == 0 leaves c undefined"),
    (lambda L: L.kern_silu_mul(None, None, 4, 12, None), "d % 8 == 0"),
    (lambda L: L.kern_rope_table_bf16(None, None, 4, 2048, 4096, 10000.0, None), "0 < half <= 1024"),
    (lambda L: L.kern_iota_i32(None, 4, 0, 1, 0, None), "stride >= 1"),
    (lambda L: L.kern_fill_f32(None, 4, 1.0, None), "a buffer"),
    # the LDS ring addresses activations by 32-bit offsets from the buffer's base: past 4 GiB is refused
    (lambda L: L.kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(*([_NZ] * 9), 256, 8192, 4200, 1, None, None), "below 4 GiB"),
    (lambda L: L.kern_mxfp4_gemm_e4m3(*([_NZ] * 6), 1 << 20, 256, 8192, None, None), "below 4 GiB"),
    (lambda L: L.kern_mxfp4_gemm_bf16(*([_NZ] * 5), 1 << 20, 256, 8192, None, None), "below 4 GiB"),
])
def test_contract_violations_are_api_errors(lib, call, msg):
    rc = call(lib)
    assert rc == 4
    assert msg in lib.kern_last_error().decode()


def test_empty_work_is_a_noop(lib):
    # tokens == 0 / ctas == 0 launch nothing and touch no device memory
    assert lib.kern_moe_quant(None, None, None, 0, 64, None) == 0
    assert lib.kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(*([ctypes.c_void_p(16)] * 9), 256, 512, 0, 1, None, None) == 0


def test_python_mirror_has_no_cpu_fallback():
    """kern_amd.ops only calls the C ABI: it names no oracle module and never computes on the host."""
    src = open(os.path.join(ROOT, "kern_amd", "ops.py")).read()
    assert "oracle" not in src.replace("no CPU", "")
    for f in os.listdir(os.path.join(ROOT, "kern_amd")):
        if f.endswith(".py"):
            assert "import oracle" not in open(os.path.join(ROOT, "kern_amd", f)).read()
            assert "from oracle" not in open(os.path.join(ROOT, "kern_amd", f)).read()


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_code_object_build_is_path_independent(tmp_path):
    """The pin is reproducible: kern_mx.hip built from a copy of the sources in another directory, to
    another output path, hashes to the sha256 kernel_index/kern_mx.toml pins (hipcc's compilation-unit
    id would otherwise follow the paths)."""
    import shutil

    src = tmp_path / "elsewhere" / "csrc"
    shutil.copytree(kb.CSRC, src)
    sha = kb.build_code_object(str(src), str(tmp_path / "out" / "copy.hsaco"))
    assert sha == kb.pinned_sha256()


_FUZZ = r"""
import ctypes, random, sys
L = ctypes.CDLL(sys.argv[1])
img = open(sys.argv[2], "rb").read()
sizes = (ctypes.c_uint32 * 64)()
n = ctypes.c_int()
def call(b):
    rc = L.kern_code_object_param_sizes(b, len(b), b"kern_mx_quant_bf16", sizes, 64, ctypes.byref(n))
    assert rc in (0, 2), rc
    return rc
assert call(img) == 0
note = img.find(b"AMDGPU")  # the metadata note's name; its msgpack follows
assert note > 0
rng = random.Random(5)
for cut in list(range(0, 256)) + [note + d for d in range(-16, 4096, 7)] + [len(img) - d for d in range(1, 64)]:
    call(img[:max(0, cut)])
for _ in range(3000):
    b = bytearray(img)
    for _ in range(rng.randint(1, 4)):
        at = rng.randrange(note, min(len(b), note + 60000)) if rng.random() < 0.9 else rng.randrange(64)
        b[at] = rng.choice([0xc4, 0xc5, 0xc6, 0xdb, 0xdd, 0xdf, 0xff, 0x00, rng.randrange(256)])
    call(bytes(b))
# section header fields pushed to the edge of 64-bit range
for off, val in [(0x28, 2**64 - 8), (0x28, len(img)), (0x3a, 0), (0x3c, 0xffff)]:
    b = bytearray(img)
    b[off:off + (8 if off == 0x28 else 2)] = val.to_bytes(8 if off == 0x28 else 2, "little")
    call(bytes(b))
print("ok")
"""


def test_metadata_parser_survives_corrupt_images(lib, tmp_path):
    """kern_code_object_param_sizes parses caller-supplied images: truncated ones, corrupted msgpack lengths
    (bin/str/array/map sizes far past the data) and section headers at the edge of the 64-bit range are
    refused with KERN_ERR_KERNEL_ARTIFACT, never read past the image (run in a child process, so an
    out-of-bounds read would show as a crash here rather than end the test session)."""
    script = tmp_path / "fuzz.py"
    script.write_text(_FUZZ)
    r = subprocess.run([sys.executable, str(script), ops.LIB_PATH, ops.HSACO_PATH], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout[-500:], r.stderr[-2000:])
