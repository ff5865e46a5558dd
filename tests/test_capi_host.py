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
    (lambda L: L.kern_fill_random_u8(None, 16, 1, 0, 0, None), "span"),
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
