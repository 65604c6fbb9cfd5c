"""CPU: the C-ABI library loads without a GPU and exports exactly the functions
include/ggml_hip_moe_cache.h declares; host-side predicates behave without a device."""
import ctypes as C
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ggml_hip_moe_cache.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ggml_hip_\w+)\s*\(", text)))


def test_header_declares_reference_api():
    fns = declared_functions()
    for name in ("enabled", "wants", "mul_mat_vec_q", "step", "active", "pin_host"):
        assert f"ggml_hip_moe_cache_{name}" in fns


def test_library_exports_every_declared_symbol(mc):
    lib_path = mc.LIB_PATH
    assert lib_path.exists(), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True, check=True).stdout
    exported = sorted(set(l.split()[-1] for l in out.splitlines() if " T " in l))
    assert exported == declared_functions()
    lib = mc.lib()                                   # binds every signature in the Python mirror
    assert {name for name, _, _ in mc.SIGNATURES} == set(declared_functions())
    assert lib.ggml_hip_moe_version().startswith(b"ggml-hip-moe-cache")


def test_host_predicates_without_device(mc):
    lib = mc.lib()
    t = mc.make_tensor(mc.Q2_K, 256, 4, 8, 0, name="x")
    assert lib.ggml_hip_moe_cache_wants(C.byref(t)) in (0, 1)
    assert lib.ggml_hip_moe_cache_active() == 0
    t.type = 3
    assert lib.ggml_hip_moe_cache_wants(C.byref(t)) == 0
    # an unsupported type is an error code, never an abort
    rc = lib.ggml_hip_mul_mat_vec_q_moe(C.byref(t), None, 1, 1, 1, 256, 4, 8, 1, 1, 1, 0, 0, 1, 2, 8, 8, 8, 4, 2, None)
    assert rc < 0 and b"unsupported" in lib.ggml_hip_moe_last_error()
