import ctypes as C
import importlib.util
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PKG_DIR = ROOT / "a6000-custom-kernels_amd"


def load_package():
    """Import the package directory (its name is not a Python identifier)."""
    name = "a6000_custom_kernels_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def mc():
    return load_package()


@pytest.fixture(scope="session")
def O():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    pkg = load_package()
    if not pkg.LIB_PATH.exists():
        pytest.fail(f"{pkg.LIB_PATH} not built: run __graft_entry__.build()")
    return torch


@pytest.fixture(scope="session")
def sim(mc):
    """The product's host code (mc_host.cpp) linked against the test-only simulated device."""
    lib_path = ROOT / "tests" / "native" / "_build" / "libmc_hostsim.so"
    srcs = [PKG_DIR / "csrc" / "mc_host.cpp", ROOT / "tests" / "native" / "sim_device.cpp",
            ROOT / "include" / "ggml_hip_moe_cache.h"]
    if not lib_path.exists() or max(p.stat().st_mtime for p in srcs) > lib_path.stat().st_mtime:
        spec = importlib.util.spec_from_file_location("mc_build", PKG_DIR / "build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_hostsim()
    lib = mc.bind(lib_path)
    lib.mc_sim_host_alloc.restype, lib.mc_sim_host_alloc.argtypes = C.c_void_p, [C.c_uint64]
    lib.mc_sim_plain_alloc.restype, lib.mc_sim_plain_alloc.argtypes = C.c_void_p, [C.c_uint64]
    lib.mc_sim_dev_alloc.restype, lib.mc_sim_dev_alloc.argtypes = C.c_void_p, [C.c_uint64]
    lib.mc_sim_set_mem_info.argtypes = [C.c_uint64, C.c_uint64]
    lib.mc_sim_fail_alloc_after.argtypes = [C.c_int]
    lib.mc_sim_fail_h2d_after.argtypes = [C.c_int]
    lib.mc_sim_live_regions.restype = C.c_longlong
    lib.mc_sim_counters.argtypes = [C.c_void_p]
    lib.mc_sim_live_streams_events.argtypes = [C.c_void_p]
    return lib
