"""The product's cache index math (lumen-rs_amd/csrc/cache_plan.hpp), run by
a host-memory executor, against the digests the reference recorded for every
cache kind and plan (golden_tests.rs:413-497): step-256 growth, the legacy
concatenating path, ring writes, wrap-around, trims, rewinds and refusals.
No GPU: the device executor replays the same plans in test_gpu_cache.py."""
import ctypes
import os
import subprocess

import pytest

from test_oracle_golden import RECORDED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "_build")
LIB = os.path.join(BUILD, "libcacheplanhost.so")


@pytest.fixture(scope="module")
def host():
    import oracle_lib
    oracle_lib.lib()  # builds liboracle.so if needed
    os.makedirs(BUILD, exist_ok=True)
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC",
                    "-I", os.path.join(ROOT, "lumen-rs_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cache_plan_host.cpp"),
                    "-L", os.path.join(ROOT, "oracle"), "-loracle",
                    "-Wl,-rpath," + os.path.join(ROOT, "oracle"), "-o", LIB], check=True)
    lib = ctypes.CDLL(LIB)
    lib.planhost_golden_digest.restype = ctypes.c_uint64
    lib.planhost_golden_digest.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
    return lib


@pytest.mark.parametrize("kind,plan,prealloc,want", RECORDED)
def test_planner_reproduces_reference_recording(host, kind, plan, prealloc, want):
    got = host.planhost_golden_digest(kind.encode(), plan.encode(), int(prealloc))
    assert got == want, f"{kind}/{plan}/prealloc={prealloc}: {got:#x} != {want:#x}"
