"""The LKV2 reader and writer (lumen-rs_amd/csrc/lkv.cpp) under
AddressSanitizer and UndefinedBehaviorSanitizer, on the host only (no GPU):
tests/lkv_sanitize_main.cpp runs the reference's fault sweeps
(crates/lumen-mlx/tests/kv_disk_faults.rs: every truncation, every
single-byte flip, a trailing byte) and 20000 seeded mutations per snapshot
over the snapshots written here, each input in a heap block of exactly its
own size, so any read past the end of a truncated file, any overflow in the
length arithmetic and any leak fails the run.

The sanitizers instrument the host pass only (-Xarch_host before each
-fsanitize=); the library's device code is not built into this binary.
"""
import os
import shutil
import struct
import subprocess
import sys

import pytest

import lkv_py as L
from test_lkv_format import sample

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "_build")
EXE = os.path.join(BUILD, "lkv_sanitize")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def exe():
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc is not installed")
    os.makedirs(BUILD, exist_ok=True)
    csrc = os.path.join(ROOT, "lumen-rs_amd", "csrc")
    san = []
    for s in ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all",
              "-fno-omit-frame-pointer"]:
        san += ["-Xarch_host", s]
    cmd = [HIPCC if os.path.exists(HIPCC) else "hipcc", "-x", "hip", "--offload-arch=gfx950",
           "-O1", "-g", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-I", csrc, *san,
           os.path.join(csrc, "lkv.cpp"), os.path.join(csrc, "status.cpp"),
           os.path.join(ROOT, "tests", "lkv_sanitize_main.cpp"), "-o", EXE]
    subprocess.run(cmd, check=True, capture_output=True)
    return EXE


def snapshots(tmp_path):
    m, recs = sample()
    files = {"sample.lkv": L.write(m, recs)}
    layers = [
        L.layer("SlidingQuantized", 5000, 0, [0, 1, None, 3], max_size=1024, keep=0, idx=17,
                bits=4, group_size=64),
        L.layer("FullTurboquant", 77, 3, [None, None], max_size=2 ** 64 - 1, keep=4, idx=9,
                bits=3, qjl_m=128),
        L.layer("Linear", 2, 0, [], lengths_id=1, left_padding_id=0),
    ]
    m2 = L.manifest("fp \"quoted\" \\ \x01\t\n é☃", 2 ** 64 - 1, 0, [], None, False, layers)
    recs2 = [(L.DTYPES["U8"], [0], b""), (L.DTYPES["I64"], [2, 1], struct.pack("<2q", -1, 2)),
             (L.DTYPES["Bool"], [], b""), (L.DTYPES["BF16"], [1, 2, 1, 1], b"\x80\x3f\x80\xbf")]
    files["options.lkv"] = L.write(m2, recs2)
    loose = b'{ "layers": [ ], "is_deep": false, "prefix_tokens": [ 9 ],\n' \
            b'  "position": 1, "created_at_unix": 2, "model_fingerprint": "\\u0041\\ud83d\\ude00" }'
    files["loose.lkv"] = L.write(None, [], raw_json=loose)
    js = L.manifest_bytes(m)
    files["duplicate.bad"] = L.write(m, recs, raw_json=js[:-1] + b',"position":7}')
    files["garbage.bad"] = L.write(m, recs, raw_json=b"#" * len(js))
    files["bigshape.bad"] = L.write(m, [(L.DTYPES["U64"], [2 ** 31 - 1] * 8, b"")])
    paths = []
    for name, data in files.items():
        p = tmp_path / name
        p.write_bytes(data)
        paths.append(str(p))
    return paths


def test_fault_sweeps_under_sanitizers(exe, tmp_path):
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([exe, *snapshots(tmp_path)], env=env, capture_output=True, text=True,
                       timeout=600)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    assert r.stdout.startswith("lkv_sanitize:")
