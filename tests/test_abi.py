"""libtqkv.so loads and exports every entry point include/tqkv.h declares
(no GPU needed: nothing here launches a kernel)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "tqkv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tqkv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import tqkv
    lib = tqkv.lib()
    names = declared()
    assert len(names) >= 6
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_status_strings_without_a_gpu():
    import tqkv
    assert tqkv.status_name(tqkv.EUNSUPPORTED) == "TQKV_EUNSUPPORTED"
    assert tqkv.status_name(12345) == "TQKV_UNKNOWN"
    assert tqkv.lib().tqkv_version() == 200


def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of the header's structs have the C compiler's sizes
    and field offsets, and the library reports the header's ABI version."""
    import ctypes
    import subprocess
    import tqkv
    structs = {"tqkv_cache_config": tqkv.CacheConfig, "tqkv_cache_view": tqkv.CacheView,
               "tqkv_cache_state": tqkv.CacheState, "tqkv_tq_config": tqkv.TqConfig}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "tqkv.h"', "int main(void) {",
             '  printf("version %d\\n", TQKV_ABI_VERSION);']
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "abi.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:-1]): int(l.split()[-1]) for l in out if l}
    assert got[("version",)] == tqkv.lib().tqkv_version()
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)
    assert got[("tqkv_cache_config", "size")] == 72


def test_argument_checks_come_before_any_launch():
    import tqkv
    assert tqkv.lib().tqkv_empty_launch(0, None) == tqkv.EINVAL_ARG
    assert tqkv.lib().tqkv_read_probe(None, 16, None, 0, None, None) == tqkv.EINVAL_ARG


def test_workspace_size_is_host_arithmetic():
    import tqkv
    n = tqkv.decode_workspace_size(32, 16, 8, 256, 32768)
    assert n > 32 * 16 * 256 * 4
    assert tqkv.decode_workspace_size(0, 16, 8, 256, 10) == 0
    # The prefill's dequantize-once rows: K and V, 2 bytes a value; at head
    # dim 128 a slab holds whole 64-key tiles.
    assert tqkv.prefill_workspace_size(4, 8, 128, 16384) == 2 * 4 * 8 * 16384 * 128 * 2
    assert tqkv.prefill_workspace_size(4, 8, 128, 3071) == 2 * 4 * 8 * 3072 * 128 * 2
    assert tqkv.prefill_workspace_size(1, 2, 256, 3071) == 2 * 1 * 2 * 3071 * 256 * 2
    assert tqkv.prefill_workspace_size(1, 2, 128, 0) == 0


def test_baseline_layouts_take_the_mfma_kernel(monkeypatch):
    import tqkv
    monkeypatch.delenv("TQKV_DECODE_KERNEL", raising=False)
    assert tqkv.decode_kernel_name(16, 8, 256, 64, 3, 3) == "mfma"  # config 2
    assert tqkv.decode_kernel_name(32, 8, 128, 64, 4, 4) == "mfma"  # configs 1 and 3
    assert tqkv.decode_kernel_name(32, 8, 128, 64, 8, 4) == "mfma"  # config 4
    assert tqkv.decode_kernel_name(16, 2, 512, 64, 8, 8) == "tiles"  # D = 512: tile kernel
    assert tqkv.decode_kernel_name(16, 8, 256, 64, 5, 5) == "mfma"  # bit-anchored windows
    assert tqkv.decode_kernel_name(32, 8, 128, 64, 6, 6) == "mfma"  # Gemma's 6-bit cache
    assert tqkv.decode_kernel_name(32, 4, 128, 64, 3, 3) == "dot2"  # 8 heads: two launches
    assert tqkv.decode_kernel_name(16, 8, 256, 32, 4, 4) == "mfma"  # gs32 (16 A rows)
    assert tqkv.decode_kernel_name(32, 8, 128, 32, 6, 6) == "mfma"
    assert tqkv.decode_kernel_name(16, 8, 128, 128, 8, 4) == "mfma"
    assert tqkv.decode_kernel_name(32, 8, 256, 32, 4, 4) == "mfma"  # 32 A rows: 2 launches of 16
    assert tqkv.decode_kernel_name(16, 8, 256, 64, 7, 7) == ""
    assert tqkv.decode_kernel_name(16, 8, 256, 64, 5, 4) == ""
    assert tqkv.decode_kernel_name(20, 4, 128, 64, 4, 4) == "mfma"  # 5 heads: 5 launches of 1
    assert tqkv.decode_kernel_name(32, 2, 512, 64, 4, 4) == "tiles"  # Gemma 4 full attention
    assert tqkv.decode_kernel_name(32, 2, 128, 64, 4, 4) == "mfma"  # 16 heads: 2 launches of 8
    assert tqkv.decode_kernel_name(66, 2, 128, 64, 4, 4) == ""  # 33 heads: past the limit
    assert tqkv.decode_kernel_name(64, 8, 256, 64, 4, 4) == "mfma"  # 8 heads: 2 MFMA launches of 4
    monkeypatch.setenv("TQKV_DECODE_KERNEL", "dot2")
    assert tqkv.decode_kernel_name(16, 8, 256, 64, 3, 3) == "dot2"


def test_long_segments_take_the_dot2_kernel(monkeypatch):
    """The MFMA kernel addresses a unit's rows with 32-bit byte offsets: a
    segment of max_rows rows with max_rows * D >= 2^31 takes the dot2 kernel,
    and tqkv_cache_append_decode checks this with the real segment lengths
    before it commits an update (a fused append needs the MFMA kernel)."""
    import tqkv
    monkeypatch.delenv("TQKV_DECODE_KERNEL", raising=False)
    for D in (64, 128, 256):
        edge = (1 << 31) // D
        assert tqkv.decode_kernel_for_rows(16, 8, D, 64, 4, 4, edge - 1) == "mfma"
        assert tqkv.decode_kernel_for_rows(16, 8, D, 64, 4, 4, edge) == "dot2"
    assert tqkv.decode_kernel_for_rows(16, 8, 256, 64, 4, 4, 0) == \
        tqkv.decode_kernel_name(16, 8, 256, 64, 4, 4)
    assert tqkv.decode_kernel_for_rows(16, 8, 256, 64, 4, 4, -1) == ""


def test_codebook_decode_refuses_other_head_groups_without_a_gpu():
    """Query heads per KV head must be 1, 2, 4, 8 or 16: the decode splits a
    KV head's heads into power-of-two groups across wavefronts, so 3 or 12
    heads a KV head would leave heads out. The refusal comes before any
    device call (the pointers below are never dereferenced)."""
    import tqkv
    lib = tqkv.lib()
    p = ctypes.c_void_p(4096)
    for H, H_kv in ((6, 2), (24, 2), (64, 2)):
        rc = lib.tqkv_decode_attend_codebook(p, 1, H, H_kv, 512, ctypes.c_float(1.0), p, p, 4, p,
                                             4, p, p, p, p, 64, 64, p, p, 1 << 20, None)
        assert rc == tqkv.EUNSUPPORTED, (H, H_kv, rc)
