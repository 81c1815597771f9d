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
    assert tqkv.lib().tqkv_version() >= 100


def test_argument_checks_come_before_any_launch():
    import tqkv
    assert tqkv.lib().tqkv_empty_launch(0, None) == tqkv.EINVAL_ARG
    assert tqkv.lib().tqkv_read_probe(None, 16, None, 0, None, None) == tqkv.EINVAL_ARG


def test_workspace_size_is_host_arithmetic():
    import tqkv
    n = tqkv.decode_workspace_size(32, 16, 8, 256, 32768)
    assert n > 32 * 16 * 256 * 4
    assert tqkv.decode_workspace_size(0, 16, 8, 256, 10) == 0


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
