"""The Rust -sys crate (lumen-rs_amd/rust/tqkv-sys) against include/tqkv.h.

No Rust toolchain exists in this image, so the crate is not compiled here;
its bindings are generated from the header, and this test keeps them in step:
the committed src/bindings.rs must equal a fresh generation, declare every
function the header declares, and carry every struct with its fields.
"""
import importlib.util
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "lumen-rs_amd", "rust", "tqkv-sys")


def _gen():
    spec = importlib.util.spec_from_file_location("gen_bindings",
                                                  os.path.join(CRATE, "gen_bindings.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bindings_are_current():
    g = _gen()
    header = open(os.path.join(ROOT, "include", "tqkv.h")).read()
    committed = open(os.path.join(CRATE, "src", "bindings.rs")).read()
    assert committed == g.generate(header), "rerun gen_bindings.py"


def test_every_header_function_is_bound():
    g = _gen()
    header = open(os.path.join(ROOT, "include", "tqkv.h")).read()
    rs = open(os.path.join(CRATE, "src", "bindings.rs")).read()
    bound = set(re.findall(r"pub fn (tqkv_[a-z0-9_]+)\(", rs))
    assert set(g.header_functions(header)) == bound


def test_type_mapping():
    g = _gen()
    assert g.rust_type("const void* const*", set()) == "*const *const c_void"
    assert g.rust_type("tqkv_cache**", set()) == "*mut *mut tqkv_cache"
    assert g.rust_type("const char*", set()) == "*const c_char"
    assert g.rust_type("size_t", set()) == "usize"
    assert g.rust_type("const tqkv_cache* const*", set()) == "*const *const tqkv_cache"
    rs = open(os.path.join(CRATE, "src", "bindings.rs")).read()
    # A struct whose layout the kernels rely on: field order and widths.
    seg = re.search(r"pub struct tqkv_affine_seg \{(.*?)\}", rs, flags=re.S).group(1)
    assert [f.split(":")[0].strip().replace("pub ", "") for f in seg.strip().splitlines()] == \
        ["k_packed", "k_scales", "k_biases", "v_packed", "v_scales", "v_biases", "cap", "n",
         "shared", "reserved"]
    assert "pub slot: [*mut c_void; 6]," in rs and "pub row_bytes: [i64; 6]," in rs
