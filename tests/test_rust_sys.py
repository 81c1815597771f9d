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


# ---------------------------------------------------------------- the safe crate
SAFE = os.path.join(ROOT, "lumen-rs_amd", "rust", "tqkv")

# turboquant_cache::KVCache (crates/turboquant-cache/src/traits.rs:9-36): the
# six required methods, their receivers and argument types, as the trait
# declares them.
KVCACHE_TRAIT = {
    "store": "&mut self, layer: usize, head: usize, keys: &[f32], values: &[f32], n_tokens: usize",
    "attend_keys": "&self, layer: usize, head: usize, query: &[f32]",
    "attend_values": "&self, layer: usize, head: usize, weights: &[f32]",
    "seq_len": "&self, layer: usize, head: usize",
    "clear": "&mut self",
    "truncate": "&mut self, layer: usize, n_keep: usize",
}


def _split_top(args):
    """Split a call's argument text at top-level commas."""
    out, depth, cur = [], 0, ""
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [a.strip() for a in out if a.strip()]


def _calls(src, prefix):
    """(name, [args]) for every `prefix<name>(...)` call in src."""
    found = []
    for m in re.finditer(re.escape(prefix) + r"(tqkv_[a-z0-9_]+)\(", src):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(src[i], 0)
            i += 1
        found.append((m.group(1), _split_top(src[m.end():i - 1])))
    return found


def _bound_arity():
    rs = open(os.path.join(CRATE, "src", "bindings.rs")).read()
    return {m.group(1): len(_split_top(m.group(2)))
            for m in re.finditer(r"pub fn (tqkv_[a-z0-9_]+)\((.*?)\)( ->|;)", rs)}


def test_safe_crate_calls_match_the_header():
    """Every libtqkv call in the safe crate names a function the header
    declares, with as many arguments as it takes; every tqkv_kvcache_*
    entry is used; every constant it names is bound."""
    src = open(os.path.join(SAFE, "src", "lib.rs")).read()
    arity = _bound_arity()
    calls = _calls(src, "sys::")
    assert calls, "no libtqkv calls found"
    for name, args in calls:
        assert name in arity, f"{name} is not in include/tqkv.h"
        assert len(args) == arity[name], f"{name}: {len(args)} arguments, header has {arity[name]}"
    header = open(os.path.join(ROOT, "include", "tqkv.h")).read()
    kv = {f for f in _gen().header_functions(header) if f.startswith("tqkv_kvcache_")}
    assert kv <= {n for n, _ in calls}, f"unused: {sorted(kv - {n for n, _ in calls})}"
    rs = open(os.path.join(CRATE, "src", "bindings.rs")).read()
    for const in set(re.findall(r"sys::(TQKV_[A-Z0-9_]+)", src)):
        assert f"pub const {const}:" in rs, const
    start = src.index("sys::tqkv_tq_config {") + len("sys::tqkv_tq_config {")
    body = src[start:src.index("\n        })", start)]
    fields = [f.split(":")[0].strip() for f in _split_top(body)]
    struct = re.search(r"pub struct tqkv_tq_config \{([^}]*)\}", rs).group(1)
    assert sorted(fields) == sorted(re.findall(r"pub (\w+):", struct))


def test_safe_crate_implements_the_reference_trait():
    src = open(os.path.join(SAFE, "src", "lib.rs")).read()
    body = src[src.index("impl KVCache for DeviceCache {"):]
    got = {m.group(1): re.sub(r"\s+", " ", m.group(2)).strip()
           for m in re.finditer(r"\bfn (\w+)\((.*?)\)", body, flags=re.S)}
    assert got == KVCACHE_TRAIT
    assert "use turboquant_cache::traits::KVCache;" in src
    # Send + Sync (the trait's supertraits) come through the Mutex over a
    # Send handle; no blanket unsafe impl Sync.
    assert "unsafe impl Send for Raw {}" in src and "unsafe impl Sync" not in src


def test_safe_crate_hygiene():
    """Every unsafe block carries a SAFETY comment; brackets balance (no
    Rust toolchain here to parse the crate); the manifest names the sys
    crate and the reference's trait crate."""
    import tomli
    for path in [os.path.join(SAFE, "src", "lib.rs"),
                 os.path.join(SAFE, "tests", "simple_cache_parity.rs")]:
        src = open(path).read()
        lines = src.splitlines()
        for i, line in enumerate(lines):
            if re.search(r"\bunsafe \{", line):
                window = "\n".join(lines[max(0, i - 8):i + 1])
                assert "// SAFETY:" in window, f"{path}:{i + 1} unsafe block without SAFETY"
        code = re.sub(r"//[^\n]*", "", src)
        code = re.sub(r'"(\\.|[^"\\])*"', '""', code)
        code = re.sub(r"'(\\.|[^'\\])'", "' '", code)
        for o, c in ["()", "[]", "{}"]:
            assert code.count(o) == code.count(c), f"{path}: unbalanced {o}{c}"
    with open(os.path.join(SAFE, "Cargo.toml"), "rb") as f:
        man = tomli.load(f)
    assert man["dependencies"]["tqkv-sys"]["path"] == "../tqkv-sys"
    assert man["dependencies"]["turboquant-cache"] == {"workspace": True}
