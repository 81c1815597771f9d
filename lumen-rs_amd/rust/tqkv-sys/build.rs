// Links libtqkv.so: from TQKV_LIB_DIR if set, else the in-tree build
// (lumen-rs_amd/libtqkv.so, two directories up), plus the HIP runtime.
fn main() {
    let dir = std::env::var("TQKV_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR");
        format!("{}/../..", here)
    });
    println!("cargo:rustc-link-search=native={}", dir);
    println!("cargo:rustc-link-lib=dylib=tqkv");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=TQKV_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
