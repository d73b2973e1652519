// Links libmivi_hip.so (built by `python mivi-v4_amd/build.py`, found through
// MIVI_HIP_LIB_DIR, default: the library's in-tree location next to this
// crate) and ROCm's HIP runtime (ROCM_PATH, default /opt/rocm).
fn main() {
    let here = std::env::var("CARGO_MANIFEST_DIR").unwrap_or_else(|_| ".".to_string());
    let lib_dir = std::env::var("MIVI_HIP_LIB_DIR").unwrap_or_else(|_| format!("{here}/../mivi_hip"));
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rerun-if-env-changed=MIVI_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rustc-link-search=native={lib_dir}");
    println!("cargo:rustc-link-lib=dylib=mivi_hip");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
