//! Links libkiln_hip.so (built by `python -m kiln_amd.build`, or installed) and
//! the HIP runtime it depends on.
fn main() {
    let dir = std::env::var("KILN_HIP_LIB_DIR").unwrap_or_else(|_| "/opt/kiln_hip/lib".into());
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=kiln_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=KILN_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
