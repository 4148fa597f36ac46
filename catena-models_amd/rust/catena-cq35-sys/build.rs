// Link against libcq35.so. CQ35_LIB_DIR points at the directory holding it
// (the repository's catena-models_amd/cq35 after `__graft_entry__.build()`,
// or wherever it was installed); the HIP runtime it needs is found through
// ROCM_PATH (default /opt/rocm).
fn main() {
    println!("cargo:rerun-if-env-changed=CQ35_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if let Ok(dir) = std::env::var("CQ35_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=cq35");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
