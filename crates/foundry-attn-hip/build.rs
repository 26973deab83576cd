// Links libfoundry_attn.so (built by `make -C foundry-trainer_amd`) and the
// HIP runtime.  FOUNDRY_ATTN_LIB_DIR names the directory holding the library;
// ROCM_PATH defaults to /opt/rocm.
fn main() {
    println!("cargo:rerun-if-env-changed=FOUNDRY_ATTN_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let dir = std::env::var("FOUNDRY_ATTN_LIB_DIR")
        .expect("set FOUNDRY_ATTN_LIB_DIR to the directory holding libfoundry_attn.so");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=foundry_attn");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // find both at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{rocm}/lib");
}
