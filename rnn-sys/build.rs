// Links librnn.so (built by `python -m rustnn_amd.build` into rustnn_amd/)
// and the HIP runtime it needs.  RNN_LIB_DIR overrides the library folder,
// ROCM_PATH the ROCm install (default /opt/rocm).
fn main() {
    let dir = std::env::var("RNN_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR");
        format!("{here}/../rustnn_amd")
    });
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=rnn");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=RNN_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed=../include/rnn.h");
}
