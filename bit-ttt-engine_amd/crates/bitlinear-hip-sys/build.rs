//! Links libbitlinear_hip.so (built by `python bit-ttt-engine_amd/build.py`, which
//! runs hipcc --offload-arch=gfx950) and the HIP runtime.
//!
//!   BTL_LIB_DIR   directory holding libbitlinear_hip.so (default: the package
//!                 directory two levels up, where build.py writes it)
//!   ROCM_PATH     ROCm install (default /opt/rocm), for libamdhip64.so

use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=BTL_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    let lib_dir = env::var("BTL_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join(".."));
    if !lib_dir.join("libbitlinear_hip.so").exists() {
        println!(
            "cargo:warning=libbitlinear_hip.so not found in {} (run python bit-ttt-engine_amd/build.py or set BTL_LIB_DIR)",
            lib_dir.display()
        );
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=bitlinear_hip");
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the library's directory on the runtime search path of binaries built against it
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
}
