// Links liblnskv.so (built by `make -C lns-ml_amd`, one directory up unless
// LNSKV_LIB_DIR says otherwise) and the HIP runtime (ROCM_PATH, default
// /opt/rocm), and records the library directory as an rpath so tests and
// binaries find liblnskv.so without LD_LIBRARY_PATH.
use std::env;
use std::path::PathBuf;

fn main() {
    let here = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let lib_dir = env::var("LNSKV_LIB_DIR").map(PathBuf::from).unwrap_or_else(|_| here.join(".."));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-lib=dylib=lnskv");
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=LNSKV_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed=../../include/lnskv.h");
}
