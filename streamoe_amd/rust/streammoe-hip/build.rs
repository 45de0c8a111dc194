//! Links libsmoe.so (built in-tree by `python streamoe_amd/build.py`) and
//! the HIP runtime. SMOE_LIB_DIR overrides where libsmoe.so is found (default:
//! the package directory two levels up, streamoe_amd/); ROCM_PATH overrides
//! /opt/rocm.
use std::env;
use std::path::PathBuf;

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let lib_dir = env::var("SMOE_LIB_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("..").join(".."));
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=smoe");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=SMOE_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}
