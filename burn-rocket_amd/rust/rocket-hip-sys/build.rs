//! Builds `libburn_rocket_amd.so` for gfx950 (hipcc, through the package's own
//! build script) and links it. The library is built in-tree, next to the HIP
//! sources: `burn-rocket_amd/lib/`.
use std::{env, path::PathBuf, process::Command};

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"));
    // rust/rocket-hip-sys -> the burn-rocket_amd package
    let pkg = manifest.join("../..").canonicalize().expect("burn-rocket_amd package directory");
    let status = Command::new(env::var("PYTHON").unwrap_or_else(|_| "python3".into()))
        .arg(pkg.join("build.py"))
        .status()
        .expect("run burn-rocket_amd/build.py (needs hipcc from ROCm)");
    assert!(status.success(), "hipcc build of the gfx950 library failed");
    let lib = pkg.join("lib");
    println!("cargo:rustc-link-search=native={}", lib.display());
    println!("cargo:rustc-link-lib=dylib=burn_rocket_amd");
    // Let dependents find the .so at run time without LD_LIBRARY_PATH.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib.display());
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", pkg.join("../include/burn_rocket_amd.h").display());
}
