//! Builds `libstarlight_hip.so` (the gfx950 code objects and the C ABI of
//! `include/starlight_hip.h`) with the repository's own Makefile and links
//! the crate against it.
//!
//! The repository root is `STARLIGHT_AMD_DIR` when set, else two directories
//! above this crate (`starlight_amd/backend-hip` -> the root). `hipcc` must be
//! on the path the Makefile uses (`/opt/rocm/bin/hipcc` by default; override
//! with `HIPCC`).
use std::env;
use std::path::PathBuf;
use std::process::Command;

fn main() {
    let root = match env::var("STARLIGHT_AMD_DIR") {
        Ok(dir) => PathBuf::from(dir),
        Err(_) => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("../..")
            .canonicalize()
            .expect("repository root"),
    };
    let csrc = root.join("starlight_amd").join("csrc");
    let jobs = env::var("NUM_JOBS").unwrap_or_else(|_| "8".to_string());
    let mut make = Command::new("make");
    make.arg("-C").arg(&csrc).arg(format!("-j{jobs}")).arg("ARCH=gfx950");
    if let Ok(hipcc) = env::var("HIPCC") {
        make.arg(format!("HIPCC={hipcc}"));
    }
    let status = make.status().expect("make could not be started");
    assert!(status.success(), "building libstarlight_hip.so failed");

    let lib = root.join("starlight_amd").join("lib");
    println!("cargo:rustc-link-search=native={}", lib.display());
    println!("cargo:rustc-link-lib=dylib=starlight_hip");
    // the shared library is found at run time next to the build's own rpath
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib.display());
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", root.join("include").display());
    println!("cargo:rerun-if-env-changed=STARLIGHT_AMD_DIR");
    println!("cargo:rerun-if-env-changed=HIPCC");
}
