//! Links libitts_hip.so: from ITTS_HIP_LIB_DIR, else the library's in-tree build
//! (index-tts-rs_amd/lib, next to this crate's parent folder).
use std::env;
use std::path::PathBuf;

fn main() {
    let dir = env::var_os("ITTS_HIP_LIB_DIR").map(PathBuf::from).unwrap_or_else(|| {
        PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("..")
            .join("..")
            .join("lib")
    });
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=itts_hip");
    println!("cargo:rerun-if-env-changed=ITTS_HIP_LIB_DIR");
}
