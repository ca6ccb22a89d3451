// Link libferrum_hip.so.  FERRUM_HIP_LIB_DIR names the directory holding it;
// by default the in-tree build (`make -C ferrum-cpu_amd` writes
// ferrum-cpu_amd/lib/libferrum_hip.so, two levels above this crate).  The
// library needs the ROCm runtime (libamdhip64) at run time.
use std::env;
use std::path::PathBuf;

fn main() {
    println!("cargo:rerun-if-env-changed=FERRUM_HIP_LIB_DIR");
    let dir = match env::var_os("FERRUM_HIP_LIB_DIR") {
        Some(d) => PathBuf::from(d),
        None => PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR"))
            .join("..")
            .join("..")
            .join("lib"),
    };
    println!("cargo:rustc-link-search=native={}", dir.display());
    println!("cargo:rustc-link-lib=dylib=ferrum_hip");
    // the same directory at run time, for tests and examples run from the tree
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", dir.display());
}
