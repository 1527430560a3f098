//! Links `libhardshell_hip.so`, the gfx950 backend built by `taco_amd/build.py` (hipcc, no
//! cargo step compiles HIP). `HARDSHELL_HIP_LIB_DIR` names the directory that holds it.

fn main() {
    println!("cargo:rerun-if-env-changed=HARDSHELL_HIP_LIB_DIR");
    if let Ok(dir) = std::env::var("HARDSHELL_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=hardshell_hip");
}
