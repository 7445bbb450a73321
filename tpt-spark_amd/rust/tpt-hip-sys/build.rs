// NOT COMPILED HERE (no Rust toolchain in the build image).
// Links the prebuilt libtpthip.so (`make -C tpt-spark_amd/csrc`).  TPTHIP_LIB_DIR names the
// directory that holds it; the library itself needs only the ROCm runtime (libamdhip64).
fn main() {
    let dir = std::env::var("TPTHIP_LIB_DIR")
        .expect("set TPTHIP_LIB_DIR to the directory holding libtpthip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=tpthip");
    println!("cargo:rerun-if-env-changed=TPTHIP_LIB_DIR");
}
