//! Link libw4a16.so. Its directory comes from W4A16_LIB_DIR (the `triton-rs_amd/` directory
//! of a built checkout of the MI355X library), else the system search path; the HIP runtime
//! (libamdhip64) is a dependency of libw4a16 itself.
fn main() {
    println!("cargo:rerun-if-env-changed=W4A16_LIB_DIR");
    if let Ok(dir) = std::env::var("W4A16_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=w4a16");
}
