//! Links liblbt_hip.so, built for gfx950 by the lemonade-burn_amd package
//! (`python lemonade-burn_amd/build.py`).  LBT_HIP_LIB_DIR names the folder
//! that holds it.
fn main() {
    println!("cargo:rerun-if-env-changed=LBT_HIP_LIB_DIR");
    if let Ok(dir) = std::env::var("LBT_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=lbt_hip");
}
