// Links libwebyiq_q4q8.so, built in-tree by `python -m webyiq_amd.build`
// (hipcc --offload-arch=gfx950).  WEBYIQ_HIP_LIB_DIR names the directory
// holding it (webyiq_amd/ of this repository by default layout).
fn main() {
    let dir = std::env::var("WEBYIQ_HIP_LIB_DIR").unwrap_or_else(|_| {
        let root = std::path::Path::new(env!("CARGO_MANIFEST_DIR")).join("../../webyiq_amd");
        root.to_string_lossy().into_owned()
    });
    println!("cargo:rerun-if-env-changed=WEBYIQ_HIP_LIB_DIR");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=webyiq_q4q8");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
