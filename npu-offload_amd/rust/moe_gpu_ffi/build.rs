// Links the prebuilt libmoe_gpu.so (built for gfx950 by `python npu-offload_amd/build.py` of this repository; cargo does
// not drive hipcc).  MOE_GPU_LIB_DIR names the directory that holds it (default: ../../lib relative to this crate).
fn main() {
    let dir = std::env::var("MOE_GPU_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").unwrap();
        format!("{here}/../../lib")
    });
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=moe_gpu");
    if std::env::var("CARGO_FEATURE_CK_SHIM").is_ok() {
        println!("cargo:rustc-link-lib=dylib=ck_gpu");
    }
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=MOE_GPU_LIB_DIR");
}
