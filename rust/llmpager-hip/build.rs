//! Link against libllmpager_hip.so, the C ABI of the gfx950 MoE path, built
//! by `python -m llmpager_amd.build` into llmpager_amd/lib/ (its gfx950 code
//! objects sit beside it and are found by lp_init).
fn main() {
    let lib = std::env::var("LLMPAGER_HIP_LIB").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").unwrap();
        format!("{here}/../../llmpager_amd/lib")
    });
    println!("cargo:rerun-if-env-changed=LLMPAGER_HIP_LIB");
    println!("cargo:rustc-link-search=native={lib}");
    println!("cargo:rustc-link-lib=dylib=llmpager_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{lib}");
}
