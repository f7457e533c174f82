// Fragment for the reference's build.rs (build.rs:1-44): call link_mvr_attn()
// from main() after the proto build.  It links libmvr_attn.so, built by
// `make -C mini-vllm-rs_amd` (hipcc, gfx950), and records the rpath so the
// binary finds it at run time.  MVR_ATTN_DIR overrides the library's folder.

fn link_mvr_attn() {
    println!("cargo:rerun-if-env-changed=MVR_ATTN_DIR");
    let dir = std::env::var("MVR_ATTN_DIR").unwrap_or_else(|_| "mini-vllm-rs_amd".into());
    println!("cargo:rerun-if-changed={dir}/libmvr_attn.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=mvr_attn");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
