// build.rs of the wave-engine crate: builds and links the MI355X attention tier
// (libwave_hip_attn.so, gfx950 code objects) when the `hip` feature is on, so
// the default build needs no ROCm.  The `--hip` flag (src/cli.rs:208-210)
// then selects hip_tier::HipBackend at the GpuBackend construction site
// (src/cpu/train_loop.rs:209-214).
fn main() {
    if std::env::var_os("CARGO_FEATURE_HIP").is_some() {
        let dir = std::env::var("WAVE_HIP_DIR").unwrap_or_else(|_| "../wave-engine_amd".into());
        let ok = std::process::Command::new("make").args(["-C", &dir]).status()
            .expect("make not found");
        assert!(ok.success(), "building libwave_hip_attn.so failed");
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-lib=dylib=wave_hip_attn");
        // hip_tier::device binds hipMalloc / hipMemcpy / hipFree for caller-owned device buffers
        let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
        println!("cargo:rustc-link-search=native={rocm}/lib");
        println!("cargo:rustc-link-lib=dylib=amdhip64");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
        println!("cargo:rerun-if-changed={dir}/csrc");
    }
}
