// The HIP half of the crate's build.rs: compiles the backend's sources (this
// repository's swin2sr-rs_amd/csrc and include/swin2sr_hip.h, copied together
// to the crate as hip/) into libswin2sr_hip.so with hipcc
// for gfx950, and links it. Replaces the nvcc/fatbin step of the `cuda`
// feature (reference build.rs:79-128). Included from build.rs:
//
//     include!("build_hip.rs");
//     fn main() {
//         #[cfg(feature = "cuda")] build_cuda();   // the existing steps
//         if std::env::var_os("CARGO_FEATURE_HIP").is_some() { build_hip(); }
//     }
//
// Packed fp32 VALU ops are disabled for all device code (they have given wrong
// results on MI355X pools); no CUDA headers or dual paths are involved.
#[allow(dead_code)]
fn build_hip() {
    use std::path::Path;
    use std::process::Command;
    let dir = Path::new("hip");
    let out = std::env::var("OUT_DIR").expect("OUT_DIR");
    let hipcc = std::env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let arch = std::env::var("SWIN2SR_HIP_ARCH").unwrap_or_else(|_| "gfx950".into());
    let srcs = ["s2s_kernels.hip", "s2s_api.cpp", "s2s_test_api.cpp", "s2s_selftest.cpp"];
    let status = Command::new(&hipcc)
        .arg(format!("--offload-arch={arch}"))
        .args(["-O3", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-DS2S_EXPORT", "-I"])
        .arg(dir)
        // the .cpp files hold device code too (the no-alloc workspace, the
        // launch wrappers): compile every source as HIP
        .args(["-x", "hip"])
        .args(srcs.iter().map(|s| dir.join(s)))
        .arg("-o")
        .arg(format!("{out}/libswin2sr_hip.so"))
        .status()
        .expect("running hipcc (set HIPCC=/path/to/hipcc)");
    assert!(status.success(), "hipcc failed building libswin2sr_hip.so");
    println!("cargo:rustc-link-search=native={out}");
    println!("cargo:rustc-link-lib=dylib=swin2sr_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{out}");
    for s in srcs.iter().chain(["s2s_kernels.h", "swin2sr_hip.h"].iter()) {
        println!("cargo:rerun-if-changed=hip/{s}");
    }
    println!("cargo:rerun-if-env-changed=HIPCC");
    println!("cargo:rerun-if-env-changed=SWIN2SR_HIP_ARCH");
}
