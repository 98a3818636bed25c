//! The FFI to libswin2sr_hip.so (include/swin2sr_hip.h), in the place
//! `src/cuda.rs` and `lightgpu::vm` take in the CUDA build.
//!
//! Copy to the crate as `src/hip.rs`; `src/lib.rs` declares it under the `hip`
//! feature (see `gpu_hip.rs` for the module wiring). Every call returns the
//! library's message as the crate's `Result<_, String>` error; an allocation
//! failure's message contains "out of memory", which is what
//! `run_with_fallback`'s `is_out_of_memory` keys its tile-halving retry on
//! (reference src/main.rs:655-662).
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr};

/// `s2s_arch`: the checkpoint's `__metadata__` (reference src/weights.rs:66-137).
#[repr(C)]
pub struct S2sArch {
    pub upsampler: c_int,
    pub scale: c_int,
    pub window: c_int,
    pub embed: c_int,
    pub heads: c_int,
    pub mlp_ratio: c_int,
    pub n_stages: c_int,
    pub depths: [c_int; 16],
    pub img_range: f32,
    pub mean: [f32; 3],
}

/// `s2s_tensor`: one named f32 tensor, borrowed for the duration of a call.
#[repr(C)]
pub struct S2sTensor {
    pub name: *const c_char,
    pub data: *const f32,
    pub ndim: c_int,
    pub shape: [i64; 4],
}

/// The opaque `s2s_ctx`.
#[repr(C)]
pub struct S2sCtx {
    _p: [u8; 0],
}

#[link(name = "swin2sr_hip")]
extern "C" {
    pub fn s2s_create(arch: *const S2sArch, t: *const S2sTensor, n: usize, out: *mut *mut S2sCtx) -> c_int;
    pub fn s2s_destroy(ctx: *mut S2sCtx);
    pub fn s2s_name() -> *const c_char;
    pub fn s2s_uploaded_bytes(ctx: *const S2sCtx) -> u64;
    pub fn s2s_uploaded_bytes_for(arch: *const S2sArch, t: *const S2sTensor, n: usize, bytes: *mut u64) -> c_int;
    pub fn s2s_plan_bytes(ctx: *mut S2sCtx, h: c_int, w: c_int, bytes: *mut u64) -> c_int;
    pub fn s2s_set_alloc_limit(ctx: *mut S2sCtx, bytes: u64) -> c_int;
    pub fn s2s_forward(ctx: *mut S2sCtx, h: c_int, w: c_int, inp: *const f32, out: *mut f32) -> c_int;
    pub fn s2s_forward_device(ctx: *mut S2sCtx, h: c_int, w: c_int, d_in: *const f32, d_out: *mut f32) -> c_int;
    pub fn s2s_forward_batch(
        ctx: *mut S2sCtx,
        n: c_int,
        h: *const c_int,
        w: *const c_int,
        inp: *const *const f32,
        out: *const *mut f32,
        aux_out: *const *mut f32,
    ) -> c_int;
    pub fn s2s_aux(ctx: *mut S2sCtx, ptr: *mut *const f32, n: *mut usize) -> c_int;
    pub fn s2s_last_error() -> *const c_char;
    pub fn s2s_device_info(name: *mut c_char, cap: usize, arch: *mut c_char, acap: usize) -> c_int;
    pub fn s2s_vram(free: *mut u64, total: *mut u64) -> c_int;
    pub fn s2s_sync() -> c_int;
    pub fn s2s_stream(ctx: *mut S2sCtx) -> *mut c_void;
    pub fn s2s_selftest(arch: *const S2sArch, t: *const S2sTensor, n: usize) -> c_int;
    pub fn s2s_profile_enable(ctx: *mut S2sCtx, on: c_int) -> c_int;
    pub fn s2s_profile_reset(ctx: *mut S2sCtx) -> c_int;
    pub fn s2s_profile_report(ctx: *mut S2sCtx, wall_ms: f32) -> c_int;
}

/// The library's message as the crate's `Result` error.
pub fn check(rc: c_int, what: &str) -> Result<(), String> {
    if rc == 0 {
        return Ok(());
    }
    let m = unsafe { CStr::from_ptr(s2s_last_error()) }.to_string_lossy().into_owned();
    Err(format!("{what}: {m}"))
}

/// `lightgpu::vm::Device` as this backend reports it: the device name and its
/// architecture string (gfx950..., where the CUDA build prints sm_xx).
pub struct Device {
    pub name: String,
    pub arch: String,
}

/// `vm::device()` (reference src/main.rs:169,516-517).
pub fn device() -> Result<Device, String> {
    let (mut n, mut a) = ([0 as c_char; 256], [0 as c_char; 64]);
    check(unsafe { s2s_device_info(n.as_mut_ptr(), n.len(), a.as_mut_ptr(), a.len()) }, "hipGetDeviceProperties")?;
    let s = |p: &[c_char]| unsafe { CStr::from_ptr(p.as_ptr()) }.to_string_lossy().into_owned();
    Ok(Device { name: s(&n), arch: s(&a) })
}

/// `vm::vram()` (reference src/main.rs:461): free and total device bytes.
pub fn vram() -> Result<(usize, usize), String> {
    let (mut f, mut t) = (0u64, 0u64);
    check(unsafe { s2s_vram(&mut f, &mut t) }, "hipMemGetInfo")?;
    Ok((f as usize, t as usize))
}

/// `vm::sync()` (reference src/main.rs:342).
pub fn sync() -> Result<(), String> {
    check(unsafe { s2s_sync() }, "hipDeviceSynchronize")
}
