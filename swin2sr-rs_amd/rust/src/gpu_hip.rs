//! The HIP device backend: `Gpu` implementing `Backend` over libswin2sr_hip.so,
//! in the place `src/gpu.rs` takes in the CUDA build, with the same public
//! names the CLI calls there (`Gpu::new`, `uploaded_bytes`, `selftest`) plus the
//! two it reaches through `lightgpu` and `src/cuda.rs` (`vm`, `Profile`).
//!
//! Copy to the crate as `src/gpu_hip.rs` and mount it under the name the CLI
//! already uses, in `src/lib.rs`:
//!
//! ```ignore
//! #[cfg(feature = "cuda")]
//! pub mod cuda;
//! #[cfg(feature = "cuda")]
//! pub mod gpu;
//! #[cfg(feature = "hip")]
//! pub mod hip;
//! #[cfg(feature = "hip")]
//! #[path = "gpu_hip.rs"]
//! pub mod gpu;
//! ```
use std::cell::Cell;
use std::ffi::{c_int, CString};

use crate::backend::Backend;
use crate::hip::*;
use crate::weights::{Upsampler, Weights};

/// The architecture and the borrowed tensor table of a checkpoint, as the C
/// ABI takes them. `names` keeps the C strings alive while `tabs` points at
/// them; the data pointers borrow `wt`'s memory-mapped tensors.
struct Table {
    arch: S2sArch,
    _names: Vec<CString>,
    tabs: Vec<S2sTensor>,
}

fn table(wt: &Weights) -> Result<Table, String> {
    if wt.depths.len() > 16 {
        return Err(format!("{} stages: the device backend takes at most 16", wt.depths.len()));
    }
    let mut depths = [0 as c_int; 16];
    for (i, d) in wt.depths.iter().enumerate() {
        depths[i] = *d as c_int;
    }
    let arch = S2sArch {
        upsampler: match wt.upsampler {
            Upsampler::PixelShuffle => 0,
            Upsampler::PixelShuffleDirect => 1,
            Upsampler::NearestConv => 2,
            Upsampler::PixelShuffleAux => 3,
        },
        scale: wt.scale as c_int,
        window: wt.window as c_int,
        embed: wt.embed as c_int,
        heads: wt.heads as c_int,
        mlp_ratio: wt.mlp_ratio as c_int,
        n_stages: wt.depths.len() as c_int,
        depths,
        img_range: wt.img_range,
        mean: wt.mean,
    };
    // `Weights` exposes its tensors by name: the `names` field (the file's own
    // order), `t(name)` for the data and `shape(name)` (src/weights.rs:85,240-250)
    let names: Vec<CString> = wt
        .names
        .iter()
        .map(|n| CString::new(n.as_str()).map_err(|_| format!("tensor name `{n}` holds a NUL")))
        .collect::<Result<_, _>>()?;
    let mut tabs = Vec::with_capacity(names.len());
    for (cn, n) in names.iter().zip(wt.names.iter()) {
        let shape = wt.shape(n);
        if shape.len() > 4 {
            return Err(format!("tensor `{n}` has {} dimensions; the device backend takes at most 4", shape.len()));
        }
        let mut s = [0i64; 4];
        for (i, d) in shape.iter().enumerate() {
            s[i] = *d as i64;
        }
        tabs.push(S2sTensor { name: cn.as_ptr(), data: wt.t(n).as_ptr(), ndim: shape.len() as c_int, shape: s });
    }
    Ok(Table { arch, _names: names, tabs })
}

thread_local! {
    /// The context `Profile::report` reports on: the last `Gpu` made on this
    /// thread (the CUDA build's profile state is thread-local too,
    /// src/cuda.rs:173-175).
    static CURRENT: Cell<*mut S2sCtx> = Cell::new(std::ptr::null_mut());
}

pub struct Gpu {
    ctx: *mut S2sCtx,
    scale: usize,
    aux: Option<Vec<f32>>,
    want_aux: bool,
}

impl Gpu {
    /// `Gpu::new(&Weights)` (reference src/gpu.rs:101-125): the tensors are
    /// borrowed for the call and copied to the device, re-laid-out for the
    /// kernels. `SWIN2SR_PROFILE_GPU` switches the event profiler on here.
    pub fn new(wt: &Weights) -> Result<Gpu, String> {
        let t = table(wt)?;
        let mut ctx = std::ptr::null_mut();
        check(unsafe { s2s_create(&t.arch, t.tabs.as_ptr(), t.tabs.len(), &mut ctx) }, "hip backend")?;
        CURRENT.with(|c| c.set(ctx));
        Ok(Gpu { ctx, scale: wt.scale, aux: None, want_aux: matches!(wt.upsampler, Upsampler::PixelShuffleAux) })
    }

    /// The device bytes a forward of an h x w image allocates (never above the
    /// crate's own `activation_bytes` model of its device).
    pub fn plan_bytes(&mut self, h: usize, w: usize) -> Result<u64, String> {
        let mut b = 0u64;
        check(unsafe { s2s_plan_bytes(self.ctx, h as c_int, w as c_int, &mut b) }, "plan")?;
        Ok(b)
    }
}

impl Gpu {
    /// Several images at once, e.g. all of an image's tiles: `s2s_forward_batch`
    /// pipelines them over the context's two lanes (one computes while the
    /// other's result is copied out). Each result equals `forward`'s for its
    /// input; `aux()` afterwards is the last image's. No counterpart in the
    /// crate: its `run_tiled` calls `Backend::forward` once per tile
    /// (src/backend.rs:92-165); a tile loop that gathers an image's crops
    /// first can call this instead and paste the results in the same order.
    pub fn forward_batch(&mut self, items: &[(usize, usize, &[f32])]) -> Result<Vec<Vec<f32>>, String> {
        let mut hs = Vec::with_capacity(items.len());
        let mut ws = Vec::with_capacity(items.len());
        let mut ins = Vec::with_capacity(items.len());
        let mut outs = Vec::with_capacity(items.len());
        for &(h, w, input) in items {
            if input.len() != 3 * h * w {
                return Err(format!("forward_batch: {} input floats for a {h}x{w} image", input.len()));
            }
            hs.push(h as c_int);
            ws.push(w as c_int);
            ins.push(input.as_ptr());
            outs.push(vec![0f32; 3 * h * self.scale * w * self.scale]);
        }
        let optrs: Vec<*mut f32> = outs.iter_mut().map(|o| o.as_mut_ptr()).collect();
        check(
            unsafe {
                s2s_forward_batch(
                    self.ctx,
                    items.len() as c_int,
                    hs.as_ptr(),
                    ws.as_ptr(),
                    ins.as_ptr(),
                    optrs.as_ptr(),
                    std::ptr::null(),
                )
            },
            "forward_batch",
        )?;
        self.aux = None;
        if self.want_aux && !items.is_empty() {
            let (mut p, mut n) = (std::ptr::null(), 0usize);
            check(unsafe { s2s_aux(self.ctx, &mut p, &mut n) }, "aux")?;
            if n > 0 {
                self.aux = Some(unsafe { std::slice::from_raw_parts(p, n) }.to_vec());
            }
        }
        Ok(outs)
    }
}

impl Backend for Gpu {
    fn name(&self) -> &'static str {
        "hip"
    }

    /// `input` is the mean-adjusted `[3][h][w]` plane `run_tiled` passes
    /// (src/backend.rs:101-104); the result is denormalised and cropped,
    /// `[3][h*s][w*s]`.
    fn forward(&mut self, h: usize, w: usize, input: &[f32]) -> Result<Vec<f32>, String> {
        if input.len() != 3 * h * w {
            return Err(format!("forward: {} input floats for a {h}x{w} image", input.len()));
        }
        let mut out = vec![0f32; 3 * h * self.scale * w * self.scale];
        check(
            unsafe { s2s_forward(self.ctx, h as c_int, w as c_int, input.as_ptr(), out.as_mut_ptr()) },
            "forward",
        )?;
        self.aux = None;
        if self.want_aux {
            let (mut p, mut n) = (std::ptr::null(), 0usize);
            check(unsafe { s2s_aux(self.ctx, &mut p, &mut n) }, "aux")?;
            if n > 0 {
                self.aux = Some(unsafe { std::slice::from_raw_parts(p, n) }.to_vec());
            }
        }
        Ok(out)
    }

    fn aux(&self) -> Option<&[f32]> {
        self.aux.as_deref()
    }
}

impl Drop for Gpu {
    fn drop(&mut self) {
        CURRENT.with(|c| {
            if c.get() == self.ctx {
                c.set(std::ptr::null_mut())
            }
        });
        unsafe { s2s_destroy(self.ctx) }
    }
}

/// `gpu::uploaded_bytes(&Weights)` (reference src/gpu.rs:792-799), from the
/// checkpoint alone, before any backend exists (`memory_budget`,
/// src/main.rs:459-471): exactly what `Gpu::new` will upload. A checkpoint the
/// device would refuse reports 0 (`Gpu::new` then says why).
pub fn uploaded_bytes(wt: &Weights) -> u64 {
    let Ok(t) = table(wt) else { return 0 };
    let mut b = 0u64;
    match check(unsafe { s2s_uploaded_bytes_for(&t.arch, t.tabs.as_ptr(), t.tabs.len(), &mut b) }, "uploaded bytes") {
        Ok(()) => b,
        Err(_) => 0,
    }
}

/// `gpu::selftest(&Weights)` behind `--cuda-selftest` (reference
/// src/gpu.rs:889-1265): every kernel against its definition at the
/// reference's shapes and the checkpoint's own width and head shape, and the
/// checkpoint's CPB tables. The library prints the count of checks.
pub fn selftest(wt: &Weights) -> Result<(), String> {
    let t = table(wt)?;
    check(unsafe { s2s_selftest(&t.arch, t.tabs.as_ptr(), t.tabs.len()) }, "hip selftest")
}

/// `lightgpu::vm` for this backend (device, vram, sync).
pub mod vm {
    pub use crate::hip::{device, sync, vram, Device};
}

/// `cuda::Profile` for this backend: `report(total_wall_ms)` prints the
/// per-kernel rows of the last `Gpu` made on this thread when
/// `SWIN2SR_PROFILE_GPU` switched its profiler on (reference src/cuda.rs:239-259).
pub struct Profile;

impl Profile {
    pub fn report(wall_ms: f32) {
        CURRENT.with(|c| {
            let ctx = c.get();
            if !ctx.is_null() {
                let _ = unsafe { s2s_profile_report(ctx, wall_ms) };
            }
        });
    }
}
