//! Both backends, on the SAME image, at widths above one 64-lane wavefront -
//! the reference's tests/gpu.rs (whole network at real widths, 56^2, 64^2 and
//! 128^2, against the CPU backend) for the HIP build. Copy to the crate as
//! tests/gpu_hip.rs; it uses the crate's tests/common (the converted
//! checkpoints, skipped when absent) and runs under `--features hip`.
#![cfg(feature = "hip")]

mod common;

use common::weights;
use swin2sr::backend::{Backend, Pre};
use swin2sr::cpu::Cpu;
use swin2sr::weights::Weights;

/// A level and a half of 8 bits, as the CUDA test holds (tests/gpu.rs:41).
const TOL: f32 = 6e-3;

fn image(h: usize, w: usize) -> Vec<f32> {
    let mut v = Vec::with_capacity(3 * h * w);
    for c in 0..3 {
        for y in 0..h {
            for x in 0..w {
                let t = ((x as f32) * 0.31 + (y as f32) * 0.17 + c as f32 * 1.7).sin();
                v.push(0.5 + 0.45 * t);
            }
        }
    }
    v
}

fn run<B: Backend>(wt: &Weights, b: &mut B, h: usize, w: usize) -> Vec<f32> {
    let pre = Pre::new(wt, h, w).expect("at least one window across");
    let adjusted = pre.adjust(wt, &image(h, w));
    b.forward(h, w, &adjusted).expect("forward")
}

fn worst(a: &[f32], b: &[f32]) -> (f32, usize) {
    assert_eq!(a.len(), b.len(), "the two backends returned different sizes");
    let mut worst = 0.0f32;
    let mut at = 0usize;
    for i in 0..a.len() {
        let d = (a[i] - b[i]).abs();
        if d > worst {
            worst = d;
            at = i;
        }
    }
    (worst, at)
}

fn agree(task: &str, h: usize, w: usize) {
    let Some(wt) = weights(task) else { return };
    let mut cpu = Cpu::new(&wt).expect("the CPU backend");
    let want = run(&wt, &mut cpu, h, w);
    let mut gpu = swin2sr::gpu::Gpu::new(&wt).expect("open the device");
    assert_eq!(gpu.name(), "hip");
    let got = run(&wt, &mut gpu, h, w);
    let (d, at) = worst(&want, &got);
    eprintln!("{task} {h}x{w}: max |diff| {d:.3e} at {at}");
    assert!(d <= TOL, "the two backends disagree by {d:.3e} at {at} ({:.0} 8-bit levels)", d * 255.0);
    if let (Some(a), Some(b)) = (cpu.aux().map(|s| s.to_vec()), gpu.aux()) {
        let (d, at) = worst(&a, b);
        assert!(d <= TOL, "the two aux planes disagree by {d:.3e} at {at}");
    }
}

#[test]
fn classical_x4_below_and_above_one_wavefront() {
    agree("classical-x4", 56, 56);
    agree("classical-x4", 64, 64);
    agree("classical-x4", 128, 128);
}

#[test]
fn classical_x2_wide() {
    agree("classical-x2", 128, 128);
}

#[test]
fn compressed_x4_with_its_aux() {
    agree("compressed-x4", 64, 64);
}

/// `uploaded_bytes` from the checkpoint alone equals what the backend holds,
/// and the selftest passes on the checkpoint's own shapes.
#[test]
fn memory_figure_and_selftest() {
    let Some(wt) = weights("classical-x4") else { return };
    let before = swin2sr::gpu::uploaded_bytes(&wt);
    assert!(before > 0);
    swin2sr::gpu::selftest(&wt).expect("hip selftest");
    let mut gpu = swin2sr::gpu::Gpu::new(&wt).expect("open the device");
    let plan = gpu.plan_bytes(256, 256).expect("plan");
    let model = swin2sr::backend::activation_bytes(&wt, 256, 256, 0, 0, true);
    assert!(plan <= model, "the device plan ({plan} B) exceeds the crate's model ({model} B)");
}
