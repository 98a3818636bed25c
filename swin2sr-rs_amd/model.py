"""Architectures, synthetic checkpoints and synthetic inputs for the swin2sr hot path.

There is no network and no published checkpoint in this environment, so every
weight set is generated: random-init by the rules the benchmark configurations
state (linears N(0, 0.02^2) with zero biases, convolutions torch's default
Kaiming-uniform U(+-1/sqrt(fan_in)) for weight and bias, LayerNorm 1/0,
logit_scale = log(10), cpb MLP 2->512->heads N(0, 0.02^2)), under the crate's
tensor names and shapes (reference src/weights.rs:142-235, the upload set of
src/gpu.rs:801-872), including the converter's derived tensors: the qkv slices
and the cpb_pre table (reference tools/convert.py:122-167).

`perturb=True` moves every bias, LayerNorm affine and logit scale off its
trivial init (and widens the cpb MLP) so a parity test exercises each term;
the benchmark uses the plain rules.

The generator is numpy's PCG64 seeded per configuration; tensors are drawn in
the fixed order `tensor_names` lists.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Dict, List

import numpy as np

UPSAMPLERS = {"pixelshuffle": 0, "pixelshuffledirect": 1, "nearest+conv": 2, "pixelshuffle_aux": 3}
RGB_MEAN = (0.4488, 0.4371, 0.4040)


@dataclasses.dataclass
class Arch:
    """The checkpoint's `__metadata__` (reference src/weights.rs:66-137)."""

    upsampler: str = "pixelshuffle"
    scale: int = 4
    window: int = 8
    embed: int = 180
    heads: int = 6
    mlp_ratio: int = 2
    depths: List[int] = dataclasses.field(default_factory=lambda: [6] * 6)
    img_range: float = 1.0
    mean: tuple = RGB_MEAN
    feat: int = 64  # num_feat of the reconstruction heads (network_swin2sr.py:726)

    @property
    def head_dim(self) -> int:
        return self.embed // self.heads

    @property
    def octaves(self) -> int:
        if self.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
            return int(round(math.log2(self.scale)))
        return 1 if self.upsampler == "pixelshuffledirect" else 2


def classical(scale: int = 4) -> Arch:
    return Arch(upsampler="pixelshuffle", scale=scale)


def lightweight(scale: int = 2) -> Arch:
    return Arch(upsampler="pixelshuffledirect", scale=scale, embed=60, depths=[6] * 4)


def realworld() -> Arch:
    return Arch(upsampler="nearest+conv", scale=4)


def compressed() -> Arch:
    return Arch(upsampler="pixelshuffle_aux", scale=4)


def relative_coords_table(win: int) -> np.ndarray:
    """network_swin2sr.py:107-120: [(2w-1)^2][2] log-spaced offsets, float32."""
    r = np.arange(-(win - 1), win, dtype=np.float32)
    t = np.stack(np.meshgrid(r, r, indexing="ij"), axis=-1).astype(np.float32)
    t = t / np.float32(win - 1)
    t = t * np.float32(8)
    t = np.sign(t) * np.log2(np.abs(t) + np.float32(1.0)) / np.float32(np.log2(8))
    return t.reshape(-1, 2).astype(np.float32)


def relative_position_index(win: int) -> np.ndarray:
    """network_swin2sr.py:124-136: idx[q][k] = (yq-yk+w-1)(2w-1) + (xq-xk+w-1)."""
    ys, xs = np.meshgrid(np.arange(win), np.arange(win), indexing="ij")
    y, x = ys.reshape(-1), xs.reshape(-1)
    return (y[:, None] - y[None, :] + win - 1) * (2 * win - 1) + (x[:, None] - x[None, :] + win - 1)


def cpb_pre(w0: np.ndarray, b0: np.ndarray, w2: np.ndarray, win: int) -> np.ndarray:
    """tools/convert.py:141-167: 16*sigmoid(MLP(table))[index], [n*n][heads], float32."""
    t = relative_coords_table(win)
    h = t @ w0.T + b0
    h = np.maximum(h, np.float32(0))
    h = h @ w2.T
    bias = h[relative_position_index(win).reshape(-1)]
    return (np.float32(16.0) / (np.float32(1.0) + np.exp(-bias))).astype(np.float32)


def tensor_names(a: Arch) -> List[str]:
    names = ["conv_first.weight", "conv_first.bias", "patch_embed.proj.weight",
             "patch_embed.proj.bias", "patch_embed.norm.weight", "patch_embed.norm.bias"]
    for s, d in enumerate(a.depths):
        for b in range(d):
            p = f"layers.{s}.residual_group.blocks.{b}."
            names += [p + k for k in (
                "attn.qkv.wq", "attn.qkv.wk", "attn.qkv.wv", "attn.qkv.q_bias", "attn.qkv.v_bias",
                "attn.logit_scale", "attn.cpb_mlp.0.weight", "attn.cpb_mlp.0.bias",
                "attn.cpb_mlp.2.weight", "attn.cpb_pre", "attn.proj.weight", "attn.proj.bias",
                "norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                "mlp.fc1.weight", "mlp.fc1.bias", "mlp.fc2.weight", "mlp.fc2.bias")]
        names += [f"layers.{s}.conv.weight", f"layers.{s}.conv.bias",
                  f"layers.{s}.patch_embed.proj.weight", f"layers.{s}.patch_embed.proj.bias"]
    names += ["norm.weight", "norm.bias", "conv_after_body.weight", "conv_after_body.bias"]
    if a.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
        names += ["conv_before_upsample.0.weight", "conv_before_upsample.0.bias"]
        if a.upsampler == "pixelshuffle_aux":
            names += ["conv_bicubic.weight", "conv_bicubic.bias", "conv_aux.weight", "conv_aux.bias",
                      "conv_after_aux.0.weight", "conv_after_aux.0.bias"]
        for o in range(a.octaves):
            names += [f"upsample.{2 * o}.weight", f"upsample.{2 * o}.bias"]
        names += ["conv_last.weight", "conv_last.bias"]
    elif a.upsampler == "pixelshuffledirect":
        names += ["upsample.0.weight", "upsample.0.bias"]
    else:
        names += ["conv_before_upsample.0.weight", "conv_before_upsample.0.bias",
                  "conv_up1.weight", "conv_up1.bias", "conv_up2.weight", "conv_up2.bias",
                  "conv_hr.weight", "conv_hr.bias", "conv_last.weight", "conv_last.bias"]
    return names


def _conv_shape(a: Arch, name: str):
    C, F, s = a.embed, a.feat, a.scale
    base = name.rsplit(".", 1)[0]
    table = {
        "conv_first": (C, 3, 3), "conv_after_body": (C, C, 3), "patch_embed.proj": (C, C, 1),
        "conv_before_upsample.0": (F, C, 3), "conv_last": (3, F, 3), "conv_up1": (F, F, 3),
        "conv_up2": (F, F, 3), "conv_hr": (F, F, 3), "conv_bicubic": (F, 3, 3),
        "conv_aux": (3, F, 3), "conv_after_aux.0": (F, 3, 3),
    }
    if base in table:
        return table[base]
    if base.startswith("layers.") and base.endswith(".conv"):
        return (C, C, 3)
    if base.startswith("layers.") and base.endswith("patch_embed.proj"):
        return (C, C, 1)
    if base.startswith("upsample."):
        if a.upsampler == "pixelshuffledirect":
            return (3 * s * s, C, 3)
        return (4 * F, F, 3)
    return None


def make_weights(a: Arch, seed: int, perturb: bool = False) -> Dict[str, np.ndarray]:
    """Synthetic checkpoint by the benchmark's init rules (see module doc)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    C, NH, n = a.embed, a.heads, a.window * a.window
    H = a.mlp_ratio * C
    cpb_std = 1.0 if perturb else 0.02

    def normal(shape, std):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    def small(shape, amp):
        if not perturb:
            return np.zeros(shape, np.float32)
        return rng.uniform(-amp, amp, size=shape).astype(np.float32)

    w: Dict[str, np.ndarray] = {}
    pending_qkv = {}
    for name in tensor_names(a):
        if name in w:
            continue
        cs = _conv_shape(a, name)
        if cs is not None:
            co, ci, k = cs
            bound = 1.0 / math.sqrt(ci * k * k)
            if name.endswith(".weight"):
                w[name] = rng.uniform(-bound, bound, size=(co, ci, k, k)).astype(np.float32)
            else:
                w[name] = rng.uniform(-bound, bound, size=(co,)).astype(np.float32)
            continue
        if name.endswith("attn.qkv.wq"):
            qkv = normal((3 * C, C), 0.02)
            p = name[: -len("wq")]
            w[p + "wq"], w[p + "wk"], w[p + "wv"] = (np.ascontiguousarray(qkv[:C]),
                                                     np.ascontiguousarray(qkv[C:2 * C]),
                                                     np.ascontiguousarray(qkv[2 * C:]))
            continue
        if name.endswith(("q_bias", "v_bias")):
            w[name] = small((C,), 0.05)
        elif name.endswith("logit_scale"):
            ls = np.full((NH, 1, 1), math.log(10.0), np.float32)
            if perturb:
                ls[:, 0, 0] += rng.uniform(-1.0, 1.0, size=NH).astype(np.float32)
                ls[0, 0, 0] = np.float32(math.log(200.0))  # above the log(100) clamp
            w[name] = ls
        elif name.endswith("cpb_mlp.0.weight"):
            w[name] = normal((512, 2), cpb_std)
        elif name.endswith("cpb_mlp.0.bias"):
            w[name] = small((512,), 0.5)
        elif name.endswith("cpb_mlp.2.weight"):
            w[name] = normal((NH, 512), cpb_std * (0.1 if perturb else 1.0))
        elif name.endswith("cpb_pre"):
            p = name[: -len("cpb_pre")]
            w[name] = cpb_pre(w[p + "cpb_mlp.0.weight"], w[p + "cpb_mlp.0.bias"],
                              w[p + "cpb_mlp.2.weight"], a.window)
        elif name.endswith("proj.weight"):
            w[name] = normal((C, C), 0.02)
        elif name.endswith("fc1.weight"):
            w[name] = normal((H, C), 0.02)
        elif name.endswith("fc2.weight"):
            w[name] = normal((C, H), 0.02)
        elif name.endswith("fc1.bias"):
            w[name] = small((H,), 0.05)
        elif name.endswith(("proj.bias", "fc2.bias")):
            w[name] = small((C,), 0.05)
        elif "norm" in name and name.endswith(".weight"):
            w[name] = (np.ones(C, np.float32) if not perturb
                       else (1.0 + rng.uniform(-0.2, 0.2, size=C)).astype(np.float32))
        elif "norm" in name and name.endswith(".bias"):
            w[name] = small((C,), 0.1)
        else:
            raise KeyError(f"no init rule for {name}")
    del pending_qkv
    return w


# ---------------------------------------------------------------------------
# Synthetic inputs, u8 RGB planar [3][h][w]
# ---------------------------------------------------------------------------

def input_uniform(h: int, w: int, seed: int) -> np.ndarray:
    """config 0: uniform 0..255."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, 256, size=(3, h, w), dtype=np.uint8)


def input_sinusoids(h: int, w: int, seed: int, noise: float = 4.0) -> np.ndarray:
    """configs 2/4: 8 random-frequency/phase 2-D sinusoids + N(0, noise^2), clipped."""
    rng = np.random.Generator(np.random.PCG64(seed))
    yy, xx = np.meshgrid(np.arange(h, dtype=np.float64), np.arange(w, dtype=np.float64),
                         indexing="ij")
    img = np.full((3, h, w), 128.0)
    for _ in range(8):
        fy, fx = rng.uniform(0.0, 0.15, size=2)
        amp = rng.uniform(6.0, 20.0)
        for c in range(3):
            ph = rng.uniform(0.0, 2 * math.pi)
            img[c] += amp * np.sin(2 * math.pi * (fy * yy + fx * xx) + ph)
    img += rng.normal(0.0, noise, size=img.shape)
    return np.clip(np.rint(img), 0, 255).astype(np.uint8)


def input_texture_dct(h: int, w: int, seed: int) -> np.ndarray:
    """config 3: smooth sinusoid texture + N(0, 8^2) + 8x8 DCT quantisation (step 16)."""
    img = input_sinusoids(h, w, seed, noise=8.0).astype(np.float64)
    k = np.arange(8)
    basis = np.cos((2 * k[None, :] + 1) * k[:, None] * math.pi / 16) * np.sqrt(2 / 8)
    basis[0] /= np.sqrt(2)
    out = img.copy()
    for c in range(3):
        for by in range(0, h - h % 8, 8):
            for bx in range(0, w - w % 8, 8):
                blk = img[c, by:by + 8, bx:bx + 8] - 128.0
                coef = basis @ blk @ basis.T
                coef = np.round(coef / 16.0) * 16.0
                out[c, by:by + 8, bx:bx + 8] = basis.T @ coef @ basis + 128.0
    return np.clip(np.rint(out), 0, 255).astype(np.uint8)


def to_unit(img_u8: np.ndarray) -> np.ndarray:
    return (img_u8.astype(np.float32) / np.float32(255.0)).astype(np.float32)


def adjust(a: Arch, img: np.ndarray) -> np.ndarray:
    """`Pre::adjust` (reference src/backend.rs:76-86): (x - mean) * img_range, f32."""
    out = img.astype(np.float32).copy()
    for c in range(3):
        out[c] = (out[c] - np.float32(a.mean[c])) * np.float32(a.img_range)
    return out


def to_rgb8(x: np.ndarray) -> np.ndarray:
    """`Image::to_rgb8` (reference src/image.rs:29-39): floor(clamp01(v)*255 + 0.5)."""
    return np.floor(np.clip(x, 0.0, 1.0).astype(np.float32) * np.float32(255.0)
                    + np.float32(0.5)).astype(np.uint8)
