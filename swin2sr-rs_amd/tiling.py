"""The crate's tiling and memory policy, host side (reference src/backend.rs:88-383).

`north_star` keeps this logic in the crate's Rust host unchanged; this module is
its mirror over the `Backend` interface, so the tiled path (config 4: 256-pixel
tiles with 64 pixels of context) runs on the HIP backend exactly as the crate
would drive it:

  - `run_tiled`: tile and context rounded to window multiples (the context UP,
    and never below one window), each crop clamped to the image,
    mean-adjusted (`Pre::adjust`), run through `backend.forward`, and its
    interior copied to the output on the OUTPUT grid; `tile == 0` is one exact
    pass over the whole image;
  - `crop_side`: the padded plane a crop runs on, `(n // win + 1) * win`;
  - `per_pixel_floats`: this backend's device floats per padded pixel (its
    buffer plan, `s2s_ctx::plan_body` / `plan_image`), which stays at or below
    the figure the crate models for its device (`src/backend.rs:300-383`), so a
    budget computed with the crate's model never under-counts this backend;
  - `auto_tile`: the largest window-multiple tile (from 1024, halving) whose
    crop fits a byte budget and the launch ceiling.
"""
from __future__ import annotations

import numpy as np

from . import model as M

# reference src/backend.rs:230: the CUDA token-grid ceiling the crate's policy
# and tests are written against. This backend has no such limit (its grids are
# 1-D and persistent), so honouring it only ever tiles earlier than necessary.
GPU_MAX_PLANE_PIXELS = 65535 * 16


def _round_pad(pad: int, win: int) -> int:
    return max(-(-pad // win), 1) * win


def crop_side(h: int, w: int, tile: int, pad: int, win: int) -> int:
    """reference src/backend.rs:249-259."""
    if tile == 0:
        th, tw = h, w
    else:
        t = max(tile // win, 1) * win
        p = _round_pad(pad, win)
        th, tw = min(t + 2 * p, h), min(t + 2 * p, w)
    return max((th // win + 1) * win, (tw // win + 1) * win)


def per_pixel_floats(arch: M.Arch) -> int:
    """Device floats per padded pixel of this backend's buffer plan."""
    c = arch.embed
    hidden = arch.mlp_ratio * c
    s = arch.scale
    body = 4 * c + 3 * c + c + hidden          # cur, work, tmp, body skip; qkv; attn out; mlp
    f = arch.feat
    if arch.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
        head = sum(f * 4 ** o for o in range(arch.octaves + 1))
        if arch.upsampler == "pixelshuffle_aux":
            head += 4 + 3 + 4 * s * s            # aux conv, aux image, bicubic input
    elif arch.upsampler == "nearest+conv":
        head = f * (1 + 4 + 16 + 16)
    else:
        head = 0
    io = 3 + 4 + 3 * s * s                      # input, padded input, output
    return body + head + io


def auto_tile(arch: M.Arch, budget: int, h: int, w: int, pad: int) -> int:
    """reference src/backend.rs:169-189 with this backend's per-pixel figure."""
    win = arch.window
    per_px = per_pixel_floats(arch)
    pad = _round_pad(pad, win)

    def fits(side):
        return per_px * side * side * 4 <= budget and side * side <= GPU_MAX_PLANE_PIXELS

    if fits(crop_side(h, w, 0, pad, win)):
        return 0
    t = (max(1024, win) // win) * win
    while True:
        if fits(crop_side(h, w, t, pad, win)) or t == win:
            return t
        t = max(t // 2 // win, 1) * win


def run_tiled(arch: M.Arch, backend, img: np.ndarray, tile: int, pad: int) -> np.ndarray:
    """reference src/backend.rs:92-165. `img` is `[3][h][w]` in [0,1] (not
    mean-adjusted); the result is `[3][h*s][w*s]`."""
    _, h, w = img.shape
    s = arch.scale
    if tile == 0:
        return backend.forward(h, w, M.adjust(arch, img))
    win = arch.window
    tile = max(tile // win, 1) * win
    pad = _round_pad(pad, win)
    out = np.zeros((3, h * s, w * s), np.float32)
    for ty in range(0, h, tile):
        for tx in range(0, w, tile):
            y0, x0 = max(ty - pad, 0), max(tx - pad, 0)
            y1, x1 = min(ty + tile + pad, h), min(tx + tile + pad, w)
            th, tw = y1 - y0, x1 - x0
            sub = np.ascontiguousarray(img[:, y0:y1, x0:x1])
            res = backend.forward(th, tw, M.adjust(arch, sub))
            oy0, ox0 = ty - y0, tx - x0
            ch = min(ty + tile, h) - ty
            cw = min(tx + tile, w) - tx
            # the copy is on the OUTPUT grid: ch*s rows of cw*s pixels
            out[:, ty * s:(ty + ch) * s, tx * s:(tx + cw) * s] = \
                res[:, oy0 * s:(oy0 + ch) * s, ox0 * s:(ox0 + cw) * s]
    return out
