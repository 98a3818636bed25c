"""The crate's tiling and memory policy, host side (reference src/backend.rs:88-383,
src/main.rs:579-662).

`north_star` keeps this logic in the crate's Rust host unchanged; this module is
its mirror over the `Backend` interface, so the tiled path (config 4: 256-pixel
tiles with 64 pixels of context) runs on the HIP backend exactly as the crate
would drive it:

  - `run_tiled`: tile and context rounded to window multiples (the context UP,
    and never below one window), each crop clamped to the image,
    mean-adjusted (`Pre::adjust`), run through `backend.forward`, and its
    interior copied to the output on the OUTPUT grid; `tile == 0` is one exact
    pass over the whole image;
  - `run_with_fallback`: `run_tiled`, retried with the tile halved (the whole
    image's first retry at half its longer side) while the backend reports
    "out of memory", announced on stderr;
  - `crop_side`: the padded plane a crop runs on, `(n // win + 1) * win`;
  - `crate_per_pixel_floats`: the crate's own model of its device's floats per
    padded pixel (`per_pixel_floats(wt, gpu = true)`), which `auto_tile` and
    `activation_bytes` budget with - the policy is the crate's, unchanged;
  - `plan_floats` / `per_pixel_floats`: this backend's exact buffer plan for an
    image (what `s2s_plan_bytes` reports) and its bound per padded pixel, which
    stays below the crate's model, so a budget computed with that model never
    under-counts this backend;
  - `auto_tile`: the largest window-multiple tile (from 1024, halving) whose
    crop fits a byte budget and the launch ceiling.
"""
from __future__ import annotations

import sys

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


def crate_per_pixel_floats(arch: M.Arch) -> int:
    """reference src/backend.rs:300-383 with `gpu = true`: the crate's device
    inventory per padded pixel (activations, the head's peak, the io images)."""
    c, mlp, r2, f = arch.embed, arch.embed * arch.mlp_ratio, arch.scale ** 2, arch.feat
    acts = 5 * c + 3 * c + 3 * c + mlp
    if arch.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
        prev, peak = f, 0
        for o in range(arch.octaves):
            shuf = 4 * f * 4 ** o
            peak, prev = max(peak, prev + shuf), shuf
        head = max(peak, prev + 3 * r2)
    elif arch.upsampler == "nearest+conv":
        head = max(max(4 * f * 4 ** s + f * 4 ** (s + 1) for s in range(2)), 4 * f + 3 * r2)
    else:
        head = 2 * 3 * r2
    return acts + head + 3 + 3 * r2


def _unit_layout(arch: M.Arch) -> bool:
    """Whether the forward keeps qkv in the window attention's unit layout
    (the library's qkv_unit_layout)."""
    hd, heads, c = arch.head_dim, arch.heads, arch.embed
    if hd not in (2, 10, 30, 32) or c != heads * hd or c % 4:
        return False
    if heads % 2 and hd % 4:
        return False
    return c in (180, 60, 360, 120)


def _fused_octaves(arch: M.Arch) -> int:
    """Octaves of the pixel-shuffle heads (the compressed one's too) composed
    into their last kernel."""
    if arch.upsampler not in ("pixelshuffle", "pixelshuffle_aux") or arch.feat % 8:
        return 0
    return 2 if arch.octaves >= 2 and arch.feat == 64 else 1


def _wino_before_upsample(arch: M.Arch) -> bool:
    """conv_before_upsample runs as Winograd (its products in the MLP buffer)."""
    return (arch.upsampler in ("pixelshuffle", "pixelshuffle_aux", "nearest+conv")
            and arch.embed in (60, 120, 180) and arch.feat % 4 == 0 and arch.feat <= 64)


def _wino_up2(arch: M.Arch) -> bool:
    """The x4 head's composed 5x5 conv runs as Winograd F(2x2,5x5)."""
    return _fused_octaves(arch) == 2 and arch.octaves == 2


def _plan_terms(arch: M.Arch, h: int, w: int):
    """(floats per buffer) of the library's plan for an h x w image, in
    s2s_ctx::body_specs + image_specs order (host-path copies included)."""
    win, c, s, f = arch.window, arch.embed, arch.scale, arch.feat
    hp, wp = (h // win + 1) * win, (w // win + 1) * win
    P = hp * wp
    qkv = P * 3 * c
    if _unit_layout(arch):
        qkv = max(qkv, P * ((arch.heads + 1) // 2) * (6 * arch.head_dim + 2))
    if c in (60, 120, 180):
        # the Winograd convs' 36 transform planes of 4x4-pixel tiles
        qkv = max(qkv, 36 * ((hp + 3) // 4) * ((wp + 3) // 4) * c)
    if _wino_up2(arch):
        # the x4 head's Winograd 5x5 conv: 36 planes of 2x2-pixel tiles x F
        qkv = max(qkv, 36 * ((hp + 1) // 2) * ((wp + 1) // 2) * f)
    hid = P * arch.mlp_ratio * c
    if _wino_before_upsample(arch):
        # conv_before_upsample's Winograd products (36 planes of F per tile)
        hid = max(hid, 36 * ((hp + 3) // 4) * ((wp + 3) // 4) * f)
    terms = [P * c] * 3 + [qkv, P * c, hid]
    terms += [3 * h * w, 3 * h * s * w * s, P * 4]
    if arch.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
        terms += [P * 4 ** o * f for o in range(arch.octaves - _fused_octaves(arch) + 1)]
        if arch.upsampler == "pixelshuffle_aux":
            terms += [P * 4, P * 3, P * s * s * 4]
    elif arch.upsampler == "nearest+conv":
        terms += [P * f, 4 * P * f, 16 * P * f, 16 * P * f]
    return terms


def plan_floats(arch: M.Arch, h: int, w: int) -> int:
    """This backend's device floats for an h x w image: exactly what
    `s2s_plan_bytes` reports, / 4."""
    return sum(max(t, 1) for t in _plan_terms(arch, h, w))


def per_pixel_floats(arch: M.Arch) -> int:
    """This backend's device floats per padded pixel: `plan_floats` divided by
    the padded plane, bounded over image sizes (the io images counted at the
    padded size)."""
    c, s, f = arch.embed, arch.scale, arch.feat
    qkv = 3 * c
    if _unit_layout(arch):
        qkv = max(qkv, ((arch.heads + 1) // 2) * (6 * arch.head_dim + 2))
    if c in (60, 120, 180):
        # 36 planes per 16 pixels, at most ceil(win/4)^2 tiles per win^2 pixels
        t = (arch.window + 3) // 4
        qkv = max(qkv, -(-36 * t * t * c // (arch.window * arch.window)))
    if _wino_up2(arch):
        t = (arch.window + 1) // 2
        qkv = max(qkv, -(-36 * t * t * f // (arch.window * arch.window)))
    hid = arch.mlp_ratio * c
    if _wino_before_upsample(arch):
        t = (arch.window + 3) // 4
        hid = max(hid, -(-36 * t * t * f // (arch.window * arch.window)))
    body = 3 * c + qkv + c + hid
    if arch.upsampler in ("pixelshuffle", "pixelshuffle_aux"):
        head = sum(f * 4 ** o for o in range(arch.octaves - _fused_octaves(arch) + 1))
        if arch.upsampler == "pixelshuffle_aux":
            head += 4 + 3 + 4 * s * s
    elif arch.upsampler == "nearest+conv":
        head = f * (1 + 4 + 16 + 16)
    else:
        head = 0
    io = 3 + 3 * s * s + 4
    return body + head + io


def auto_tile(arch: M.Arch, budget: int, h: int, w: int, pad: int) -> int:
    """reference src/backend.rs:169-189, with the crate's own device model."""
    win = arch.window
    per_px = crate_per_pixel_floats(arch)
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


def is_out_of_memory(err: str) -> bool:
    """reference src/main.rs:660-662: the one failure a smaller tile can fix."""
    return "OUT_OF_MEMORY" in err or "out of memory" in err


def run_with_fallback(arch: M.Arch, backend, img: np.ndarray, tile: int, pad: int,
                      quiet: bool = False, log=None, batch: bool = False):
    """reference src/main.rs:579-662: `run_tiled`, and while the backend fails
    with an out-of-memory error, again with the tile halved - a failed
    whole-image pass (`tile == 0`) falls back to half the image's longer side -
    down to one window. Only out-of-memory errors are retried; a retry out of
    `tile == 0` (the only exact mode) is announced even when `quiet`. `batch`
    is passed to `run_tiled` (an image's crops in one batched call).
    Returns (image, tile used)."""
    log = log or (lambda m: print(m, file=sys.stderr, flush=True))
    win = arch.window
    _, h, w = img.shape
    for _ in range(64):
        try:
            return run_tiled(arch, backend, img, tile, pad, batch=batch), tile
        except Exception as e:  # the backend's error type carries the message
            msg = str(e)
            if not (is_out_of_memory(msg) and (tile > win or tile == 0)):
                raise
            nxt = (max(h, w) // 2 // win if tile == 0 else tile // 2 // win)
            nxt = max(nxt, 1) * win
            shrinking = nxt != 0 if tile == 0 else nxt < tile
            if not shrinking or nxt == 0:
                raise type(e)(f"{msg}\n(a {win}-pixel tile is the smallest this engine will "
                              "run, and it did not fit either)") from e
            note = msg.rstrip(".")
            if tile == 0:
                log(f"note: {note} - retrying with a {nxt}x{nxt} tile (--tile 0 is the only "
                    "exact mode; this run is now tiled, and tiled results differ slightly from "
                    "one pass - see README)")
            elif not quiet:
                log(f"note: {note} - retrying with a {nxt}x{nxt} tile")
            tile = nxt
    raise RuntimeError(f"gave up after 64 tile reductions at tile {tile}")


def run_tiled(arch: M.Arch, backend, img: np.ndarray, tile: int, pad: int,
              batch: bool = False) -> np.ndarray:
    """reference src/backend.rs:92-165. `img` is `[3][h][w]` in [0,1] (not
    mean-adjusted); the result is `[3][h*s][w*s]`. With `batch` and a backend
    that has `forward_batch` (the HIP backend: its two lanes), the image's
    crops go through one batched call, then are pasted in the same order;
    every tile's result is what `forward` gives for it."""
    _, h, w = img.shape
    s = arch.scale
    if tile == 0:
        return backend.forward(h, w, M.adjust(arch, img))
    win = arch.window
    tile = max(tile // win, 1) * win
    pad = _round_pad(pad, win)
    out = np.zeros((3, h * s, w * s), np.float32)

    def paste(job, res):
        ty, tx, y0, x0 = job
        oy0, ox0 = ty - y0, tx - x0
        ch = min(ty + tile, h) - ty
        cw = min(tx + tile, w) - tx
        # the copy is on the OUTPUT grid: ch*s rows of cw*s pixels
        out[:, ty * s:(ty + ch) * s, tx * s:(tx + cw) * s] = \
            res[:, oy0 * s:(oy0 + ch) * s, ox0 * s:(ox0 + cw) * s]

    jobs, shapes, crops = [], [], []
    for ty in range(0, h, tile):
        for tx in range(0, w, tile):
            y0, x0 = max(ty - pad, 0), max(tx - pad, 0)
            y1, x1 = min(ty + tile + pad, h), min(tx + tile + pad, w)
            th, tw = y1 - y0, x1 - x0
            sub = M.adjust(arch, np.ascontiguousarray(img[:, y0:y1, x0:x1]))
            if batch and hasattr(backend, "forward_batch"):
                jobs.append((ty, tx, y0, x0))
                shapes.append((th, tw))
                crops.append(sub)
            else:
                paste((ty, tx, y0, x0), backend.forward(th, tw, sub))
    if jobs:
        for job, res in zip(jobs, backend.forward_batch(shapes, crops)):
            paste(job, res)
    return out
