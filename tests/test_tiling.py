"""The crate's tiling and memory policy (reference src/backend.rs:88-383,
tests/tiling.rs) over the Backend interface.

CPU tests drive `run_tiled` with the oracle as the backend (the crate's own
tiling tests run it on the CPU backend); GPU tests hold the HIP backend's tiled
output against the oracle's, tile for tile, including config 4's geometry
(256-pixel tiles with 64 pixels of context).
"""
import numpy as np
import pytest


class OracleBackend:
    """The oracle behind the `Backend` shape (test code only)."""

    def __init__(self, orc, arch, weights):
        self.orc, self.arch, self.weights = orc, arch, weights

    def forward(self, h, w, x):
        out, _ = self.orc.forward(self.arch, self.weights, h, w, x)
        return out


def tiny(pkg, **kw):
    base = dict(upsampler="pixelshuffledirect", scale=2, embed=12, heads=2, depths=[1, 1])
    base.update(kw)
    return pkg.model.Arch(**base)


def test_crop_side_is_the_reference_rule(pkg):
    T = pkg.tiling
    # (n // win + 1) * win, never ceil: a 256 image runs on 264
    assert T.crop_side(256, 256, 0, 0, 8) == 264
    assert T.crop_side(648, 640, 0, 0, 8) == 656
    # a 256 tile with 64 of context on a 1024 image: 384 -> 392
    assert T.crop_side(1024, 1024, 256, 64, 8) == 392
    # the crop is clamped to the image
    assert T.crop_side(100, 300, 256, 64, 8) == 304
    # the context rounds UP to a window and is never zero
    assert T.crop_side(1024, 1024, 256, 1, 8) == T.crop_side(1024, 1024, 256, 8, 8)
    assert T.crop_side(1024, 1024, 256, 9, 8) == T.crop_side(1024, 1024, 256, 16, 8)


def test_crate_device_model_is_the_references(pkg):
    """reference src/backend.rs:300-383 (gpu = true), checked against the
    figures its own comments quote: 3671 floats a padded pixel for the
    180-wide classical x4, 819 for the lightweight x2."""
    M, T = pkg.model, pkg.tiling
    assert T.crate_per_pixel_floats(M.classical(4)) == 3671
    assert T.crate_per_pixel_floats(M.lightweight(2)) == 819


def test_per_pixel_floats_stays_within_the_crates_device_model(pkg):
    """The crate budgets with its own device inventory (src/backend.rs:300-383);
    this backend must not allocate more per padded pixel than that model says,
    and its exact plan must stay within its own per-pixel bound."""
    M, T = pkg.model, pkg.tiling
    for a in (M.classical(4), M.classical(2), M.lightweight(2), M.realworld(), M.compressed()):
        assert T.per_pixel_floats(a) <= T.crate_per_pixel_floats(a), a.upsampler
        for h, w in [(8, 8), (37, 29), (256, 256), (480, 640)]:
            P = (h // 8 + 1) * 8 * ((w // 8 + 1) * 8)
            assert T.plan_floats(a, h, w) <= T.per_pixel_floats(a) * P


def test_plan_floats_counts_the_unit_layout_and_the_composed_octaves(pkg):
    """The terms the old figure missed: the qkv buffer's real size (the
    attention's unit layout, (heads+1)/2 x (6 hd + 2) floats a pixel = 546 at
    hd = 30; the body's Winograd convs' 36 transform planes of 4x4-pixel
    tiles, 9 C / 4 = 405 floats a pixel; the x4 head's Winograd 5x5 conv's 36
    planes of 2x2-pixel tiles of F = 64, 576 a pixel: whichever is largest)
    and the head planes the composed octaves never allocate."""
    M, T = pkg.model, pkg.tiling
    a = M.classical(4)
    P = 264 * 264
    terms = T._plan_terms(a, 256, 256)
    assert terms[3] == P * 576                  # qkv: the head's 5x5 products > unit layout (546)
    assert T._plan_terms(M.classical(2), 256, 256)[3] == P * 546  # x2: no 5x5 conv
    assert terms[-1] == P * 64                  # one head plane: both octaves composed
    assert T.plan_floats(M.classical(2), 256, 256) - T.plan_floats(a, 256, 256) == \
        3 * 256 * 256 * (4 - 16) - P * 30       # x2: one composed octave, plane 0 only; no 5x5


def test_auto_tile(pkg):
    T = pkg.tiling
    a = pkg.model.classical(4)
    per = T.crate_per_pixel_floats(a)
    # a budget the whole image fits: one pass
    assert T.auto_tile(a, per * 264 * 264 * 4, 256, 256, 32) == 0
    # a budget a 256 tile with 32 of context fits but the image does not
    side = T.crop_side(1024, 1024, 256, 32, 8)
    t = T.auto_tile(a, per * side * side * 4, 1024, 1024, 32)
    assert t == 256 and t % 8 == 0
    # the launch ceiling tiles even an unlimited budget
    big = T.auto_tile(a, 1 << 62, 2000, 2000, 32)
    assert big != 0 and T.crop_side(2000, 2000, big, 32, 8) ** 2 <= T.GPU_MAX_PLANE_PIXELS


class CappedBackend:
    """A backend that fails like a device out of memory above a crop size, or
    with another error when asked (test code only)."""

    def __init__(self, inner, max_side, error="hipMalloc(qkv) failed: out of memory"):
        self.inner, self.max_side, self.error, self.sizes = inner, max_side, error, []

    def forward(self, h, w, x):
        self.sizes.append((h, w))
        if max(h, w) > self.max_side:
            raise RuntimeError(self.error)
        return self.inner.forward(h, w, x)


def test_run_with_fallback_halves_until_the_tile_fits(pkg, orc):
    """reference src/main.rs:579-662: tile 0 falls back to half the image's
    longer side, then halves; each retry is announced; the result is
    run_tiled's at the tile that fitted."""
    M, T = pkg.model, pkg.tiling
    a = tiny(pkg)
    inner = OracleBackend(orc, a, M.make_weights(a, seed=8, perturb=True))
    img = M.to_unit(M.input_uniform(64, 48, seed=9))
    be = CappedBackend(inner, 32)
    notes = []
    got, tile = T.run_with_fallback(a, be, img, 0, 8, log=notes.append)
    assert tile == 16
    assert be.sizes[:2] == [(64, 48), (40, 40)]
    assert len(notes) == 2 and "--tile 0 is the only exact mode" in notes[0]
    assert "retrying with a 32x32 tile" in notes[0] and "retrying with a 16x16 tile" in notes[1]
    assert np.array_equal(got, T.run_tiled(a, inner, img, 16, 8))
    # quiet silences the note for a tile the user chose, never the one out of tile 0
    notes.clear()
    T.run_with_fallback(a, CappedBackend(inner, 32), img, 32, 8, quiet=True, log=notes.append)
    assert notes == []


class BatchingBackend:
    """A backend with `forward_batch` (the HIP backend's two-lane entry) over
    another one, recording each batch's shapes; out of memory above a crop
    size, like CappedBackend (test code only)."""

    def __init__(self, inner, max_side=1 << 30):
        self.inner, self.max_side, self.batches = inner, max_side, []

    def forward(self, h, w, x):
        raise AssertionError("the batched tile loop calls forward_batch only")

    def forward_batch(self, shapes, xs):
        self.batches.append(list(shapes))
        if max(max(s) for s in shapes) > self.max_side:
            raise RuntimeError("hipMalloc(qkv) failed: out of memory")
        return [self.inner.forward(h, w, x) for (h, w), x in zip(shapes, xs)]


def test_batched_tile_loop_is_the_sequential_one(pkg, orc):
    """run_tiled with `batch`: the image's crops go to one forward_batch call
    in the sequential loop's order, and the image is the sequential loop's;
    through run_with_fallback the out-of-memory retry halves the tile as for
    forward."""
    M, T = pkg.model, pkg.tiling
    a = tiny(pkg)
    inner = OracleBackend(orc, a, M.make_weights(a, seed=10, perturb=True))
    img = M.to_unit(M.input_uniform(40, 56, seed=11))
    seq = T.run_tiled(a, inner, img, 16, 8)
    bb = BatchingBackend(inner)
    assert np.array_equal(T.run_tiled(a, bb, img, 16, 8, batch=True), seq)
    assert len(bb.batches) == 1 and len(bb.batches[0]) == 3 * 4
    assert bb.batches[0][0] == (24, 24) and bb.batches[0][-1] == (16, 16)
    # tile 0 stays one whole-image forward
    assert np.array_equal(T.run_tiled(a, inner, img, 0, 8, batch=True), T.run_tiled(a, inner, img, 0, 8))
    capped = BatchingBackend(inner, max_side=32)
    got, tile = T.run_with_fallback(a, capped, img, 32, 8, quiet=True, batch=True)
    assert tile == 16 and np.array_equal(got, seq)


def test_run_with_fallback_retries_only_out_of_memory(pkg, orc):
    M, T = pkg.model, pkg.tiling
    a = tiny(pkg)
    inner = OracleBackend(orc, a, M.make_weights(a, seed=8, perturb=True))
    img = M.to_unit(M.input_uniform(32, 32, seed=9))
    be = CappedBackend(inner, 8, error="k_gemm failed: hipErrorIllegalAddress")
    with pytest.raises(RuntimeError, match="IllegalAddress"):
        T.run_with_fallback(a, be, img, 0, 8, log=lambda m: None)
    assert len(be.sizes) == 1
    # a one-window tile that still does not fit is not retried: the device's
    # own error ends the run (the guard is tile > win or tile == 0)
    be = CappedBackend(inner, 4)
    notes = []
    with pytest.raises(RuntimeError, match="out of memory"):
        T.run_with_fallback(a, be, img, 0, 8, log=notes.append)
    assert len(notes) == 2 and "retrying with a 8x8 tile" in notes[1]
    assert T.is_out_of_memory("cuMemAlloc failed: CUDA_ERROR_OUT_OF_MEMORY")
    assert not T.is_out_of_memory("launch failed")


def test_tile_covering_the_image_is_one_exact_pass(pkg, orc):
    M = pkg.model
    a = tiny(pkg)
    be = OracleBackend(orc, a, M.make_weights(a, seed=3, perturb=True))
    img = M.to_unit(M.input_uniform(20, 28, seed=2))
    whole = pkg.tiling.run_tiled(a, be, img, 0, 0)
    got = pkg.tiling.run_tiled(a, be, img, 64, 8)
    assert np.array_equal(got, whole)


@pytest.mark.parametrize("tile,pad", [(8, 0), (8, 8), (16, 0), (16, 16), (24, 8)])
def test_tiled_output_covers_the_image(pkg, orc, tile, pad):
    """reference tests/tiling.rs:79-109: a flat input leaves no pixel unwritten
    and the mosaic stays close to one pass."""
    M = pkg.model
    a = tiny(pkg)
    be = OracleBackend(orc, a, M.make_weights(a, seed=4, perturb=True))
    img = np.full((3, 32, 32), 0.55, np.float32)
    whole = pkg.tiling.run_tiled(a, be, img, 0, 0)
    got = pkg.tiling.run_tiled(a, be, img, tile, pad)
    assert np.count_nonzero(got == 0.0) == 0
    assert np.abs(got - whole).max() <= 1e-2


def test_the_pad_rounds_up_to_a_whole_window(pkg, orc):
    M = pkg.model
    a = tiny(pkg)
    be = OracleBackend(orc, a, M.make_weights(a, seed=5, perturb=True))
    img = M.to_unit(M.input_uniform(40, 40, seed=6))
    one = pkg.tiling.run_tiled(a, be, img, 8, 8)
    for asked in (0, 1, 7, 8):
        assert np.array_equal(pkg.tiling.run_tiled(a, be, img, 8, asked), one)
    # one more pixel of context asks for a second window
    two = pkg.tiling.run_tiled(a, be, img, 8, 9)
    assert np.array_equal(two, pkg.tiling.run_tiled(a, be, img, 8, 16))
    assert not np.array_equal(two, one)


def seam_image():
    """reference tests/tiling.rs:258-261: frac(0.618034 (3c + 11y + 29x)) on 32x32."""
    c = np.arange(3)[:, None, None]
    y = np.arange(32)[None, :, None]
    x = np.arange(32)[None, None, :]
    t = (c * 3 + y * 11 + x * 29).astype(np.float32) * np.float32(0.618034)
    return (t - np.floor(t)).astype(np.float32)


def seam_errors(pkg, a, be):
    """(one window of context, two windows) around 16-pixel tiles: the largest
    difference from the whole-image pass (reference tests/tiling.rs:262-265)."""
    T, img = pkg.tiling, seam_image()
    whole = T.run_tiled(a, be, img, 0, 0)
    win = a.window
    thin = float(np.abs(T.run_tiled(a, be, img, 2 * win, win) - whole).max())
    thick = float(np.abs(T.run_tiled(a, be, img, 2 * win, 2 * win) - whole).max())
    return thin, thick


def test_context_reduces_the_tiling_error(pkg, orc):
    """reference tests/tiling.rs:252-274 on the lightweight x2 model (random
    weights by the benchmark's rules, seed 0; the reference uses the published
    checkpoint): one window of context must leave more seam error than two,
    and two at most 0.02 (here, as in the reference's comment, exactly 0)."""
    M = pkg.model
    a = M.lightweight(2)
    thin, thick = seam_errors(pkg, a, OracleBackend(orc, a, M.make_weights(a, seed=0)))
    assert thin > thick, (thin, thick)
    assert thick <= 0.02, thick


# ---- the HIP backend through the tile loop ---------------------------------------

@pytest.mark.gpu
def test_context_reduces_the_tiling_error_on_the_device(pkg, orc):
    """The same property with the HIP backend behind the tile loop: one window
    of context leaves more error than two, two leave at most 0.02, and both
    figures equal the oracle's to 1e-4."""
    M = pkg.model
    a = M.lightweight(2)
    wts = M.make_weights(a, seed=0)
    be = pkg.abi.HipBackend(a, wts)
    try:
        thin, thick = seam_errors(pkg, a, be)
    finally:
        be.close()
    assert thin > thick, (thin, thick)
    assert thick <= 0.02, thick
    o_thin, o_thick = seam_errors(pkg, a, OracleBackend(orc, a, wts))
    assert abs(thin - o_thin) <= 1e-4 and abs(thick - o_thick) <= 1e-4, (thin, o_thin, thick, o_thick)


@pytest.mark.gpu
@pytest.mark.parametrize("tile,pad", [(16, 8), (24, 16), (0, 0)])
def test_tiled_device_matches_tiled_oracle(pkg, orc, tile, pad):
    M = pkg.model
    a = M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[1, 1])
    wts = M.make_weights(a, seed=7, perturb=True)
    img = M.to_unit(M.input_sinusoids(40, 52, seed=8))
    want = pkg.tiling.run_tiled(a, OracleBackend(orc, a, wts), img, tile, pad)
    be = pkg.abi.HipBackend(a, wts)
    try:
        got = pkg.tiling.run_tiled(a, be, img, tile, pad)
    finally:
        be.close()
    assert np.abs(got - want).max() < 1e-4


@pytest.mark.gpu
def test_config4_tile_geometry(pkg, orc):
    """Config 4's tiling (1024x1024, 256-pixel tiles, 64 of context, the
    compressed head) on a two-block model of the released width: every tile's
    crop runs on a 392x392 plane; a corner and an interior tile are each held
    against the oracle on the same crop, and the assembled image is finite and
    fully written."""
    M = pkg.model
    a = M.Arch(upsampler="pixelshuffle_aux", scale=4, embed=180, heads=6, depths=[1, 1])
    wts = M.make_weights(a, seed=5, perturb=True)
    img = M.to_unit(M.input_sinusoids(1024, 1024, seed=5))
    be = pkg.abi.HipBackend(a, wts)
    try:
        out = pkg.tiling.run_tiled(a, be, img, 256, 64)
        for (y0, y1, x0, x1) in [(0, 320, 0, 320), (192, 576, 448, 832)]:
            sub = np.ascontiguousarray(img[:, y0:y1, x0:x1])
            x = M.adjust(a, sub)
            got = be.forward(y1 - y0, x1 - x0, x)
            got_aux = be.aux()
            want, want_aux = orc.forward(a, wts, y1 - y0, x1 - x0, x)
            assert np.abs(got - want).max() < 1e-4
            assert np.abs(got_aux.reshape(want_aux.shape) - want_aux).max() < 1e-4
    finally:
        be.close()
    assert out.shape == (3, 4096, 4096)
    assert np.isfinite(out).all() and np.count_nonzero(out == 0.0) == 0
