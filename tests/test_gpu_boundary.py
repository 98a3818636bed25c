"""The drop-in boundary on the device: the memory queries the crate's policy
calls (`gpu::uploaded_bytes(&Weights)` before any backend exists, the per-image
plan), the aggregate self-test behind `--cuda-selftest`, the allocation cap and
the tile-halving retry it lets a test drive (`run_with_fallback`), and the
checkpoint variants of the CPB table."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def archs(M):
    return [M.classical(4), M.classical(2), M.lightweight(2), M.realworld(), M.compressed(),
            M.Arch(upsampler="pixelshuffle", scale=8, embed=24, heads=2, depths=[1, 0, 2]),
            M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[1], feat=32)]


def test_uploaded_bytes_for_is_what_create_uploads(pkg):
    """reference src/gpu.rs:792-799, called by memory_budget before any backend
    exists (src/main.rs:459-471): the context-free figure equals the context's."""
    M = pkg.model
    for arch in archs(M):
        wts = M.make_weights(arch, seed=1)
        want = pkg.abi.uploaded_bytes_for(arch, wts)
        be = pkg.HipBackend(arch, wts)
        try:
            assert be.uploaded_bytes() == want, arch
        finally:
            be.close()


def test_plan_bytes_is_the_tiling_plan(pkg):
    """s2s_plan_bytes equals the tiling mirror's exact plan, and the plan per
    padded pixel stays within both this backend's bound and the crate's own
    device model (src/backend.rs:300-383)."""
    M, T = pkg.model, pkg.tiling
    for arch in archs(M):
        be = pkg.HipBackend(arch, M.make_weights(arch, seed=1))
        try:
            for h, w in [(8, 8), (37, 29), (256, 256), (480, 640)]:
                got = be.plan_bytes(h, w)
                assert got == 4 * T.plan_floats(arch, h, w), (arch.upsampler, h, w)
                P = (h // 8 + 1) * 8 * ((w // 8 + 1) * 8)
                assert got <= 4 * T.per_pixel_floats(arch) * P
                assert T.per_pixel_floats(arch) <= T.crate_per_pixel_floats(arch)
        finally:
            be.close()


@pytest.mark.parametrize("which", ["classical", "lightweight"])
def test_selftest(pkg, which, capfd):
    """The crate's --cuda-selftest (reference src/gpu.rs:889-1265) for the
    released widths: every kernel against its definition, and the checkpoint's
    CPB tables (device MLP against cpb_pre)."""
    M = pkg.model
    arch = M.classical(4) if which == "classical" else M.lightweight(2)
    pkg.abi.selftest(arch, M.make_weights(arch, seed=2, perturb=True))
    out = capfd.readouterr().out
    assert "hip selftest:" in out
    n = int(out.split("hip selftest:")[1].split()[0])
    assert n >= 35, out


def test_alloc_limit_gives_out_of_memory_and_the_context_recovers(pkg):
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[1, 1])
    wts = M.make_weights(arch, seed=3, perturb=True)
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(64, 64, seed=3)))
    os.environ["SWIN2SR_HIP_ALLOC_LIMIT"] = "1000000"
    try:
        be = pkg.HipBackend(arch, wts)
    finally:
        del os.environ["SWIN2SR_HIP_ALLOC_LIMIT"]
    try:
        assert be.plan_bytes(64, 64) > 1000000
        with pytest.raises(pkg.abi.S2SError, match="out of memory"):
            be.forward(64, 64, x)
        be.set_alloc_limit(be.plan_bytes(64, 64))
        y = be.forward(64, 64, x)
        be.set_alloc_limit(0)
        assert np.array_equal(be.forward(64, 64, x), y)
    finally:
        be.close()


class OracleBackend:
    def __init__(self, orc, arch, weights):
        self.orc, self.arch, self.weights = orc, arch, weights

    def forward(self, h, w, x):
        return self.orc.forward(self.arch, self.weights, h, w, x)[0]


def test_run_with_fallback_halves_the_tile_on_the_device(pkg, orc):
    """reference src/main.rs:579-662 over the HIP backend: a whole-image pass
    that does not fit the cap falls back to half the image, then halves again,
    each retry announced; the result is the tiled oracle's at the final tile."""
    M, T = pkg.model, pkg.tiling
    arch = M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[1, 1])
    wts = M.make_weights(arch, seed=4, perturb=True)
    img = M.to_unit(M.input_sinusoids(64, 64, seed=4))
    be = pkg.HipBackend(arch, wts)
    notes = []
    try:
        # tile 32 + 8 of context: crops up to 40 pixels; tile 16: up to 32
        cap = be.plan_bytes(32, 32)
        assert be.plan_bytes(40, 40) > cap
        be.set_alloc_limit(cap)
        got, tile = T.run_with_fallback(arch, be, img, 0, 8, log=notes.append)
    finally:
        be.close()
    assert tile == 16
    assert len(notes) == 2
    assert "out of memory" in notes[0] and "retrying with a 32x32 tile" in notes[0]
    assert "--tile 0 is the only exact mode" in notes[0]
    assert "retrying with a 16x16 tile" in notes[1]
    want = T.run_tiled(arch, OracleBackend(orc, arch, wts), img, 16, 8)
    assert np.abs(got - want).max() < 1e-4


@pytest.mark.parametrize("keep", ["cpb_pre", "cpb_mlp"])
def test_checkpoint_with_one_cpb_source(pkg, orc, keep):
    """A checkpoint may carry the converter's cpb_pre table, the cpb_mlp
    weights, or both (tools/convert.py keeps both). The device reads cpb_pre
    when present - the table the crate itself uses - and computes the table
    from the MLP otherwise; both must give the oracle's image."""
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=60, heads=6, depths=[2])
    full = M.make_weights(arch, seed=6, perturb=True)
    drop = "cpb_mlp" if keep == "cpb_pre" else "cpb_pre"
    wts = {k: v for k, v in full.items() if drop not in k}
    assert len(wts) < len(full)
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(40, 48, seed=6)))
    be = pkg.HipBackend(arch, wts)
    try:
        got = be.forward(40, 48, x)
    finally:
        be.close()
    want, _ = orc.forward(arch, full, 40, 48, x)
    assert np.abs(got - want).max() < 1e-4


@pytest.mark.parametrize("upsampler", ["nearest+conv", "pixelshuffle_aux"])
def test_head_planes_past_2gib(pkg, upsampler):
    """The heads at a 760 x 760 image (a 768^2 padded plane): nearest+conv's
    16*P*feat planes pass 2 GiB (16*P*64*4 B = 2.4 GB each; written by the
    LeakyReLU conv epilogue, read by conv_hr's loader and by conv_last); the
    compressed head, its octaves and its bicubic branch composed with
    conv_last, holds no plane that large, and runs the composed kernels and
    the bicubic plane (16*P*4 floats) at this size. The input repeats a random
    16 x 16 patch, so away from the borders every output sees what it sees in a
    200 x 200 image of the same pattern, and the two must agree bit for bit
    there (each output's arithmetic is independent of where it sits in the
    launch)."""
    M = pkg.model
    arch = M.Arch(upsampler=upsampler, scale=4, embed=180, heads=6, depths=[1])
    be = pkg.HipBackend(arch, M.make_weights(arch, seed=1, perturb=True))
    patch = np.random.default_rng(5).uniform(0, 1, (3, 16, 16)).astype(np.float32)
    try:
        plane = 16 * 768 * 768 * 64 * 4      # nearest+conv's largest head plane, bytes
        if upsampler == "nearest+conv":
            assert plane > 2 ** 31 and be.plan_bytes(760, 760) > plane
        outs = []
        for n in (760, 200):
            img = np.tile(patch, (1, n // 16 + 1, n // 16 + 1))[:, :n, :n]
            outs.append(be.forward(n, n, M.adjust(arch, np.ascontiguousarray(img))))
        big, small = outs
        assert big.shape == (3, 3040, 3040) and np.isfinite(big).all()
        sl = (slice(None), slice(4 * 64, 4 * 128), slice(4 * 64, 4 * 128))
        assert np.array_equal(big[sl], small[sl])
    finally:
        be.close()


@pytest.mark.parametrize("upsampler", ["pixelshuffle", "pixelshuffle_aux"])
def test_held_buffers_serve_smaller_and_transposed_images(pkg, upsampler):
    """A context keeps its buffers while a new image's plan fits them (a
    smaller image after a larger one, the same pixel count transposed, as a
    tiled image alternates), and plans afresh only for a larger one. Through a
    sequence of sizes on one context, host and device entries and the graph
    replays included, every output (and aux image) equals that of a fresh
    context run at that size alone, bit for bit."""
    M, hip = pkg.model, pkg.hip
    arch = M.Arch(upsampler=upsampler, scale=4, embed=180, heads=6, depths=[1, 1])
    wts = M.make_weights(arch, seed=12, perturb=True)
    sizes = [(40, 56), (24, 40), (40, 24), (16, 16), (40, 56), (48, 64), (24, 40)]
    xs = {hw: M.adjust(arch, M.to_unit(M.input_sinusoids(*hw, seed=hw[0] + hw[1]))) for hw in set(sizes)}
    want = {}
    for hw, x in xs.items():
        fresh = pkg.HipBackend(arch, wts)
        try:
            want[hw] = (fresh.forward(*hw, x), fresh.aux())
        finally:
            fresh.close()
    be = pkg.HipBackend(arch, wts)
    try:
        for h, w in sizes:
            got = be.forward(h, w, xs[(h, w)])
            assert np.array_equal(got, want[(h, w)][0]), (h, w)
            if upsampler == "pixelshuffle_aux":
                assert np.array_equal(be.aux(), want[(h, w)][1]), (h, w)
            # the device entry three times (eager, captured, replayed)
            din = hip.DeviceBuffer.from_array(xs[(h, w)])
            dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
            for _ in range(3):
                be.forward_device(h, w, din.ptr, dout.ptr)
                hip.stream_synchronize(be.stream())
                assert np.array_equal(dout.download((3, h * 4, w * 4)), want[(h, w)][0]), (h, w)
            din.free()
            dout.free()
    finally:
        be.close()
