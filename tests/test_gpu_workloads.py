"""Parity at the real workloads: BASELINE.json's configurations and the
headline benchmark, at their full sizes, depths and seeds, with the plain
benchmark-rule weights (not the perturbed ones the unit tests use), through
the C ABI against the oracle (the C restatement of the crate's CPU path).

Bars (north_star): <= 1e-4 max-abs on the fp32 output, <= 1 level on the
8-bit image; the RSTB plane at 1e-4 relative to its magnitude (its values are
N(0, 1) activations, not a [0, 1] image). The reference's own cross-backend
test runs the whole network at real widths the same way
(tests/gpu.rs:96-173).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def check_image(M, got, want, aux=None, want_aux=None):
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    err = float(np.abs(got - want).max())
    assert err <= 1e-4, err
    d8 = int(np.abs(M.to_rgb8(got).astype(int) - M.to_rgb8(want).astype(int)).max())
    assert d8 <= 1, d8
    if want_aux is not None:
        assert aux is not None and aux.size == want_aux.size
        assert float(np.abs(aux.reshape(want_aux.shape) - want_aux).max()) <= 1e-4


def test_headline_workload(pkg, orc):
    """bench.py's exact workload: classical x4, 256x256 -> 1024x1024, weights
    by the benchmark's rules at seed 3, config 2's input generator at seed 3;
    through the host entry (s2s_forward) and the HBM-resident one the bench
    times (s2s_forward_device)."""
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=3)
    h = w = 256
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=3)))
    be = pkg.HipBackend(arch, wts)
    try:
        got = be.forward(h, w, x)
        din = hip.DeviceBuffer.from_array(x)
        dout = hip.DeviceBuffer(3 * 1024 * 1024)
        # three identical calls, as the bench makes them: launched kernel by
        # kernel, captured into the library's graph and launched, replayed
        for i in range(3):
            dout.upload(np.zeros(3 * 1024 * 1024, np.float32))
            be.forward_device(h, w, din.ptr, dout.ptr)
            hip.stream_synchronize(be.stream())
            got_dev = dout.download((3, 1024, 1024))
            assert np.array_equal(got, got_dev), (i, float(np.abs(got - got_dev).max()))
    finally:
        be.close()
    want, _ = orc.forward(arch, wts, h, w, x)
    check_image(M, got, want)


def test_config1_single_rstb(pkg, orc):
    """Config 1: one RSTB (6 Swin V2 layers, shifts 0/4, the close) on the
    UNPADDED 256x256x180 plane (1024 windows), N(0, 1) activations seed 2,
    weights seed 0 - bench.py --workload rstb's exact inputs."""
    M, hip = pkg.model, pkg.hip
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=180, heads=6, depths=[6])
    wts = M.make_weights(arch, seed=0)
    hp = wp = 256
    x = np.random.Generator(np.random.PCG64(2)).standard_normal((hp * wp, 180), dtype=np.float32)
    be = pkg.HipBackend(arch, wts)
    try:
        din = hip.DeviceBuffer.from_array(x)
        dout = hip.DeviceBuffer(din.n)
        be.rstb_device(0, hp, wp, din.ptr, dout.ptr)
        hip.synchronize()
        got = dout.download((hp * wp, 180))
    finally:
        be.close()
    p = orc.plan_explicit(hp, wp, 8, 180)
    want = orc.rstb(arch, wts, p, 0, np.ascontiguousarray(x.T.reshape(180, hp, wp)))
    want = want.reshape(180, hp * wp).T
    err = float(np.abs(got - want).max()) / max(1.0, float(np.abs(want).max()))
    assert err <= 1e-4, err


def test_config2_classical_x2(pkg, orc):
    """Config 2: classical x2, 256x256 -> 512x512, weights seed 3, the
    sinusoid input at seed 3."""
    M = pkg.model
    arch = M.classical(2)
    wts = M.make_weights(arch, seed=3)
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(256, 256, seed=3)))
    be = pkg.HipBackend(arch, wts)
    try:
        got = be.forward(256, 256, x)
    finally:
        be.close()
    want, _ = orc.forward(arch, wts, 256, 256, x)
    check_image(M, got, want)


def test_config3_realworld_x4(pkg, orc):
    """Config 3: real-world x4 (nearest+conv), 6x6 layers, 480x640 ->
    1920x2560, weights seed 4, the DCT-quantised texture input at seed 4."""
    M = pkg.model
    arch = M.realworld()
    wts = M.make_weights(arch, seed=4)
    x = M.adjust(arch, M.to_unit(M.input_texture_dct(480, 640, seed=4)))
    be = pkg.HipBackend(arch, wts)
    try:
        got = be.forward(480, 640, x)
        again = be.forward(480, 640, x)
    finally:
        be.close()
    assert np.array_equal(got, again)
    want, _ = orc.forward(arch, wts, 480, 640, x)
    check_image(M, got, want)


def test_config0_lightweight_x2(pkg, orc):
    """Config 0: lightweight x2 (C 60, 4x6 layers, pixelshuffledirect),
    64x64 uniform input seed 1 -> 128x128, weights seed 0."""
    M = pkg.model
    arch = M.lightweight(2)
    wts = M.make_weights(arch, seed=0)
    x = M.adjust(arch, M.to_unit(M.input_uniform(64, 64, seed=1)))
    be = pkg.HipBackend(arch, wts)
    try:
        got = be.forward(64, 64, x)
    finally:
        be.close()
    want, _ = orc.forward(arch, wts, 64, 64, x)
    check_image(M, got, want)


class RecordingBackend:
    """The HIP backend behind `Backend`, keeping each tile's input, output and
    aux image (test code only)."""

    def __init__(self, be):
        self.be, self.calls = be, []

    def forward(self, h, w, x):
        out = self.be.forward(h, w, x)
        self.calls.append((h, w, x, out, self.be.aux()))
        return out


def test_config4_compressed_tiled(pkg, orc):
    """Config 4: compressed x4 (pixelshuffle_aux), 6x6 layers, 1024x1024 in
    256-pixel tiles with 64 of context (16 tiles on 392x392 planes) -> 4096 x
    4096, weights seed 5, config 3's input generator at seed 5. Parity per tile
    against the oracle on the same crop (output and aux image) for one tile of
    each of the four crop shapes - a corner (320x320), the two edges (320x384
    and 384x320) and an interior tile (384x384) - and for the far corner; every
    tile of the assembled image is the device tile's interior."""
    M = pkg.model
    arch = M.compressed()
    wts = M.make_weights(arch, seed=5)
    img = M.to_unit(M.input_texture_dct(1024, 1024, seed=5))
    be = pkg.HipBackend(arch, wts)
    rec = RecordingBackend(be)
    try:
        out = pkg.tiling.run_tiled(arch, rec, img, 256, 64)
    finally:
        be.close()
    assert out.shape == (3, 4096, 4096) and np.isfinite(out).all()
    assert len(rec.calls) == 16
    assert {(h, w) for h, w, *_ in rec.calls} == {(320, 320), (320, 384), (384, 320), (384, 384)}
    for i in (0, 1, 4, 6, 15):  # tiles (0,0), (0,1), (1,0), (1,2), (3,3)
        h, w, x, got, aux = rec.calls[i]
        assert (h, w) == {0: (320, 320), 1: (320, 384), 4: (384, 320), 6: (384, 384), 15: (320, 320)}[i]
        want, want_aux = orc.forward(arch, wts, h, w, x)
        check_image(M, got, want, aux, want_aux)
        ty, tx = divmod(i, 4)
        y0, x0 = max(ty * 256 - 64, 0), max(tx * 256 - 64, 0)
        oy, ox = (ty * 256 - y0) * 4, (tx * 256 - x0) * 4
        assert np.array_equal(out[:, ty * 1024:(ty + 1) * 1024, tx * 1024:(tx + 1) * 1024],
                              got[:, oy:oy + 1024, ox:ox + 1024])


@pytest.mark.parametrize("kind", ["mean", "white", "checker"])
def test_degenerate_images(pkg, orc, kind):
    """Degenerate images against the oracle: every pixel at the normalisation
    mean (the adjusted input is exactly 0: every activation comes from the
    conv biases alone, the same at every interior pixel, so every window's
    tokens are equal and its softmax is uniform up to the position bias), a
    constant white image, and a one-pixel black/white checkerboard (the
    largest step between neighbours), through classical x4 and the
    lightweight x2 model at 24 x 40."""
    M = pkg.model
    h, w = 24, 40
    for arch, seed in ((M.classical(4), 81), (M.lightweight(2), 82)):
        wts = M.make_weights(arch, seed=seed)
        if kind == "mean":
            img = np.broadcast_to(np.asarray(arch.mean, np.float32)[:, None, None], (3, h, w)).copy()
        elif kind == "white":
            img = np.ones((3, h, w), np.float32)
        else:
            yy, xx = np.mgrid[0:h, 0:w]
            img = np.broadcast_to(((yy + xx) % 2).astype(np.float32), (3, h, w)).copy()
        x = M.adjust(arch, img)
        if kind == "mean":
            assert not np.any(x)
        be = pkg.HipBackend(arch, wts)
        try:
            got = be.forward(h, w, x)
        finally:
            be.close()
        want, _ = orc.forward(arch, wts, h, w, x)
        check_image(M, got, want)
