"""A seeded sweep of image sizes over the model families, through the device
forward against the oracle (reference src/cpu.rs:1471-1759, the crate's CPU
path), at the north-star bars: 1e-4 max-abs on the [0, 1] image and one 8-bit
level.

The sizes are drawn once from a fixed generator, so the cases are the same on
every run: widths and heights from 8 to 71, which covers planes that are exact
window multiples (the reference then pads a whole window), planes one pixel
past one, and aspect ratios far from square. Each family runs at its released
width (C = 180, or 60 for the lightweight model) with one stage of two blocks,
so both the plain and the shifted-window attention run, and four strips
narrower than two windows (up to 517 pixels long) follow. Every case is
forwarded three times on one context: the plan is reused on the second call,
the third replays the forward as a captured graph, and all three must be
equal bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FAMILIES = [
    ("pixelshuffle", 2, 180), ("pixelshuffle", 4, 180), ("pixelshuffle", 8, 180),
    ("pixelshuffledirect", 2, 60), ("pixelshuffledirect", 3, 60), ("pixelshuffledirect", 4, 60),
    ("nearest+conv", 4, 180), ("pixelshuffle_aux", 4, 180),
]


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(16):
        up, scale, c = FAMILIES[i % len(FAMILIES)]
        hi = 33 if scale == 8 else 72  # the x8 head's planes grow 64-fold
        h, w = (int(v) for v in rng.integers(8, hi, size=2))
        out.append((up, scale, c, h, w, 100 + i))
    # and strips narrower than two windows
    out += [("pixelshuffle", 4, 180, 8, 517, 200), ("pixelshuffle", 2, 180, 301, 9, 201),
            ("pixelshuffledirect", 3, 60, 13, 401, 202), ("nearest+conv", 4, 180, 260, 11, 203)]
    return out


@pytest.mark.parametrize("up,scale,c,h,w,seed", _cases(),
                         ids=lambda v: str(v) if not isinstance(v, str) else v)
def test_forward_sweep(pkg, orc, up, scale, c, h, w, seed):
    M = pkg.model
    arch = M.Arch(upsampler=up, scale=scale, embed=c, heads=6, depths=[2])
    wts = M.make_weights(arch, seed=seed, perturb=True)
    x = M.adjust(arch, M.to_unit(M.input_uniform(h, w, seed=seed)))
    want, want_aux = orc.forward(arch, wts, h, w, x)
    be = pkg.abi.HipBackend(arch, wts)
    try:
        got = [be.forward(h, w, x) for _ in range(3)]
        aux = be.aux()
    finally:
        be.close()
    assert got[0].shape == want.shape == (3, h * scale, w * scale)
    assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2])
    err = float(np.abs(got[0] - want).max())
    assert err < 1e-4, err
    d8 = np.abs(M.to_rgb8(got[0]).astype(int) - M.to_rgb8(want).astype(int)).max()
    assert d8 <= 1
    if want_aux is not None:
        assert float(np.abs(aux.reshape(want_aux.shape) - want_aux).max()) < 1e-4
