"""GPU parity: every kernel of the HIP path against the CPU oracle, through the C ABI.

Bars (north_star): index / mask maps bit-exact; fp32 ops within rounding of
the reference's own selftest tolerances (2e-5 for kernels, src/gpu.rs:892);
whole-network output within 1e-4 max-abs on the [0,1] image and within one
8-bit level after `to_rgb8`.

Widths: the reference found a race that only showed above one 32-lane warp
(tests/gpu.rs:1-21); every kernel here is also run on planes wider than one
64-lane wavefront and larger than one workgroup tile (128 rows).
"""
import numpy as np
import pytest

import refimpl as R

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def nchw_to_hwc(x):
    return np.ascontiguousarray(x.transpose(1, 2, 0).reshape(-1, x.shape[0]))


def hwc_to_nchw(x, h, w):
    return np.ascontiguousarray(x.reshape(h, w, -1).transpose(2, 0, 1))


@pytest.mark.parametrize("hp,wp", [(16, 16), (16, 24), (72, 80), (264, 264)])
@pytest.mark.parametrize("shift", [0, 4])
def test_window_map_bit_exact(pkg, orc, hp, wp, shift):
    abi = pkg.abi
    yx, reg = abi.test_window_map(hp, wp, shift)
    p = orc.plan_explicit(hp, wp, 8, 4)
    want_yx, want_reg = orc.window_map(p, shift)
    assert np.array_equal(yx, want_yx)
    assert np.array_equal(reg, want_reg)


@pytest.mark.parametrize("heads,hd", [(2, 2), (6, 30), (6, 10), (3, 32), (2, 12), (3, 4)])
@pytest.mark.parametrize("shift", [0, 4])
@pytest.mark.parametrize("hp,wp", [(16, 16), (40, 72)])
def test_attention(pkg, orc, heads, hd, shift, hp, wp):
    abi = pkg.abi
    c = heads * hd
    if c % 4:
        pytest.skip("channel count must be a multiple of 4 for the device layout")
    r = rng(heads * 100 + hd + shift + hp)
    p = orc.plan_explicit(hp, wp, 8, c)
    n = 64
    # plane-order q, k, v [P][c] each; the oracle wants window-major tokens
    q = r.standard_normal((c, hp, wp), dtype=np.float32)
    k = r.standard_normal((c, hp, wp), dtype=np.float32)
    v = r.standard_normal((c, hp, wp), dtype=np.float32)
    ls = np.array([1.3 - 0.2 * i for i in range(heads)], np.float32)
    ls[0] = np.log(300.0)  # above the log(100) clamp
    cpb = (r.standard_normal((n * n, heads), dtype=np.float32) * 3.0).astype(np.float32)
    qkv_tok = np.concatenate([orc.gather(p, t, shift) for t in (q, k, v)], axis=0)
    want_tok = orc.attention(p, heads, hd, ls, cpb, qkv_tok, shift)
    want = nchw_to_hwc(orc.scatter(p, want_tok, shift))
    qkv_plane = np.concatenate([nchw_to_hwc(t) for t in (q, k, v)], axis=1)
    got = abi.test_attention(hp, wp, heads, hd, shift, qkv_plane, ls, cpb)
    # against the oracle: the reference selftest's 2e-5 (src/gpu.rs:892), scaled by
    # the value range (its inputs were sin(); these are N(0,1)), because the
    # reference CPU's fast_exp carries 1.6e-5 relative error
    vmax = max(1.0, float(np.abs(v).max()))
    err = np.abs(got - want).max()
    assert err < 2e-5 * vmax, err
    # against exact float64 math: fp32 cosines carry ~1.2e-7 relative error, which
    # the temperature exp(min(ls, ln 100)) multiplies into the logits
    qw, kw, vw = (R.shifted_windows(t, 8, shift) for t in (q, k, v))
    mids = R.mask_regions(hp, wp, 8, shift) if shift else None
    exact = R.window_attention(qw, kw, vw, ls, cpb, mids)
    exact = nchw_to_hwc(R.unshift_windows(exact, 8, shift, hp, wp))
    temp = float(np.exp(min(ls.max(), np.log(100.0))))
    assert np.abs(got - exact).max() < vmax * (5e-6 + 1.2e-7 * temp)


def test_cpb_table(pkg, orc):
    M = pkg.model
    r = rng(5)
    w0 = r.standard_normal((512, 2), dtype=np.float32)
    b0 = r.uniform(-0.5, 0.5, 512).astype(np.float32)
    w2 = (r.standard_normal((6, 512), dtype=np.float32) * 0.1).astype(np.float32)
    want = M.cpb_pre(w0, b0, w2, 8)
    got = pkg.abi.test_cpb_table(8, 6, w0, b0, w2)
    assert np.abs(got - want).max() < 1e-4


@pytest.mark.parametrize("rows,cin,cout", [(37, 60, 43), (300, 180, 180), (513, 180, 540),
                                           (200, 360, 180), (130, 180, 360), (97, 27, 64),
                                           (150, 120, 60), (20011, 180, 540), (17003, 360, 180)])
@pytest.mark.parametrize("epi", [0, 1, 2, 5])
def test_linear(pkg, orc, rows, cin, cout, epi):
    r = rng(rows + cin + cout + epi)
    x = r.standard_normal((rows, cin), dtype=np.float32)
    w = (r.standard_normal((cout, cin), dtype=np.float32) / np.sqrt(cin)).astype(np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    res = r.standard_normal((rows, cout), dtype=np.float32)
    base = orc.linear(x, w, b)
    if epi == 0:
        want = base
    elif epi == 1:
        want = orc.gelu(base)
    elif epi == 2:
        want = base + res
    else:
        want = np.where(base < 0, base * np.float32(0.2), base)
    got = pkg.abi.test_linear(x, w, b, epilogue=epi, res=res if epi == 2 else None, slope=0.2)
    err = np.abs(got - want).max()
    assert err < 3e-5 * max(1.0, np.abs(want).max()), err


@pytest.mark.parametrize("c", [180, 60, 27])
def test_gelu_epilogue_against_exact_erf(pkg, c):
    """The device GELU (an erfc-based polynomial form, both GEMM kernels'
    epilogues: K = 180 and 60 take the weight-stationary kernel, 27 the tiled
    one) against the float64 erf GELU over [-12, 12] and at 0 / -0 / tiny
    arguments; an identity weight makes the GEMM pass each value through
    exactly. Bar: 1e-6 absolute, the rounding of a float32 erff form."""
    from scipy.special import erf
    r = rng(c)
    n = 8192
    vals = np.concatenate([np.linspace(-12, 12, n * c // 2, dtype=np.float32),
                           r.standard_normal(n * c // 2 - 6).astype(np.float32) * 2,
                           np.float32([0.0, -0.0, 1e-30, -1e-30, 1e-7, -1e-7])])
    x = vals.reshape(n, c)
    eye = np.eye(c, dtype=np.float32)
    got = pkg.abi.test_linear(x, eye, np.zeros(c, np.float32), epilogue=1)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1.0 + erf(xd / np.sqrt(2.0)))
    err = np.abs(got - want).max()
    assert err < 1e-6, err
    assert np.all(got[x >= 0] >= 0) and np.all(got[x < 0] <= 0)


@pytest.mark.parametrize("rows,cin,cout", [(37, 60, 60), (300, 180, 180), (129, 360, 180),
                                           (70, 120, 60), (23001, 180, 180), (19005, 360, 180)])
@pytest.mark.parametrize("with_res", [False, True])
def test_linear_layernorm(pkg, orc, rows, cin, cout, with_res):
    r = rng(rows * 7 + cin + with_res)
    x = r.standard_normal((rows, cin), dtype=np.float32)
    w = (r.standard_normal((cout, cin), dtype=np.float32) / np.sqrt(cin)).astype(np.float32)
    b = r.standard_normal(cout, dtype=np.float32) * np.float32(0.3)
    g = (1 + 0.2 * r.standard_normal(cout)).astype(np.float32)
    beta = (0.1 * r.standard_normal(cout)).astype(np.float32)
    res = r.standard_normal((rows, cout), dtype=np.float32)
    y = orc.linear(x, w, b)
    ln = orc.channel_layer_norm(np.ascontiguousarray(y.T), g, beta).T
    want = ln + res if with_res else ln
    got = pkg.abi.test_linear(x, w, b, epilogue=4 if with_res else 3, res=res if with_res else None,
                              ln_w=g, ln_b=beta)
    err = np.abs(got - want).max()
    assert err < 5e-5, err


@pytest.mark.parametrize("hw,c", [(100, 180), (1000, 60), (77, 64), (1, 180), (4099, 180), (9, 60)])
@pytest.mark.parametrize("with_res", [False, True])
def test_layernorm(pkg, orc, hw, c, with_res):
    r = rng(hw + c)
    x = (r.standard_normal((hw, c), dtype=np.float32) * 3 + 1).astype(np.float32)
    g = (1 + 0.2 * r.standard_normal(c)).astype(np.float32)
    b = (0.1 * r.standard_normal(c)).astype(np.float32)
    res = r.standard_normal((hw, c), dtype=np.float32)
    want = orc.channel_layer_norm(np.ascontiguousarray(x.T), g, b).T
    if with_res:
        want = want + res
    got = pkg.abi.test_ln_residual(x, g, b, res if with_res else None)
    assert np.abs(got - want).max() < 3e-5


@pytest.mark.parametrize("h,w,c", [(16, 16, 180), (24, 40, 180), (19, 23, 60), (5, 33, 24),
                                   (1, 17, 192), (72, 80, 180)])
def test_embed(pkg, orc, h, w, c):
    """The forward's first kernel (conv_first, and the folded patch_embed +
    LayerNorm, on fp32 MFMA) against the oracle's direct conv3x3 and channel
    LayerNorm: planes ending in a partial 16-pixel task, one pixel high, the
    released widths, and widths whose channels leave waves with no columns."""
    r = rng(h * w + c)
    x = (0.5 * r.standard_normal((3, h, w))).astype(np.float32)
    w1 = (r.standard_normal((c, 3, 3, 3)) / np.sqrt(27)).astype(np.float32)
    b1 = (0.1 * r.standard_normal(c)).astype(np.float32)
    w2 = (r.standard_normal((c, 3, 3, 3)) / np.sqrt(27)).astype(np.float32)
    b2 = (0.1 * r.standard_normal(c)).astype(np.float32)
    g = (1 + 0.2 * r.standard_normal(c)).astype(np.float32)
    be = (0.1 * r.standard_normal(c)).astype(np.float32)
    x_hwc = np.ascontiguousarray(x.reshape(3, h * w).T)
    body, cur = pkg.abi.test_embed(x_hwc, h, w, w1, b1, w2, b2, g, be)
    want_body = orc.conv3x3(x, w1, b1).reshape(c, h * w)
    want_cur = orc.channel_layer_norm(np.ascontiguousarray(orc.conv3x3(x, w2, b2).reshape(c, h * w)), g, be)
    assert np.abs(body - want_body.T).max() < 2e-6
    assert np.abs(cur - want_cur.T).max() < 2e-5


@pytest.mark.parametrize("h,w,cin,cout", [(5, 7, 3, 4), (7, 9, 4, 12), (33, 39, 16, 20),
                                          (20, 70, 180, 180), (9, 11, 180, 64), (16, 16, 64, 3)])
@pytest.mark.parametrize("epi", [0, 2, 5])
def test_conv3x3(pkg, orc, h, w, cin, cout, epi):
    r = rng(h * w + cin + cout + epi)
    x = r.standard_normal((cin, h, w), dtype=np.float32)
    wt = (r.standard_normal((cout, cin, 3, 3), dtype=np.float32) / np.sqrt(9 * cin)).astype(np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    res = r.standard_normal((cout, h, w), dtype=np.float32)
    base = orc.conv3x3(x, wt, b)
    if epi == 0:
        want = base
    elif epi == 2:
        want = base + res
    else:
        want = np.where(base < 0, base * np.float32(0.01), base)
    got = pkg.abi.test_conv3x3(nchw_to_hwc(x), h, w, wt, b, epilogue=epi,
                               res=nchw_to_hwc(res) if epi == 2 else None, slope=0.01)
    err = np.abs(hwc_to_nchw(got, h, w) - want).max()
    assert err < 5e-5, err


@pytest.mark.parametrize("shift", [0, 4])
@pytest.mark.parametrize("hp,wp", [(16, 16), (40, 72), (264, 264)])
def test_block_attention_fused(pkg, orc, shift, hp, wp):
    """6 heads of 30 (C = 180): the block's qkv projection and window
    attention run as one kernel (the pair's q|k|v straight from the GEMM into
    the attention's LDS unit). From x and the block's weights against the
    qkv linear in float64 and the oracle's attention, at the attention test's
    bars, up to the headline plane with its wrapped last window row and
    column."""
    abi = pkg.abi
    heads, hd = 6, 30
    c = heads * hd
    r = rng(hp * wp + shift + 11)
    P = hp * wp
    x = r.standard_normal((P, c), dtype=np.float32)
    w = (r.standard_normal((3 * c, c), dtype=np.float32) / np.sqrt(c)).astype(np.float32)
    b = r.standard_normal(3 * c, dtype=np.float32)
    b[c:2 * c] = 0.0  # k has no bias
    ls = np.array([1.3 - 0.2 * i for i in range(heads)], np.float32)
    ls[0] = np.log(300.0)  # above the log(100) clamp
    cpb = (r.standard_normal((64 * 64, heads), dtype=np.float32) * 3.0).astype(np.float32)
    qkv = (x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32)  # [P][3c]
    p = orc.plan_explicit(hp, wp, 8, c)
    planes = [hwc_to_nchw(np.ascontiguousarray(qkv[:, i * c:(i + 1) * c]), hp, wp) for i in range(3)]
    qkv_tok = np.concatenate([orc.gather(p, t, shift) for t in planes], axis=0)
    want = nchw_to_hwc(orc.scatter(p, orc.attention(p, heads, hd, ls, cpb, qkv_tok, shift), shift))
    got = abi.test_block_attention(hp, wp, heads, hd, shift, x, w, b, ls, cpb)
    vmax = max(1.0, float(np.abs(qkv[:, 2 * c:]).max()))
    err = np.abs(got - want).max()
    assert err < 2e-5 * vmax, err


@pytest.mark.parametrize("h,w,c", [(2, 2, 180), (5, 7, 60), (6, 10, 60), (34, 40, 120),
                                   (33, 39, 180), (20, 70, 180), (72, 80, 180), (264, 264, 180),
                                   (72, 72, 60)])
@pytest.mark.parametrize("epi", [0, 2, 5])
def test_conv3x3_winograd(pkg, orc, h, w, c, epi):
    """The body's C -> C convs (the stage close, conv_after_body) run as
    Winograd F(4x4,3x3) at the released widths: against the oracle's direct
    conv, at the same bar as the direct kernel, up to the headline plane
    (264 x 264 x 180, the borders' zero padding included); a 2x2 plane is
    all border, and 5x7 and 33x39 end in partial 4x4 tiles."""
    cin = cout = c
    r = rng(h * w + cin + cout + epi + 7)
    x = r.standard_normal((cin, h, w), dtype=np.float32)
    wt = (r.standard_normal((cout, cin, 3, 3), dtype=np.float32) / np.sqrt(9 * cin)).astype(np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    res = r.standard_normal((cout, h, w), dtype=np.float32)
    base = orc.conv3x3(x, wt, b)
    if epi == 0:
        want = base
    elif epi == 2:
        want = base + res
    else:
        want = np.where(base < 0, base * np.float32(0.01), base)
    got = pkg.abi.test_conv3x3_winograd(nchw_to_hwc(x), h, w, wt, b, epilogue=epi,
                                        res=nchw_to_hwc(res) if epi == 2 else None, slope=0.01)
    err = np.abs(hwc_to_nchw(got, h, w) - want).max()
    assert err < 5e-5, err


@pytest.mark.parametrize("h,w,cin,cout", [(2, 2, 180, 64), (5, 7, 60, 64), (33, 39, 180, 64),
                                         (72, 80, 120, 32), (264, 264, 180, 64), (40, 48, 180, 4)])
@pytest.mark.parametrize("epi", [0, 5])
def test_conv3x3_winograd_narrow(pkg, orc, h, w, cin, cout, epi):
    """conv_before_upsample's C -> F conv (F <= 64) as the head runs it:
    Winograd F(4x4,3x3) with the transform-domain GEMM on the weight-stationary
    kernel's narrow (64-column) build and its products in a buffer of their
    own, then LeakyReLU(0.01); against the oracle's direct conv."""
    r = rng(h * w + cin * cout + epi)
    x = r.standard_normal((cin, h, w), dtype=np.float32)
    wt = (r.standard_normal((cout, cin, 3, 3), dtype=np.float32) / np.sqrt(9 * cin)).astype(np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    base = orc.conv3x3(x, wt, b)
    want = base if epi == 0 else np.where(base < 0, base * np.float32(0.01), base)
    got = pkg.abi.test_conv3x3_winograd(nchw_to_hwc(x), h, w, wt, b, epilogue=epi, slope=0.01)
    err = np.abs(hwc_to_nchw(got, h, w) - want).max()
    assert err < 5e-5, err


@pytest.mark.parametrize("cin,feat,h,w", [(4, 3, 5, 7), (4, 4, 1, 6), (6, 24, 4, 5), (64, 64, 9, 70),
                                          (8, 8, 3, 61)])
def test_conv3x3_shuffle2(pkg, orc, cin, feat, h, w):
    r = rng(cin * feat + h * w)
    x = r.standard_normal((cin, h, w), dtype=np.float32)
    wt = (r.standard_normal((4 * feat, cin, 3, 3), dtype=np.float32) / np.sqrt(9 * cin)).astype(np.float32)
    b = r.standard_normal(4 * feat, dtype=np.float32)
    want = orc.conv3x3_shuffle2(x, wt, b)
    got = pkg.abi.test_conv3x3_shuffle2(nchw_to_hwc(x), h, w, wt, b)
    err = np.abs(hwc_to_nchw(got, 2 * h, 2 * w) - want).max()
    assert err < 5e-5, err


@pytest.mark.parametrize("c,h,w", [(4, 1, 1), (4, 3, 5), (8, 7, 2), (64, 9, 70), (64, 33, 17),
                                   (64, 122, 162)])
def test_conv3x3_nearest2(pkg, orc, c, h, w):
    """The real-world head's conv of a nearest-2x upsampling (conv_up1 /
    conv_up2, + LeakyReLU 0.2) as the device runs it, four phases of 2x2 convs
    of the plane, against the oracle's nearest upsampling (reference
    cpu::upsample2x_nearest) then its direct conv3x3, LeakyReLU in numpy; every
    border (the upsampled plane's zero padding is the plane's) included."""
    r = rng(c * 131 + h * w)
    x = r.standard_normal((c, h, w), dtype=np.float32)
    wt = (r.standard_normal((c, c, 3, 3), dtype=np.float32) / np.sqrt(9 * c)).astype(np.float32)
    b = r.standard_normal(c, dtype=np.float32)
    z = orc.conv3x3(orc.upsample2x_nearest(x), wt, b)
    want = np.where(z < 0, z * np.float32(0.2), z)
    got = pkg.abi.test_conv3x3_nearest2(nchw_to_hwc(x), h, w, wt, b, 0.2)
    err = np.abs(hwc_to_nchw(got, 2 * h, 2 * w) - want).max()
    assert err < 5e-5, err


def _forward_pair(pkg, orc, arch, seed, h, w, perturb=True):
    M = pkg.model
    wts = M.make_weights(arch, seed=seed, perturb=perturb)
    img = M.to_unit(M.input_sinusoids(h, w, seed=seed + 1))
    x = M.adjust(arch, img)
    want, _ = orc.forward(arch, wts, h, w, x)
    be = pkg.abi.HipBackend(arch, wts)
    try:
        got = be.forward(h, w, x)
        got2 = be.forward(h, w, x)  # the reused plan must give the same answer
    finally:
        be.close()
    return want, got, got2


@pytest.mark.parametrize("h,w", [(37, 29), (64, 64), (8, 8)])
def test_forward_small_model(pkg, orc, h, w):
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[2, 3])
    want, got, got2 = _forward_pair(pkg, orc, arch, 11, h, w)
    assert got.shape == want.shape
    assert np.array_equal(got, got2)
    err = np.abs(got - want).max()
    assert err < 1e-4, err
    d8 = np.abs(M.to_rgb8(got).astype(int) - M.to_rgb8(want).astype(int)).max()
    assert d8 <= 1


@pytest.mark.parametrize("scale,h,w", [(2, 13, 21), (4, 9, 11), (8, 9, 11), (2, 520, 520)])
def test_pixelshuffle_head_compositions(pkg, orc, scale, h, w):
    """The classical head's composed last stage at every octave count: x2 runs
    the last octave and conv_last composed (k_up_last), x4 the last two octaves
    (the 5x5 conv GEMM through pixel_shuffle(4)), x8 one ordinary octave before
    those two; each with its top-row / left-column edge pass, on images small
    enough that the edges are a large part of the output. x2 also at 520^2,
    where k_up_last takes its 8-row tiles (4-row tiles below 2 workgroups per
    CU)."""
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=scale, embed=24, heads=2, depths=[1])
    want, got, got2 = _forward_pair(pkg, orc, arch, 5 + scale, h, w, perturb=True)
    assert got.shape == want.shape == (3, h * scale, w * scale)
    assert np.array_equal(got, got2)
    err = np.abs(got - want).max()
    assert err < 1e-4, err
    # the edge rows and columns on their own
    assert np.abs(got[:, :scale, :] - want[:, :scale, :]).max() < 1e-4
    assert np.abs(got[:, :, :scale] - want[:, :, :scale]).max() < 1e-4


def test_forward_stage_without_blocks(pkg, orc):
    """A stage with no Swin blocks: its close (the folded 3x3 + 1x1 conv and the
    stage residual) reads the plane it must write, so it goes through scratch."""
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=24, heads=2, depths=[0, 2, 0])
    want, got, got2 = _forward_pair(pkg, orc, arch, 5, 21, 19, perturb=True)
    assert np.array_equal(got, got2)
    err = np.abs(got - want).max()
    assert err < 1e-4, err


@pytest.mark.parametrize("h,w,scale", [(37, 29, 4), (48, 72, 2)])
def test_forward_classical(pkg, orc, h, w, scale):
    M = pkg.model
    arch = M.classical(scale)
    want, got, _ = _forward_pair(pkg, orc, arch, 3, h, w, perturb=True)
    err = np.abs(got - want).max()
    assert err < 1e-4, err
    d8 = np.abs(M.to_rgb8(got).astype(int) - M.to_rgb8(want).astype(int)).max()
    assert d8 <= 1


def test_forward_rejects_tiny_image(pkg):
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=24, heads=2, depths=[1])
    be = pkg.abi.HipBackend(arch, M.make_weights(arch, seed=1))
    try:
        with pytest.raises(pkg.abi.S2SError, match="smaller than one 8x8 window"):
            be.forward(7, 20, np.zeros((3, 7, 20), np.float32))
    finally:
        be.close()


def test_forward_with_buffers_past_2gib(pkg):
    """A plane whose qkv buffer passes 2 GiB runs: at 1008^2 it is 2.34 GB, set
    by the x4 head's Winograd F(2x2,5x5) planes (36 x 504^2 tiles x 64 floats;
    the attention units alone would be 1008^2 x 546 floats = 2.22 GB), and it
    is reached through resources based per task, tile or window. (The composed
    head allocates no plane past 2 GiB; test_gpu_boundary.py's
    test_head_planes_past_2gib covers the heads that do.) The input repeats
    a random 16 x 16 patch, so away from the borders (the reflect padding and
    the shifted-window mask live there) every window, conv tap and pixel sees
    what it sees in a 200 x 200 image of the same pattern, and the outputs
    there must agree bit for bit (every kernel's per-output arithmetic is
    independent of where the output sits in the launch)."""
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=4, embed=180, heads=6, depths=[1])
    be = pkg.abi.HipBackend(arch, M.make_weights(arch, seed=1, perturb=True))
    patch = np.random.default_rng(3).uniform(0, 1, (3, 16, 16)).astype(np.float32)
    try:
        outs = []
        for n in (1000, 200):
            img = np.tile(patch, (1, n // 16 + 1, n // 16 + 1))[:, :n, :n]
            outs.append(be.forward(n, n, M.adjust(arch, np.ascontiguousarray(img))))
        big, small = outs
        assert big.shape == (3, 4000, 4000) and np.isfinite(big).all()
        sl = (slice(None), slice(4 * 64, 4 * 128), slice(4 * 64, 4 * 128))
        assert np.array_equal(big[sl], small[sl])
    finally:
        be.close()


def test_forward_refuses_plane_past_buffer_limit(pkg):
    """A plane whose MLP hidden buffer would pass the 32-bit offsets of the
    GEMM that reads it whole (1248^2 padded pixels x 360 x 4 B = 2.24 GB) is
    refused with an "out of memory" message - the condition the crate's
    tile-halving retry keys on - and the context still runs a small image
    afterwards. (The limit, 1.49 M pixels, is above the crate's
    GPU_MAX_PLANE_PIXELS of 65535 x 16.)"""
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=180, heads=6, depths=[1])
    be = pkg.abi.HipBackend(arch, M.make_weights(arch, seed=1))
    try:
        with pytest.raises(pkg.abi.S2SError, match="out of memory"):
            be.forward(1240, 1240, np.zeros((3, 1240, 1240), np.float32))
        x = M.adjust(arch, M.to_unit(M.input_sinusoids(16, 16, seed=2)))
        y = be.forward(16, 16, x)
        assert y.shape == (3, 32, 32) and np.isfinite(y).all()
    finally:
        be.close()


def test_rstb_device(pkg, orc):
    """One RSTB (config 1's op sequence) on an explicit unpadded plane, through
    the device entry and the host-buffer test entry (bit-identical)."""
    hip = pkg.hip
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=180, heads=6, depths=[6])
    wts = M.make_weights(arch, seed=2, perturb=True)
    hp = wp = 32
    x = np.random.default_rng(2).standard_normal((180, hp, wp), dtype=np.float32)
    p = orc.plan_explicit(hp, wp, 8, 180)
    want = orc.rstb(arch, wts, p, 0, x)
    be = pkg.abi.HipBackend(arch, wts)
    try:
        dx = hip.DeviceBuffer.from_array(nchw_to_hwc(x))
        dy = hip.DeviceBuffer(dx.n)
        be.rstb_device(0, hp, wp, dx.ptr, dy.ptr)
        hip.synchronize()
        got = hwc_to_nchw(dy.download((hp * wp, 180)), hp, wp)
        # the host-buffer entry runs the same launches
        assert np.array_equal(be.test_rstb(0, hp, wp, nchw_to_hwc(x)), dy.download((hp * wp, 180)))
        # in place (d_in == d_out) is allowed by the ABI
        be.rstb_device(0, hp, wp, dx.ptr, dx.ptr)
        hip.synchronize()
        assert np.array_equal(dx.download((hp * wp, 180)), dy.download((hp * wp, 180)))
        dx.free()
        dy.free()
    finally:
        be.close()
    err = np.abs(got - want).max() / max(1.0, np.abs(want).max())
    assert err < 1e-4, err


def test_forward_device_matches_host_path(pkg):
    """s2s_forward_device on HBM-resident buffers gives the host entry's bytes."""
    hip = pkg.hip
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=4, embed=24, heads=2, depths=[2])
    wts = M.make_weights(arch, seed=9, perturb=True)
    h, w = 20, 36
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=4)))
    be = pkg.abi.HipBackend(arch, wts)
    try:
        want = be.forward(h, w, x)
        din = hip.DeviceBuffer.from_array(x)
        dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
        be.forward_device(h, w, din.ptr, dout.ptr)
        hip.stream_synchronize(be.stream())
        got = dout.download((3, h * 4, w * 4))
    finally:
        be.close()
    assert np.array_equal(got, want)


def test_profiler_counts_launches(pkg):
    M = pkg.model
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=24, heads=2, depths=[2, 2])
    be = pkg.abi.HipBackend(arch, M.make_weights(arch, seed=1))
    try:
        be.profile(True)
        x = np.zeros((3, 16, 16), np.float32)
        be.forward(16, 16, x)
        ms, n = be.profile_query("window_attention")
        assert n == 4 and ms > 0
        ms, n = be.profile_query("qkv")
        assert n == 4
        be.profile_reset()
        assert be.profile_query("qkv") == (0.0, 0)
    finally:
        be.close()


# ---- the published network's own outputs (tests/golden/make_golden.py) ---------

def _golden_cases():
    import json
    from pathlib import Path
    man = Path(__file__).resolve().parent / "golden" / "net_manifest.json"
    return json.loads(man.read_text()) if man.exists() else []


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_forward_against_published_network(pkg, orc, case):
    """Every head on the device against the reference's PyTorch network (golden
    vectors) and against the oracle: <= 1e-4 max-abs, <= 1 8-bit level."""
    from pathlib import Path
    G = Path(__file__).resolve().parent / "golden"
    M = pkg.model
    arch = M.Arch(**case["arch"])
    wts = M.make_weights(arch, seed=case["seed"], perturb=True)
    img = np.load(G / f"net_{case['name']}_in.npy")
    want = np.load(G / f"net_{case['name']}_out.npy")
    h, w = case["h"], case["w"]
    x = M.adjust(arch, M.to_unit(img))
    be = pkg.abi.HipBackend(arch, wts)
    try:
        got = be.forward(h, w, x)
        aux = be.aux()
    finally:
        be.close()
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4
    d8 = np.abs(M.to_rgb8(got).astype(int) - M.to_rgb8(want).astype(int)).max()
    assert d8 <= 1
    orc_out, orc_aux = orc.forward(arch, wts, h, w, x)
    assert np.abs(got - orc_out).max() < 1e-4
    if case["aux"]:
        want_aux = np.load(G / f"net_{case['name']}_aux.npy")
        assert aux is not None and aux.size == want_aux.size
        aux = aux.reshape(want_aux.shape)
        assert np.abs(aux - want_aux).max() < 1e-4
        assert np.abs(aux - orc_aux).max() < 1e-4
    else:
        assert aux is None


@pytest.mark.parametrize("upsampler,scale,h,w", [
    ("pixelshuffledirect", 2, 64, 64),      # config 0's geometry (128x128 out)
    ("pixelshuffledirect", 3, 37, 29),
    ("nearest+conv", 4, 40, 56),
    ("pixelshuffle_aux", 4, 37, 45),
])
def test_other_heads_against_oracle(pkg, orc, upsampler, scale, h, w):
    """The non-classical heads at the released widths (C = 60 lightweight, 180
    otherwise; feat 64) and planes wider than one 64-lane wavefront."""
    M = pkg.model
    if upsampler == "pixelshuffledirect":
        arch = M.Arch(upsampler=upsampler, scale=scale, embed=60, depths=[2, 2])
    else:
        arch = M.Arch(upsampler=upsampler, scale=scale, embed=180, depths=[2])
    wts = M.make_weights(arch, seed=scale + h, perturb=True)
    x = M.adjust(arch, M.to_unit(M.input_uniform(h, w, seed=1)))
    be = pkg.abi.HipBackend(arch, wts)
    try:
        got = be.forward(h, w, x)
        aux = be.aux()
    finally:
        be.close()
    want, want_aux = orc.forward(arch, wts, h, w, x)
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4
    assert np.abs(M.to_rgb8(got).astype(int) - M.to_rgb8(want).astype(int)).max() <= 1
    if want_aux is not None:
        assert np.abs(aux.reshape(want_aux.shape) - want_aux).max() < 1e-4


def test_mfma_peak_probe(pkg):
    """The fp32 matrix peak probe returns a rate no device can exceed: at most
    the 157.3 TFLOP/s spec figure (2.4 GHz x 256 CUs x 4 SIMDs x 64 FLOPs per
    cycle) plus timing noise, and a positive one; its implied clock matches."""
    ms, tf, ghz = pkg.abi.mfma_peak(2000, 3)
    assert ms > 0 and 0 < tf <= 157.3 * 1.03, (ms, tf)
    assert abs(ghz - tf * 1e12 / (256 * 4 * 64) / 1e9) < 0.05 * ghz, (tf, ghz)
