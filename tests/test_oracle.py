"""Pinning the CPU oracle (no GPU): each restated function against a check that
is not its own formula - the PyTorch network's formulation in float64
(tests/refimpl.py), closed forms, the reference's own definitional selftests
(src/cpu.rs:2021-2356) and the reference's torch golden vectors (bicubic KAT).
"""
import math
from pathlib import Path

import numpy as np
import pytest

import refimpl as R

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32_tol(k, scale):
    """Float32 accumulation bound for a k-term sum of magnitude `scale` against float64:
    4 eps sqrt(k) |y| (random-walk rounding), plus 1e-6 absolute."""
    return 4 * 6e-8 * math.sqrt(k) * max(1.0, float(scale)) + 1e-6


def lcg(n, seed=0x12345678):
    """The reference selftest's generator (src/cpu.rs:2023-2027)."""
    out = np.empty(n, np.float32)
    x = seed
    for i in range(n):
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((x >> 8) / 16777216.0 - 0.5)
    return out


# ---- plan / index / region / padding: bit-exact ------------------------------

@pytest.mark.parametrize("h,w,win", [(19, 13, 8), (16, 16, 8), (37, 29, 8), (9, 17, 4), (64, 64, 8)])
def test_plan_padding_rule(orc, h, w, win):
    p = orc.plan_new(h, w, win, 2)
    # src/plan.rs:39-47: the NEXT window multiple, a whole extra window on exact multiples
    assert p.hp == (h // win + 1) * win and p.wp == (w // win + 1) * win
    assert p.hp > h and p.wp > w and p.hp % win == 0
    assert p.nw == (p.hp // win) * (p.wp // win) and p.n == win * win
    assert orc.shift_for(p, 0) == 0 and orc.shift_for(p, 1) == win // 2 and orc.shift_for(p, 2) == 0


@pytest.mark.parametrize("hp,wp,win,shift", [(24, 16, 8, 0), (24, 16, 8, 4), (16, 24, 8, 4),
                                             (72, 80, 8, 4), (12, 20, 4, 2), (264, 264, 8, 4)])
def test_gather_is_roll_then_partition(orc, hp, wp, win, shift):
    c = 3
    p = orc.plan_explicit(hp, wp, win, c)
    x = np.arange(c * hp * wp, dtype=np.float32).reshape(c, hp, wp)
    tok = orc.gather(p, x, shift)
    want = R.shifted_windows(x, win, shift).reshape(-1, c)
    assert np.array_equal(tok, want)
    # the scatter is the inverse, checked from tokens that are NOT a gather output
    t2 = np.random.default_rng(1).standard_normal(tok.shape).astype(np.float32)
    back = orc.scatter(p, t2, shift)
    assert np.array_equal(back, R.unshift_windows(t2.reshape(p.nw, p.n, c), win, shift, hp, wp))


@pytest.mark.parametrize("hp,wp,win,shift", [(24, 16, 8, 4), (16, 24, 8, 4), (72, 80, 8, 4),
                                             (12, 20, 4, 2), (40, 32, 8, 4)])
def test_region_is_calculate_mask(orc, hp, wp, win, shift):
    p = orc.plan_explicit(hp, wp, win, 1)
    yx, reg = orc.window_map(p, shift)
    ids = 3 * reg[:, 0].astype(np.int64) + reg[:, 1]
    assert np.array_equal(ids.reshape(p.nw, p.n), R.mask_regions(hp, wp, win, shift))
    # index = (wh*win + i + shift) % hp etc. - torch.roll(-shift)
    rows = np.arange(hp * wp).reshape(1, hp, wp).astype(np.float32)
    flat = R.shifted_windows(rows, win, shift).reshape(-1).astype(np.int64)
    assert np.array_equal(yx[:, 0] * wp + yx[:, 1], flat)


@pytest.mark.parametrize("h,w", [(9, 9), (19, 13), (37, 29), (8, 16), (15, 8)])
def test_pad_reflect_is_torch_cat_flip(orc, h, w):
    x = np.random.default_rng(h * w).standard_normal((3, h, w)).astype(np.float32)
    p = orc.plan_new(h, w, 8, 3)
    got = orc.pad_reflect(x, p.hp, p.wp)
    assert np.array_equal(got, R.pad_like_reference(x, 8).astype(np.float32))


# ---- dense ops against float64 definitions ------------------------------------

def test_conv3x3_definition_selftest_shape(orc):
    ci, h, w, co = 3, 5, 7, 4
    v = lcg(ci * h * w + co * ci * 9 + co)
    x = v[:ci * h * w].reshape(ci, h, w)
    wt = v[ci * h * w:ci * h * w + co * ci * 9].reshape(co, ci, 3, 3)
    b = v[-co:]
    assert np.abs(orc.conv3x3(x, wt, b) - R.conv3x3(x, wt, b)).max() < 1e-5


@pytest.mark.parametrize("ci,co,h,w", [(3, 180, 12, 20), (180, 180, 9, 11), (64, 3, 16, 17), (60, 27, 1, 9)])
def test_conv3x3(orc, ci, co, h, w):
    r = np.random.default_rng(ci + co)
    x = r.standard_normal((ci, h, w)).astype(np.float32)
    wt = (r.standard_normal((co, ci, 3, 3)) / math.sqrt(9 * ci)).astype(np.float32)
    b = r.standard_normal(co).astype(np.float32)
    want = R.conv3x3(x, wt, b)
    assert np.abs(orc.conv3x3(x, wt, b) - want).max() < f32_tol(9 * ci, np.abs(want).max())


@pytest.mark.parametrize("ci,feat,h,w", [(5, 3, 4, 6), (4, 3, 1, 6), (64, 64, 6, 9), (2, 2, 1, 33)])
def test_conv3x3_shuffle2(orc, ci, feat, h, w):
    r = np.random.default_rng(ci * feat + h)
    x = r.standard_normal((ci, h, w)).astype(np.float32)
    wt = (r.standard_normal((4 * feat, ci, 3, 3)) / math.sqrt(9 * ci)).astype(np.float32)
    b = r.standard_normal(4 * feat).astype(np.float32)
    want = R.pixel_shuffle(R.conv3x3(x, wt, b), 2)
    assert np.abs(orc.conv3x3_shuffle2(x, wt, b) - want).max() < f32_tol(9 * ci, np.abs(want).max())
    # and against the oracle's own conv3x3 + pixel_shuffle2 (reference selftest, src/cpu.rs:2064-2098)
    two = orc.pixel_shuffle2(orc.conv3x3(x, wt, b))
    assert np.abs(orc.conv3x3_shuffle2(x, wt, b) - two).max() < 2 * f32_tol(9 * ci, np.abs(want).max())


@pytest.mark.parametrize("rows,ci,co", [(37, 60, 43), (200, 180, 540), (19, 360, 180), (8, 7, 11)])
def test_linear_and_conv1x1(orc, rows, ci, co):
    r = np.random.default_rng(rows + ci)
    x = r.standard_normal((rows, ci)).astype(np.float32)
    w = (r.standard_normal((co, ci)) / math.sqrt(ci)).astype(np.float32)
    b = r.standard_normal(co).astype(np.float32)
    want = x.astype(np.float64) @ w.T.astype(np.float64) + b
    tol = f32_tol(ci, np.abs(want).max())
    assert np.abs(orc.linear(x, w, b) - want).max() < tol
    xt = np.ascontiguousarray(x.T).reshape(ci, 1, rows)
    got = orc.conv1x1(xt, w.reshape(co, ci, 1, 1), b).reshape(co, rows).T
    assert np.abs(got - want).max() < tol


def test_pixel_shuffle_and_nearest(orc):
    x = lcg(2 * 9 * 3 * 4).reshape(18, 3, 4)
    assert np.array_equal(orc.pixel_shuffle(x, 3), R.pixel_shuffle(x, 3).astype(np.float32))
    assert np.array_equal(orc.pixel_shuffle2(x[:8]), R.pixel_shuffle(x[:8], 2).astype(np.float32))
    up = orc.upsample2x_nearest(x)
    assert np.array_equal(up, np.repeat(np.repeat(x, 2, 1), 2, 2))


@pytest.mark.parametrize("c,hw", [(17, 400), (180, 1000), (3, 5)])
def test_channel_layer_norm(orc, c, hw):
    r = np.random.default_rng(c)
    x = (r.standard_normal((c, hw)) * 2 + 0.5).astype(np.float32)
    w = r.standard_normal(c).astype(np.float32)
    b = r.standard_normal(c).astype(np.float32)
    got = orc.channel_layer_norm(x, w, b)
    assert np.abs(got - R.layer_norm(x, w, b, axis=0)).max() < 1e-5 * max(1, np.abs(w).max() * 4)


def test_fast_exp_is_sqrt2_exp(orc):
    # What the reference's series computes (src/cpu.rs:1095-1120): 2^(t+1/2) for
    # t = x*log2(e) < 1/2, i.e. sqrt(2)*e^x, within the degree-6 series error.
    # Below 2^-126 (x < -86.99, where floor(t + 1/2) - 1/2 < -126) it returns 0.
    xs = np.concatenate([np.linspace(-86.9, 0, 20001), [-1e-7, -0.3466, -0.3465]])
    got = np.array([orc.fast_exp(v) for v in xs], np.float64)
    rel = np.abs(got / (math.sqrt(2.0) * np.exp(xs)) - 1.0)
    assert rel.max() < 1.6e-5
    assert orc.fast_exp(-100.0) == 0.0 and orc.fast_exp(-87.0) == 0.0


def test_gelu_is_erf_form(orc):
    x = np.linspace(-6, 6, 4001).astype(np.float32)
    assert np.abs(orc.gelu(x) - R.gelu(x)).max() < 2e-6


# ---- attention and the bias table -------------------------------------------

@pytest.mark.parametrize("hp,wp,win,heads,hd,shift", [
    (12, 20, 4, 2, 2, 0), (12, 20, 4, 2, 2, 2),     # the reference selftest's Plan::new(9,17,4,4)
    (16, 24, 8, 6, 30, 0), (16, 24, 8, 6, 30, 4), (24, 16, 8, 6, 10, 4)])
def test_attention_against_torch_formulation(orc, hp, wp, win, heads, hd, shift):
    r = np.random.default_rng(hp * wp + heads + shift)
    c = heads * hd
    p = orc.plan_explicit(hp, wp, win, c)
    n = win * win
    planes = [r.standard_normal((c, hp, wp)).astype(np.float32) for _ in range(3)]
    ls = np.array([1.5, 0.25, 5.3, 2.3, -0.5, 3.0][:heads], np.float32)
    cpb = (r.standard_normal((n * n, heads)) * 2).astype(np.float32)
    qkv = np.concatenate([orc.gather(p, t, shift) for t in planes], 0)
    got = orc.attention(p, heads, hd, ls, cpb, qkv, shift).reshape(p.nw, n, c)
    q, k, v = (R.shifted_windows(t, win, shift) for t in planes)
    mids = R.mask_regions(hp, wp, win, shift) if shift else None
    want = R.window_attention(q, k, v, ls, cpb, mids)
    # the reference CPU's fast_exp is 1.6e-5 relative; scale by the value range
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(planes[2]).max())


def test_cpb_table(orc, pkg):
    r = np.random.default_rng(3)
    w0 = r.standard_normal((512, 2)).astype(np.float32)
    b0 = r.uniform(-0.5, 0.5, 512).astype(np.float32)
    w2 = (r.standard_normal((6, 512)) * 0.1).astype(np.float32)
    want = R.cpb_table(w0, b0, w2, 8)
    assert np.abs(orc.cpb_table(8, 6, w0, b0, w2) - want).max() < 2e-5
    assert np.abs(pkg.model.cpb_pre(w0, b0, w2, 8) - want).max() < 2e-5
    # the log-spaced coordinates reach +-log2(9)/log2(8) at offsets +-(win-1)
    t = R.relative_coords_table(8)
    assert abs(t.max() - math.log2(9) / 3) < 1e-12 and abs(t.min() + math.log2(9) / 3) < 1e-12


# ---- golden vectors -----------------------------------------------------------

def test_bicubic_against_torch_kat(orc):
    """The reference's own torch KAT (tests/bicubic.rs, tests/data/bicubic_*.npy)."""
    x = np.load(GOLDEN / "bicubic_in_40x32.npy")
    want = np.load(GOLDEN / "bicubic_out_148x116.npy")
    assert x.shape == (1, 1, 40, 32) and want.shape == (1, 1, 148, 116)
    got = orc.bicubic_resize(x[0], 148, 116)
    assert np.abs(got - want[0]).max() < 2e-5


# ---- composition --------------------------------------------------------------

def tiny_arch(pkg, **kw):
    M = pkg.model
    base = dict(upsampler="pixelshuffle", scale=4, embed=12, heads=2, depths=[2, 3])
    base.update(kw)
    return M.Arch(**base)


def test_rstb_against_torch_formulation(orc, pkg):
    M = pkg.model
    arch = tiny_arch(pkg, depths=[4])
    wts = M.make_weights(arch, seed=21, perturb=True)
    x = np.random.default_rng(4).standard_normal((12, 16, 24)).astype(np.float32)
    p = orc.plan_explicit(16, 24, 8, 12)
    got = orc.rstb(arch, wts, p, 0, x)
    want = R.rstb(x, wts, 0, 4, 8, 2)
    assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("h,w,scale", [(16, 20, 4), (13, 9, 2), (37, 29, 4)])
def test_forward_against_torch_formulation(orc, pkg, h, w, scale):
    M = pkg.model
    arch = tiny_arch(pkg, scale=scale)
    wts = M.make_weights(arch, seed=h + w, perturb=True)
    img = M.to_unit(M.input_uniform(h, w, seed=1))
    got, _ = orc.forward(arch, wts, h, w, M.adjust(arch, img))
    want = R.network(arch, wts, img)[:, :h * scale, :w * scale]
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4


def test_oracle_threads_do_not_change_results(orc, pkg):
    M = pkg.model
    arch = tiny_arch(pkg)
    wts = M.make_weights(arch, seed=5, perturb=True)
    x = M.adjust(arch, M.to_unit(M.input_uniform(24, 16, seed=2)))
    n0 = orc.lib().orc_threads()
    try:
        orc.lib().orc_set_threads(1)
        a, _ = orc.forward(arch, wts, 24, 16, x)
    finally:
        orc.lib().orc_set_threads(n0)
    b, _ = orc.forward(arch, wts, 24, 16, x)
    assert np.array_equal(a, b)


# ---- the published network's own outputs ---------------------------------------

def _golden_cases():
    import json
    man = GOLDEN / "net_manifest.json"
    return json.loads(man.read_text()) if man.exists() else []


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_forward_against_published_network(orc, pkg, case):
    """Golden vectors written by tests/golden/make_golden.py from the reference's
    PyTorch Swin2SR (tools/network_swin2sr.py) on the same synthetic weights:
    pins the graph's composition and every head, at 1e-4 (the north_star bar)."""
    M = pkg.model
    arch = M.Arch(**case["arch"])
    wts = M.make_weights(arch, seed=case["seed"], perturb=True)
    img = np.load(GOLDEN / f"net_{case['name']}_in.npy")
    want = np.load(GOLDEN / f"net_{case['name']}_out.npy")
    got, aux = orc.forward(arch, wts, case["h"], case["w"], M.adjust(arch, M.to_unit(img)))
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4
    if case["aux"]:
        want_aux = np.load(GOLDEN / f"net_{case['name']}_aux.npy")
        assert aux.shape == want_aux.shape
        assert np.abs(aux - want_aux).max() < 1e-4
