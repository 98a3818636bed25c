"""Independent float64 references used to pin the oracle (and double-check the GPU).

Each function follows the PUBLISHED PyTorch network's formulation
(reference tools/network_swin2sr.py) rather than the crate's CPU path that the
oracle restates, so a transcription error in the oracle (a wrong sign of the
shift, a mask built on the wrapped coordinate, a transposed operand, a pre-norm
block, a missing skip) shows up as a disagreement:
  - window partition = torch.roll(-shift) then window_partition (reshape);
  - the shift mask = calculate_mask's three slices per axis;
  - padding = main_test_swin2sr.py's torch.cat([x, flip(x)]) truncation;
  - attention = F.normalize(q) @ F.normalize(k)^T * clamp(ls).exp() + 16
    sigmoid(cpb_mlp(table))[index] + mask, softmax with exact exp, @ v;
  - LayerNorm = two-pass mean/variance over channels (nn.LayerNorm);
  - convolutions = zero-padded einsum over taps.
Everything is computed in float64.
"""
import math

import numpy as np

try:
    from scipy.special import erf as _erf
except Exception:  # pragma: no cover
    _erf = np.vectorize(math.erf)


def pad_like_reference(x, win):
    """tools/make_fixture.py:80-89: torch.cat([x, flip(x)], dim)[:h + pad]."""
    c, h, w = x.shape
    hp = (h // win + 1) * win
    wp = (w // win + 1) * win
    x = np.concatenate([x, np.flip(x, 1)], 1)[:, :hp, :]
    x = np.concatenate([x, np.flip(x, 2)], 2)[:, :, :wp]
    return x


def window_partition(x_hwc, win):
    """network_swin2sr.py window_partition on [H][W][C] -> [nW][win*win][C]."""
    H, W, C = x_hwc.shape
    x = x_hwc.reshape(H // win, win, W // win, win, C).transpose(0, 2, 1, 3, 4)
    return x.reshape(-1, win * win, C)


def window_reverse(windows, win, H, W):
    C = windows.shape[-1]
    x = windows.reshape(H // win, W // win, win, win, C).transpose(0, 2, 1, 3, 4)
    return x.reshape(H, W, C)


def shifted_windows(x_chw, win, shift):
    """roll(-shift) then partition: [nW][n][C]."""
    x = np.transpose(x_chw, (1, 2, 0))
    if shift:
        x = np.roll(x, (-shift, -shift), axis=(0, 1))
    return window_partition(x, win)


def unshift_windows(windows, win, shift, H, W):
    x = window_reverse(windows, win, H, W)
    if shift:
        x = np.roll(x, (shift, shift), axis=(0, 1))
    return np.transpose(x, (2, 0, 1))


def mask_regions(H, W, win, shift):
    """calculate_mask (network_swin2sr.py:261-282): the cnt id per token, [nW][n]."""
    img = np.zeros((H, W, 1))
    sl = (slice(0, -win), slice(-win, -shift), slice(-shift, None))
    cnt = 0
    for hs in sl:
        for ws in sl:
            img[hs, ws, :] = cnt
            cnt += 1
    return window_partition(img, win)[..., 0].astype(np.int64)


def relative_coords_table(win):
    r = np.arange(-(win - 1), win, dtype=np.float64)
    t = np.stack(np.meshgrid(r, r, indexing="ij"), -1)
    t = t / (win - 1) * 8
    t = np.sign(t) * np.log2(np.abs(t) + 1.0) / np.log2(8)
    return t.reshape(-1, 2)


def relative_position_index(win):
    coords = np.stack(np.meshgrid(np.arange(win), np.arange(win), indexing="ij")).reshape(2, -1)
    rel = coords[:, :, None] - coords[:, None, :]
    rel = rel.transpose(1, 2, 0).copy()
    rel[:, :, 0] += win - 1
    rel[:, :, 1] += win - 1
    rel[:, :, 0] *= 2 * win - 1
    return rel.sum(-1)


def cpb_table(w0, b0, w2, win):
    h = relative_coords_table(win) @ np.asarray(w0, np.float64).T + np.asarray(b0, np.float64)
    h = np.maximum(h, 0) @ np.asarray(w2, np.float64).T
    bias = h[relative_position_index(win).reshape(-1)]
    return 16.0 / (1.0 + np.exp(-bias))  # [n*n][heads]


def window_attention(q, k, v, logit_scale, cpb, mask_ids=None):
    """One window set. q,k,v: [nW][n][C]; cpb: [n*n][heads]; returns [nW][n][C]."""
    nW, n, C = q.shape
    heads = len(logit_scale)
    hd = C // heads
    out = np.zeros_like(q, dtype=np.float64)
    bias = np.asarray(cpb, np.float64).reshape(n, n, heads).transpose(2, 0, 1)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        qh, kh, vh = q[..., sl], k[..., sl], v[..., sl]
        qn = qh / np.maximum(np.linalg.norm(qh, axis=-1, keepdims=True), 1e-12)
        kn = kh / np.maximum(np.linalg.norm(kh, axis=-1, keepdims=True), 1e-12)
        att = qn @ kn.transpose(0, 2, 1)
        att = att * math.exp(min(float(logit_scale[h]), math.log(100.0)))
        att = att + bias[h][None]
        if mask_ids is not None:
            att = att + np.where(mask_ids[:, :, None] != mask_ids[:, None, :], -100.0, 0.0)
        att = att - att.max(-1, keepdims=True)
        p = np.exp(att)
        p = p / p.sum(-1, keepdims=True)
        out[..., sl] = p @ vh
    return out


def layer_norm(x, w, b, axis=-1, eps=1e-5):
    x = np.asarray(x, np.float64)
    m = x.mean(axis, keepdims=True)
    v = ((x - m) ** 2).mean(axis, keepdims=True)
    shape = [1] * x.ndim
    shape[axis] = -1
    return (x - m) / np.sqrt(v + eps) * np.reshape(w, shape) + np.reshape(b, shape)


def gelu(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))


def conv3x3(x, w, b):
    """x [cin][h][w], w [cout][cin][3][3], zero pad 1, float64."""
    x = np.asarray(x, np.float64)
    cin, h, wd = x.shape
    xp = np.zeros((cin, h + 2, wd + 2))
    xp[:, 1:-1, 1:-1] = x
    out = np.zeros((w.shape[0], h, wd)) + np.asarray(b, np.float64)[:, None, None]
    for ky in range(3):
        for kx in range(3):
            out += np.einsum("oi,ihw->ohw", np.asarray(w[:, :, ky, kx], np.float64),
                             xp[:, ky:ky + h, kx:kx + wd])
    return out


def conv1x1(x, w, b):
    return np.einsum("oi,ihw->ohw", np.asarray(w, np.float64).reshape(w.shape[0], -1),
                     np.asarray(x, np.float64)) + np.asarray(b, np.float64)[:, None, None]


def pixel_shuffle(x, r):
    """F.pixel_shuffle: [C*r*r][H][W] -> [C][H*r][W*r]."""
    c, h, w = x.shape
    c //= r * r
    return x.reshape(c, r, r, h, w).transpose(0, 3, 1, 4, 2).reshape(c, h * r, w * r)


def lrelu(x, s):
    return np.where(x < 0, x * s, x)


def swin_block(x, wts, p, win, shift, heads):
    """SwinTransformerBlock.forward (network_swin2sr.py:284-323), post-norm, on [C][H][W]."""
    C, H, W = x.shape
    g = lambda k: np.asarray(wts[p + k], np.float64)
    xw = shifted_windows(x, win, shift)
    q = xw @ g("attn.qkv.wq").T + g("attn.qkv.q_bias")
    k = xw @ g("attn.qkv.wk").T
    v = xw @ g("attn.qkv.wv").T + g("attn.qkv.v_bias")
    mids = mask_regions(H, W, win, shift) if shift else None
    a = window_attention(q, k, v, wts[p + "attn.logit_scale"].reshape(-1),
                         cpb_table(wts[p + "attn.cpb_mlp.0.weight"], wts[p + "attn.cpb_mlp.0.bias"],
                                   wts[p + "attn.cpb_mlp.2.weight"], win), mids)
    a = a @ g("attn.proj.weight").T + g("attn.proj.bias")
    a = unshift_windows(a, win, shift, H, W)
    x = x + layer_norm(a, g("norm1.weight"), g("norm1.bias"), axis=0)
    t = np.transpose(x, (1, 2, 0))
    hmid = gelu(t @ g("mlp.fc1.weight").T + g("mlp.fc1.bias"))
    m = np.transpose(hmid @ g("mlp.fc2.weight").T + g("mlp.fc2.bias"), (2, 0, 1))
    return x + layer_norm(m, g("norm2.weight"), g("norm2.bias"), axis=0)


def rstb(x, wts, s, depth, win, heads):
    """RSTB.forward (network_swin2sr.py:574-575)."""
    y = x
    for b in range(depth):
        y = swin_block(y, wts, f"layers.{s}.residual_group.blocks.{b}.", win,
                       0 if b % 2 == 0 else win // 2, heads)
    y = conv3x3(y, wts[f"layers.{s}.conv.weight"], wts[f"layers.{s}.conv.bias"])
    y = conv1x1(y, wts[f"layers.{s}.patch_embed.proj.weight"], wts[f"layers.{s}.patch_embed.proj.bias"])
    return y + x


def network(arch, wts, img01):
    """Swin2SR.forward (network_swin2sr.py:940-1006) for the pixelshuffle head on an
    image already padded the reference way; returns the uncropped output."""
    win = arch.window
    x = pad_like_reference(np.asarray(img01, np.float64), win)
    mean = np.asarray(arch.mean, np.float64)[:, None, None]
    x = (x - mean) * arch.img_range
    x = conv3x3(x, wts["conv_first.weight"], wts["conv_first.bias"])
    first = x
    f = conv1x1(x, wts["patch_embed.proj.weight"], wts["patch_embed.proj.bias"])
    f = layer_norm(f, wts["patch_embed.norm.weight"], wts["patch_embed.norm.bias"], axis=0)
    for s, d in enumerate(arch.depths):
        f = rstb(f, wts, s, d, win, arch.heads)
    f = layer_norm(f, wts["norm.weight"], wts["norm.bias"], axis=0)
    x = conv3x3(f, wts["conv_after_body.weight"], wts["conv_after_body.bias"]) + first
    assert arch.upsampler == "pixelshuffle"
    x = lrelu(conv3x3(x, wts["conv_before_upsample.0.weight"], wts["conv_before_upsample.0.bias"]), 0.01)
    for o in range(arch.octaves):
        x = pixel_shuffle(conv3x3(x, wts[f"upsample.{2 * o}.weight"], wts[f"upsample.{2 * o}.bias"]), 2)
    x = conv3x3(x, wts["conv_last.weight"], wts["conv_last.bias"])
    return x / arch.img_range + mean
