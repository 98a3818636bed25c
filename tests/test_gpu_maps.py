"""The production shifted-window maps, bit-exact, through the kernels the
forward runs (north_star: "shift/mask/window index maps bit-exact").

The maps live inline in three places of the forward: the qkv GEMM's
shifted-window gather into the attention's unit layout (EPI_QKV_WIN, with the
per-token path of windows that wrap around the plane edge), the window
attention's -100 band mask, and its scatter of the output back to the plane.
Each probe feeds those kernels exactly representable data whose answer is
decided by the map alone, and holds the result against the oracle's
`Plan::index` / `Plan::region` tables (reference src/plan.rs:72-108,
oracle `orc_window_map`) with `np.array_equal`:

  gather  - an identity qkv weight carries each pixel's index (and, in a
            second probe, each channel's) into every q/k/v column of the unit
            layout; every float must equal the index map's pixel.
  scatter - q = k = 0 (so the cosine logit is exactly 0) and a CPB table that
            puts 0 on one chosen key per query and -200 elsewhere: the softmax
            is exactly one-hot, the output is exactly that key's v, written to
            the query's pixel.
  mask    - the same table with -50 on the query's own key: when the chosen key
            lies in another mask band the -100 shift mask makes the query's
            own key win instead (exp(-50) vanishes against 1 in f32), so each
            output float says, exactly, whether the band rule separated the
            pair.
Each head gets its own choice of key (itself, the row/column neighbour, the
mirror, the transpose, ...), at 264 x 264 (the headline plane) and 40 x 72,
shifts 0 and 4, so the wrapped last window row and column are covered.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PLANES = [(264, 264), (40, 72)]

# per head: the key each query is made to attend to
CHOICES = [
    lambda q: q,                       # itself: the scatter alone
    lambda q: q ^ 1,                   # column neighbour
    lambda q: q ^ 8,                   # row neighbour
    lambda q: (q + 9) % 64,            # diagonal step, wrapping inside the window
    lambda q: 63 - q,                  # the mirror token: crosses both bands
    lambda q: (q % 8) * 8 + q // 8,    # the transpose
    lambda q: (q + 1) % 64,
    lambda q: (q + 56) % 64,
    lambda q: (5 * q) % 64,
    lambda q: (q + 27) % 64,
    lambda q: 7 - q % 8 + (q // 8) * 8,
    lambda q: (q + 36) % 64,
]


def _pixels(orc, hp, wp, shift):
    p = orc.plan_explicit(hp, wp, 8, 4)
    yx, reg = orc.window_map(p, shift)
    pix = (yx[:, 0].astype(np.int64) * wp + yx[:, 1]).reshape(-1, 64)
    return pix, reg.reshape(-1, 64, 2)


@pytest.mark.parametrize("hp,wp", PLANES)
@pytest.mark.parametrize("shift", [0, 4])
@pytest.mark.parametrize("heads,hd", [(6, 30), (6, 10), (4, 30)])
def test_qkv_window_gather_bit_exact(pkg, orc, hp, wp, shift, heads, hd):
    abi = pkg.abi
    c = heads * hd
    P = hp * wp
    pix, _ = _pixels(orc, hp, wp, shift)
    hg = (heads + 1) // 2
    # probe 1: every channel of pixel p holds p; W = [I; I; I]
    x = np.repeat(np.arange(P, dtype=np.float32)[:, None], c, axis=1)
    w = np.concatenate([np.eye(c, dtype=np.float32)] * 3, axis=0)
    b = np.zeros(3 * c, np.float32)
    unit = abi.test_qkv_windows(hp, wp, heads, hd, shift, x, w, b)
    want = pix.astype(np.float32)  # [window][token]
    for h in range(heads):
        for seg in range(3):
            col = (2 * seg + (h & 1)) * hd
            got = unit[:, h // 2, :, col:col + hd]
            assert np.array_equal(got, np.broadcast_to(want[:, :, None], got.shape)), (h, seg)
    # the two padding floats per row stay unwritten
    assert np.isnan(unit[:, :, :, 6 * hd:]).all()
    # probe 2: channel ch holds ch + 1, segment s scaled by 256^s: each column
    # of the unit must hold its own (segment, head, d)
    x = np.broadcast_to(np.arange(1, c + 1, dtype=np.float32), (P, c)).copy()
    w = np.concatenate([np.eye(c, dtype=np.float32) * np.float32(256.0 ** s) for s in range(3)])
    unit = abi.test_qkv_windows(hp, wp, heads, hd, shift, x, w, b)
    for h in range(heads):
        for seg in range(3):
            col = (2 * seg + (h & 1)) * hd
            want_c = (np.arange(h * hd, (h + 1) * hd, dtype=np.float32) + 1) * np.float32(256.0 ** seg)
            got = unit[:, h // 2, :, col:col + hd]
            assert np.array_equal(got, np.broadcast_to(want_c, got.shape)), (h, seg)
    assert hg == unit.shape[1]


def _one_hot_probe(pkg, orc, hp, wp, shift, heads, hd):
    c = heads * hd
    P = hp * wp
    x = np.repeat((np.arange(P, dtype=np.float32) + 1)[:, None], c, axis=1)
    w = np.zeros((3 * c, c), np.float32)
    w[2 * c:] = np.eye(c, dtype=np.float32)           # q = k = 0, v = x
    b = np.zeros(3 * c, np.float32)
    ls = np.full(heads, np.log(10.0), np.float32)
    cpb = np.full((64, 64, heads), -200.0, np.float32)
    q = np.arange(64)
    for h in range(heads):
        k = np.array([CHOICES[h % len(CHOICES)](int(t)) for t in q])
        cpb[q, q, h] = -50.0
        cpb[q, k, h] = 0.0
    got = pkg.abi.test_block_attention(hp, wp, heads, hd, shift, x, w, b, ls,
                                       cpb.reshape(64 * 64, heads))
    # expected from the oracle's index and band maps alone
    pix, reg = _pixels(orc, hp, wp, shift)
    want = np.zeros((P, c), np.float32)
    for h in range(heads):
        k = np.array([CHOICES[h % len(CHOICES)](int(t)) for t in q])
        same = np.all(reg[:, q, :] == reg[:, k, :], axis=2) if shift else np.ones(pix.shape, bool)
        src = np.where(same, pix[:, k], pix[:, q])      # [window][query]
        want[pix.reshape(-1), h * hd:(h + 1) * hd] = (src.reshape(-1) + 1).astype(np.float32)[:, None]
    return got, want, pix, reg


@pytest.mark.parametrize("hp,wp", PLANES)
@pytest.mark.parametrize("shift", [0, 4])
@pytest.mark.parametrize("heads,hd", [(6, 30), (6, 10), (12, 10), (2, 12), (3, 32)])
def test_attention_scatter_and_mask_bit_exact(pkg, orc, hp, wp, shift, heads, hd):
    """(6, 30), (6, 10) and (12, 10) run the unit-layout kernels; (2, 12) and
    (3, 32) the plane-layout ones."""
    got, want, pix, reg = _one_hot_probe(pkg, orc, hp, wp, shift, heads, hd)
    assert np.array_equal(got, want)
    if shift:
        # the probe really exercised the mask: some chosen keys crossed a band
        q = np.arange(64)
        k = np.array([CHOICES[4](int(t)) for t in q])
        assert not np.all(reg[:, q, :] == reg[:, k, :])
