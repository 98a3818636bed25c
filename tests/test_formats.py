"""On-disk formats (host side, no GPU): the converted-checkpoint safetensors
with the crate's __metadata__ validation (reference src/weights.rs:90-235,
tools/convert.py:224-266), the SW2F golden fixture (src/fixture.rs) pinned
against two of the reference's own fixture files, and PNG IO (src/image.rs)
pinned against the PNG specification's filter definitions."""
import json
import struct
import zlib
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT

GOLDEN = ROOT / "tests" / "golden"


@pytest.fixture(scope="module")
def F(pkg):
    return pkg.formats


def tiny(M, ups="pixelshuffle", scale=2):
    return M.Arch(upsampler=ups, scale=scale, embed=24, heads=2, depths=[2, 1])


# ---------------------------------------------------------------------------
# safetensors
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ups,scale", [("pixelshuffle", 2), ("pixelshuffle", 4),
                                       ("pixelshuffledirect", 2), ("nearest+conv", 4),
                                       ("pixelshuffle_aux", 4)])
def test_safetensors_round_trip(pkg, F, tmp_path, ups, scale):
    M = pkg.model
    arch = tiny(M, ups, scale)
    w = M.make_weights(arch, seed=5, perturb=True)
    p = tmp_path / "m.safetensors"
    F.save_weights(p, arch, w, task="test_sr")
    wt = F.Weights.load(p)
    assert (wt.task, wt.upsampler, wt.scale, wt.window, wt.embed, wt.heads, wt.head_dim,
            wt.mlp_ratio, wt.depths) == ("test_sr", ups, scale, 8, 24, 2, 12, 2, [2, 1])
    assert wt.img_range == 1.0 and np.allclose(wt.mean, M.RGB_MEAN)
    assert wt.names == sorted(w)
    got = wt.tensors()
    for k, v in w.items():
        assert got[k].shape == v.shape and np.array_equal(got[k], v), k
    a2 = wt.arch()
    assert (a2.upsampler, a2.scale, a2.embed, a2.heads, a2.depths, a2.feat) == \
        (arch.upsampler, arch.scale, arch.embed, arch.heads, arch.depths, arch.feat)


def test_safetensors_layout_is_the_converters(pkg, F, tmp_path):
    """tools/convert.py:238-266: 8-byte length field counting the space
    padding, payload start 8-byte aligned, names sorted, every payload offset
    4-byte aligned and contiguous in name order."""
    M = pkg.model
    arch = tiny(M)
    w = M.make_weights(arch, seed=1)
    p = tmp_path / "m.safetensors"
    F.save_weights(p, arch, w, task="classical_sr")
    b = p.read_bytes()
    (n,) = struct.unpack_from("<Q", b, 0)
    assert (8 + n) % 8 == 0
    hdr = json.loads(b[8:8 + n].decode().rstrip(" "))
    meta = hdr.pop("__metadata__")
    assert meta["depths"] == "2,1" and meta["rgb_mean"] == "0.4488,0.4371,0.4040"
    names = list(hdr)
    assert names == sorted(names)
    off = 0
    for k in names:
        b0, b1 = hdr[k]["data_offsets"]
        assert b0 == off and b0 % 4 == 0 and hdr[k]["dtype"] == "F32"
        assert b1 - b0 == 4 * int(np.prod(hdr[k]["shape"]))
        raw = np.frombuffer(b, "<f4", count=(b1 - b0) // 4, offset=8 + n + b0)
        assert np.array_equal(raw.reshape(hdr[k]["shape"]), w[k])
        off = (b1 + 3) & ~3
    assert len(b) == 8 + n + off


def _rewrite(F, src, dst, drop_meta=None, set_meta=None, reshape=None, dtype=None):
    st = F.SafeTensors(src)
    tensors = {k: np.array(st.tensor(k)) for k in st.order}
    meta = dict(st.metadata)
    if drop_meta:
        meta.pop(drop_meta)
    if set_meta:
        meta.update(set_meta)
    if reshape:
        k, shape = reshape
        tensors[k] = np.zeros(shape, np.float32)
    F.write_safetensors(dst, tensors, meta)
    if dtype:
        b = bytearray(Path(dst).read_bytes())
        (n,) = struct.unpack_from("<Q", b, 0)
        hdr = b[8:8 + n].decode()
        hdr = hdr.replace('"dtype":"F32"', f'"dtype":"{dtype}"', 1)
        b[8:8 + n] = hdr.encode()
        Path(dst).write_bytes(bytes(b))


@pytest.fixture(scope="module")
def saved(pkg, F, tmp_path_factory):
    M = pkg.model
    arch = tiny(M)
    p = tmp_path_factory.mktemp("st") / "ok.safetensors"
    F.save_weights(p, arch, M.make_weights(arch, seed=2), task="classical_sr")
    return p


@pytest.mark.parametrize("key", ["task", "upsampler", "scale", "window_size", "embed_dim",
                                 "num_heads", "mlp_ratio", "depths", "img_range", "rgb_mean"])
def test_weights_require_every_metadata_key(F, saved, tmp_path, key):
    p = tmp_path / "m.safetensors"
    _rewrite(F, saved, p, drop_meta=key)
    with pytest.raises(F.FormatError, match=f"no `{key}` in __metadata__ - convert"):
        F.Weights.load(p)


@pytest.mark.parametrize("meta,msg", [
    ({"upsampler": "bilinear"}, "upsampler `bilinear` is not one this engine implements"),
    ({"scale": "four"}, "`scale` = 'four'"),
    ({"depths": "6,x"}, "depths:"),
    ({"rgb_mean": "0.1,0.2"}, "rgb_mean has 2 entries, expected 3"),
    ({"embed_dim": "36"}, r"conv_first.weight is \[24, 3, 3, 3\], the 2-stage/36-wide"),
    ({"mlp_ratio": "4"}, r"mlp.fc1.weight is \[48, 24\], expected \[96, 24\]"),
    ({"num_heads": "3"}, r"attn.cpb_pre is \[4096, 2\], expected \[4096, 3\]"),
    ({"depths": "2,2"}, r"layers.1.residual_group.blocks.1.attn.qkv.wq: no such tensor"),
    ({"upsampler": "pixelshuffle_aux"}, "conv_bicubic.weight: no such tensor"),
    ({"upsampler": "pixelshuffledirect"}, "implies upsample.0.weight 12x24x3x3, found"),
])
def test_weights_validation_messages(F, saved, tmp_path, meta, msg):
    """The checks of reference src/weights.rs:142-235: a checkpoint whose header
    disagrees with its tensors fails at load with the field that disagrees."""
    p = tmp_path / "m.safetensors"
    _rewrite(F, saved, p, set_meta=meta)
    with pytest.raises(F.FormatError, match=msg):
        F.Weights.load(p)


def test_weights_shape_and_dtype_errors(F, saved, tmp_path):
    p = tmp_path / "m.safetensors"
    _rewrite(F, saved, p, reshape=("layers.0.residual_group.blocks.1.mlp.fc2.weight", (24, 24)))
    with pytest.raises(F.FormatError, match=r"mlp.fc2.weight is \[24, 24\], expected \[24, 48\]"):
        F.Weights.load(p)
    _rewrite(F, saved, p, dtype="F16")
    with pytest.raises(F.FormatError, match="dtype F16, this engine reads F32"):
        F.Weights.load(p)
    b = Path(saved).read_bytes()
    (tmp_path / "short.safetensors").write_bytes(b[:len(b) - 8])
    with pytest.raises(F.FormatError, match="outside the"):
        F.Weights.load(tmp_path / "short.safetensors")
    (tmp_path / "junk.safetensors").write_bytes(struct.pack("<Q", 4) + b"{nop")
    with pytest.raises(F.FormatError, match="not JSON"):
        F.Weights.load(tmp_path / "junk.safetensors")


# ---------------------------------------------------------------------------
# SW2F fixtures: the reference's own files
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name,scale,aux", [("ref_fixture_classical_x2.bin", 2, False),
                                            ("ref_fixture_compressed_x4.bin", 4, True)])
def test_reference_fixtures_parse_and_round_trip(F, tmp_path, name, scale, aux):
    src = GOLDEN / name
    f = F.Fixture.load(src)
    assert (f.version, f.h, f.w, f.c, f.scale, f.win) == (1, 37, 29, 3, scale, 8)
    assert (f.aux is not None) == aux and f.flags == (1 if aux else 0)
    assert f.input.size == 3 * 37 * 29 and f.expected.size == 3 * 37 * scale * 29 * scale
    # the input is the [0, 1] image the reference network saw
    assert 0.0 <= f.input.min() and f.input.max() <= 1.0
    if aux:
        assert f.aux_plane() == (40, 32) and f.aux.size == 3 * 40 * 32
    out = tmp_path / "again.bin"
    f.save(out)
    assert out.read_bytes() == src.read_bytes()


def test_fixture_compare_and_locate(F):
    f = F.Fixture.load(GOLDEN / "ref_fixture_classical_x2.bin")
    got = f.expected.copy()
    oh, ow = 74, 58
    idx = 2 * oh * ow + 5 * ow + 7
    got[idx] += 0.25
    worst, at, mean = f.compare(got)
    assert at == idx and abs(worst - 0.25) < 1e-6 and abs(mean - 0.25 / got.size) < 1e-9
    assert f.locate(at) == (5, 7, 2)


def test_fixture_errors(F, tmp_path):
    b = (GOLDEN / "ref_fixture_compressed_x4.bin").read_bytes()
    cases = [
        (b"XXXX" + b[4:], "not a swin2sr fixture"),
        (b[:4] + struct.pack("<I", 2) + b[8:], "fixture version 2, this engine reads 1"),
        (b[:28] + struct.pack("<I", 3) + b[32:], "unknown fixture flags 0x3"),
        (b[:-4], r"234288 bytes expected for 37x29x3 at scale 4 with a 40x32 aux plane, 234284 present"),
    ]
    for i, (data, msg) in enumerate(cases):
        p = tmp_path / f"bad{i}.bin"
        p.write_bytes(data)
        with pytest.raises(F.FormatError, match=msg):
            F.Fixture.load(p)


# ---------------------------------------------------------------------------
# PNG
# ---------------------------------------------------------------------------

def _filter_row(ft, cur, prev, bpp):
    """The forward filters of the PNG specification (section 9.2), per byte,
    written from the definitions: residual = raw - predictor (mod 256)."""
    out = []
    for i, x in enumerate(cur):
        a = cur[i - bpp] if i >= bpp else 0
        b = prev[i]
        c = prev[i - bpp] if i >= bpp else 0
        if ft == 0:
            pr = 0
        elif ft == 1:
            pr = a
        elif ft == 2:
            pr = b
        elif ft == 3:
            pr = (a + b) // 2
        else:
            p = a + b - c
            pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
            pr = a if pa <= pb and pa <= pc else (b if pb <= pc else c)
        out.append((x - pr) % 256)
    return bytes([ft] + out)


def _png(w, h, depth, ctype, rows_bytes, filters):
    bpp = {0: 1, 4: 2, 2: 3, 6: 4}[ctype] * depth // 8
    prev = [0] * len(rows_bytes[0])
    raw = b""
    for y, row in enumerate(rows_bytes):
        raw += _filter_row(filters[y % len(filters)], list(row), prev, bpp)
        prev = list(row)

    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)

    return (b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, depth, ctype, 0, 0, 0))
            + chunk(b"IDAT", zlib.compress(raw)) + chunk(b"IEND", b""))


@pytest.mark.parametrize("depth,ctype", [(8, 2), (8, 6), (8, 0), (8, 4), (16, 2), (16, 0)])
def test_png_decode_every_filter(F, depth, ctype):
    rng = np.random.default_rng(depth * 10 + ctype)
    h, w = 7, 11
    ch = {0: 1, 4: 2, 2: 3, 6: 4}[ctype]
    if depth == 8:
        samples = rng.integers(0, 256, size=(h, w, ch), dtype=np.uint16)
        rows = [bytes(samples[y].reshape(-1).astype(np.uint8)) for y in range(h)]
        scale = 255.0
    else:
        samples = rng.integers(0, 65536, size=(h, w, ch), dtype=np.uint32)
        rows = [bytes(np.stack([samples[y] >> 8, samples[y] & 255], -1).reshape(-1).astype(np.uint8))
                for y in range(h)]
        scale = 65535.0
    b = _png(w, h, depth, ctype, rows, filters=[0, 1, 2, 3, 4])
    hh, ww, img = F.decode_png(b)
    assert (hh, ww) == (h, w)
    want = samples.astype(np.float64) / scale
    if ch <= 2:
        want = np.repeat(want[..., :1], 3, axis=2)
    else:
        want = want[..., :3]
    assert np.allclose(img, want.transpose(2, 0, 1), atol=1e-7)


def test_png_round_trip_and_rounding(pkg, F, tmp_path):
    M = pkg.model
    rng = np.random.default_rng(3)
    x = rng.uniform(-0.1, 1.1, size=(3, 9, 13)).astype(np.float32)
    x[0, 0, 0] = 0.5 / 255.0   # rounds half up, like floor(v*255 + 0.5)
    p = tmp_path / "o.png"
    F.save_rgb(p, x)
    y = F.load_rgb(p)
    assert y.shape == x.shape
    assert np.array_equal(np.rint(y * 255.0).astype(np.uint8), M.to_rgb8(x))
    assert np.rint(y[0, 0, 0] * 255) == 1


def test_png_errors(F, tmp_path):
    with pytest.raises(F.FormatError, match="not a PNG"):
        F.decode_png(b"GIF89a")
    good = F.encode_png(np.zeros((2, 2, 3), np.uint8))
    bad = bytearray(good)
    bad[20] ^= 0xFF           # inside IHDR: the CRC no longer matches
    with pytest.raises(F.FormatError, match="CRC mismatch"):
        F.decode_png(bytes(bad))
    p = tmp_path / "pal.png"
    p.write_bytes(_png(1, 1, 8, 2, [b"\0\0\0"], [0]).replace(b"\x08\x02\x00\x00\x00", b"\x08\x03\x00\x00\x00"))
    with pytest.raises(F.FormatError):
        F.load_rgb(p)
