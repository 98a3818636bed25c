"""The crate's on-disk formats, host side of the device boundary.

- The converted checkpoint: a `.safetensors` file whose `__metadata__` records
  the architecture. `Weights.load` reads it (memory-mapped, no copy) and
  validates the tensors against the architecture the header claims, with the
  crate's rules and messages (reference src/weights.rs:90-235);
  `write_safetensors` / `save_weights` write the converter's layout (reference
  tools/convert.py:224-266: names sorted, payloads 4-byte aligned, the JSON
  header padded with spaces to an 8-byte boundary).
- The golden fixture `SW2F` v1: a 36-byte header and raw little-endian f32
  planes, with an optional aux plane (reference src/fixture.rs,
  tools/make_fixture.py:17-24).
- PNG: decode 8/16-bit grey, grey+alpha, RGB and RGBA into planar f32 RGB in
  [0,1]; encode 8-bit RGB (reference src/image.rs). Written from the PNG
  specification (ISO/IEC 15948): zlib stream, per-scanline filter types 0-4.

Errors raise `FormatError` carrying the crate's message text.
"""
from __future__ import annotations

import json
import struct
import zlib
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import model as M


class FormatError(ValueError):
    pass


# ---------------------------------------------------------------------------
# safetensors
# ---------------------------------------------------------------------------

class SafeTensors:
    """A read-only, memory-mapped `.safetensors` file: the tensor table in the
    file's own order, the `__metadata__` strings, and zero-copy f32 views."""

    def __init__(self, path):
        self.path = Path(path)
        try:
            size = self.path.stat().st_size
        except OSError as e:
            raise FormatError(f"{self.path}: {e.strerror or e}") from None
        if size < 8:
            raise FormatError(f"{self.path}: {size} bytes, too short for a safetensors header")
        with open(self.path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            if n > size - 8:
                raise FormatError(f"{self.path}: header length {n} runs past the end of the file "
                                  f"({size} bytes)")
            raw = f.read(n)
        try:
            header = json.loads(raw.decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise FormatError(f"{self.path}: the header is not JSON: {e}") from None
        if not isinstance(header, dict):
            raise FormatError(f"{self.path}: the header is not a JSON object")
        meta = header.pop("__metadata__", {}) or {}
        if not isinstance(meta, dict) or not all(isinstance(v, str) for v in meta.values()):
            raise FormatError(f"{self.path}: __metadata__ must map names to strings")
        self.metadata: Dict[str, str] = dict(meta)
        self.data_start = 8 + n
        data_len = size - self.data_start
        self.order: List[str] = []
        self._info: Dict[str, Tuple[Tuple[int, ...], int, int]] = {}
        for name, e in header.items():
            if not isinstance(e, dict):
                raise FormatError(f"{self.path}: {name}: malformed entry")
            dtype, shape, offs = e.get("dtype"), e.get("shape"), e.get("data_offsets")
            if dtype != "F32":
                raise FormatError(f"{self.path}: {name}: dtype {dtype}, this engine reads F32")
            if (not isinstance(shape, list) or not all(isinstance(d, int) and d >= 0 for d in shape)
                    or not isinstance(offs, list) or len(offs) != 2
                    or not all(isinstance(o, int) for o in offs)):
                raise FormatError(f"{self.path}: {name}: malformed shape or data_offsets")
            b, end = offs
            count = int(np.prod(shape, dtype=np.int64)) if shape else 1
            if not (0 <= b <= end <= data_len):
                raise FormatError(f"{self.path}: {name}: data_offsets {offs} outside the "
                                  f"{data_len}-byte payload")
            if end - b != 4 * count:
                raise FormatError(f"{self.path}: {name}: {end - b} bytes for shape {shape} "
                                  f"({4 * count} expected)")
            if b % 4:
                raise FormatError(f"{self.path}: {name}: payload offset {b} is not 4-byte aligned")
            self.order.append(name)
            self._info[name] = (tuple(shape), b, count)
        self.size = size
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r") if size > 0 else None

    def __contains__(self, name: str) -> bool:
        return name in self._info

    def shape(self, name: str) -> Tuple[int, ...]:
        if name not in self._info:
            raise FormatError(f"{self.path}: {name}: no such tensor")
        return self._info[name][0]

    def tensor(self, name: str) -> np.ndarray:
        shape, b, count = self._info[name]
        start = self.data_start + b
        return np.frombuffer(self._map, dtype="<f4", count=count, offset=start).reshape(shape)


def write_safetensors(path, tensors: Dict[str, np.ndarray], metadata: Dict[str, str]) -> None:
    """The converter's layout (reference tools/convert.py:238-266)."""
    items = sorted(tensors.items())
    header = {}
    offset = 0
    for name, a in items:
        a = np.ascontiguousarray(a, dtype="<f4")
        n = a.size * 4
        header[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [offset, offset + n]}
        offset += (n + 3) & ~3
    header["__metadata__"] = {k: str(v) for k, v in metadata.items()}
    hjson = json.dumps(header, separators=(",", ":")).encode()
    pad = (-(8 + len(hjson))) & 7
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hjson) + pad))
        f.write(hjson)
        f.write(b" " * pad)
        written = 0
        for name, a in items:
            raw = np.ascontiguousarray(a, dtype="<f4").tobytes()
            want = header[name]["data_offsets"][0]
            if written < want:
                f.write(b"\0" * (want - written))
                written = want
            f.write(raw)
            written += len(raw)


METADATA_KEYS = ("task", "upsampler", "scale", "window_size", "embed_dim", "num_heads",
                 "mlp_ratio", "depths", "img_range", "rgb_mean")


def metadata_for(arch: M.Arch, task: str) -> Dict[str, str]:
    """The `__metadata__` the converter records (reference tools/convert.py:224-236)."""
    return {
        "task": task, "upsampler": arch.upsampler, "scale": str(arch.scale),
        "window_size": str(arch.window), "embed_dim": str(arch.embed),
        "num_heads": str(arch.heads), "mlp_ratio": str(arch.mlp_ratio),
        "depths": ",".join(str(d) for d in arch.depths), "img_range": repr(float(arch.img_range)),
        "rgb_mean": ",".join(f"{m:.4f}" for m in arch.mean), "format": "pt",
    }


def save_weights(path, arch: M.Arch, tensors: Dict[str, np.ndarray], task: str) -> None:
    write_safetensors(path, tensors, metadata_for(arch, task))


class Weights:
    """The checkpoint plus the architecture it describes (reference
    src/weights.rs:66-137): `Weights.load(path)` reads the `__metadata__`,
    parses it, and validates the tensor set against it."""

    def __init__(self, st: SafeTensors, meta: Dict[str, str]):
        p = st.path

        def num(k):
            try:
                return int(meta[k])
            except ValueError as e:
                raise FormatError(f"{p}: `{k}` = {meta[k]!r}: {e}") from None

        try:
            depths = [int(s.strip()) for s in meta["depths"].split(",")]
        except ValueError as e:
            raise FormatError(f"depths: {e}") from None
        try:
            mean = [float(s.strip()) for s in meta["rgb_mean"].split(",")]
        except ValueError as e:
            raise FormatError(f"rgb_mean: {e}") from None
        if len(mean) != 3:
            raise FormatError(f"rgb_mean has {len(mean)} entries, expected 3")
        ups = meta["upsampler"]
        if ups not in M.UPSAMPLERS:
            raise FormatError(
                f"upsampler `{ups}` is not one this engine implements (pixelshuffle, "
                "pixelshuffledirect, nearest+conv, pixelshuffle_aux)")
        try:
            img_range = float(meta["img_range"])
        except ValueError as e:
            raise FormatError(f"img_range: {e}") from None
        self.file = st
        self.path = p
        self.task = meta["task"]
        self.upsampler = ups
        self.scale = num("scale")
        self.window = num("window_size")
        self.embed = num("embed_dim")
        self.heads = num("num_heads")
        if self.heads == 0:
            raise FormatError(f"{p}: `num_heads` = {meta['num_heads']!r}: zero heads")
        self.head_dim = self.embed // self.heads
        self.mlp_ratio = num("mlp_ratio")
        self.depths = depths
        self.img_range = img_range
        self.mean = tuple(np.float32(m).item() for m in mean)
        self.names = list(st.order)
        self.bytes = st.size

    @classmethod
    def load(cls, path) -> "Weights":
        st = SafeTensors(path)
        meta = {}
        for k in METADATA_KEYS:
            if k not in st.metadata:
                raise FormatError(
                    f"{st.path}: no `{k}` in __metadata__ - convert the checkpoint with "
                    "tools/convert.py, which records the architecture; a plain state_dict "
                    "cannot be checked")
            meta[k] = st.metadata[k]
        w = cls(st, meta)
        w.validate()
        return w

    def _shape(self, name: str) -> List[int]:
        if name not in self.file:
            raise FormatError(f"{self.path}: {name}: no such tensor")
        return list(self.file.shape(name))

    def validate(self) -> None:
        """reference src/weights.rs:142-235: the mistakes that otherwise surface
        as a wrong image rather than an error."""
        e, p = self.embed, self.path
        want = [("conv_first.weight", [e, 3, 3, 3]), ("conv_after_body.weight", [e, e, 3, 3]),
                ("norm.weight", [e]), ("patch_embed.proj.weight", [e, e, 1, 1]),
                ("patch_embed.norm.weight", [e])]
        if self.upsampler != "pixelshuffledirect":
            want.append(("conv_last.bias", [3]))
        for name, shape in want:
            got = self._shape(name)
            if got != shape:
                raise FormatError(
                    f"{p}: {name} is {got}, the {len(self.depths)}-stage/{e}-wide architecture "
                    f"in the header implies {shape}")
        win4 = self.window ** 4
        for l, d in enumerate(self.depths):
            for b in range(d):
                q = f"layers.{l}.residual_group.blocks.{b}"
                for name, shape in [
                    (f"{q}.attn.qkv.wq", [e, e]), (f"{q}.attn.qkv.wv", [e, e]),
                    (f"{q}.attn.proj.weight", [e, e]),
                    (f"{q}.mlp.fc1.weight", [self.mlp_ratio * e, e]),
                    (f"{q}.mlp.fc2.weight", [e, self.mlp_ratio * e]),
                    (f"{q}.attn.cpb_pre", [win4, self.heads]),
                ]:
                    got = self._shape(name)
                    if got != shape:
                        raise FormatError(f"{p}: {name} is {got}, expected {shape}")
        if self.upsampler == "pixelshuffle_aux":
            feat = self._shape("conv_before_upsample.0.weight")[0]
            for name, shape in [
                ("conv_bicubic.weight", [feat, 3, 3, 3]), ("conv_bicubic.bias", [feat]),
                ("conv_aux.weight", [3, feat, 3, 3]), ("conv_aux.bias", [3]),
                ("conv_after_aux.0.weight", [feat, 3, 3, 3]), ("conv_after_aux.0.bias", [feat]),
            ]:
                got = self._shape(name)
                if got != shape:
                    raise FormatError(f"{p}: {name} is {got}, the compressed head implies {shape}")
        if self.upsampler == "pixelshuffledirect":
            out = self.scale * self.scale * 3
            got = self._shape("upsample.0.weight")
            if got != [out, self.embed, 3, 3]:
                raise FormatError(
                    f"{p}: upsampler pixelshuffledirect implies upsample.0.weight "
                    f"{out}x{self.embed}x3x3, found {got}")

    def t(self, name: str) -> np.ndarray:
        return self.file.tensor(name)

    def shape(self, name: str) -> Tuple[int, ...]:
        return self.file.shape(name)

    def has(self, name: str) -> bool:
        return name in self.file

    def arch(self) -> M.Arch:
        """The architecture as the device backend takes it."""
        feat = 64
        if self.has("conv_before_upsample.0.weight"):
            feat = int(self.shape("conv_before_upsample.0.weight")[0])
        return M.Arch(upsampler=self.upsampler, scale=self.scale, window=self.window,
                      embed=self.embed, heads=self.heads, mlp_ratio=self.mlp_ratio,
                      depths=list(self.depths), img_range=self.img_range, mean=self.mean,
                      feat=feat)

    def tensors(self) -> Dict[str, np.ndarray]:
        """Every tensor, as zero-copy views of the mapping."""
        return {n: self.t(n) for n in self.names}


# ---------------------------------------------------------------------------
# SW2F golden fixtures
# ---------------------------------------------------------------------------

SW2F_MAGIC = b"SW2F"
FLAG_AUX = 1


class Fixture:
    """reference src/fixture.rs: `[3][h][w]` input in [0,1], the expected
    `[3][h*s][w*s]` output and, with flag bit 0, the aux plane at the padded
    geometry."""

    def __init__(self, h, w, c, scale, win, input, expected, aux=None, version=1):
        self.version, self.h, self.w, self.c = version, h, w, c
        self.scale, self.win = scale, win
        self.flags = FLAG_AUX if aux is not None else 0
        self.input = np.asarray(input, np.float32).reshape(-1)
        self.expected = np.asarray(expected, np.float32).reshape(-1)
        self.aux = None if aux is None else np.asarray(aux, np.float32).reshape(-1)

    def aux_plane(self) -> Tuple[int, int]:
        return ((self.h // self.win + 1) * self.win, (self.w // self.win + 1) * self.win)

    @classmethod
    def load(cls, path) -> "Fixture":
        p = Path(path)
        try:
            b = p.read_bytes()
        except OSError as e:
            raise FormatError(f"{p}: {e.strerror or e}") from None
        if len(b) < 36 or b[:4] != SW2F_MAGIC:
            raise FormatError(f"{p}: not a swin2sr fixture (want 4-byte magic SW2F)")
        version, h, w, c, scale, win, flags, _ = struct.unpack_from("<8I", b, 4)
        if version != 1:
            raise FormatError(f"{p}: fixture version {version}, this engine reads 1")
        if flags & ~FLAG_AUX:
            raise FormatError(
                f"{p}: unknown fixture flags {flags:#x} - this engine knows only bit 0 "
                f"({FLAG_AUX:#x}, an aux plane follows)")
        ah, aw = (((h // win + 1) * win, (w // win + 1) * win) if flags & FLAG_AUX else (0, 0))
        n_in, n_out, n_aux = h * w * c, h * scale * w * scale * c, ah * aw * c
        need = 36 + 4 * (n_in + n_out + n_aux)
        if len(b) != need:
            extra = f" with a {ah}x{aw} aux plane" if flags & FLAG_AUX else ""
            raise FormatError(f"{p}: {need} bytes expected for {h}x{w}x{c} at scale {scale}"
                              f"{extra}, {len(b)} present")
        f32 = np.frombuffer(b, dtype="<f4", offset=36)
        inp = f32[:n_in].copy()
        exp = f32[n_in:n_in + n_out].copy()
        aux = f32[n_in + n_out:].copy() if flags & FLAG_AUX else None
        return cls(h, w, c, scale, win, inp, exp, aux, version)

    def save(self, path) -> None:
        """tools/make_fixture.py:104-110."""
        with open(path, "wb") as f:
            f.write(SW2F_MAGIC)
            f.write(struct.pack("<8I", 1, self.h, self.w, self.c, self.scale, self.win,
                                self.flags, 0))
            f.write(self.input.astype("<f4").tobytes())
            f.write(self.expected.astype("<f4").tobytes())
            if self.aux is not None:
                f.write(self.aux.astype("<f4").tobytes())

    def compare(self, got: np.ndarray) -> Tuple[float, int, float]:
        """(worst |diff|, its flat index, mean |diff|), reference src/fixture.rs:96-110."""
        g = np.asarray(got, np.float32).reshape(-1)
        if g.size != self.expected.size:
            raise FormatError("backend returned the wrong number of pixels")
        d = np.abs(self.expected - g)
        at = int(np.argmax(d))
        return float(d[at]), at, float(d.astype(np.float64).mean())

    def locate(self, idx: int) -> Tuple[int, int, int]:
        """(y, x, channel) of a flat index of the expected tensor."""
        oh, ow = self.h * self.scale, self.w * self.scale
        plane = oh * ow
        c, rem = divmod(idx, plane)
        return rem // ow, rem % ow, c


# ---------------------------------------------------------------------------
# PNG
# ---------------------------------------------------------------------------

PNG_SIG = b"\x89PNG\r\n\x1a\n"


def _chunks(b: bytes):
    pos = 8
    while pos + 8 <= len(b):
        (n,) = struct.unpack_from(">I", b, pos)
        typ = b[pos + 4:pos + 8]
        data = b[pos + 8:pos + 8 + n]
        if len(data) != n or pos + 12 + n > len(b):
            raise FormatError("truncated PNG chunk")
        (crc,) = struct.unpack_from(">I", b, pos + 8 + n)
        if zlib.crc32(typ + data) & 0xFFFFFFFF != crc:
            raise FormatError(f"PNG chunk {typ.decode('latin-1')}: CRC mismatch")
        yield typ, data
        pos += 12 + n


def _unfilter(raw: bytes, h: int, stride: int, bpp: int) -> np.ndarray:
    """Undo the per-scanline filters (PNG spec section 9.2) into [h][stride] bytes."""
    if len(raw) < h * (stride + 1):
        raise FormatError("PNG image data too short")
    rows = np.frombuffer(raw, np.uint8, count=h * (stride + 1)).reshape(h, stride + 1)
    out = np.zeros((h, stride), np.uint8)
    prev = np.zeros(stride, np.int32)
    for y in range(h):
        ft = int(rows[y, 0])
        line = rows[y, 1:].astype(np.int32)
        if ft == 0:
            cur = line
        elif ft == 1:   # Sub: running sum per byte lane of a pixel
            cur = np.zeros(stride, np.int32)
            for k in range(bpp):
                cur[k::bpp] = np.cumsum(line[k::bpp]) & 0xFF
        elif ft == 2:   # Up
            cur = (line + prev) & 0xFF
        elif ft in (3, 4):
            cur = np.zeros(stride, np.int32)
            ln, pv = line.tolist(), prev.tolist()
            c = [0] * stride
            for i in range(stride):
                a = c[i - bpp] if i >= bpp else 0
                up = pv[i]
                if ft == 3:   # Average
                    c[i] = (ln[i] + ((a + up) >> 1)) & 0xFF
                else:         # Paeth
                    ul = pv[i - bpp] if i >= bpp else 0
                    p = a + up - ul
                    pa, pb, pc = abs(p - a), abs(p - up), abs(p - ul)
                    pred = a if (pa <= pb and pa <= pc) else (up if pb <= pc else ul)
                    c[i] = (ln[i] + pred) & 0xFF
            cur = np.asarray(c, np.int32)
        else:
            raise FormatError(f"PNG filter type {ft} on row {y}")
        out[y] = cur.astype(np.uint8)
        prev = cur
    return out


def decode_png(b: bytes) -> Tuple[int, int, np.ndarray]:
    """(h, w, planar f32 RGB [3][h][w] in [0,1]) - reference src/image.rs:48-107:
    grey and grey+alpha replicate the grey sample, alpha is dropped, 16-bit
    samples scale by 1/65535 and 8-bit by 1/255."""
    if b[:8] != PNG_SIG:
        raise FormatError("not a PNG file")
    ihdr = None
    idat = []
    for typ, data in _chunks(b):
        if typ == b"IHDR":
            ihdr = struct.unpack(">IIBBBBB", data)
        elif typ == b"IDAT":
            idat.append(data)
        elif typ == b"IEND":
            break
    if ihdr is None:
        raise FormatError("PNG without IHDR")
    w, h, depth, ctype, comp, filt, interlace = ihdr
    channels = {0: 1, 4: 2, 2: 3, 6: 4}.get(ctype)
    if channels is None:
        raise FormatError(f"unsupported png colour type {ctype}")
    if depth not in (8, 16):
        raise FormatError(f"unsupported png bit depth {depth}")
    if comp != 0 or filt != 0 or interlace != 0:
        raise FormatError("unsupported PNG compression, filter method or interlacing")
    bpp = channels * depth // 8
    stride = w * bpp
    raw = zlib.decompress(b"".join(idat))
    px = _unfilter(raw, h, stride, bpp)
    if depth == 16:
        s = px.reshape(h, w * channels, 2).astype(np.uint32)
        samples = ((s[..., 0] << 8) | s[..., 1]).astype(np.float32) * np.float32(1.0 / 65535.0)
    else:
        samples = px.astype(np.float32) * np.float32(1.0 / 255.0)
    samples = samples.reshape(h, w, channels)
    if channels <= 2:
        rgb = np.repeat(samples[..., :1], 3, axis=2)
    else:
        rgb = samples[..., :3]
    return h, w, np.ascontiguousarray(rgb.transpose(2, 0, 1)).astype(np.float32)


def load_rgb(path) -> np.ndarray:
    """Planar f32 RGB `[3][h][w]` in [0,1] from a PNG file."""
    p = Path(path)
    try:
        b = p.read_bytes()
    except OSError as e:
        raise FormatError(f"open {p}: {e.strerror or e}") from None
    try:
        return decode_png(b)[2]
    except FormatError as e:
        raise FormatError(f"{p}: {e}") from None


def encode_png(rgb8: np.ndarray) -> bytes:
    """8-bit RGB PNG of an interleaved `[h][w][3]` u8 array (filter 0 rows)."""
    a = np.ascontiguousarray(rgb8, np.uint8)
    if a.ndim != 3 or a.shape[2] != 3:
        raise FormatError("encode_png takes [h][w][3] bytes")
    h, w, _ = a.shape
    rows = np.zeros((h, 1 + 3 * w), np.uint8)
    rows[:, 1:] = a.reshape(h, 3 * w)

    def chunk(typ, data):
        return (struct.pack(">I", len(data)) + typ + data +
                struct.pack(">I", zlib.crc32(typ + data) & 0xFFFFFFFF))

    return (PNG_SIG + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0)) +
            chunk(b"IDAT", zlib.compress(rows.tobytes(), 6)) + chunk(b"IEND", b""))


def save_rgb(path, planar: np.ndarray) -> None:
    """Write `[3][h][w]` f32 in [0,1] as 8-bit RGB with the crate's rounding
    (`Image::to_rgb8`, reference src/image.rs:29-39)."""
    rgb8 = M.to_rgb8(np.asarray(planar, np.float32)).transpose(1, 2, 0)
    Path(path).write_bytes(encode_png(rgb8))


# ---------------------------------------------------------------------------
# The --device gpu flow around the backend
# ---------------------------------------------------------------------------

def verify_fixture(weights: Weights, fixture: Fixture, backend) -> Dict[str, object]:
    """reference src/main.rs:665-760: run a fixture's input through a backend
    and report the worst difference (and the aux plane's, when there is one)."""
    if fixture.c != 3:
        raise FormatError(f"the fixture has {fixture.c} channels, this engine restores RGB")
    if fixture.scale != weights.scale:
        raise FormatError(f"the fixture is scale {fixture.scale}, the checkpoint is x{weights.scale}")
    if fixture.win != weights.window:
        raise FormatError(f"the fixture was made with window {fixture.win}, the checkpoint uses "
                          f"{weights.window}")
    arch = weights.arch()
    x = M.adjust(arch, fixture.input.reshape(3, fixture.h, fixture.w))
    got = backend.forward(fixture.h, fixture.w, x)
    worst, at, mean = fixture.compare(got)
    rep = {"worst": worst, "at": fixture.locate(at), "mean": mean, "aux_worst": None}
    aux_got = backend.aux()
    if (fixture.aux is None) != (aux_got is None):
        raise FormatError("aux: the fixture and the backend disagree about a second image")
    if fixture.aux is not None:
        if aux_got.size != fixture.aux.size:
            raise FormatError(f"aux: {aux_got.size} values, the fixture has {fixture.aux.size}")
        rep["aux_worst"] = float(np.abs(fixture.aux - aux_got.reshape(-1)).max())
    return rep
