"""ctypes binding of include/swin2sr_hip.h, and the `Backend` mirror over it.

`HipBackend` is the host-side mirror of the crate's `Backend` trait
(reference src/backend.rs:29-49) for the device: `name()`, `forward(h, w,
input)` on a mean-adjusted `[3][h][w]` plane returning the denormalised,
cropped `[3][h*s][w*s]` image, and `aux()`. Errors surface as `S2SError`
carrying the library's message (which contains "out of memory" for
allocation failures, the condition the crate's tile-halving retry keys on).

The library is REQUIRED: there is no CPU fallback anywhere in this package.
If `libswin2sr_hip.so` is missing, loading fails with an error that says how
to build it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Dict, Optional, Tuple

import numpy as np

from . import model as M

LIB_PATH = Path(__file__).resolve().parent / "libswin2sr_hip.so"


class S2SError(RuntimeError):
    pass


class Arch_(C.Structure):
    _fields_ = [("upsampler", C.c_int), ("scale", C.c_int), ("window", C.c_int),
                ("embed", C.c_int), ("heads", C.c_int), ("mlp_ratio", C.c_int),
                ("n_stages", C.c_int), ("depths", C.c_int * 16), ("img_range", C.c_float),
                ("mean", C.c_float * 3)]


class Tensor_(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.POINTER(C.c_float)), ("ndim", C.c_int),
                ("shape", C.c_int64 * 4)]


_lib = None

FP = C.POINTER(C.c_float)
EXPORTS = {
    "s2s_create": (C.c_int, [C.POINTER(Arch_), C.POINTER(Tensor_), C.c_size_t, C.POINTER(C.c_void_p)]),
    "s2s_destroy": (None, [C.c_void_p]),
    "s2s_name": (C.c_char_p, []),
    "s2s_uploaded_bytes": (C.c_uint64, [C.c_void_p]),
    "s2s_uploaded_bytes_for": (C.c_int, [C.POINTER(Arch_), C.POINTER(Tensor_), C.c_size_t,
                                         C.POINTER(C.c_uint64)]),
    "s2s_plan_bytes": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_uint64)]),
    "s2s_set_alloc_limit": (C.c_int, [C.c_void_p, C.c_uint64]),
    "s2s_selftest": (C.c_int, [C.POINTER(Arch_), C.POINTER(Tensor_), C.c_size_t]),
    "s2s_forward": (C.c_int, [C.c_void_p, C.c_int, C.c_int, FP, FP]),
    "s2s_forward_device": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "s2s_forward_batch": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                    C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                    C.POINTER(C.c_void_p)]),
    "s2s_forward_device_batch": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int,
                                           C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "s2s_forward_device_noalloc": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                             C.c_void_p]),
    "s2s_aux": (C.c_int, [C.c_void_p, C.POINTER(FP), C.POINTER(C.c_size_t)]),
    "s2s_last_error": (C.c_char_p, []),
    "s2s_device_info": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    "s2s_vram": (C.c_int, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "s2s_sync": (C.c_int, []),
    "s2s_stream": (C.c_void_p, [C.c_void_p]),
    "s2s_profile_enable": (C.c_int, [C.c_void_p, C.c_int]),
    "s2s_profile_reset": (C.c_int, [C.c_void_p]),
    "s2s_profile_report": (C.c_int, [C.c_void_p, C.c_float]),
    "s2s_profile_query": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_int)]),
    "s2s_profile_only": (C.c_int, [C.c_void_p, C.c_char_p]),
    "s2s_rstb_device": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "s2s_test_window_map": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int32),
                                      C.POINTER(C.c_uint8)]),
    "s2s_test_qkv_windows": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP,
                                       FP, C.c_size_t]),
    "s2s_test_block_attention": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP,
                                           FP, FP, FP, FP]),
    "s2s_test_attention": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP, FP]),
    "s2s_test_cpb_table": (C.c_int, [C.c_int, C.c_int, FP, FP, FP, FP]),
    "s2s_test_linear": (C.c_int, [C.c_int, C.c_int, C.c_int, FP, FP, FP, C.c_int, FP, FP, FP,
                                  C.c_float, FP]),
    "s2s_test_ln_residual": (C.c_int, [C.c_int, C.c_int, FP, FP, FP, FP, FP]),
    "s2s_test_embed": (C.c_int, [C.c_int, C.c_int, C.c_int, FP, FP, FP, FP, FP, FP, FP, FP, FP]),
    "s2s_test_conv3x3": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP, C.c_int, FP,
                                   C.c_float, FP]),
    "s2s_test_conv3x3_winograd": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP,
                                            C.c_int, FP, C.c_float, FP]),
    "s2s_test_conv3x3_shuffle2": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP, FP]),
    "s2s_test_rstb": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, FP, FP]),
    "s2s_test_mfma_peak": (C.c_int, [C.c_int, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                     C.POINTER(C.c_double)]),
    "s2s_test_conv3x3_nearest2": (C.c_int, [C.c_int, C.c_int, C.c_int, FP, FP, FP, C.c_float, FP]),
}


def load_library():
    """Load libswin2sr_hip.so (loud failure if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise S2SError(f"{LIB_PATH} is not built: run `make -C {LIB_PATH.parent}` "
                       "(or __graft_entry__.build()); there is no CPU fallback")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in EXPORTS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return (load_library().s2s_last_error() or b"").decode()


def check(rc: int, what: str):
    if rc != 0:
        raise S2SError(f"{what}: {last_error()}")


def fptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "float32 C-contiguous required"
    return a.ctypes.data_as(FP)


def arch_struct(a: M.Arch) -> Arch_:
    s = Arch_()
    s.upsampler = M.UPSAMPLERS[a.upsampler]
    s.scale, s.window, s.embed, s.heads, s.mlp_ratio = a.scale, a.window, a.embed, a.heads, a.mlp_ratio
    s.n_stages = len(a.depths)
    for i, d in enumerate(a.depths):
        s.depths[i] = d
    s.img_range = a.img_range
    for i in range(3):
        s.mean[i] = a.mean[i]
    return s


def tensor_table(weights: Dict[str, np.ndarray]):
    """(array of Tensor_, keep-alive list) for a name -> array dict."""
    keep = []
    arr = (Tensor_ * len(weights))()
    for i, (name, t) in enumerate(weights.items()):
        t = np.ascontiguousarray(t, dtype=np.float32)
        nb = name.encode()
        keep += [t, nb]
        arr[i].name = nb
        arr[i].data = t.ctypes.data_as(FP)
        arr[i].ndim = t.ndim
        for d in range(t.ndim):
            arr[i].shape[d] = t.shape[d]
    return arr, keep


class HipBackend:
    """The device `Backend` (reference src/backend.rs:29-49 / src/gpu.rs:736-759)."""

    def __init__(self, arch: M.Arch, weights: Dict[str, np.ndarray]):
        lib = load_library()
        self.arch = arch
        a = arch_struct(arch)
        tabs, keep = tensor_table(weights)
        ctx = C.c_void_p()
        check(lib.s2s_create(C.byref(a), tabs, len(weights), C.byref(ctx)), "s2s_create")
        self._ctx = ctx
        self._lib = lib
        del keep

    def close(self):
        if getattr(self, "_ctx", None):
            self._lib.s2s_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def ctx(self):
        return self._ctx

    def name(self) -> str:
        return self._lib.s2s_name().decode()

    def uploaded_bytes(self) -> int:
        return int(self._lib.s2s_uploaded_bytes(self._ctx))

    def plan_bytes(self, h: int, w: int) -> int:
        """Device bytes a forward of an h x w image allocates (s2s_plan_bytes)."""
        b = C.c_uint64()
        check(self._lib.s2s_plan_bytes(self._ctx, h, w, C.byref(b)), "s2s_plan_bytes")
        return int(b.value)

    def set_alloc_limit(self, nbytes: int):
        """Cap the per-image plans at `nbytes` (0 = none): past it a forward
        fails with "out of memory"."""
        check(self._lib.s2s_set_alloc_limit(self._ctx, int(nbytes)), "s2s_set_alloc_limit")

    def forward(self, h: int, w: int, input_adjusted: np.ndarray,
                out: Optional[np.ndarray] = None) -> np.ndarray:
        """`Backend::forward`: a new output image per call, as the crate's
        backend returns a new Vec (or into `out`, a caller-owned float32
        [3][h*s][w*s] array)."""
        x = np.ascontiguousarray(input_adjusted, dtype=np.float32)
        assert x.shape == (3, h, w), x.shape
        s = self.arch.scale
        if out is None:
            out = np.empty((3, h * s, w * s), np.float32)
        assert out.shape == (3, h * s, w * s) and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
        check(self._lib.s2s_forward(self._ctx, h, w, fptr(x), fptr(out)), "s2s_forward")
        return out

    def forward_batch(self, shapes, inputs, aux=False):
        """`forward` over several images (a tiled image's crops) at once, on the
        context's two lanes: a list of new output images, and with `aux` a list
        of each image's aux image (None where the head makes none)."""
        n = len(inputs)
        s = self.arch.scale
        xs = [np.ascontiguousarray(x, dtype=np.float32) for x in inputs]
        for (h, w), x in zip(shapes, xs):
            assert x.shape == (3, h, w), x.shape
        outs = [np.empty((3, h * s, w * s), np.float32) for h, w in shapes]
        win = self.arch.window
        has_aux = aux and self.arch.upsampler == "pixelshuffle_aux"
        auxs = ([np.empty((3, (h // win + 1) * win, (w // win + 1) * win), np.float32) for h, w in shapes]
                if has_aux else None)
        vp = lambda a: C.c_void_p(a.ctypes.data)
        hs = (C.c_int * max(n, 1))(*[h for h, _ in shapes])
        ws = (C.c_int * max(n, 1))(*[w for _, w in shapes])
        ins = (C.c_void_p * max(n, 1))(*[vp(x) for x in xs])
        os_ = (C.c_void_p * max(n, 1))(*[vp(o) for o in outs])
        ax = (C.c_void_p * max(n, 1))(*[vp(a) for a in auxs]) if has_aux else None
        check(self._lib.s2s_forward_batch(self._ctx, n, hs, ws, ins, os_, ax), "s2s_forward_batch")
        if aux:
            return outs, (auxs if has_aux else [None] * n)
        return outs

    def forward_device(self, h: int, w: int, d_in: int, d_out: int):
        check(self._lib.s2s_forward_device(self._ctx, h, w, C.c_void_p(d_in), C.c_void_p(d_out)),
              "s2s_forward_device")

    def forward_device_batch(self, h: int, w: int, d_ins, d_outs):
        """n images of one size (device pointers), over the context's stream
        and its second lane; ordered on the context's stream."""
        n = len(d_ins)
        assert len(d_outs) == n
        ins = (C.c_void_p * max(n, 1))(*[C.c_void_p(p) for p in d_ins])
        outs = (C.c_void_p * max(n, 1))(*[C.c_void_p(p) for p in d_outs])
        check(self._lib.s2s_forward_device_batch(self._ctx, n, h, w, ins, outs),
              "s2s_forward_device_batch")

    def forward_device_noalloc(self, h: int, w: int, d_in: int, d_out: int):
        """The forward on the library's static per-GPU workspace (no allocation)."""
        check(self._lib.s2s_forward_device_noalloc(self._ctx, h, w, C.c_void_p(d_in),
                                                   C.c_void_p(d_out)),
              "s2s_forward_device_noalloc")

    def rstb_device(self, stage: int, hp: int, wp: int, d_in: int, d_out: int):
        check(self._lib.s2s_rstb_device(self._ctx, stage, hp, wp, C.c_void_p(d_in),
                                        C.c_void_p(d_out)), "s2s_rstb_device")

    def test_rstb(self, stage: int, hp: int, wp: int, x_hwc: np.ndarray) -> np.ndarray:
        """One RSTB stage on host buffers (channel-last `[hp*wp][embed]`)."""
        x = np.ascontiguousarray(x_hwc, dtype=np.float32)
        assert x.size == hp * wp * self.arch.embed, x.shape
        out = np.empty((hp * wp, self.arch.embed), np.float32)
        check(self._lib.s2s_test_rstb(self._ctx, stage, hp, wp, fptr(x), fptr(out)), "s2s_test_rstb")
        return out

    def aux(self) -> Optional[np.ndarray]:
        p = FP()
        n = C.c_size_t()
        check(self._lib.s2s_aux(self._ctx, C.byref(p), C.byref(n)), "s2s_aux")
        if n.value == 0:
            return None
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()

    def stream(self) -> int:
        return int(self._lib.s2s_stream(self._ctx) or 0)

    def profile(self, on: bool):
        check(self._lib.s2s_profile_enable(self._ctx, 1 if on else 0), "s2s_profile_enable")

    def profile_reset(self):
        check(self._lib.s2s_profile_reset(self._ctx), "s2s_profile_reset")

    def profile_report(self, wall_ms: float = 0.0):
        check(self._lib.s2s_profile_report(self._ctx, wall_ms), "s2s_profile_report")

    def profile_only(self, kernel: Optional[str]):
        """Bracket only launches named `kernel` with events (None = all)."""
        check(self._lib.s2s_profile_only(self._ctx, kernel.encode() if kernel else None),
              "s2s_profile_only")

    def profile_query(self, kernel: str) -> Tuple[float, int]:
        ms = C.c_double()
        n = C.c_int()
        check(self._lib.s2s_profile_query(self._ctx, kernel.encode(), C.byref(ms), C.byref(n)),
              "s2s_profile_query")
        return ms.value, n.value


def device_info() -> Tuple[str, str]:
    lib = load_library()
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(256)
    check(lib.s2s_device_info(name, 256, arch, 256), "s2s_device_info")
    return name.value.decode(), arch.value.decode()


def uploaded_bytes_for(arch: M.Arch, weights: Dict[str, np.ndarray]) -> int:
    """`gpu::uploaded_bytes(&Weights)`: what s2s_create will upload, no context."""
    lib = load_library()
    a = arch_struct(arch)
    tabs, keep = tensor_table(weights)
    b = C.c_uint64()
    check(lib.s2s_uploaded_bytes_for(C.byref(a), tabs, len(weights), C.byref(b)),
          "s2s_uploaded_bytes_for")
    del keep
    return int(b.value)


def selftest(arch: M.Arch, weights: Optional[Dict[str, np.ndarray]] = None):
    """`gpu::selftest` (the crate's --cuda-selftest): raises S2SError naming the
    failing check; prints the count of checks on success."""
    lib = load_library()
    a = arch_struct(arch)
    if weights:
        tabs, keep = tensor_table(weights)
        rc = lib.s2s_selftest(C.byref(a), tabs, len(weights))
        del keep
    else:
        rc = lib.s2s_selftest(C.byref(a), None, 0)
    check(rc, "s2s_selftest")


# ---- per-op test entry points ------------------------------------------------

def unit_floats(hp, wp, heads, head_dim):
    """Floats of the window attention's unit layout of qkv for a plane."""
    return (hp // 8) * (wp // 8) * ((heads + 1) // 2) * 64 * (6 * head_dim + 2)


def mfma_peak(iters: int = 20000, reps: int = 5) -> Tuple[float, float, float]:
    """(ms per launch, TFLOP/s, implied shader clock in GHz) of the fp32 MFMA
    peak probe."""
    ms, tf, ghz = C.c_double(), C.c_double(), C.c_double()
    check(load_library().s2s_test_mfma_peak(iters, reps, C.byref(ms), C.byref(tf), C.byref(ghz)),
          "s2s_test_mfma_peak")
    return ms.value, tf.value, ghz.value


def test_qkv_windows(hp, wp, heads, head_dim, shift, x, wqkv, bqkv):
    """The production qkv GEMM's raw unit-layout output, shape
    [windows][head pairs][64][6*head_dim + 2] (unwritten padding is NaN)."""
    lib = load_library()
    n = unit_floats(hp, wp, heads, head_dim)
    out = np.empty(n, np.float32)
    c32 = lambda a: np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_qkv_windows(hp, wp, heads, head_dim, shift, fptr(c32(x)), fptr(c32(wqkv)),
                                   fptr(c32(bqkv)), fptr(out), n), "s2s_test_qkv_windows")
    return out.reshape((hp // 8) * (wp // 8), (heads + 1) // 2, 64, 6 * head_dim + 2)


def test_block_attention(hp, wp, heads, head_dim, shift, x, wqkv, bqkv, logit_scale, cpb):
    """The production qkv projection + window attention (one fused kernel for
    6 heads of 30); the plane [hp*wp][c]."""
    lib = load_library()
    c = heads * head_dim
    out = np.empty((hp * wp, c), np.float32)
    c32 = lambda a: np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_block_attention(hp, wp, heads, head_dim, shift, fptr(c32(x)),
                                       fptr(c32(wqkv)), fptr(c32(bqkv)),
                                       fptr(c32(logit_scale).reshape(-1)), fptr(c32(cpb)),
                                       fptr(out)), "s2s_test_block_attention")
    return out


def test_window_map(hp, wp, shift, win=8):
    lib = load_library()
    n = (hp // win) * (wp // win) * win * win
    yx = np.empty((n, 2), np.int32)
    reg = np.empty((n, 2), np.uint8)
    check(lib.s2s_test_window_map(hp, wp, win, shift, yx.ctypes.data_as(C.POINTER(C.c_int32)),
                                  reg.ctypes.data_as(C.POINTER(C.c_uint8))), "s2s_test_window_map")
    return yx, reg


def test_attention(hp, wp, heads, head_dim, shift, qkv_plane, logit_scale, cpb, win=8):
    lib = load_library()
    c = heads * head_dim
    out = np.empty((hp * wp, c), np.float32)
    check(lib.s2s_test_attention(hp, wp, win, heads, head_dim, shift,
                                 fptr(np.ascontiguousarray(qkv_plane, np.float32)),
                                 fptr(np.ascontiguousarray(logit_scale, np.float32).reshape(-1)),
                                 fptr(np.ascontiguousarray(cpb, np.float32)), fptr(out)),
          "s2s_test_attention")
    return out


def test_cpb_table(win, heads, w0, b0, w2):
    lib = load_library()
    out = np.empty((win ** 4, heads), np.float32)
    check(lib.s2s_test_cpb_table(win, heads, fptr(np.ascontiguousarray(w0, np.float32)),
                                 fptr(np.ascontiguousarray(b0, np.float32)),
                                 fptr(np.ascontiguousarray(w2, np.float32)), fptr(out)),
          "s2s_test_cpb_table")
    return out


def test_linear(x, w, bias=None, epilogue=0, res=None, ln_w=None, ln_b=None, slope=0.0):
    lib = load_library()
    rows, cin = x.shape
    cout = w.shape[0]
    out = np.empty((rows, cout), np.float32)
    c32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    args = [c32(x), c32(w), c32(bias), c32(res), c32(ln_w), c32(ln_b)]
    check(lib.s2s_test_linear(rows, cin, cout, fptr(args[0]), fptr(args[1]), fptr(args[2]),
                              epilogue, fptr(args[3]), fptr(args[4]), fptr(args[5]), slope,
                              fptr(out)), "s2s_test_linear")
    return out


def test_ln_residual(x, ln_w, ln_b, res=None):
    lib = load_library()
    hw, c = x.shape
    out = np.empty_like(x, dtype=np.float32)
    c32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_ln_residual(hw, c, fptr(c32(x)), fptr(c32(ln_w)), fptr(c32(ln_b)),
                                   fptr(c32(res)), fptr(out)), "s2s_test_ln_residual")
    return out


def test_embed(x_hwc, h, w, w_first, b_first, w_fold, b_fold, ln_w, ln_b):
    """conv_first and the folded patch_embed + LayerNorm through the forward's
    kernel: `x_hwc` [h*w][3], weights [c][3][3][3]; returns (body, cur), each
    [h*w][c]."""
    lib = load_library()
    c = w_first.shape[0]
    body = np.empty((h * w, c), np.float32)
    cur = np.empty((h * w, c), np.float32)
    c32 = lambda a: np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_embed(h, w, c, fptr(c32(x_hwc)), fptr(c32(w_first)), fptr(c32(b_first)),
                             fptr(c32(w_fold)), fptr(c32(b_fold)), fptr(c32(ln_w)), fptr(c32(ln_b)),
                             fptr(body), fptr(cur)), "s2s_test_embed")
    return body, cur


def test_conv3x3(x_hwc, h, w, wgt, bias, epilogue=0, res=None, slope=0.0):
    lib = load_library()
    cout, cin = wgt.shape[0], wgt.shape[1]
    out = np.empty((h * w, cout), np.float32)
    c32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_conv3x3(h, w, cin, cout, fptr(c32(x_hwc)), fptr(c32(wgt)), fptr(c32(bias)),
                               epilogue, fptr(c32(res)), slope, fptr(out)), "s2s_test_conv3x3")
    return out


def test_conv3x3_nearest2(x_hwc, h, w, wgt, bias, slope):
    """conv3x3 (c -> c) + LeakyReLU of the nearest-2x upsampling of an h x w
    plane, as the four phases' 2x2 convs the real-world head runs."""
    lib = load_library()
    c = wgt.shape[0]
    out = np.empty((4 * h * w, c), np.float32)
    c32 = lambda a: np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_conv3x3_nearest2(h, w, c, fptr(c32(x_hwc)), fptr(c32(wgt)), fptr(c32(bias)),
                                        slope, fptr(out)), "s2s_test_conv3x3_nearest2")
    return out


def test_conv3x3_winograd(x_hwc, h, w, wgt, bias, epilogue=0, res=None, slope=0.0):
    """The Winograd F(4x4,3x3) conv path: the body's C -> C convs (c_in ==
    c_out in {60, 120, 180}) and conv_before_upsample's C -> F (F <= 64)."""
    lib = load_library()
    cout, cin = wgt.shape[0], wgt.shape[1]
    out = np.empty((h * w, cout), np.float32)
    c32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_conv3x3_winograd(h, w, cin, cout, fptr(c32(x_hwc)), fptr(c32(wgt)),
                                        fptr(c32(bias)), epilogue, fptr(c32(res)), slope, fptr(out)),
          "s2s_test_conv3x3_winograd")
    return out


def test_conv3x3_shuffle2(x_hwc, h, w, wgt, bias):
    lib = load_library()
    c4, cin = wgt.shape[0], wgt.shape[1]
    feat = c4 // 4
    out = np.empty((4 * h * w, feat), np.float32)
    c32 = lambda a: np.ascontiguousarray(a, np.float32)
    check(lib.s2s_test_conv3x3_shuffle2(h, w, cin, feat, fptr(c32(x_hwc)), fptr(c32(wgt)),
                                        fptr(c32(bias)), fptr(out)), "s2s_test_conv3x3_shuffle2")
    return out
