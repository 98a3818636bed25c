"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline. The
HIP backend never loads it.

Layouts are the reference CPU path's: planes NCHW `[c][h][w]`, window tokens
`[nw*n][c]` window-major, qkv `[3][tokens][c]`.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Dict, Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
FP = C.POINTER(C.c_float)


class Plan(C.Structure):
    _fields_ = [(k, C.c_int) for k in ("h", "w", "hp", "wp", "win", "nwh", "nww", "nw", "n", "c")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} not built: run `make -C {HERE}`")
        L = C.CDLL(str(LIB_PATH))
        P = C.POINTER(Plan)
        sig = {
            "orc_plan_new": (None, [C.c_int, C.c_int, C.c_int, C.c_int, P]),
            "orc_plan_explicit": (None, [C.c_int, C.c_int, C.c_int, C.c_int, P]),
            "orc_shift_for": (C.c_int, [P, C.c_int]),
            "orc_window_map": (None, [P, C.c_int, C.POINTER(C.c_int32), C.POINTER(C.c_uint8)]),
            "orc_region_of": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int]),
            "orc_pad_reflect": (None, [FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP]),
            "orc_conv3x3": (None, [FP, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP, FP]),
            "orc_conv3x3_shuffle2": (None, [FP, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP, FP]),
            "orc_conv1x1": (None, [FP, C.c_int, C.c_long, FP, C.c_int, FP, FP]),
            "orc_linear": (None, [FP, C.c_long, C.c_int, FP, C.c_int, FP, FP]),
            "orc_pixel_shuffle2": (None, [FP, C.c_int, C.c_int, C.c_int, FP]),
            "orc_pixel_shuffle": (None, [FP, C.c_int, C.c_int, C.c_int, C.c_int, FP]),
            "orc_bicubic_resize": (None, [FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP]),
            "orc_upsample2x_nearest": (None, [FP, C.c_int, C.c_int, C.c_int, FP]),
            "orc_leaky_relu": (None, [FP, C.c_long, C.c_float]),
            "orc_add_into": (None, [FP, FP, C.c_long]),
            "orc_channel_layer_norm": (None, [FP, FP, FP, FP, C.c_int, C.c_long, C.c_float]),
            "orc_fast_exp": (C.c_float, [C.c_float]),
            "orc_gelu_erf_inplace": (None, [FP, C.c_long]),
            "orc_gather": (None, [P, FP, C.c_int, FP]),
            "orc_scatter": (None, [P, FP, C.c_int, FP]),
            "orc_attention": (None, [P, C.c_int, C.c_int, FP, FP, FP, C.c_int, FP]),
            "orc_cpb_table": (None, [C.c_int, C.c_int, FP, FP, FP, FP]),
            "orc_to_rgb8": (None, [FP, C.c_long, C.POINTER(C.c_uint8)]),
            # arch / tensor-table arguments are the ABI's structs (swin2sr_rs_amd.abi)
            "orc_rstb": (C.c_int, None),
            "orc_forward": (C.c_int, None),
            "orc_last_error": (C.c_char_p, []),
            "orc_threads": (C.c_int, []),
            "orc_set_threads": (None, [C.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            if args is not None:
                f.argtypes = args
        _lib = L
    return _lib


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def ptr(a):
    return None if a is None else a.ctypes.data_as(FP)


def plan_new(h, w, win, c) -> Plan:
    p = Plan()
    lib().orc_plan_new(h, w, win, c, C.byref(p))
    return p


def plan_explicit(hp, wp, win, c) -> Plan:
    p = Plan()
    lib().orc_plan_explicit(hp, wp, win, c, C.byref(p))
    return p


def shift_for(p: Plan, b: int) -> int:
    return lib().orc_shift_for(C.byref(p), b)


def window_map(p: Plan, shift: int):
    n = p.nw * p.n
    yx = np.empty((n, 2), np.int32)
    reg = np.empty((n, 2), np.uint8)
    lib().orc_window_map(C.byref(p), shift, yx.ctypes.data_as(C.POINTER(C.c_int32)),
                         reg.ctypes.data_as(C.POINTER(C.c_uint8)))
    return yx, reg


def region_of(a, length, win, shift):
    return lib().orc_region_of(a, length, win, shift)


def pad_reflect(x, hp, wp):
    x = f32(x)
    c, h, w = x.shape
    out = np.empty((c, hp, wp), np.float32)
    lib().orc_pad_reflect(ptr(x), c, h, w, hp, wp, ptr(out))
    return out


def conv3x3(x, wgt, bias):
    x, wgt, bias = f32(x), f32(wgt), f32(bias)
    cin, h, w = x.shape
    cout = wgt.shape[0]
    out = np.empty((cout, h, w), np.float32)
    lib().orc_conv3x3(ptr(x), cin, h, w, ptr(wgt), cout, ptr(bias), ptr(out))
    return out


def conv3x3_shuffle2(x, wgt, bias):
    x, wgt, bias = f32(x), f32(wgt), f32(bias)
    cin, h, w = x.shape
    feat = wgt.shape[0] // 4
    out = np.empty((feat, 2 * h, 2 * w), np.float32)
    lib().orc_conv3x3_shuffle2(ptr(x), cin, h, w, ptr(wgt), feat, ptr(bias), ptr(out))
    return out


def conv1x1(x, wgt, bias):
    x, wgt, bias = f32(x), f32(wgt.reshape(wgt.shape[0], -1)), f32(bias)
    cin, h, w = x.shape
    cout = wgt.shape[0]
    out = np.empty((cout, h, w), np.float32)
    lib().orc_conv1x1(ptr(x), cin, h * w, ptr(wgt), cout, ptr(bias), ptr(out))
    return out


def linear(x, wgt, bias):
    x, wgt, bias = f32(x), f32(wgt), f32(bias)
    rows, cin = x.shape
    cout = wgt.shape[0]
    out = np.empty((rows, cout), np.float32)
    lib().orc_linear(ptr(x), rows, cin, ptr(wgt), cout, ptr(bias), ptr(out))
    return out


def pixel_shuffle2(x):
    x = f32(x)
    c4, h, w = x.shape
    out = np.empty((c4 // 4, 2 * h, 2 * w), np.float32)
    lib().orc_pixel_shuffle2(ptr(x), c4, h, w, ptr(out))
    return out


def pixel_shuffle(x, scale):
    x = f32(x)
    cs, h, w = x.shape
    c = cs // (scale * scale)
    out = np.empty((c, h * scale, w * scale), np.float32)
    lib().orc_pixel_shuffle(ptr(x), c, h, w, scale, ptr(out))
    return out


def bicubic_resize(x, oh, ow):
    x = f32(x)
    c, h, w = x.shape
    out = np.empty((c, oh, ow), np.float32)
    lib().orc_bicubic_resize(ptr(x), c, h, w, oh, ow, ptr(out))
    return out


def upsample2x_nearest(x):
    x = f32(x)
    c, h, w = x.shape
    out = np.empty((c, 2 * h, 2 * w), np.float32)
    lib().orc_upsample2x_nearest(ptr(x), c, h, w, ptr(out))
    return out


def channel_layer_norm(x, w, b, eps=1e-5):
    x = f32(x)
    c = x.shape[0]
    hw = x.size // c
    out = np.empty_like(x)
    lib().orc_channel_layer_norm(ptr(x), ptr(f32(w)), ptr(f32(b)), ptr(out), c, hw, eps)
    return out


def fast_exp(x: float) -> float:
    return lib().orc_fast_exp(float(x))


def gelu(x):
    y = f32(x).copy()
    lib().orc_gelu_erf_inplace(ptr(y), y.size)
    return y


def gather(p: Plan, x, shift):
    x = f32(x)
    tok = np.empty((p.nw * p.n, p.c), np.float32)
    lib().orc_gather(C.byref(p), ptr(x), shift, ptr(tok))
    return tok


def scatter(p: Plan, tok, shift):
    tok = f32(tok)
    x = np.empty((p.c, p.hp, p.wp), np.float32)
    lib().orc_scatter(C.byref(p), ptr(tok), shift, ptr(x))
    return x


def attention(p: Plan, heads, head_dim, logit_scale, cpb, qkv, shift):
    qkv = f32(qkv)
    out = np.empty((p.nw * p.n, p.c), np.float32)
    lib().orc_attention(C.byref(p), heads, head_dim, ptr(f32(logit_scale).reshape(-1)),
                        ptr(f32(cpb)), ptr(qkv), shift, ptr(out))
    return out


def cpb_table(win, heads, w0, b0, w2):
    out = np.empty((win ** 4, heads), np.float32)
    lib().orc_cpb_table(win, heads, ptr(f32(w0)), ptr(f32(b0)), ptr(f32(w2)), ptr(out))
    return out


def to_rgb8(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().orc_to_rgb8(ptr(x), x.size, out.ctypes.data_as(C.POINTER(C.c_uint8)))
    return out


def _arch_and_tables(arch, weights):
    import importlib
    abi = importlib.import_module("swin2sr_rs_amd.abi")
    a = abi.arch_struct(arch)
    tabs, keep = abi.tensor_table(weights)
    return a, tabs, keep


def forward(arch, weights: Dict[str, np.ndarray], h, w, in_adjusted):
    """Whole-image forward (reference cpu::forward + head + finish)."""
    a, tabs, keep = _arch_and_tables(arch, weights)
    x = f32(in_adjusted)
    s = arch.scale
    out = np.empty((3, h * s, w * s), np.float32)
    win = arch.window
    hp, wp = (h // win + 1) * win, (w // win + 1) * win
    aux = np.empty((3, hp, wp), np.float32) if arch.upsampler == "pixelshuffle_aux" else None
    rc = lib().orc_forward(C.byref(a), tabs, C.c_size_t(len(weights)), C.c_int(h), C.c_int(w),
                           ptr(x), ptr(out), ptr(aux))
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    del keep
    return out, aux


def rstb(arch, weights, p: Plan, stage, x_nchw):
    """One RSTB stage on an explicit plan, NCHW in/out (config-1 reference)."""
    a, tabs, keep = _arch_and_tables(arch, weights)
    x = f32(x_nchw).copy()
    rc = lib().orc_rstb(C.byref(a), tabs, C.c_size_t(len(weights)), C.byref(p), C.c_int(stage),
                        ptr(x))
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())
    del keep
    return x
