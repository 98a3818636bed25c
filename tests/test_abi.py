"""The C ABI library, without a GPU: it loads, exports every symbol the header
declares, and its host-only paths behave (name, error slot, weight-set
validation messages). No kernel is launched here."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "swin2sr_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s2s_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("s2s_create", "s2s_forward", "s2s_aux", "s2s_destroy", "s2s_last_error",
              "s2s_device_info", "s2s_vram", "s2s_sync", "s2s_profile_report",
              "s2s_uploaded_bytes", "s2s_test_attention", "s2s_test_window_map"):
        assert s in syms


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_name_and_error_slot(pkg):
    lib = pkg.load_library()
    assert lib.s2s_name() == b"hip"
    assert isinstance(lib.s2s_last_error(), bytes)


def test_synthetic_checkpoint_has_the_crate_tensor_set(pkg):
    """The shapes `Weights::validate` checks (reference src/weights.rs:142-235)."""
    M = pkg.model
    for arch in (M.classical(4), M.classical(2), M.lightweight(2), M.realworld(), M.compressed()):
        w = M.make_weights(arch, seed=0)
        C_, F = arch.embed, arch.feat
        assert w["conv_first.weight"].shape == (C_, 3, 3, 3)
        assert w["conv_after_body.weight"].shape == (C_, C_, 3, 3)
        assert w["patch_embed.proj.weight"].shape == (C_, C_, 1, 1)
        for s, d in enumerate(arch.depths):
            for b in range(d):
                p = f"layers.{s}.residual_group.blocks.{b}."
                assert w[p + "attn.qkv.wq"].shape == (C_, C_)
                assert w[p + "mlp.fc1.weight"].shape == (arch.mlp_ratio * C_, C_)
                assert w[p + "attn.cpb_pre"].shape == (arch.window ** 4, arch.heads)
                assert w[p + "attn.logit_scale"].shape == (arch.heads, 1, 1)
        if arch.upsampler != "pixelshuffledirect":
            assert w["conv_last.bias"].shape == (3,)
        else:
            assert w["upsample.0.weight"].shape == (3 * arch.scale ** 2, C_, 3, 3)
        if arch.upsampler == "pixelshuffle_aux":
            assert w["conv_aux.weight"].shape == (3, F, 3, 3)
        assert all(v.dtype == np.float32 for v in w.values())


def test_benchmark_init_rules(pkg):
    M = pkg.model
    arch = M.classical(4)
    w = M.make_weights(arch, seed=3)
    assert np.all(w["layers.0.residual_group.blocks.0.attn.logit_scale"] == np.float32(np.log(10)))
    assert np.all(w["layers.0.residual_group.blocks.0.attn.qkv.q_bias"] == 0)
    assert np.all(w["norm.weight"] == 1) and np.all(w["norm.bias"] == 0)
    s = w["layers.0.residual_group.blocks.0.mlp.fc1.weight"].std()
    assert 0.018 < s < 0.022
    bound = 1 / np.sqrt(180 * 9)
    assert np.abs(w["layers.0.conv.weight"]).max() <= bound


def _rust_externs(text):
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    return re.findall(r"pub fn (s2s_[a-z0-9_]+)\(", block)


def _rust_struct(text, name):
    body = re.search(r"pub struct %s \{(.*?)\n\}" % name, text, re.S).group(1)
    return re.findall(r"pub (\w+): ([^,\n]+),", body)


def _c_struct(text, name):
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.match(r"(.+?)\s*(\*?)\s*(\w+)(\[[^\]]+\])?$", decl)
        fields.append((m.group(3), (m.group(1) + m.group(2)).replace(" ", ""), m.group(4)))
    return fields


def test_rust_ffi_matches_the_header(pkg):
    """The Rust binding a maintainer adds (swin2sr-rs_amd/rust/src/hip.rs) cannot be
    compiled in this image: hold it against the header instead - every function it
    declares is declared in include/swin2sr_hip.h and exported by the library, and
    its #[repr(C)] structs have the C structs' fields in the same order and types."""
    rs = (ROOT / "swin2sr-rs_amd" / "rust" / "src" / "hip.rs").read_text()
    lib = pkg.load_library()
    syms = declared_symbols()
    fns = _rust_externs(rs)
    assert len(fns) >= 15
    for f in fns:
        assert f in syms and hasattr(lib, f), f
    ctype = {"int": "c_int", "float": "f32", "constchar*": "*const c_char",
             "constfloat*": "*const f32", "int64_t": "i64"}
    h = HEADER.read_text()
    for rname, cname in (("S2sArch", "s2s_arch"), ("S2sTensor", "s2s_tensor")):
        r = _rust_struct(rs, rname)
        c = _c_struct(h, cname)
        assert [n for n, _ in r] == [n for n, _, _ in c], (rname, r, c)
        for (rn, rt), (cn, ct, arr) in zip(r, c):
            want = ctype[ct]
            if arr:
                n = arr.strip("[]").replace("S2S_MAX_STAGES", "16")
                want = f"[{want}; {n}]"
            assert rt.strip() == want, (rn, rt, want)
