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
