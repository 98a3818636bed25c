"""The on-disk formats around the device backend (the crate's `--device gpu`
flow, reference src/main.rs:592-760): a converted checkpoint loaded from its
safetensors file drives the HIP backend exactly as the in-memory weights do,
a SW2F fixture written from the CPU oracle verifies through it, and a PNG
goes through the tiled path and back to PNG."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _tiny(M, ups, scale):
    return M.Arch(upsampler=ups, scale=scale, embed=24, heads=2, depths=[2, 1])


@pytest.mark.parametrize("ups,scale", [("pixelshuffle", 4), ("pixelshuffle_aux", 4),
                                       ("nearest+conv", 4), ("pixelshuffledirect", 2)])
def test_checkpoint_file_drives_the_backend(pkg, orc, tmp_path, ups, scale):
    M, F = pkg.model, pkg.formats
    arch = _tiny(M, ups, scale)
    wts = M.make_weights(arch, seed=11, perturb=True)
    path = tmp_path / "m.safetensors"
    F.save_weights(path, arch, wts, task="test_sr")
    wt = F.Weights.load(path)
    h, w = 21, 30
    img = M.to_unit(M.input_sinusoids(h, w, seed=6))
    x = M.adjust(wt.arch(), img)
    be_file = pkg.HipBackend(wt.arch(), wt.tensors())
    be_mem = pkg.HipBackend(arch, wts)
    try:
        a = be_file.forward(h, w, x)
        b = be_mem.forward(h, w, x)
        assert np.array_equal(a, b)
        if ups == "pixelshuffle_aux":
            assert np.array_equal(be_file.aux(), be_mem.aux())
        # an SW2F fixture of the CPU oracle's output verifies through the file
        want, aux = orc.forward(arch, wts, h, w, x)
        fx = F.Fixture(h, w, 3, scale, 8, img, want, aux)
        fpath = tmp_path / "f.bin"
        fx.save(fpath)
        rep = F.verify_fixture(wt, F.Fixture.load(fpath), be_file)
        assert rep["worst"] <= 1e-4, rep
        if aux is not None:
            assert rep["aux_worst"] <= 1e-4, rep
    finally:
        be_file.close()
        be_mem.close()


def test_png_through_the_tiled_path(pkg, tmp_path):
    """PNG in -> run_tiled on the device -> PNG out, against the in-memory
    result of the same tiled run."""
    M, F, T = pkg.model, pkg.formats, pkg.tiling
    arch = _tiny(M, "pixelshuffle", 2)
    wts = M.make_weights(arch, seed=4, perturb=True)
    img8 = M.input_sinusoids(40, 52, seed=2)
    src = tmp_path / "in.png"
    src.write_bytes(F.encode_png(img8.transpose(1, 2, 0)))
    img = F.load_rgb(src)
    # the crate decodes with a multiply by the f32 reciprocal 1/255 (src/image.rs:65-68)
    assert np.array_equal(img, img8.astype(np.float32) * np.float32(1.0 / 255.0))
    be = pkg.HipBackend(arch, wts)
    try:
        out = T.run_tiled(arch, be, img, 16, 8)
        dst = tmp_path / "out.png"
        F.save_rgb(dst, out)
        back = F.load_rgb(dst)
        assert back.shape == (3, 80, 104)
        assert np.array_equal(np.rint(back * 255).astype(np.uint8), M.to_rgb8(out))
    finally:
        be.close()
