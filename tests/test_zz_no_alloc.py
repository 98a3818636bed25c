"""The allocation-free forward (s2s_forward_device_noalloc) against the
allocating one (s2s_forward_device) through the C ABI: the same kernels on a
static per-GPU workspace, so the outputs must agree bit for bit - on two calls
in a row, the second on a smaller image (the workspace keeps the first call's
contents), for every head (the compressed model's aux planes, the x2 composed
octave, pixelshuffledirect, nearest+conv) and the lightweight width. A
plane past the workspace is refused with an error and the context still runs."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(pkg, be, arch, h, w, seed):
    M, hip = pkg.model, pkg.hip
    s = arch.scale
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=seed)))
    din = hip.DeviceBuffer.from_array(x)
    want_buf = hip.DeviceBuffer(3 * h * s * w * s)
    got_buf = hip.DeviceBuffer(3 * h * s * w * s)
    be.forward_device(h, w, din.ptr, want_buf.ptr)
    be.forward_device_noalloc(h, w, din.ptr, got_buf.ptr)
    hip.stream_synchronize(be.stream())
    want = want_buf.download((3, h * s, w * s))
    got = got_buf.download((3, h * s, w * s))
    for b in (din, want_buf, got_buf):
        b.free()
    return got, want


@pytest.mark.parametrize("which", ["classical-x4", "compressed-x4", "classical-x2", "lightweight-x2",
                                   "realworld-x4"])
def test_noalloc_forward_matches_the_allocating_one(pkg, which):
    M = pkg.model
    sizes = [(120, 96, 1), (40, 56, 2)]
    if which == "classical-x4":
        arch = M.classical(4)
    elif which == "compressed-x4":
        arch = M.Arch(upsampler="pixelshuffle_aux", scale=4, embed=180, heads=6, depths=[2, 2])
    elif which == "classical-x2":
        arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=180, heads=6, depths=[2, 2])
    elif which == "lightweight-x2":
        arch = M.lightweight(2)
    else:
        # the nearest+conv head's planes are 16 times the body's: smaller images
        arch = M.Arch(upsampler="nearest+conv", scale=4, embed=180, heads=6, depths=[2, 2])
        sizes = [(64, 72, 1), (40, 56, 2)]
    be = pkg.HipBackend(arch, M.make_weights(arch, seed=7, perturb=True))
    try:
        for h, w, seed in sizes:
            got, want = _pair(pkg, be, arch, h, w, seed)
            assert np.isfinite(got).all()
            assert np.array_equal(got, want), (h, w)
    finally:
        be.close()


def test_noalloc_refuses_a_plane_past_the_workspace(pkg):
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    be = pkg.HipBackend(arch, M.make_weights(arch, seed=1))
    try:
        h = w = 256
        din = hip.DeviceBuffer(3 * h * w)
        dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
        with pytest.raises(pkg.abi.S2SError, match="bytes of workspace, above this entry's maximum"):
            be.forward_device_noalloc(h, w, din.ptr, dout.ptr)
        din.free()
        dout.free()
        got, want = _pair(pkg, be, arch, 64, 64, 3)
        assert np.array_equal(got, want)
    finally:
        be.close()


def test_noalloc_between_graph_replays(pkg):
    """The allocation-free entry carves its buffers out of the workspace for
    the call and puts the context's own plan back, so a graph the context
    captured before the call replays unchanged after it (and the entry itself
    launches eagerly, never into that graph)."""
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    be = pkg.HipBackend(arch, M.make_weights(arch, seed=4, perturb=True))
    h, w = 40, 56
    shape = (3, h * 4, w * 4)
    xs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=s))) for s in (4, 5, 6)]
    din = hip.DeviceBuffer(3 * h * w)
    dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
    dna = hip.DeviceBuffer(3 * h * 4 * w * 4)
    try:
        want = [be.forward(h, w, x) for x in xs]  # the host path: other buffers
        din.upload(xs[0])
        for _ in range(3):  # eager, captured and launched, replayed
            be.forward_device(h, w, din.ptr, dout.ptr)
        hip.stream_synchronize(be.stream())
        assert np.array_equal(dout.download(shape), want[0])
        for i in (1, 2):
            din.upload(xs[i])
            be.forward_device_noalloc(h, w, din.ptr, dna.ptr)
            be.forward_device(h, w, din.ptr, dout.ptr)  # a replay
            hip.stream_synchronize(be.stream())
            assert np.array_equal(dna.download(shape), want[i]), i
            assert np.array_equal(dout.download(shape), want[i]), i
    finally:
        for b in (din, dout, dna):
            b.free()
        be.close()


def test_noalloc_contexts_on_two_streams_take_turns(pkg):
    """Two contexts (two streams) calling the allocation-free entry back to
    back with no synchronisation between the calls share the GPU's one
    workspace; the library orders them on the device (each call waits for the
    workspace's previous user), so every output equals the same call run on
    its own, bit for bit."""
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    bes = [pkg.HipBackend(arch, M.make_weights(arch, seed=s, perturb=True)) for s in (21, 22)]
    h, w = 120, 96
    n_out = 3 * h * 4 * w * 4
    xs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=s))) for s in (31, 32, 33)]
    dins = [hip.DeviceBuffer.from_array(x) for x in xs]
    # (context, input) per call, interleaved between the two contexts
    calls = [(0, 0), (1, 1), (0, 2), (1, 0), (0, 1), (1, 2)]
    outs = [hip.DeviceBuffer(n_out) for _ in calls]
    try:
        want = {}
        for b, i in set(calls):  # each call on its own, synchronised
            d = hip.DeviceBuffer(n_out)
            bes[b].forward_device_noalloc(h, w, dins[i].ptr, d.ptr)
            hip.stream_synchronize(bes[b].stream())
            want[(b, i)] = d.download((3, h * 4, w * 4))
            d.free()
        for (b, i), o in zip(calls, outs):
            bes[b].forward_device_noalloc(h, w, dins[i].ptr, o.ptr)
        for be in bes:
            hip.stream_synchronize(be.stream())
        for k, ((b, i), o) in enumerate(zip(calls, outs)):
            got = o.download((3, h * 4, w * 4))
            assert np.array_equal(got, want[(b, i)]), (k, b, i, float(np.abs(got - want[(b, i)]).max()))
    finally:
        for buf in dins + outs:
            buf.free()
        for be in bes:
            be.close()
