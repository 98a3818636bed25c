"""The batched entries. s2s_forward_device_batch: n images of one size
alternating between the context's stream and its second lane (a stream, buffer
plans and graphs of its own over the same weights), against the same images
forwarded one by one on a plain context, bit for bit - over repeated calls
(each lane capturing and replaying its graphs), odd and even batch sizes, a
size change between batches, and single-image calls on the same context in
between. The reference forwards one image at a time (src/backend.rs:29-49);
equality with the single-image path, whose parity with the oracle the other
GPU tests establish, is the bar. s2s_forward_batch (host images of mixed
sizes, a tiled image's crops) and the tile loop over it are held to the same
bar."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(M, arch, h, w, seeds):
    return [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=s))) for s in seeds]


def test_batch_matches_single_forwards(pkg):
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=17, perturb=True)
    single = pkg.HipBackend(arch, wts)
    batch = pkg.HipBackend(arch, wts)
    bufs = []
    try:
        def want_of(h, w, xs):
            return [single.forward(h, w, x) for x in xs]

        def run(h, w, xs):
            s = arch.scale
            dins = [hip.DeviceBuffer.from_array(x) for x in xs]
            douts = [hip.DeviceBuffer(3 * h * s * w * s) for _ in xs]
            bufs.extend(dins + douts)
            return dins, douts

        h, w = 40, 56
        xs = _inputs(M, arch, h, w, range(20, 24))
        want = want_of(h, w, xs)
        dins, douts = run(h, w, xs[:2])
        for rep in range(4):  # eager, captured per lane, replayed; new inputs each time
            for k in range(2):
                dins[k].upload(xs[(rep + k) % 4])
            batch.forward_device_batch(h, w, [d.ptr for d in dins], [d.ptr for d in douts])
            hip.stream_synchronize(batch.stream())
            for k in range(2):
                got = douts[k].download((3, h * 4, w * 4))
                assert np.array_equal(got, want[(rep + k) % 4]), (rep, k)
        # an odd batch, a single-image call on the same context, another size
        d3, o3 = run(h, w, xs[:3])
        batch.forward_device_batch(h, w, [d.ptr for d in d3], [d.ptr for d in o3])
        hip.stream_synchronize(batch.stream())
        for k in range(3):
            assert np.array_equal(o3[k].download((3, h * 4, w * 4)), want[k]), k
        assert np.array_equal(batch.forward(h, w, xs[3]), want[3])
        h2, w2 = 24, 32
        ys = _inputs(M, arch, h2, w2, (40, 41))
        want2 = want_of(h2, w2, ys)
        d2, o2 = run(h2, w2, ys)
        for _ in range(3):
            batch.forward_device_batch(h2, w2, [d.ptr for d in d2], [d.ptr for d in o2])
            hip.stream_synchronize(batch.stream())
            for k in range(2):
                assert np.array_equal(o2[k].download((3, h2 * 4, w2 * 4)), want2[k]), k
        # a batch of one and of none
        batch.forward_device_batch(h2, w2, [d2[1].ptr], [o2[0].ptr])
        batch.forward_device_batch(h2, w2, [], [])
        hip.stream_synchronize(batch.stream())
        assert np.array_equal(o2[0].download((3, h2 * 4, w2 * 4)), want2[1])
    finally:
        for b in bufs:
            b.free()
        batch.close()
        single.close()


def test_batch_waits_for_the_contexts_stream(pkg):
    """The lane starts after the work already queued on the context's stream:
    inputs written by a copy ordered on that stream, enqueued just before the
    batch with no synchronisation, are what the lane's image reads."""
    import ctypes as C

    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=18, perturb=True)
    h, w = 32, 40
    xs = _inputs(M, arch, h, w, (51, 52))
    zero = np.zeros_like(xs[0])
    be = pkg.HipBackend(arch, wts)
    try:
        want = [be.forward(h, w, x) for x in xs]
        src = [hip.DeviceBuffer.from_array(x) for x in xs]
        dins = [hip.DeviceBuffer.from_array(zero) for _ in xs]
        douts = [hip.DeviceBuffer(3 * h * 4 * w * 4) for _ in xs]
        h_ = hip.rt()
        h_.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        h_.hipMemcpyAsync.restype = C.c_int
        st = be.stream()
        for rep in range(3):
            for d in dins:
                d.upload(zero)
            for d, s_ in zip(dins, src):
                assert h_.hipMemcpyAsync(C.c_void_p(d.ptr), C.c_void_p(s_.ptr), xs[0].size * 4, hip.D2D,
                                         C.c_void_p(st)) == 0
            be.forward_device_batch(h, w, [d.ptr for d in dins], [d.ptr for d in douts])
            hip.stream_synchronize(st)
            for k in range(2):
                assert np.array_equal(douts[k].download((3, h * 4, w * 4)), want[k]), (rep, k)
        for b in src + dins + douts:
            b.free()
    finally:
        be.close()


def test_host_batch_matches_single_forwards(pkg):
    """s2s_forward_batch (host images of mixed sizes, pipelined over the two
    lanes) against s2s_forward per image on a plain context, bit for bit: odd
    and even batches, a batch of one and of none, repeated so each lane
    replays its graphs, for the classical, compressed, lightweight and
    real-world heads; with the compressed head, each image's aux image too,
    and s2s_aux afterwards is the last image's."""
    M = pkg.model
    for arch, seed in ((M.classical(4), 61), (M.compressed(), 62), (M.lightweight(2), 65),
                       (M.Arch(upsampler="nearest+conv", scale=4, embed=180, heads=6, depths=[2, 2]), 66)):
        wts = M.make_weights(arch, seed=seed, perturb=True)
        shapes = [(40, 56), (24, 32), (40, 56), (32, 40), (24, 32)]
        xs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=70 + i)))
              for i, (h, w) in enumerate(shapes)]
        single = pkg.HipBackend(arch, wts)
        batch = pkg.HipBackend(arch, wts)
        try:
            want, want_aux = [], []
            for (h, w), x in zip(shapes, xs):
                want.append(single.forward(h, w, x))
                want_aux.append(single.aux())
            aux_head = arch.upsampler == "pixelshuffle_aux"
            assert (want_aux[0] is not None) == aux_head
            for sel in ([0, 1, 2, 3, 4], [1, 3], [2, 0, 4, 1], [3], [], [4, 3, 2, 1, 0]):
                outs, auxs = batch.forward_batch([shapes[i] for i in sel], [xs[i] for i in sel], aux=True)
                assert len(outs) == len(sel)
                for k, i in enumerate(sel):
                    assert np.array_equal(outs[k], want[i]), (arch.upsampler, sel, k)
                    if aux_head:
                        assert np.array_equal(auxs[k].ravel(), want_aux[i]), (sel, k)
                    else:
                        assert auxs[k] is None
                if sel and aux_head:
                    assert np.array_equal(batch.aux(), want_aux[sel[-1]]), sel
            # a single-image call on the same context afterwards
            assert np.array_equal(batch.forward(*shapes[2], xs[2]), want[2])
        finally:
            batch.close()
            single.close()


def test_tiled_image_batched_matches_sequential(pkg):
    """The tile loop with its crops in one batched call gives the image the
    sequential loop gives (compressed head, tiles of 32 with 8 of context on a
    ragged 88x120 image: corner, edge, interior and clipped crops)."""
    M = pkg.model
    arch = M.compressed()
    wts = M.make_weights(arch, seed=63, perturb=True)
    img = M.to_unit(M.input_texture_dct(88, 120, seed=63))
    be = pkg.HipBackend(arch, wts)
    try:
        seq = pkg.tiling.run_tiled(arch, be, img, 32, 8)
        bat = pkg.tiling.run_tiled(arch, be, img, 32, 8, batch=True)
        bat2 = pkg.tiling.run_tiled(arch, be, img, 32, 8, batch=True)
    finally:
        be.close()
    assert seq.shape == (3, 352, 480) and np.isfinite(seq).all()
    assert np.array_equal(bat, seq) and np.array_equal(bat2, seq)


def test_batch_entries_refuse_bad_arguments(pkg):
    """Errors come back through s2s_last_error and leave the context usable:
    an image smaller than a window anywhere in a host batch, null image
    pointers, a negative count; then both entries still run."""
    import ctypes as C

    M = pkg.model
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=64, perturb=True)
    be = pkg.HipBackend(arch, wts)
    try:
        x = M.adjust(arch, M.to_unit(M.input_sinusoids(24, 32, seed=64)))
        want = be.forward(24, 32, x)
        small = np.zeros((3, 4, 32), np.float32)
        with pytest.raises(pkg.abi.S2SError, match="s2s_forward_batch"):
            be.forward_batch([(24, 32), (4, 32)], [x, small])
        lib, ctx = be._lib, be._ctx
        hs = (C.c_int * 1)(24)
        ws = (C.c_int * 1)(32)
        nul = (C.c_void_p * 1)(None)
        assert lib.s2s_forward_batch(ctx, 1, hs, ws, nul, nul, None) != 0
        assert "null" in pkg.abi.last_error()
        assert lib.s2s_forward_batch(ctx, -1, hs, ws, nul, nul, None) != 0
        assert lib.s2s_forward_device_batch(ctx, -1, 24, 32, nul, nul) != 0
        outs = be.forward_batch([(24, 32), (24, 32)], [x, x])
        assert all(np.array_equal(o, want) for o in outs)
        assert np.array_equal(be.forward(24, 32, x), want)
    finally:
        be.close()
