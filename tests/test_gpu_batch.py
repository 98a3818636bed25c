"""The batched device entry (s2s_forward_device_batch): n images of one size
alternating between the context's stream and its second lane (a stream, buffer
plans and graphs of its own over the same weights), against the same images
forwarded one by one on a plain context, bit for bit - over repeated calls
(each lane capturing and replaying its graphs), odd and even batch sizes, a
size change between batches, and single-image calls on the same context in
between. The reference forwards one image at a time (src/backend.rs:29-49);
equality with the single-image path, whose parity with the oracle the other
GPU tests establish, is the bar."""
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
