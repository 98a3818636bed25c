"""The device forward's HIP-graph replay (s2s_forward_device called again with
the same image size, pointers and buffer plan) against the same forward
launched kernel by kernel, through the C ABI.

The second identical call in a row captures the launches and the calls after
it replay the graph, so every replay here gets a fresh input written into the
same device buffer, with the program's own eager work (copies, other
forwards, synchronisations) between replays, and each output must equal the
eager context's output for that input bit for bit (the same kernels in the
same order). The reference has no graph path: its CUDA backend launches
kernel by kernel (src/gpu.rs:462-583); equality with the eager launches, whose
parity with the oracle the other GPU tests establish, is the bar.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def make_backend(pkg, arch, wts, graphs):
    old = os.environ.get("SWIN2SR_HIP_GRAPHS")
    os.environ["SWIN2SR_HIP_GRAPHS"] = "1" if graphs else "0"
    try:
        return pkg.HipBackend(arch, wts)
    finally:
        if old is None:
            del os.environ["SWIN2SR_HIP_GRAPHS"]
        else:
            os.environ["SWIN2SR_HIP_GRAPHS"] = old


def test_graph_replays_match_eager_launches(pkg, orc):
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=5, perturb=True)
    h, w = 24, 40
    h2, w2 = 16, 24
    inputs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=s))) for s in range(6)]
    other = M.adjust(arch, M.to_unit(M.input_sinusoids(h2, w2, seed=9)))
    eager = make_backend(pkg, arch, wts, graphs=False)
    graph = make_backend(pkg, arch, wts, graphs=True)
    try:
        want = [eager.forward(h, w, x) for x in inputs]
        want_other = eager.forward(h2, w2, other)
        din = hip.DeviceBuffer(3 * h * w)
        dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
        din2 = hip.DeviceBuffer.from_array(other)
        dout2 = hip.DeviceBuffer(3 * h2 * 4 * w2 * 4)

        def run(i):
            din.upload(inputs[i])
            graph.forward_device(h, w, din.ptr, dout.ptr)
            hip.stream_synchronize(graph.stream())
            got = dout.download((3, h * 4, w * 4))
            assert np.array_equal(got, want[i]), (i, float(np.abs(got - want[i]).max()))

        # eager (first sight), captured + launched, then replays
        for i in (0, 1, 2, 3):
            run(i)
        # a host-path forward of the same size in between: other buffers, eager
        assert np.array_equal(graph.forward(h, w, inputs[4]), want[4])
        run(5)
        run(0)
        # another image size re-plans the buffers (the graph is dropped); back
        # at the first size: eager, captured, replayed again
        graph.forward_device(h2, w2, din2.ptr, dout2.ptr)
        hip.stream_synchronize(graph.stream())
        assert np.array_equal(dout2.download((3, h2 * 4, w2 * 4)), want_other)
        for i in (1, 2, 3, 4):
            run(i)
    finally:
        graph.close()
        eager.close()
    # and the eager context itself against the oracle on one of the inputs
    ref, _ = orc.forward(arch, wts, h, w, inputs[2])
    assert float(np.abs(want[2] - ref).max()) <= 1e-4


def test_caller_capture_records_the_launches(pkg):
    """A caller that captures the context's stream (s2s_stream) into a graph of
    its own gets the forward's launches in it, not the library's graph: its
    graph, replayed on new inputs, equals the eager context bit for bit."""
    import ctypes as C

    M, hip = pkg.model, pkg.hip
    h_ = hip.rt()
    vp = C.c_void_p
    for name, args in {"hipStreamBeginCapture": [vp, C.c_int], "hipStreamEndCapture": [vp, C.POINTER(vp)],
                       "hipGraphInstantiate": [C.POINTER(vp), vp, vp, vp, C.c_size_t],
                       "hipGraphLaunch": [vp, vp], "hipGraphExecDestroy": [vp],
                       "hipGraphDestroy": [vp]}.items():
        getattr(h_, name).argtypes = args
        getattr(h_, name).restype = C.c_int
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=6, perturb=True)
    h, w = 16, 24
    inputs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=s))) for s in range(3)]
    eager = make_backend(pkg, arch, wts, graphs=False)
    graph = make_backend(pkg, arch, wts, graphs=True)
    g = vp()
    ge = vp()
    try:
        want = [eager.forward(h, w, x) for x in inputs]
        din = hip.DeviceBuffer(3 * h * w)
        dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
        st = vp(graph.stream())
        # the same call twice first: the library has captured a graph of its own
        din.upload(inputs[0])
        for _ in range(2):
            graph.forward_device(h, w, din.ptr, dout.ptr)
        hip.stream_synchronize(graph.stream())
        assert np.array_equal(dout.download((3, h * 4, w * 4)), want[0])
        # now the caller captures the stream (relaxed mode) around the same call
        assert h_.hipStreamBeginCapture(st, 2) == 0
        graph.forward_device(h, w, din.ptr, dout.ptr)
        assert h_.hipStreamEndCapture(st, C.byref(g)) == 0
        assert h_.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
        for i in (1, 2, 0):
            din.upload(inputs[i])
            assert h_.hipGraphLaunch(ge, st) == 0
            hip.stream_synchronize(graph.stream())
            got = dout.download((3, h * 4, w * 4))
            assert np.array_equal(got, want[i]), (i, float(np.abs(got - want[i]).max()))
    finally:
        if ge.value:
            h_.hipGraphExecDestroy(ge)
        if g.value:
            h_.hipGraphDestroy(g)
        graph.close()
        eager.close()


@pytest.mark.parametrize("name", ["lightweight", "realworld", "compressed"])
def test_graph_replays_other_models(pkg, name):
    """The released models' other shapes (lightweight: 6 heads of 10, the
    two-kernel attention on packed K = 60 weights, pixelshuffledirect;
    real-world: nearest+conv; compressed: the aux head) replay bit-exact too."""
    M, hip = pkg.model, pkg.hip
    arch = {"lightweight": M.lightweight(2), "realworld": M.realworld(), "compressed": M.compressed()}[name]
    wts = M.make_weights(arch, seed=7, perturb=True)
    h, w = 16, 24
    s = arch.scale
    inputs = [M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=sd))) for sd in range(4)]
    eager = make_backend(pkg, arch, wts, graphs=False)
    graph = make_backend(pkg, arch, wts, graphs=True)
    try:
        want = [eager.forward(h, w, x) for x in inputs]
        din = hip.DeviceBuffer(3 * h * w)
        dout = hip.DeviceBuffer(3 * h * s * w * s)
        for i in (0, 1, 2, 3, 0):  # eager, captured + launched, replays
            din.upload(inputs[i])
            graph.forward_device(h, w, din.ptr, dout.ptr)
            hip.stream_synchronize(graph.stream())
            got = dout.download((3, h * s, w * s))
            assert np.array_equal(got, want[i]), (name, i, float(np.abs(got - want[i]).max()))
    finally:
        graph.close()
        eager.close()


def _async_copy(hip, stream, dst, src, nbytes):
    """A device-to-device copy ordered on `stream` (hipMemcpyAsync)."""
    import ctypes as C

    h_ = hip.rt()
    h_.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    h_.hipMemcpyAsync.restype = C.c_int
    assert h_.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), nbytes, hip.D2D, C.c_void_p(stream)) == 0


def test_graph_replaced_while_a_replay_is_in_flight(pkg):
    """Calls A, A, A, B, B, A and then six calls' pairs each twice (input/output
    pairs of one size) enqueued with no synchronisation between them: the
    context keeps four graphs, so captures past the fourth evict the least
    recently used one while replays are still queued. Each call's output,
    snapshotted by a copy ordered on the stream right after it, equals the
    eager context's bit for bit."""
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=8, perturb=True)
    h, w = 40, 56
    n_out = 3 * h * 4 * w * 4
    xa = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=11)))
    xb = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=12)))
    eager = make_backend(pkg, arch, wts, graphs=False)
    graph = make_backend(pkg, arch, wts, graphs=True)
    bufs = []
    try:
        want = {"A": eager.forward(h, w, xa), "B": eager.forward(h, w, xb)}
        pairs = {"A": (hip.DeviceBuffer.from_array(xa), hip.DeviceBuffer(n_out)),
                 "B": (hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer(n_out))}
        for i, k in enumerate("CDEFGH"):
            xk = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=13 + i)))
            want[k] = eager.forward(h, w, xk)
            pairs[k] = (hip.DeviceBuffer.from_array(xk), hip.DeviceBuffer(n_out))
        bufs = [b for p in pairs.values() for b in p]
        seq = ["A", "A", "A", "B", "B", "A"] + [k for k in "CDEFGH" for _ in range(2)] + ["A", "H", "A", "A"]
        snaps = [hip.DeviceBuffer(n_out) for _ in seq]
        bufs += snaps
        st = graph.stream()
        for k, snap in zip(seq, snaps):
            din, dout = pairs[k]
            graph.forward_device(h, w, din.ptr, dout.ptr)
            _async_copy(hip, st, snap.ptr, dout.ptr, n_out * 4)
        hip.stream_synchronize(st)
        for i, (k, snap) in enumerate(zip(seq, snaps)):
            got = snap.download((3, h * 4, w * 4))
            assert np.array_equal(got, want[k]), (i, k, float(np.abs(got - want[k]).max()))
    finally:
        for b in bufs:
            b.free()
        graph.close()
        eager.close()


def test_capture_around_a_new_size_is_refused(pkg):
    """A caller capturing the context's stream around a call whose image size
    needs a new buffer plan gets an error naming the cause (planning would
    allocate and synchronise the captured stream); its capture ends cleanly,
    and the context still runs both sizes afterwards, bit-exact against an
    eager context."""
    import ctypes as C

    M, hip = pkg.model, pkg.hip
    h_ = hip.rt()
    vp = C.c_void_p
    for name, args in {"hipStreamBeginCapture": [vp, C.c_int], "hipStreamEndCapture": [vp, C.POINTER(vp)],
                       "hipGraphDestroy": [vp]}.items():
        getattr(h_, name).argtypes = args
        getattr(h_, name).restype = C.c_int
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=9, perturb=True)
    (h, w), (h2, w2) = (16, 24), (24, 40)
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=1)))
    x2 = M.adjust(arch, M.to_unit(M.input_sinusoids(h2, w2, seed=2)))
    eager = make_backend(pkg, arch, wts, graphs=False)
    graph = make_backend(pkg, arch, wts, graphs=True)
    g = vp()
    try:
        want, want2 = eager.forward(h, w, x), eager.forward(h2, w2, x2)
        din, dout = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer(3 * h * 4 * w * 4)
        din2, dout2 = hip.DeviceBuffer.from_array(x2), hip.DeviceBuffer(3 * h2 * 4 * w2 * 4)
        graph.forward_device(h, w, din.ptr, dout.ptr)
        hip.stream_synchronize(graph.stream())
        st = vp(graph.stream())
        assert h_.hipStreamBeginCapture(st, 2) == 0
        with pytest.raises(pkg.abi.S2SError, match="needs a new buffer plan"):
            graph.forward_device(h2, w2, din2.ptr, dout2.ptr)
        assert h_.hipStreamEndCapture(st, C.byref(g)) == 0
        for _ in range(3):  # eager, captured + launched, replayed
            graph.forward_device(h, w, din.ptr, dout.ptr)
            hip.stream_synchronize(graph.stream())
            assert np.array_equal(dout.download((3, h * 4, w * 4)), want)
        graph.forward_device(h2, w2, din2.ptr, dout2.ptr)
        hip.stream_synchronize(graph.stream())
        assert np.array_equal(dout2.download((3, h2 * 4, w2 * 4)), want2)
        for b in (din, dout, din2, dout2):
            b.free()
    finally:
        if g.value:
            h_.hipGraphDestroy(g)
        graph.close()
        eager.close()


def test_many_replays_and_batches_are_identical(pkg):
    """Determinism under repetition: classical x4 at 64 x 64, 200 graph replays
    and 100 two-lane batches of the same input, every output equal to the
    first eager forward's bit for bit (the kernels have no atomics and a fixed
    reduction order, so any difference would be a race or a hardware fault)."""
    M, hip = pkg.model, pkg.hip
    arch = M.classical(4)
    wts = M.make_weights(arch, seed=91, perturb=True)
    h = w = 64
    x = M.adjust(arch, M.to_unit(M.input_sinusoids(h, w, seed=91)))
    shape = (3, h * 4, w * 4)
    be = make_backend(pkg, arch, wts, graphs=True)
    bufs = []
    try:
        din = hip.DeviceBuffer.from_array(x)
        dout = hip.DeviceBuffer(3 * h * 4 * w * 4)
        d2 = [hip.DeviceBuffer(3 * h * 4 * w * 4) for _ in range(2)]
        bufs += [din, dout] + d2
        be.forward_device(h, w, din.ptr, dout.ptr)
        hip.stream_synchronize(be.stream())
        want = dout.download(shape)
        st = be.stream()
        for rep in range(200):
            be.forward_device(h, w, din.ptr, dout.ptr)
            if rep % 20 == 19:
                hip.stream_synchronize(st)
                assert np.array_equal(dout.download(shape), want), rep
        for rep in range(100):
            be.forward_device_batch(h, w, [din.ptr, din.ptr], [d.ptr for d in d2])
            if rep % 10 == 9:
                hip.stream_synchronize(st)
                for k, d in enumerate(d2):
                    assert np.array_equal(d.download(shape), want), (rep, k)
    finally:
        for b in bufs:
            b.free()
        be.close()
