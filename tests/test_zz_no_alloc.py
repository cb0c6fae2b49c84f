"""qasr_hip_argmax_int8_noalloc (no counterpart in the reference): the LM-head
argmax for callers that cannot allocate, its block partials in a static
device array.  Through the C ABI it must return the index the handle-based
entry point returns (qasr_hip_argmax_int8 / qasr_hip_rmsnorm_argmax_int8, its
partials in the handle's scratch), on two calls in a row with the second
smaller (the array keeps the first call's partials), and reject what it
cannot hold before launching anything."""
import ctypes as C

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def both(dev, x, norm_w, w, ws, K, N):
    from qwenasr_amd import kernels as K_
    from qwenasr_amd._lib import check, lib
    dx, dw, dws = dev.upload(x), dev.upload(w), dev.upload(ws)
    dn = dev.upload(norm_w) if norm_w is not None else None
    ref_out, out = dev.zeros(1, np.int32), dev.zeros(1, np.int32)
    ref = K_.argmax_matvec_int8(dx, dw, dws, K, N, ref_out, norm_w=dn, eps=1e-6)
    stream = lib().qasr_hip_stream(dev.h)
    check(lib().qasr_hip_argmax_int8_noalloc(stream, dx.ptr, dn.ptr if dn is not None else None, C.c_float(1e-6),
                                             dw.ptr, dws.ptr, K, N, out.ptr))
    dev.sync()
    return int(out.numpy().reshape(-1)[0]), ref


@pytest.mark.parametrize("norm", [False, True])
def test_noalloc_argmax_matches_handle_entry_point(dev, orc, norm):
    r = rng(77 + norm)
    for K, N in ((1024, 151936), (512, 5000)):       # the second call is smaller
        print(f"noalloc argmax K={K} N={N} norm={norm}", flush=True)
        w = r.integers(-127, 128, (N, K), dtype=np.int8)
        ws = r.uniform(1e-4, 2e-3, N).astype(np.float32)
        x = r.normal(0, 1, K).astype(np.float32)
        g = r.uniform(0.5, 1.5, K).astype(np.float32) if norm else None
        got, ref = both(dev, x, g, w, ws, K, N)
        assert got == ref, (K, N, got, ref)
        want = orc.argmax_int8(orc.rms_norm(x, g, 1e-6) if norm else x, w, ws)[0]
        assert got == want, (K, N, got, want)


def test_noalloc_argmax_rejects_bad_shapes(dev):
    from qwenasr_amd import QasrError
    from qwenasr_amd._lib import check, lib
    buf = dev.zeros(64, np.float32)
    for K, N in ((4160, 10), (100, 10), (1024, 0)):
        with pytest.raises(QasrError):
            check(lib().qasr_hip_argmax_int8_noalloc(None, buf.ptr, None, C.c_float(0.0), buf.ptr, buf.ptr, K, N,
                                                     buf.ptr))


def test_noalloc_argmax_in_a_captured_graph(dev, orc):
    """The call captured into a HIP graph on the handle's stream (its scratch
    address was resolved when the handle was created, so nothing is loaded or
    allocated during capture) and replayed four times, with new inputs
    uploaded eagerly and a synchronisation between replays: every replay
    returns the index the handle-based entry point returns for that input."""
    from qwenasr_amd import kernels as K_
    from qwenasr_amd._lib import check, lib
    hip = C.CDLL("libamdhip64.so.7")     # the HIP runtime the library already loaded
    K, N = 1024, 151936
    r = rng(91)
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, N).astype(np.float32)
    g = r.uniform(0.5, 1.5, K).astype(np.float32)
    dx, dw, dws, dn = dev.upload(r.normal(0, 1, K).astype(np.float32)), dev.upload(w), dev.upload(ws), dev.upload(g)
    out, ref_out = dev.zeros(1, np.int32), dev.zeros(1, np.int32)
    stream = C.c_void_p(lib().qasr_hip_stream(dev.h))
    graph, exe = C.c_void_p(), C.c_void_p()
    dev.sync()
    print("noalloc argmax: capture", flush=True)
    assert hip.hipStreamBeginCapture(stream, 0) == 0
    rc = lib().qasr_hip_argmax_int8_noalloc(stream, dx.ptr, dn.ptr, C.c_float(1e-6), dw.ptr, dws.ptr, K, N, out.ptr)
    assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
    check(rc)
    assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0
    try:
        for rep in range(4):
            x = r.normal(0, 1, K).astype(np.float32)
            dx.copy_from(x)
            dev.sync()
            assert hip.hipGraphLaunch(exe, stream) == 0
            dev.sync()
            got = int(out.numpy().reshape(-1)[0])
            ref = K_.argmax_matvec_int8(dx, dw, dws, K, N, ref_out, norm_w=dn, eps=1e-6)
            want = orc.argmax_int8(orc.rms_norm(x, g, 1e-6), w, ws)[0]
            print(f"replay {rep}: {got} (handle entry point {ref}, oracle {want})", flush=True)
            assert got == ref == want, (rep, got, ref, want)
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
