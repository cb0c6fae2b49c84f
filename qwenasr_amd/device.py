"""Device handle and device arrays over the qasr_hip C ABI."""
import ctypes as C
import weakref

import numpy as np

from ._lib import P, check, lib


class Device:
    """One qasr_hip handle: a GPU, one HIP stream and a scratch area."""

    def __init__(self, index=0):
        h = P()
        check(lib().qasr_hip_create(index, C.byref(h)))
        self.h = h
        self.index = index
        self._children = weakref.WeakSet()   # decoders / encoders created on this handle

    def adopt(self, obj):
        """Register an object whose close() must run before the handle is destroyed."""
        self._children.add(obj)

    def close(self):
        if self.h:
            # the C ABI requires them freed first; streams before the decoders they borrow
            for c in sorted(self._children, key=lambda o: getattr(o, "_close_first", 1), reverse=True):
                c.close()
            lib().qasr_hip_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        check(lib().qasr_hip_synchronize(self.h))

    def empty(self, shape, dtype):
        return DeviceArray(self, shape, dtype)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        d = DeviceArray(self, arr.shape, arr.dtype)
        d.copy_from(arr)
        return d

    def zeros(self, shape, dtype):
        d = DeviceArray(self, shape, dtype)
        check(lib().qasr_hip_memset(self.h, d.ptr, 0, d.nbytes))
        return d

    def copy(self, dst, src, nbytes=None):
        """Device-to-device copy with the library's copy kernel (asynchronous)."""
        n = src.nbytes if nbytes is None else int(nbytes)
        check(lib().qasr_hip_copy(self.h, dst.ptr, src.ptr, n))

    def timer_hold(self, us):
        """Hold the stream for `us` microseconds, so that launches enqueued
        meanwhile run back to back (see qasr_hip_timer_hold)."""
        check(lib().qasr_hip_timer_hold(self.h, int(us)))

    def timer_start(self):
        check(lib().qasr_hip_timer_start(self.h))

    def timer_stop(self):
        ms = C.c_float()
        check(lib().qasr_hip_timer_stop(self.h, C.byref(ms)))
        return ms.value


def device_count():
    n = C.c_int()
    check(lib().qasr_hip_device_count(C.byref(n)))
    return n.value


class DeviceArray:
    """A contiguous device allocation with a numpy shape/dtype."""

    def __init__(self, dev, shape, dtype):
        self.dev = dev
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = P()
        check(lib().qasr_hip_malloc(dev.h, max(self.nbytes, 1), C.byref(p)))
        self._p = p

    @property
    def ptr(self):
        return self._p

    def offset(self, elems):
        """Raw pointer `elems` elements past the start."""
        return P(self._p.value + int(elems) * self.dtype.itemsize)

    def copy_from(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes == self.nbytes, (arr.shape, self.shape)
        check(lib().qasr_hip_upload(self.dev.h, self._p, arr.ctypes.data_as(P), self.nbytes))

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(lib().qasr_hip_download(self.dev.h, out.ctypes.data_as(P), self._p, self.nbytes))
        return out

    def free(self):
        if self._p and self.dev.h:
            lib().qasr_hip_free(self.dev.h, self._p)
        self._p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
