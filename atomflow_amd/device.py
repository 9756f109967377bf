"""Device memory, streams, events and graphs through libatomflow_kv.so's af_rt_* ABI.

Used by the tests and the benchmark so that no second GPU runtime (e.g. torch's
bundled one) is loaded into the process.
"""
import ctypes

import numpy as np

from . import check, lib


def device_count():
    n = ctypes.c_int(0)
    st = lib().af_rt_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


def set_device(index):
    check(lib().af_rt_set_device(index), "af_rt_set_device")


def add_i32(ptr, n, delta, stream=None):
    check(lib().af_rt_add_i32(ptr, n, delta, _s(stream)), "af_rt_add_i32")


def read_probe(ptr, nbytes, workgroups, sink_ptr, segment_bytes=0, row_bytes=0, stream=None,
               nontemporal=False):
    """One streaming-read launch over nbytes at ptr (af_rt_read_probe)."""
    check(lib().af_rt_read_probe(ptr, nbytes, workgroups, segment_bytes, row_bytes,
                                 int(nontemporal), sink_ptr, _s(stream)), "af_rt_read_probe")


def device_info():
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    cus = ctypes.c_int(0)
    check(lib().af_rt_device_info(name, 256, ctypes.byref(cus), arch, 64), "af_rt_device_info")
    return {"name": name.value.decode(), "arch": arch.value.decode(), "compute_units": cus.value}


def synchronize():
    check(lib().af_rt_device_sync(), "af_rt_device_sync")


def mem_info():
    free = ctypes.c_size_t(0)
    total = ctypes.c_size_t(0)
    check(lib().af_rt_mem_info(ctypes.byref(free), ctypes.byref(total)), "af_rt_mem_info")
    return free.value, total.value


class DeviceBuffer:
    """An owned device allocation of ``nbytes`` bytes."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().af_rt_malloc(ctypes.byref(p), max(self.nbytes, 1)), f"af_rt_malloc({nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a, stream=None):
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a, stream)
        return buf

    def upload(self, a, stream=None, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().af_rt_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes, _s(stream)), "h2d")
        sync(stream)  # the host array may be freed after return

    def download(self, dtype, shape=None, stream=None, offset=0, count=None):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(count, dtype)
        check(lib().af_rt_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, _s(stream)),
              "d2h")
        sync(stream)
        return out.reshape(shape) if shape is not None else out

    def fill_u32(self, value=0, stream=None):
        check(lib().af_rt_fill_u32(self.ptr, value, self.nbytes // 4, _s(stream)), "fill")

    def free(self):
        if self.ptr:
            check(lib().af_rt_free(self.ptr), "af_rt_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                lib().af_rt_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().af_rt_stream_create(ctypes.byref(p)), "af_rt_stream_create")
        self.handle = p.value

    def sync(self):
        check(lib().af_rt_stream_sync(self.handle), "af_rt_stream_sync")

    def destroy(self):
        if self.handle:
            check(lib().af_rt_stream_destroy(self.handle), "af_rt_stream_destroy")
            self.handle = None


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().af_rt_event_create(ctypes.byref(p)), "af_rt_event_create")
        self.handle = p.value

    def record(self, stream=None):
        check(lib().af_rt_event_record(self.handle, _s(stream)), "af_rt_event_record")

    def sync(self):
        check(lib().af_rt_event_sync(self.handle), "af_rt_event_sync")

    def elapsed_ms(self, end):
        ms = ctypes.c_float(0)
        check(lib().af_rt_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle), "elapsed")
        return ms.value

    def destroy(self):
        if self.handle:
            lib().af_rt_event_destroy(self.handle)
            self.handle = None


class Graph:
    """A captured and instantiated hipGraph."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def capture(cls, stream, fn):
        check(lib().af_rt_capture_begin(_s(stream)), "af_rt_capture_begin")
        try:
            fn()
        except Exception:
            g = ctypes.c_void_p()
            lib().af_rt_capture_end(_s(stream), ctypes.byref(g))
            if g.value:
                lib().af_rt_graph_destroy(g.value)
            raise
        g = ctypes.c_void_p()
        check(lib().af_rt_capture_end(_s(stream), ctypes.byref(g)), "af_rt_capture_end")
        return cls(g.value)

    def launch(self, stream):
        check(lib().af_rt_graph_launch(self.handle, _s(stream)), "af_rt_graph_launch")

    def destroy(self):
        if self.handle:
            check(lib().af_rt_graph_destroy(self.handle), "af_rt_graph_destroy")
            self.handle = None


def _s(stream):
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


def sync(stream=None):
    if stream is None:
        synchronize()
    else:
        check(lib().af_rt_stream_sync(_s(stream)), "af_rt_stream_sync")
