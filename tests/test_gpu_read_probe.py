"""af_rt_read_probe, the streaming-read measurement aid: both access patterns
run to completion over small buffers and leave the sink word untouched (the
fold of a constant fill never equals the probe's sentinel), and arguments the
patterns cannot cover are rejected before any launch."""
import numpy as np
import pytest

import atomflow_amd
from atomflow_amd import device as dev

pytestmark = pytest.mark.gpu


def test_read_probe_patterns(gpu):
    print("[case] read probe: contiguous and head-row patterns", flush=True)
    rows, row_bytes = 1000, 2048
    nbytes = 2 * rows * row_bytes
    buf = dev.DeviceBuffer(nbytes)
    buf.fill_u32(0x3C003C00)
    sink = dev.DeviceBuffer(256)
    sink.fill_u32(0x12345678)
    for nt in (False, True):  # default and non-temporal loads
        for g in (1, 7, 256, 4096):
            dev.read_probe(buf.ptr, nbytes, g, sink.ptr, nontemporal=nt)
        for seg, rb in ((256, 2048), (128, 1024), (128, 2048)):
            for splits in (1, 3, 64, 2000):
                dev.read_probe(buf.ptr, nbytes, splits * (rb // seg), sink.ptr, seg, rb,
                               nontemporal=nt)
    dev.synchronize()
    assert np.all(sink.download(np.uint32) == 0x12345678)


def test_read_probe_rejects_bad_arguments(gpu):
    print("[case] read probe argument checks", flush=True)
    lib = atomflow_amd.lib()
    buf = dev.DeviceBuffer(1 << 20)
    sink = dev.DeviceBuffer(256)
    E = atomflow_amd
    assert lib.af_rt_read_probe(None, 1 << 20, 8, 0, 0, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 8, 0, 0, 0, None, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 0, 0, 0, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr + 8, 1024, 8, 0, 0, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1000, 8, 0, 0, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 8, 64, 2048, 0, sink.ptr, None) == E.AF_ERR_UNSUPPORTED
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 8, 256, 1000, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 3 * 2048, 8, 256, 2048, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 9, 256, 2048, 0, sink.ptr, None) == E.AF_ERR_INVALID_ARG
    assert lib.af_rt_read_probe(buf.ptr, 1 << 20, 16, 256, 2048, 0, sink.ptr, None) == 0
    dev.synchronize()
