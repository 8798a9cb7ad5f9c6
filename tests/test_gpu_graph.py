"""Graph capture through the C ABI (g4_graph_begin_capture / end_capture / launch / destroy): what
a captured graph may hold. A kernel node keeps copies of its arguments, so a replay reads only the
device buffers they name; a copy to or from host memory would be touched at every replay after the
enqueuing call returned, so end_capture refuses it, and the stream stays usable afterwards."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_kernels_and_device_copies_replay(gpu):
    print("graph: fill kernel + device-to-device copy, three replays", flush=True)
    st = gpu.Stream()
    src = gpu.DeviceBuffer.from_array(np.arange(4096, dtype=np.uint8))
    dst = gpu.DeviceBuffer.empty((4096,), np.uint8)

    def record():
        dst.fill(0x11, st.handle)
        gpu._check(gpu.lib().g4_memcpy_d2d(dst.ptr, src.ptr, 2048, st.handle))

    g = gpu.Graph(st, record)
    want = np.concatenate([np.arange(2048, dtype=np.uint8), np.full(2048, 0x11, np.uint8)])
    for rep in range(3):
        dst.fill(0x7B, st.handle)  # eager work between replays
        g.launch()
        st.synchronize()
        assert np.array_equal(dst.download(), want), rep
    g.close()
    st.close()


def test_host_copy_in_a_capture_is_refused(gpu):
    print("graph: device-to-host copy inside a capture", flush=True)
    st = gpu.Stream()
    src = gpu.DeviceBuffer.from_array(np.arange(256, dtype=np.uint8))
    host = ctypes.c_void_p()
    gpu._check(gpu.lib().g4_host_alloc(ctypes.byref(host), 256))
    try:
        with pytest.raises(gpu.G4Error, match="host memory|cannot be inspected"):
            gpu.Graph(st, lambda: gpu._check(
                gpu.lib().g4_memcpy_d2h_async(host.value, src.ptr, 256, st.handle)))
        # the stream left the capture and runs work as before
        out = gpu.DeviceBuffer.empty((256,), np.uint8)
        gpu._check(gpu.lib().g4_memcpy_d2d(out.ptr, src.ptr, 256, st.handle))
        st.synchronize()
        assert np.array_equal(out.download(), np.arange(256, dtype=np.uint8))
    finally:
        gpu.lib().g4_host_free(host.value)
        st.close()
