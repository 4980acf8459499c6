"""Runtime behaviour on the MI355X: asynchronous uploads through the pinned
staging ring keep stream order and data (uploads that wrap the ring many
times, interleaved with kernels that read and overwrite the destinations),
and the synchronous path for large buffers."""
from array import array

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def test_staged_uploads_wrap_and_stay_ordered(amd):
    runtime = amd.get_runtime()
    ring = runtime.STAGING_BYTES
    rng = np.random.default_rng(5)
    sizes = [int(s) for s in rng.integers(1, ring // 16, size=64)]  # ~ 32 MiB in all: the ring wraps
    expected, storages = [], []
    for i, n in enumerate(sizes):
        values = rng.standard_normal(n // 4 + 1).astype(np.float32)
        target = amd.AMDStorage(values.size, "float32")
        runtime.upload(target.ptr, array("f", values.tobytes()))
        # a kernel reading the fresh upload, queued behind the copy
        doubled = amd.add(target, target)
        # the destination is overwritten again at once: the first copy must land first
        again = values + 1.0
        runtime.upload(target.ptr, array("f", again.tobytes()))
        expected.append((values * 2, again))
        storages.append((doubled, target))
    for (want_doubled, want_again), (doubled, target) in zip(expected, storages):
        assert np.array_equal(np.frombuffer(doubled.to_array(), dtype=np.float32), want_doubled)
        assert np.array_equal(np.frombuffer(target.to_array(), dtype=np.float32), want_again)


def test_large_upload_takes_the_synchronous_path(amd):
    runtime = amd.get_runtime()
    n = runtime.STAGING_BYTES // 4 + 1024  # more than a quarter of the ring, in floats
    values = np.arange(n, dtype=np.float32)
    target = amd.storage(array("f", values.tobytes()), dtype="float32")
    assert np.array_equal(np.frombuffer(target.to_array(), dtype=np.float32), values)
