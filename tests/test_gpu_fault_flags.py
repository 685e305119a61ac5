"""GPU: fkv_paged_take_fault_flags is ordered on the stream it is given.

The read and the clear are one device-side exchange enqueued on that stream, followed by
a wait for that stream only: a fault raised by work enqueued on the same stream before
the call is reported by it, the next call reports nothing, and a bit that work on
another stream raised is reported once that work is done. fkv_paged_read and
fkv_paged_write order on their stream the same way.
"""
import numpy as np
import pytest

from tests.helpers import make_pools

pytestmark = pytest.mark.gpu


def _bad_append(pool, stream):
    import torch
    with torch.cuda.stream(stream):
        k = torch.ones((2, 1, 64), dtype=torch.float32, device="cuda")
        slots = torch.tensor([0, pool.config.num_blocks * 16], dtype=torch.int64, device="cuda")
        pool.append(0, k, k, slots, stream=stream)


def test_fault_read_on_the_raising_stream():
    import torch

    import ferrum_amd as fa
    pool, _ = make_pools(1, 1, 64, 4)
    side = torch.cuda.Stream()
    _bad_append(pool, side)
    assert pool.take_fault_flags(stream=side) == fa.FAULT_SLOT_RANGE
    assert pool.take_fault_flags(stream=side) == 0


def test_fault_raised_on_another_stream_is_kept():
    import torch

    import ferrum_amd as fa
    pool, _ = make_pools(1, 1, 64, 4)
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    _bad_append(pool, a)
    a.synchronize()  # finished: a read on any stream reports it
    assert pool.take_fault_flags(stream=b) == fa.FAULT_SLOT_RANGE
    _bad_append(pool, a)
    a.synchronize()
    assert pool.take_fault_flags() == fa.FAULT_SLOT_RANGE  # the current stream
    assert pool.take_fault_flags(stream=a) == 0


def test_image_read_and_write_order_on_their_stream():
    import torch
    from oracle import ref
    pool, layout = make_pools(1, 2, 64, 8)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(3)
    image = rng.integers(0, 256, layout.pool_bytes, dtype=np.uint8)
    pool.write(image, stream=side)
    assert np.array_equal(pool.read(stream=side), image)
    k_host = rng.standard_normal((3, 2, 64), dtype=np.float32)
    slots_host = np.array([1, 17, 40], np.int64)
    with torch.cuda.stream(side):
        k = torch.from_numpy(k_host).cuda()
        slots = torch.from_numpy(slots_host).cuda()
        pool.append(0, k, k, slots, stream=side)
    want = image.copy()
    ref.append(layout, want, 0, k_host, k_host, slots_host)
    assert np.array_equal(pool.read(stream=side), want)  # after the append on `side`
    assert pool.take_fault_flags(stream=side) == 0
