"""bpd_stage_int64 on the device: thousands of uploads in flight wrap the
pinned ring several times (the host never waits while they fit), uploads
larger than a quarter of the ring take buffers of their own, and every
destination holds exactly the values its call was given, although each
host array is overwritten as soon as its call returns."""

from __future__ import annotations

import array

import pytest
import torch

from bpdecode_amd import _lib

pytestmark = pytest.mark.gpu


def test_stage_ring_wraps_and_oversize(dev):
    print("case staging ring: 6000 uploads + oversize", flush=True)
    lib = _lib.lib()
    stream = _lib.stream_of(dev)
    n_small, width = 6000, 300  # 2,400 bytes each: about 15 MB through a 4 MB ring
    out = torch.empty((n_small, width), dtype=torch.int64, device=dev)
    host = array.array("q", [0] * width)
    addr, _ = host.buffer_info()
    big_every, big_n = 1500, (1 << 20) // 8 + 3  # just over a quarter of the ring
    bigs = []
    for i in range(n_small):
        for j in range(width):
            host[j] = i * 1000 + j
        _lib.check(lib.bpd_stage_int64(out[i].data_ptr(), addr, width, stream))
        if i % big_every == 0:
            src = torch.arange(big_n, dtype=torch.int64) * 7 + i
            dst = torch.empty(big_n, dtype=torch.int64, device=dev)
            _lib.check(lib.bpd_stage_int64(dst.data_ptr(), src.data_ptr(), big_n, stream))
            bigs.append((dst, src.clone()))
            src.zero_()  # the call has copied it
    torch.cuda.synchronize()
    want = torch.arange(n_small, dtype=torch.int64)[:, None] * 1000 + torch.arange(width)[None, :]
    assert torch.equal(out.cpu(), want)
    for dst, src in bigs:
        assert torch.equal(dst.cpu(), src)


def test_stage_rejects_bad_arguments(dev):
    lib = _lib.lib()
    assert lib.bpd_stage_int64(None, None, 0, _lib.stream_of(dev)) == 0
    assert lib.bpd_stage_int64(None, None, -1, _lib.stream_of(dev)) != 0
    assert lib.bpd_stage_int64(None, None, 4, _lib.stream_of(dev)) != 0
