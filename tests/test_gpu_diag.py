"""Diagnostic kernels behind the bench's ceilings: the plain read (checksum against numpy)
and the scaled-MFMA throughput loop (every output equals its closed form)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 48, (1 << 20) + 16 * 37])
def test_read_bytes_checksum(gpu, nbytes):
    from mambo_amd import _native
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=max(nbytes // 4, 1), dtype=np.uint32)[: nbytes // 4]
    src = torch.from_numpy(host.view(np.int32).copy()).to(gpu) if nbytes else torch.empty(4, dtype=torch.int32,
                                                                                           device=gpu)
    sink = torch.full((_native.READ_SINK_WORDS,), -1, dtype=torch.int32, device=gpu)
    step(f"read_bytes {nbytes} bytes")
    _native.check(_native.lib().mambo_read_bytes(src.data_ptr(), nbytes, sink.data_ptr(),
                                                 _native.stream_handle(None)), "read_bytes")
    torch.cuda.synchronize()
    got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
    want = int(np.bitwise_xor.reduce(host)) if nbytes else 0
    assert got == want


def test_read_bytes_rejects_bad_arguments(gpu):
    from mambo_amd import _native
    sink = torch.empty(_native.READ_SINK_WORDS, dtype=torch.int32, device=gpu)
    src = torch.empty(64, dtype=torch.int32, device=gpu)
    assert _native.lib().mambo_read_bytes(src.data_ptr(), 24, sink.data_ptr(), None) == _native.MAMBO_ERR_VALUE
    assert _native.lib().mambo_read_bytes(src.data_ptr() + 4, 32, sink.data_ptr(), None) == _native.MAMBO_ERR_VALUE


@pytest.mark.parametrize("workgroups,iters", [(1, 0), (3, 7), (512, 50)])
def test_mfma_peak_sums(gpu, workgroups, iters):
    from mambo_amd import _native
    out = torch.full((workgroups * 256,), -1.0, dtype=torch.float32, device=gpu)
    step(f"mfma_peak workgroups={workgroups} iters={iters}")
    _native.check(_native.lib().mambo_mfma_peak(workgroups, iters, out.data_ptr(), _native.stream_handle(None)),
                  "mfma_peak")
    torch.cuda.synchronize()
    # each MFMA adds 128 (E4M3 1.0 x 1.0 over K=128) to all 4 accumulators of 8 chains
    assert bool((out == 4096.0 * iters).all())
