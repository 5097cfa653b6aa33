"""The projection sweep's layer tables on the CPU: the Llama-3 shapes and one GPU's
tensor-parallel shard of them (column-parallel q/k/v and gate/up split N, row-parallel
o and down split K, in whole 16-row tiles and 256-weight blocks)."""

from __future__ import annotations

import pytest

from mambo_amd.utils.sweep import MODELS, layer_shapes


def test_full_layers():
    assert [s[0] for s in layer_shapes("llama70b")] == ["q", "k", "v", "o", "gate", "up", "down"]
    # 70B: hidden 8192, 64 query heads and 8 key/value heads of 128, FFN 28672
    assert layer_shapes("llama70b")[1] == ("k", 1024, 8192, 0)
    assert layer_shapes("llama8b")[6] == ("down", 4096, 14336, 3)
    assert MODELS["llama70b"][1] == 80 and MODELS["llama8b"][1] == 32


@pytest.mark.parametrize("model", ["llama70b", "llama8b"])
@pytest.mark.parametrize("tp", [2, 4, 8])
def test_tensor_parallel_shard(model, tp):
    full = layer_shapes(model)
    for (name, n, k, slot), (sname, sn, sk, sslot) in zip(full, layer_shapes(model, tp)):
        assert (name, slot) == (sname, sslot)
        if slot in (0, 2):
            assert (sn * tp, sk) == (n, k) and sn % 16 == 0
        else:
            assert (sn, sk * tp) == (n, k) and sk % 256 == 0


def test_shard_that_breaks_a_tile_or_block_is_refused():
    with pytest.raises(ValueError, match="q: N=4096 does not split into 3 shards of whole 16-row tiles"):
        layer_shapes("llama8b", 3)
    with pytest.raises(ValueError, match="down: K=28672 does not split into 32 shards of whole 256-weight blocks"):
        layer_shapes("llama70b", 32)


def test_profile_segmentation_finds_each_points_timed_steps():
    """The per-point profile summary cuts a kernel trace into the points' timed steps: runs
    of GEMM / K-split fill dispatches that other kernels (input set-up, copies, checks)
    separate. A point whose K-split adds a fill per launch has up to twice its launches."""
    from mambo_amd.utils.rocprof_summary import segment_points

    def step(launches, fills):
        return ["gemm_stream_kernel"] * launches + ["zero_rows_kernel"] * fills

    names = ["randn"] + step(3, 0) + ["copy"] + step(3, 0) + ["allclose"]  # eager step, check replay
    names += step(3, 0) * 4 + ["randn"]                                      # W=2 + K=2 replays
    names += step(2, 2) + ["copy"] + step(2, 2) + ["allclose"] + step(2, 2) * 4
    points = [{"workload": "a", "launches": 3}, {"workload": "b", "launches": 2}]
    a, b = segment_points(names, points, 4, 2)
    assert [names[i] for i in a] == step(3, 0) * 2 and a.stop == names.index("randn", 1)
    assert [names[i] for i in b] == step(2, 2) * 2 and b.stop == len(names)
    with pytest.raises(ValueError, match="no run of steps for point c"):
        segment_points(names, points + [{"workload": "c", "launches": 1}], 4, 2)
