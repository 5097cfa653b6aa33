"""Chained projections (mambo_iq3s_fp8_matmul_chain, one persistent launch for up to 16
launches at 1..4 tokens) on the GPU: bit-identical to the same grouped launches run one
after the other, against the oracle, with a real dependency (each launch reading the
previous launch's output), across HIP-graph replays, and with a host-forced wait timeout
that is reported and leaves the sync words clean."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import make_synthetic_iq3_s
from oracle import oracle
from test_gpu_matmul import check

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def weight(gpu, n, k, seed):
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = make_synthetic_iq3_s(n, k, seed=seed)
    return raw, prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu), fields=False)


def mxfp8(gpu, m, k, seed):
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32))
    return xv, xs, torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)


# One 8B-shaped layer at M tokens: q/k/v grouped, o, gate/up grouped (narrowed), down,
# plus a ragged launch (N not a multiple of 16, K of one block).
LAYER = [([("q", 4096), ("k", 1024), ("v", 1024)], 4096), ([("o", 4096)], 4096),
         ([("gate", 2048), ("up", 2048)], 4096), ([("down", 4096)], 14336), ([("r", 40), ("s", 1000)], 256)]


def build_layer(gpu, m):
    launches = []
    for i, (projs, k) in enumerate(LAYER):
        ws = [weight(gpu, n, k, seed=0xC0 + 10 * i + j) for j, (_, n) in enumerate(projs)]
        xv, xs, xvg, xsg = mxfp8(gpu, m, k, seed=0x5EED + i)
        launches.append((ws, xv, xs, xvg, xsg))
    return launches


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("waves", [4, 8, 16])
def test_chain_equals_grouped_launches(gpu, m, waves):
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, chain_status, launch_iq3_s_fp8_matmul_chain, \
        launch_iq3_s_fp8_matmul_grouped, new_chain_sync
    layer = build_layer(gpu, m)
    sync = new_chain_sync(gpu)
    step(f"chain of {len(layer)} launches, M={m}, waves={waves}")
    chained = launch_iq3_s_fp8_matmul_chain(
        [ChainLaunch(xvg, [w for _, w in ws], x_scales=xsg) for ws, _, _, xvg, xsg in layer], waves=waves,
        sync=sync)
    cfg = {"kernel": _native.GEMM_STREAM, "waves": waves, "split_k": 1}
    step("the same launches one by one (stream kernel, same waves)")
    single = [launch_iq3_s_fp8_matmul_grouped(xvg, xsg, [w for _, w in ws], config=cfg)
              for ws, _, _, xvg, xsg in layer]
    torch.cuda.synchronize()
    for i, (outs, refs) in enumerate(zip(chained, single)):
        for j, (o, r) in enumerate(zip(outs, refs)):
            assert torch.equal(o, r), f"launch {i} projection {j}"
    chain_status(sync)  # no wait timed out
    assert int(sync.abs().sum()) == 0  # counters back to zero
    step("oracle on the ragged launch and sampled rows of the others")
    for i, (ws, xv, xs, _, _) in enumerate(layer):
        for j, (raw, _) in enumerate(ws):
            rows = np.arange(raw.shape[0]) if raw.shape[0] <= 1024 else \
                np.random.default_rng(i + j).choice(raw.shape[0], 48, replace=False)
            expected = oracle.iq3s_fp8_matmul(xv, xs, raw[rows])
            check(chained[i][j].cpu().numpy()[:, rows], expected)


@pytest.mark.parametrize("tpw", [2, 7, 300])
def test_chain_runs_of_tiles(gpu, tpw):
    """Several tiles per workgroup (the last run of a launch ragged, a run holding a whole
    launch): the same bits as the stream kernel with runs of the same length."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, chain_status, launch_iq3_s_fp8_matmul_chain, \
        launch_iq3_s_fp8_matmul_grouped, new_chain_sync
    m = 2
    layer = build_layer(gpu, m)[1:]
    sync = new_chain_sync(gpu)
    step(f"chain with {tpw} tiles per workgroup")
    chained = launch_iq3_s_fp8_matmul_chain(
        [ChainLaunch(xvg, [w for _, w in ws], x_scales=xsg) for ws, _, _, xvg, xsg in layer], waves=4,
        tiles_per_workgroup=tpw, sync=sync)
    cfg = {"kernel": _native.GEMM_STREAM, "waves": 4, "split_k": 1, "tile_n": 16 * tpw}
    single = [launch_iq3_s_fp8_matmul_grouped(xvg, xsg, [w for _, w in ws], config=cfg)
              for ws, _, _, xvg, xsg in layer]
    torch.cuda.synchronize()
    chain_status(sync)
    for outs, refs in zip(chained, single):
        for o, r in zip(outs, refs):
            assert torch.equal(o, r)


@pytest.mark.parametrize("m", [1, 4])
def test_chain_dependency_through_outputs(gpu, m):
    """Launch i+1 takes launch i's float32 output as its activations (quantized in the
    kernel). The outputs start as 1e30 everywhere, so an activation read before the
    previous launch finished would show; a second run with new inputs over the same
    buffers would show a read served from a cache line the first run left behind.
    Checked bit for bit against the same launches one by one (quantization inside each
    projection) and against the oracle fed with the GPU's previous output."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, chain_status, launch_iq3_s_fp8_matmul_chain, \
        launch_iq3_s_matmul_quantize, new_chain_sync
    dims = [(4096, 2048), (2048, 4096), (4096, 1024), (1024, 8192)]  # (K, N) per launch
    ws = [weight(gpu, n, k, seed=0xD0 + i) for i, (k, n) in enumerate(dims)]
    x0 = torch.empty((m, dims[0][0]), dtype=torch.bfloat16, device=gpu)
    outs = [torch.full((m, n), 1e30, dtype=torch.float32, device=gpu) for _, n in dims]
    launches = [ChainLaunch(x0 if i == 0 else outs[i - 1], [ws[i][1]], outs=[outs[i]]) for i in range(len(dims))]
    sync = new_chain_sync(gpu)
    for run in range(2):
        x0.copy_(torch.from_numpy(np.random.default_rng(10 * m + run).standard_normal(
            (m, dims[0][0])).astype(np.float32)).to(gpu))
        torch.cuda.synchronize()
        step(f"dependent chain of {len(dims)} launches, M={m}, run {run}")
        launch_iq3_s_fp8_matmul_chain(launches, waves=8, sync=sync)
        torch.cuda.synchronize()
        chain_status(sync)
        check_dependent_run(gpu, ws, x0, outs)


def check_dependent_run(gpu, ws, x0, outs):
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_matmul_quantize
    cfg = {"kernel": _native.GEMM_STREAM, "waves": 8, "split_k": 1}
    x = x0
    for i, (raw, w) in enumerate(ws):
        step(f"launch {i} alone")
        ref = launch_iq3_s_matmul_quantize(x, w, config=cfg)
        torch.cuda.synchronize()
        assert torch.equal(outs[i], ref), f"launch {i}"
        xin = (x.float() if i == 0 else x).cpu().numpy()
        xv, xs = oracle.quantize_mxfp8(xin)
        expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
        # rel-L2 <= 1e-3 as everywhere; elementwise, the f32 accumulation error grows with
        # the magnitudes (each launch multiplies them by ~20 here), so the absolute
        # tolerance is 1e-4 of the largest output instead of the N(0,1)-scaled 5e-3
        check(outs[i].cpu().numpy(), expected, elementwise=False)
        np.testing.assert_allclose(outs[i].cpu().numpy(), expected, rtol=5e-4,
                                   atol=1e-4 * float(np.abs(expected).max()))
        x = outs[i]
    assert bool(torch.isfinite(outs[-1]).all())


def test_chain_graph_replays(gpu):
    """A chain captured in a HIP graph with its sync words: every replay (eager work and
    synchronisations between them) equals the eager call, and the words end at zero."""
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, chain_status, launch_iq3_s_fp8_matmul_chain, \
        new_chain_sync
    layer = build_layer(gpu, 1)
    launches = [ChainLaunch(xvg, [w for _, w in ws], x_scales=xsg) for ws, _, _, xvg, xsg in layer]
    sync = new_chain_sync(gpu)
    step("eager chain")
    eager = [[o.clone() for o in outs] for outs in launch_iq3_s_fp8_matmul_chain(launches, sync=sync)]
    outs = [[torch.empty_like(o) for o in group] for group in eager]
    for cl, group in zip(launches, outs):
        cl.outs = group
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    step("capture")
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            launch_iq3_s_fp8_matmul_chain(launches, sync=sync)
    torch.cuda.current_stream().wait_stream(stream)
    for r in range(4):
        for group in outs:
            for o in group:
                o.fill_(-1.0)
        step(f"replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            for o, e in zip(a, b):
                assert torch.equal(o, e), f"replay {r}"
        assert int(sync.abs().sum()) == 0
    chain_status(sync)


def test_chain_timeout_is_reported(gpu):
    """wait_bias makes every dependency wait unreachable: each workgroup's first wait times
    out after timeout_us, the kernel still finishes, chain_status raises once, and the
    same sync words then serve a normal call."""
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, chain_status, launch_iq3_s_fp8_matmul_chain, \
        new_chain_sync
    layer = build_layer(gpu, 1)[:3]
    launches = [ChainLaunch(xvg, [w for _, w in ws], x_scales=xsg) for ws, _, _, xvg, xsg in layer]
    sync = new_chain_sync(gpu)
    step("chain with unreachable waits (2 ms bound)")
    launch_iq3_s_fp8_matmul_chain(launches, sync=sync, wait_bias=1, timeout_us=2000, tiles_per_workgroup=8)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="timed out"):
        chain_status(sync)
    assert int(sync.abs().sum()) == 0
    chain_status(sync)  # reported once
    step("normal chain on the same sync words")
    good = launch_iq3_s_fp8_matmul_chain(launches, sync=sync)
    torch.cuda.synchronize()
    chain_status(sync)
    for (ws, xv, xs, _, _), outs in zip(layer, good):
        raw = ws[0][0]
        check(outs[0].cpu().numpy()[:, :64], oracle.iq3s_fp8_matmul(xv, xs, raw[:64]))


def test_chain_validation(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import ChainLaunch, launch_iq3_s_fp8_matmul_chain
    _, w = weight(gpu, 32, 512, seed=1)
    _, _, xvg, xsg = mxfp8(gpu, 5, 512, seed=2)
    with pytest.raises(ValueError, match="1..4 tokens"):
        launch_iq3_s_fp8_matmul_chain([ChainLaunch(xvg, [w], x_scales=xsg)])
    _, _, xvg, xsg = mxfp8(gpu, 2, 512, seed=2)
    with pytest.raises(ValueError, match="between 1 and 16"):
        launch_iq3_s_fp8_matmul_chain([ChainLaunch(xvg, [w], x_scales=xsg)] * 17)
    with pytest.raises(ValueError, match="waves"):
        launch_iq3_s_fp8_matmul_chain([ChainLaunch(xvg, [w], x_scales=xsg)], waves=6)
    _, _, xv3, xs3 = mxfp8(gpu, 3, 512, seed=2)
    with pytest.raises(ValueError, match="same M"):
        launch_iq3_s_fp8_matmul_chain([ChainLaunch(xvg, [w], x_scales=xsg), ChainLaunch(xv3, [w], x_scales=xs3)])
