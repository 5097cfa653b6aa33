"""The projection sweep that bench.py times and the in-sweep tuner replays, on one
Llama-3-8B layer: its three ways of feeding activations give the same outputs, a
captured step replays to the eager results, and the grouped launches (q/k/v, gate/up)
match one launch per projection."""

from __future__ import annotations

import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def layer(gpu):
    from mambo_amd.utils.sweep import build_weights
    step("one llama8b layer of synthetic IQ3_S weights")
    return build_weights("llama8b", 1)


def _outputs(launches):
    return list({id(p[3]): p[3] for (_, projs, _) in launches for p in projs}.values())


def _run(launches, configs, with_quant):
    from mambo_amd.utils.sweep import make_step
    outs = _outputs(launches)
    for o in outs:
        o.fill_(float("nan"))
    make_step(launches, configs, with_quant)()
    torch.cuda.synchronize()
    return [o.clone() for o in outs]


@pytest.mark.parametrize("m", [1, 4, 16])
def test_quantization_modes_agree(layer, m):
    """Activations quantized beforehand, by a quantizer launch in the step, or inside the
    GEMM (at M <= 4 on the stream kernel: bit-identical by construction; elsewhere the
    library runs the quantizer and then the GEMM): the same outputs."""
    from mambo_amd.kernels.iq3_s_fp8 import select_config
    from mambo_amd.utils.sweep import build_launches, launch_shape
    launches = build_launches(layer, m)
    assert [names for names, _, _ in launches] == [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
    configs = [select_config(m, *launch_shape(projs)) for _, projs, _ in launches]
    step(f"M={m}: pre-quantized activations")
    ref = _run(launches, configs, "none")
    assert all(torch.isfinite(r).all() for r in ref)
    for mode in ("separate", "fused"):
        step(f"M={m}: {mode} quantization")
        got = _run(launches, configs, mode)
        for g, r in zip(got, ref):
            if mode == "separate":
                assert torch.equal(g, r) or rel_l2(g.cpu().numpy(), r.cpu().numpy()) <= 1e-5, mode
            else:
                assert rel_l2(g.cpu().numpy(), r.cpu().numpy()) <= 1e-5, mode


@pytest.mark.parametrize("m", [1, 32])
def test_graph_replay_and_grouping(layer, m):
    from mambo_amd.kernels.iq3_s_fp8 import select_config
    from mambo_amd.utils.sweep import build_launches, capture, launch_shape, make_step, time_replays
    grouped = build_launches(layer, m)
    configs = [select_config(m, *launch_shape(projs)) for _, projs, _ in grouped]
    step(f"M={m}: eager step, then a captured graph replayed three times")
    ref = _run(grouped, configs, "none")
    graph = capture(make_step(grouped, configs))
    outs = _outputs(grouped)
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert rel_l2(o.cpu().numpy(), r.cpu().numpy()) <= 1e-6
    ms, wall = time_replays(graph.replay, 3, 1)
    assert ms > 0 and wall > 0
    step(f"M={m}: one launch per projection")
    single = build_launches(layer, m, no_group=True)
    assert len(single) == 7
    cfg1 = [select_config(m, *launch_shape(projs)) for _, projs, _ in single]
    got = _run(single, cfg1, "none")
    by_name = {names[0]: projs[0][3] for names, projs, _ in single}
    grouped_out = {name: p[3] for names, projs, _ in grouped for name, p in zip(names, projs)}
    for name, o in by_name.items():
        assert rel_l2(o.cpu().numpy(), grouped_out[name].cpu().numpy()) <= 1e-5, name
    assert len(got) == 7
