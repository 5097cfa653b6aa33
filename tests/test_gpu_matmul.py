"""Fused IQ3_S x MXFP8 projection on the GPU against the CPU oracle.

Tolerances: rel-L2 <= 1e-3 against the float64-accumulated product of the decoded
operands (the acceptance bar of the path), plus the reference test's elementwise
rtol 5e-4 / atol 5e-3 (test_iq3_s_fp8.py:201)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, make_synthetic_iq3_s, rel_l2
from oracle import oracle

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3
RTOL, ATOL = 5e-4, 5e-3


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def check(out: np.ndarray, expected: np.ndarray, *, elementwise: bool = True) -> None:
    assert out.shape == expected.shape and out.dtype == np.float32
    err = rel_l2(out, expected)
    assert err <= REL_L2, f"rel-L2 {err:.3e}"
    if elementwise:
        np.testing.assert_allclose(out, expected, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 17, 33, 128, 129])
def test_synthetic_iq3_s_fp8_matmul_matches_oracle(gpu, m):
    """test_iq3_s_fp8.py:178-210: N=7, K=768, reference block generator; also strided
    activations (column stride 2, as the reference test passes them)."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n_rows, k = 7, 768
    raw = make_synthetic_iq3_s(n_rows, k, seed=0x3F8)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(20261016 + m).standard_normal((m, k)).astype(np.float32)
    step(f"quantize + matmul M={m} N=7 K=768")
    xq, xs = launch_quantize_fp8(torch.from_numpy(x).to(gpu))
    out = launch_iq3_s_fp8_matmul(xq, xs, fields)
    torch.cuda.synchronize()
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw)
    check(out.cpu().numpy(), expected)
    strided_values = torch.empty((m, 2 * k), dtype=torch.uint8, device=gpu)
    strided_values[:, ::2] = xq
    strided_scales = torch.empty((m, 2 * k // 32), dtype=torch.uint8, device=gpu)
    strided_scales[:, ::2] = xs
    step(f"matmul strided activations M={m}")
    out2 = launch_iq3_s_fp8_matmul(strided_values[:, ::2], strided_scales[:, ::2], fields)
    torch.cuda.synchronize()
    check(out2.cpu().numpy(), expected)


def test_golden_matmul_small(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    g = np.load(GOLDEN / "matmul_small.npz")
    fields = prepare_iq3_s_fields(torch.from_numpy(g["raw"]).to(gpu))
    step("matmul golden M=9 N=7 K=768")
    out = launch_iq3_s_fp8_matmul(torch.from_numpy(g["x_values"]).to(gpu), torch.from_numpy(g["x_scales"]).to(gpu),
                                  fields)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), g["out"])


def test_every_search_space_config_agrees(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import gemm_search_space, launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n_rows, k = 100, 2048
    raw = make_synthetic_iq3_s(n_rows, k, seed=17)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    for m in (1, 6, 16, 37):
        x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
        xv, xs = oracle.quantize_mxfp8(x)
        expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
        xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
        for cfg in gemm_search_space(m, n_rows, k):
            step(f"matmul M={m} N=100 K=2048 cfg={cfg}")
            out = launch_iq3_s_fp8_matmul(xvg, xsg, fields, config=cfg)
            torch.cuda.synchronize()
            check(out.cpu().numpy(), expected)


def test_every_stream_config_at_long_k(gpu):
    """Every stream-kernel candidate at K=8192, where 1, 2 and 4 tokens take one, four and
    sixteen codebook copies in LDS (every wave count, run length and K split of the
    search space), against the oracle."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import gemm_search_space, launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n_rows, k = 48, 8192
    raw = make_synthetic_iq3_s(n_rows, k, seed=23)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    for m in (1, 2, 4):
        x = np.random.default_rng(100 + m).standard_normal((m, k)).astype(np.float32)
        xv, xs = oracle.quantize_mxfp8(x)
        expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
        xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
        cfgs = [c for c in gemm_search_space(m, n_rows, k) if c["kernel"] == _native.GEMM_STREAM]
        assert cfgs
        for cfg in cfgs:
            step(f"stream M={m} N=48 K=8192 cfg={cfg}")
            out = launch_iq3_s_fp8_matmul(xvg, xsg, fields, config=cfg)
            torch.cuda.synchronize()
            check(out.cpu().numpy(), expected, elementwise=False)


def test_output_row_stride_and_preallocated_out(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = make_synthetic_iq3_s(40, 1024, seed=21)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(1).standard_normal((6, 1024)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
    big = torch.full((6, 64), 7.0, dtype=torch.float32, device=gpu)
    for cfg in ({"waves": 4, "split_k": 1}, {"waves": 2, "split_k": 4}):
        step(f"matmul into strided out cfg={cfg}")
        launch_iq3_s_fp8_matmul(torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu), fields,
                                config=cfg, out=big[:, 8:48])
        torch.cuda.synchronize()
        b = big.cpu().numpy()
        check(b[:, 8:48], expected)
        assert np.all(b[:, :8] == 7.0) and np.all(b[:, 48:] == 7.0)


def _synth_weight(gpu, n: int, k: int, seed: int):
    from mambo_amd import _native
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = torch.empty((n, k // 256, 110), dtype=torch.uint8, device=gpu)
    _native.check(_native.lib().mambo_synth_iq3s(seed, k // 256, 0, n, raw.data_ptr(), _native.stream_handle(None)))
    return prepare_iq3_s_fields(raw, fields=False)


def _synth_act(gpu, m: int, k: int, seed: int = 1):
    from mambo_amd import _native
    bits = torch.empty(m * k, dtype=torch.int16, device=gpu)
    _native.check(_native.lib().mambo_synth_bf16(seed, 2, 0.0, 0, m * k, bits.data_ptr(), _native.stream_handle(None)))
    return bits.view(torch.bfloat16).view(m, k)


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_llama3_8b_decode_shapes(gpu, n, k, m):
    """Decode-shaped projections on the 8B shapes, weights from the counter-based
    generator: full output for the smaller shapes, sampled rows for the larger."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=0)
    step(f"quantize + matmul M={m} {n}x{k}")
    xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k))
    out = launch_iq3_s_fp8_matmul(xq, xs, fields).cpu().numpy()
    torch.cuda.synchronize()
    rows = np.arange(n) if n * k <= 4096 * 4096 else np.concatenate(
        [np.arange(256), np.random.default_rng(n).choice(n, 256, replace=False)])
    raw = np.concatenate([oracle.gen_iq3s(0, 1, k // 256, row0=int(r)) for r in rows]) if len(rows) < n \
        else oracle.gen_iq3s(0, n, k // 256)
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw, threads=oracle.default_threads())
    check(out[:, rows], expected, elementwise=False)
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("m", [1, 32])
def test_llama3_70b_gate_shape_sampled(gpu, m):
    """28672 x 8192 (gate/up), sampled output rows against the oracle."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    n, k = 28672, 8192
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=5)
    step(f"quantize + matmul M={m} {n}x{k}")
    xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=9))
    out = launch_iq3_s_fp8_matmul(xq, xs, fields).cpu().numpy()
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(n, 192, replace=False))
    raw = np.concatenate([oracle.gen_iq3s(5, 1, k // 256, row0=int(r)) for r in rows])
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw, threads=oracle.default_threads())
    check(out[:, rows], expected, elementwise=False)


@pytest.mark.parametrize("m", [2, 3, 4])
def test_llama3_70b_down_shape_staged_rows(gpu, m):
    """8192 x 28672 (down) at 2-4 tokens: 57-115 KiB of activation rows, staged in LDS for
    one 16-wave workgroup per CU by the default configuration (and, as a check of the
    other form, read from L2 by an 8-wave configuration); sampled rows against the
    oracle."""
    import ctypes

    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    n, k = 8192, 28672
    c = _native.GemmConfig()
    assert _native.lib().mambo_gemm_default_config(m, n, k // 256, ctypes.byref(c)) == 0
    assert (c.kernel, c.waves) == (_native.GEMM_STREAM, 16), c.as_dict()
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=6)
    xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=10 + m))
    rows = np.sort(np.random.default_rng(2).choice(n, 128, replace=False))
    raw = np.concatenate([oracle.gen_iq3s(6, 1, k // 256, row0=int(r)) for r in rows])
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw, threads=oracle.default_threads())
    for cfg in (c.as_dict(), {"kernel": _native.GEMM_STREAM, "waves": 8, "split_k": 1, "tile_n": 16}):
        step(f"matmul M={m} {n}x{k} cfg={cfg}")
        out = launch_iq3_s_fp8_matmul(xq, xs, fields, config=cfg).cpu().numpy()
        torch.cuda.synchronize()
        check(out[:, rows], expected, elementwise=False)


def test_graph_capture_replays_match_eager(gpu):
    """Split-K launches (zero-fill kernel + atomics) captured in a HIP graph: every replay,
    with eager work between replays, matches the eager result."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    fields = [_synth_weight(gpu, 1024, 4096, seed=s) for s in (11, 12)]
    xq, xs = launch_quantize_fp8(_synth_act(gpu, 4, 4096))
    outs = [torch.empty((4, 1024), dtype=torch.float32, device=gpu) for _ in fields]
    cfgs = [{"waves": 4, "split_k": 4}, {"waves": 2, "split_k": 1}]

    def step_fn():
        for f, o, c in zip(fields, outs, cfgs):
            launch_iq3_s_fp8_matmul(xq, xs, f, config=c, out=o)

    step("eager reference")
    step_fn()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    step("capture")
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step_fn()
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        step(f"replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            torch.testing.assert_close(o, r, rtol=1e-5, atol=1e-5)
        _ = (xq.float().sum()).item()  # eager work between replays


@pytest.mark.parametrize("m", [1, 5, 16, 33, 130])
def test_grouped_projections_match_single_launches(gpu, m):
    """Three projections of one input in one launch (q/k/v-like, ragged N): each output
    is bit-identical to its own launch under the same configuration and matches the
    oracle; a K-split grouped launch (zero fill + atomics) matches the oracle too."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul, launch_iq3_s_fp8_matmul_grouped
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    k = 2048
    raws = [make_synthetic_iq3_s(n, k, seed=40 + i) for i, n in enumerate((100, 37, 64))]
    fields = [prepare_iq3_s_fields(torch.from_numpy(r).to(gpu)) for r in raws]
    x = np.random.default_rng(7 + m).standard_normal((m, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    expected = [oracle.iq3s_fp8_matmul(xv, xs, r) for r in raws]
    from mambo_amd import _native
    cfg = {"kernel": _native.GEMM_DENSE, "waves": 2, "split_k": 1} if m < 64 else \
        {"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 1, "tile_m": 64, "tile_n": 64}
    step(f"grouped matmul M={m} N=100+37+64 K=2048 cfg={cfg}")
    outs = launch_iq3_s_fp8_matmul_grouped(xvg, xsg, fields, config=cfg)
    singles = [launch_iq3_s_fp8_matmul(xvg, xsg, f, config=cfg) for f in fields]
    torch.cuda.synchronize()
    for o, s_, e in zip(outs, singles, expected):
        np.testing.assert_array_equal(o.cpu().numpy(), s_.cpu().numpy())
        check(o.cpu().numpy(), e)
    step(f"grouped matmul M={m} default config and split_k=4")
    for c in (None, {"kernel": _native.GEMM_DENSE, "waves": 2, "split_k": 4}):
        outs = launch_iq3_s_fp8_matmul_grouped(xvg, xsg, fields, config=c)
        torch.cuda.synchronize()
        for o, e in zip(outs, expected):
            check(o.cpu().numpy(), e)


@pytest.mark.parametrize("m", [1, 3, 4, 9])
def test_stream_kernel_multi_tile_runs(gpu, m):
    """Stream kernel workgroups that walk a run of row tiles: runs of 1..14 tiles over a
    grouped launch whose projections (N = 100, 37, 64: 7 + 3 + 4 tiles, the last of each
    partial) make runs cross projection boundaries and leave the last run short; more
    waves than K blocks (idle waves), and a K split over workgroups. Every run length
    gives the same bits as one tile per workgroup (same summation order) and matches the
    oracle."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul_grouped
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    k = 2048
    raws = [make_synthetic_iq3_s(n, k, seed=140 + i) for i, n in enumerate((100, 37, 64))]
    fields = [prepare_iq3_s_fields(torch.from_numpy(r).to(gpu)) for r in raws]
    x = np.random.default_rng(11 + m).standard_normal((m, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    expected = [oracle.iq3s_fp8_matmul(xv, xs, r) for r in raws]
    for waves in (1, 4, 8, 16):
        for split in (1, 3):
            base = None
            for tiles_per_wg in (1, 2, 3, 5, 14, 20):
                cfg = {"kernel": _native.GEMM_STREAM, "waves": waves, "split_k": split, "tile_n": 16 * tiles_per_wg}
                step(f"stream multi-tile M={m} N=100+37+64 K=2048 cfg={cfg}")
                outs = [o.cpu().numpy() for o in launch_iq3_s_fp8_matmul_grouped(xvg, xsg, fields, config=cfg)]
                for o, e in zip(outs, expected):
                    check(o, e)
                if split == 1:
                    if base is None:
                        base = outs
                    for o, b in zip(outs, base):
                        np.testing.assert_array_equal(o, b)


@pytest.mark.parametrize("k", [2048, 8192])
def test_stream_kernel_codebook_copies(gpu, k):
    """The stream kernel keeps 1, 4 or 16 copies of its codebook in LDS, chosen by the
    launch's tokens and K (1 token on K >= 8192: one copy; 2 tokens: four; 3-4 tokens on
    K >= 8192: sixteen; K < 8192: four). Every token count against the oracle, for 1, 4
    and 16 waves with runs of tiles; and each token's outputs bit for bit equal to a
    one-token launch of that token (the block-diagonal MFMA computes every token's
    outputs alone, so only a wrong codebook word could change them)."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n = 200
    raw = make_synthetic_iq3_s(n, k, seed=k + 7)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(k).standard_normal((4, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
    for waves, tiles_per_wg in ((1, 1), (4, 1), (4, 3), (16, 2)):
        cfg = {"kernel": _native.GEMM_STREAM, "waves": waves, "split_k": 1, "tile_n": 16 * tiles_per_wg}
        single = []
        for t in range(4):
            step(f"stream codebook copies: token {t} alone K={k} cfg={cfg}")
            single.append(launch_iq3_s_fp8_matmul(xvg[t:t + 1], xsg[t:t + 1], fields, config=cfg).cpu().numpy())
        for m in (1, 2, 3, 4):
            step(f"stream codebook copies: M={m} K={k} cfg={cfg}")
            out = launch_iq3_s_fp8_matmul(xvg[:m], xsg[:m], fields, config=cfg).cpu().numpy()
            check(out, expected[:m])
            for t in range(m):
                np.testing.assert_array_equal(out[t:t + 1], single[t], err_msg=f"token {t} of M={m}")


def test_grouped_into_strided_outputs(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul_grouped
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    k, m = 1024, 3
    raws = [make_synthetic_iq3_s(n, k, seed=60 + n) for n in (20, 33)]
    fields = [prepare_iq3_s_fields(torch.from_numpy(r).to(gpu)) for r in raws]
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(3).standard_normal((m, k)).astype(np.float32))
    from mambo_amd import _native
    # the K-split form zeroes the slices first (one dispatch for all projections) and
    # must leave the columns between them alone
    for cfg in (None, {"kernel": _native.GEMM_STREAM, "waves": 2, "split_k": 2},
                {"kernel": _native.GEMM_DENSE, "waves": 1, "split_k": 4}):
        big = torch.full((m, 80), 7.0, dtype=torch.float32, device=gpu)
        step(f"grouped matmul into column slices of one buffer, cfg={cfg}")
        launch_iq3_s_fp8_matmul_grouped(torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu), fields,
                                        outs=[big[:, 4:24], big[:, 40:73]], config=cfg)
        torch.cuda.synchronize()
        b = big.cpu().numpy()
        check(b[:, 4:24], oracle.iq3s_fp8_matmul(xv, xs, raws[0]))
        check(b[:, 40:73], oracle.iq3s_fp8_matmul(xv, xs, raws[1]))
        assert np.all(b[:, :4] == 7.0) and np.all(b[:, 24:40] == 7.0) and np.all(b[:, 73:] == 7.0)


@pytest.mark.parametrize("m", [64, 100, 128, 257])
def test_tiled_kernel_every_tile_shape(gpu, m):
    """The tiled (prefill) kernel at ragged M and N (N=100: a partial weight tile and
    partial workgroups), every tile shape it is built for (at M=100 with split_k=3, which
    the library rounds to two splits of the 4 K blocks), against the oracle."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n_rows, k = 100, 1024
    raw = make_synthetic_iq3_s(n_rows, k, seed=70 + m)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(90 + m).standard_normal((m, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    expected = oracle.iq3s_fp8_matmul(xv, xs, raw, threads=oracle.default_threads())
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    shapes = [(tile_m, waves, rows) for tile_m in (64, 128) for waves in (4, 8) for rows in (16, 32)]
    shapes += [(256, 8, 16), (256, 16, 16)]
    for tile_m, waves, rows_per_wave in shapes:
        cfg = {"kernel": _native.GEMM_TILED, "waves": waves, "split_k": 1 if m != 100 else 3,
               "tile_m": tile_m, "tile_n": rows_per_wave * waves}
        step(f"tiled M={m} N=100 K=1024 cfg={cfg}")
        out = launch_iq3_s_fp8_matmul(xvg, xsg, fields, config=cfg)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), expected)


@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 14336)])
def test_prefill_shape_sampled(gpu, n, k):
    """M=2048 prefill on 8B shapes (default config: the tiled kernel), sampled output
    columns against the oracle."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    m = 2048
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=3)
    step(f"quantize + matmul M={m} {n}x{k}")
    xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=4))
    out = launch_iq3_s_fp8_matmul(xq, xs, fields).cpu().numpy()
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(n + k).choice(n, 48, replace=False))
    raw = np.concatenate([oracle.gen_iq3s(3, 1, k // 256, row0=int(r)) for r in rows])
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw, threads=oracle.default_threads())
    check(out[:, rows], expected, elementwise=False)
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("m,k,split", [(700, 2048, 4), (700, 1024, 4), (1100, 1024, 1)])
def test_prefill_form_many_items(gpu, m, k, split):
    """The 256-token x 128-row prefill form with more work items than CUs, so each
    workgroup runs several items through one pipeline: a ragged last token tile (rows
    past M read as zero and are not stored), ragged last weight groups, K splits of two
    blocks and of one block (the block after next then lies two items ahead), and a
    grouped launch into column slices of one buffer. Sampled weight rows against the
    oracle; the columns around the slices and the rows past M keep their contents."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul_grouped
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    n1, n2 = 3000, 4100
    step(f"synth weights {n1}+{n2} x {k}")
    fields = [_synth_weight(gpu, n1, k, seed=11), _synth_weight(gpu, n2, k, seed=12)]
    xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=13))
    cfg = {"kernel": _native.GEMM_TILED, "waves": 8, "split_k": split, "tile_m": 256, "tile_n": 128}
    big = torch.full((m + 5, n1 + n2 + 40), 7.0, dtype=torch.float32, device=gpu)
    c1, c2 = 8, 24 + n1
    step(f"grouped prefill form M={m} K={k} cfg={cfg}")
    launch_iq3_s_fp8_matmul_grouped(xq, xs, fields, outs=[big[:m, c1:c1 + n1], big[:m, c2:c2 + n2]], config=cfg)
    torch.cuda.synchronize()
    b = big.cpu().numpy()
    assert np.all(b[m:] == 7.0) and np.all(b[:, :c1] == 7.0)
    assert np.all(b[:, c1 + n1:c2] == 7.0) and np.all(b[:, c2 + n2:] == 7.0)
    xqn, xsn = xq.cpu().numpy(), xs.cpu().numpy()
    for seed, n, c in ((11, n1, c1), (12, n2, c2)):
        rng = np.random.default_rng(seed + m)
        rows = np.unique(np.concatenate([rng.choice(n, 20, replace=False), [0, 127, 128, n - 1]]))
        raw = np.concatenate([oracle.gen_iq3s(seed, 1, k // 256, row0=int(r)) for r in rows])
        expected = oracle.iq3s_fp8_matmul(xqn, xsn, raw, threads=oracle.default_threads())
        check(b[:m, c + rows], expected, elementwise=False)


def test_default_32_token_tiles(gpu):
    """17-32 tokens on a wide enough grid: the library default is the tiled kernel's
    32-token tile (four waves sharing each activation block) with K split."""
    import ctypes

    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n, k, m = 4096, 8192, 24
    c = _native.GemmConfig()
    assert _native.lib().mambo_gemm_default_config(m, n, k // 256, ctypes.byref(c)) == 0
    assert (c.kernel, c.tile_m, c.split_k) == (_native.GEMM_TILED, 32, 4), c.as_dict()
    raw = oracle.gen_iq3s(31, n, k // 256)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(24).standard_normal((m, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    step(f"default config M={m} N={n} K={k}: {c.as_dict()}")
    out = launch_iq3_s_fp8_matmul(torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu), fields,
                                  config={"kernel": _native.GEMM_AUTO})
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.iq3s_fp8_matmul(xv, xs, raw))


@pytest.mark.parametrize("m", [7, 16, 23, 32])
def test_tiled_k_groups(gpu, m):
    """16- and 32-token tiles whose workgroups hold 2 to 16 K groups of one, two or four
    waves (each group takes every G-th K block, the groups' sums added in LDS at the end),
    on 7 K blocks (a K range that the groups do not divide evenly, and groups with no
    block at all) and N=100 (a partial weight tile), with no K split and with split_k=3
    (ranges of 3, 3 and 1 blocks), against the oracle."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n_rows, k = 100, 7 * 256
    raw = make_synthetic_iq3_s(n_rows, k, seed=300 + m)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    x = np.random.default_rng(310 + m).standard_normal((m, k)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    expected = oracle.iq3s_fp8_matmul(xv, xs, raw)
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    shapes = [(16, 8, 64), (16, 8, 128), (16, 16, 64), (16, 4, 16), (16, 4, 32), (16, 8, 16), (16, 8, 32),
              (16, 16, 16), (16, 16, 32)]
    shapes += [(32, 8, 64), (32, 8, 32), (32, 8, 16)] if m > 16 else []
    for tile_m, waves, tile_n in shapes:
        for split in (1, 3):
            cfg = {"kernel": _native.GEMM_TILED, "waves": waves, "split_k": split, "tile_m": tile_m,
                   "tile_n": tile_n}
            step(f"tiled K groups M={m} N=100 K={k} cfg={cfg}")
            out = launch_iq3_s_fp8_matmul(xvg, xsg, fields, config=cfg)
            torch.cuda.synchronize()
            check(out.cpu().numpy(), expected)
