"""Host-side robustness on the GPU: an error left behind by an unrelated HIP call is not
reported as a launch failure; a weight whose SoA fields change after its first
projection is repacked; activation scales in row-strided views that the tiled kernel
cannot read in place are copied; and the library's own kernels exit cleanly after each
of these."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import make_synthetic_iq3_s
from oracle import oracle
from test_gpu_matmul import check, step

pytestmark = pytest.mark.gpu


def test_stale_hip_error_is_not_blamed_on_the_next_launch(gpu):
    from mambo_amd import _native
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime instance torch and the library share
    hip.hipSetDevice.argtypes = [ctypes.c_int]
    hip.hipGetLastError.restype = ctypes.c_int
    buf = torch.zeros(1000, dtype=torch.float32, device=gpu)
    torch.cuda.synchronize()
    step("hipSetDevice(9999) leaves an error behind; then a valid fill")
    assert hip.hipSetDevice(9999) != 0
    rc = _native.lib().mambo_fill_f32(buf.data_ptr(), buf.numel(), 2.5, _native.stream_handle(None))
    assert rc == _native.MAMBO_OK, _native.lib().mambo_last_error()
    # the earlier error is no longer pending on the thread, but the call names it
    message = _native.lib().mambo_last_error().decode()
    assert "earlier HIP error" in message and "fill_f32: ok" in message, message
    torch.cuda.synchronize()
    assert bool((buf == 2.5).all())
    assert hip.hipGetLastError() == 0
    step("a second fill with nothing pending leaves no message")
    rc = _native.lib().mambo_fill_f32(buf.data_ptr(), buf.numel(), 1.5, _native.stream_handle(None))
    assert rc == _native.MAMBO_OK and _native.lib().mambo_last_error() == b""


def test_packed_weight_follows_field_writes(gpu):
    """The first projection builds the packed tile from the SoA fields; after the fields
    are written in place (d and a group's scale nibbles) the next projection uses the
    new weights."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n, k, m = 48, 1024, 5
    raw = make_synthetic_iq3_s(n, k, seed=91)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(9).standard_normal((m, k)).astype(np.float32))
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    step("matmul with the prepared weight")
    first = launch_iq3_s_fp8_matmul(xvg, xsg, fields)
    torch.cuda.synchronize()
    check(first.cpu().numpy(), oracle.iq3s_fp8_matmul(xv, xs, raw))
    packed_before = fields.packed
    # new d for row 7, block 2 and new scale bytes for row 30, block 0 (fields are [B, N, ...])
    new_d = np.array([0.03125], dtype=np.float16)
    fields.d[2, 7] = torch.from_numpy(new_d).to(gpu)[0]
    fields.scales.view(torch.uint8).view(-1, n, 4)[0, 30, :] = torch.tensor([0x5A, 0xF0, 0x0F, 0x33],
                                                                           dtype=torch.uint8, device=gpu)
    edited = raw.copy()
    edited[7, 2, :2] = new_d.view(np.uint8)
    edited[30, 0, 106:110] = [0x5A, 0xF0, 0x0F, 0x33]
    step("matmul after writing the SoA fields in place")
    second = launch_iq3_s_fp8_matmul(xvg, xsg, fields)
    torch.cuda.synchronize()
    assert fields.packed is not packed_before
    expected = oracle.iq3s_fp8_matmul(xv, xs, edited)
    check(second.cpu().numpy(), expected)
    assert not np.array_equal(second.cpu().numpy()[:, [7, 30]], first.cpu().numpy()[:, [7, 30]])



def test_release_soa_fields_on_the_gpu(gpu):
    """A weight prepared the reference's way holds only its SoA fields until the first
    projection builds the tile; release_soa_fields then frees the fields (device memory
    drops by their 110 bytes per block) and the next projections return the same bits."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import has_soa_fields, prepare_iq3_s_fields, release_soa_fields
    n, k, m = 512, 4096, 3
    raw = make_synthetic_iq3_s(n, k, seed=0x5E1)
    source = torch.from_numpy(raw).to(gpu)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(gpu)
    step(f"prepare [{n},{k // 256},110] with SoA fields only")
    fields = prepare_iq3_s_fields(source)
    torch.cuda.synchronize()
    soa = torch.cuda.memory_allocated(gpu) - base
    assert fields.packed is None and soa >= raw.nbytes
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(5).standard_normal((m, k)).astype(np.float32))
    xvg, xsg = torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu)
    step("first projection builds the tile")
    first = launch_iq3_s_fp8_matmul(xvg, xsg, fields)
    torch.cuda.synchronize()
    check(first.cpu().numpy(), oracle.iq3s_fp8_matmul(xv, xs, raw))
    assert fields.packed is not None
    before = torch.cuda.memory_allocated(gpu)
    step("release the SoA fields")
    release_soa_fields(fields)
    torch.cuda.synchronize()
    assert not has_soa_fields(fields)
    # the five placeholders each take one 512-byte block of torch's caching allocator
    assert before - torch.cuda.memory_allocated(gpu) >= raw.nbytes - 5 * 512
    step("projection after the release")
    second = launch_iq3_s_fp8_matmul(xvg, xsg, fields)
    torch.cuda.synchronize()
    assert torch.equal(second, first)

def test_row_strided_scales_through_the_tiled_kernel(gpu):
    """M = 24 (the tiled kernel's 32-token tile by default on wide grids, and as an
    explicit config): scale rows with a stride of K/32 + 4 bytes (not 8-byte aligned)
    are copied by the launcher; the result matches the contiguous call and the oracle."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n, k, m = 4096, 8192, 24
    raw = oracle.gen_iq3s(55, n, k // 256)
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu), fields=False)
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(24).standard_normal((m, k)).astype(np.float32))
    xvg = torch.from_numpy(xv).to(gpu)
    wide = torch.zeros((m, k // 32 + 4), dtype=torch.uint8, device=gpu)
    wide[:, :k // 32] = torch.from_numpy(xs).to(gpu)
    strided = wide[:, :k // 32]
    assert strided.stride(0) % 8 == 4
    expected = oracle.iq3s_fp8_matmul(xv, xs, raw, threads=oracle.default_threads())
    for cfg in (None, {"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 4, "tile_m": 32, "tile_n": 64}):
        step(f"matmul M={m} row-strided scales cfg={cfg}")
        out = launch_iq3_s_fp8_matmul(xvg, strided, fields, config=cfg)
        ref = launch_iq3_s_fp8_matmul(xvg, torch.from_numpy(xs).to(gpu), fields, config=cfg)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), expected)
        check(ref.cpu().numpy(), expected)


@pytest.mark.parametrize("m", [1, 3])
def test_odd_scale_rows_through_the_stream_kernel(gpu, m):
    """C ABI call at 1 and 3 tokens with the activation scale rows at an odd address and
    an odd row stride (K/32 + 1 bytes): the stream kernel then reads the scales from
    global memory a byte at a time (its LDS copy moves them as dwords, so it is not
    used); the result matches the oracle."""
    from mambo_amd import _native
    from mambo_amd.utils.iq3_s_weight import ensure_packed, prepare_iq3_s_fields
    n, k = 256, 4096
    raw = oracle.gen_iq3s(57, n, k // 256)
    packed = ensure_packed(prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu), fields=False))
    xv, xs = oracle.quantize_mxfp8(np.random.default_rng(30 + m).standard_normal((m, k)).astype(np.float32))
    xvg = torch.from_numpy(xv).to(gpu)
    ld = k // 32 + 1
    buf = torch.zeros(1 + m * ld, dtype=torch.uint8, device=gpu)
    scales = buf[1:].view(m, ld)
    scales[:, :k // 32] = torch.from_numpy(xs).to(gpu)
    assert scales.data_ptr() % 2 == 1 and ld % 2 == 1
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=gpu)
    cfg = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 4, "split_k": 1, "tile_n": 16})
    lib = _native.lib()
    step(f"matmul M={m} scales at an odd address, row stride {ld}")
    rc = lib.mambo_iq3s_fp8_matmul(xvg.data_ptr(), k, scales.data_ptr(), ld, m, packed.data_ptr(), n, k // 256,
                                   out.data_ptr(), n, ctypes.byref(cfg), None)
    assert rc == 0, lib.mambo_last_error()
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.iq3s_fp8_matmul(xv, xs, raw, threads=oracle.default_threads()))
