"""IQ3_S preparation and the standalone decoder on the GPU against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, all_codes_blocks, make_synthetic_iq3_s
from oracle import oracle

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("n_rows,blocks", [(7, 3), (1, 1), (33, 2)])
def test_soa_fields_preserve_every_byte(gpu, n_rows, blocks):
    """test_iq3_s_fp8.py:134-148."""
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = make_synthetic_iq3_s(n_rows, blocks * 256, seed=0x50A)
    step(f"prepare [{n_rows},{blocks},110]")
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu), pack=True)
    torch.cuda.synchronize()
    reconstructed = np.empty_like(raw)
    for field, start, end in ((fields.d, 0, 2), (fields.qs, 2, 66), (fields.qh, 66, 74),
                              (fields.signs, 74, 106), (fields.scales, 106, 110)):
        assert field.is_contiguous()
        assert field.data_ptr() % field.element_size() == 0
        data = field.cpu().view(torch.uint8).numpy().reshape(blocks, n_rows, end - start)
        reconstructed[..., start:end] = data.transpose(1, 0, 2)
    np.testing.assert_array_equal(reconstructed, raw)
    assert sum(f.numel() * f.element_size() for f in (fields.d, fields.qs, fields.qh, fields.signs,
                                                      fields.scales)) == raw.nbytes
    # the private tile layout is a lossless permutation of the same bytes
    np.testing.assert_array_equal(unpack_tiles(fields.packed.cpu().numpy(), n_rows, blocks), raw)


def _tile_group(kb: int, h: int) -> int:
    """Weight group in K block kb of MFMA half h (tile layout in mambo_amd/csrc/mambo_common.h)."""
    return ((kb & 1) << 2) + ((kb >> 1) << 1) + h


def _slot_code(q: int, i: int) -> int:
    """Code (0..63) of the block held in slot i (0..15) of lane group q."""
    h, c = i >> 3, i & 7
    return 8 * _tile_group(2 * (c >> 2) + (q >> 1), h) + 4 * (q & 1) + (c & 3)


def unpack_tiles(packed: np.ndarray, n: int, blocks: int) -> np.ndarray:
    """Inverse of the 16-row x 1-block tile layout (mambo_amd/csrc/mambo_common.h)."""
    tiles = (n + 15) // 16
    p = packed.reshape(tiles, blocks, 1760)
    raw = np.zeros((tiles, 16, blocks, 110), dtype=np.uint8)
    for lane in range(64):
        r, q = lane & 15, lane >> 4
        words = p[:, :, 16 * lane:16 * lane + 16].copy().view("<u4").astype(np.uint64)
        tail = p[:, :, 1024 + 2 * lane:1026 + 2 * lane].copy().view("<u2").astype(np.uint64)
        w = [words[..., i] for i in range(4)] + [tail[..., 0], np.zeros_like(tail[..., 0])]
        for i in range(16):
            c = _slot_code(q, i)
            pos = 9 * i
            wi, sh = pos // 32, pos % 32
            val = ((w[wi] >> np.uint64(sh)) | (w[wi + 1] << np.uint64(32 - sh))) & np.uint64(0x1FF)
            raw[:, r, :, 2 + c] = (val & np.uint64(0xFF)).astype(np.uint8)
            raw[:, r, :, 66 + c // 8] |= ((val >> np.uint64(8)).astype(np.uint8) << np.uint8(c % 8))
        for h in range(2):
            t = p[:, :, 1152 + 8 * lane + 4 * h:1152 + 8 * lane + 4 * h + 4].copy().view("<u4")[..., 0]
            for c in range(8):
                code = _slot_code(q, 8 * h + c)
                for j in range(4):
                    bit = ((t >> np.uint32(c + 8 * j)) & np.uint32(1)).astype(np.uint8)
                    k = 4 * code + j
                    raw[:, r, :, 74 + k // 8] |= bit << np.uint8(k % 8)
        raw[:, r, :, 106 + q] = p[:, :, 1664 + lane]
        if q == 0:
            raw[:, r, :, 0:2] = p[:, :, 1728 + 2 * r:1730 + 2 * r]
    return raw.reshape(tiles * 16, blocks, 110)[:n]


def test_packed_decode_all_codes_and_sign_nibbles(gpu):
    """test_iq3_s_fp8.py:105-131: aligned, odd-address and strided sources all decode
    exactly to +-grid magnitudes."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_dequant_iq3_s
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    from conftest import e4m3_values
    raw, code, sign = all_codes_blocks()
    expected = oracle.dequant_iq3s(raw)
    aligned = torch.from_numpy(raw).to(gpu)
    allocation = torch.empty(raw.size + 1, dtype=torch.uint8, device=gpu)
    unaligned = allocation[1:].view(raw.shape)
    unaligned.copy_(aligned)
    strided_allocation = torch.empty((8, 16, 2 * 110), dtype=torch.uint8, device=gpu)
    strided = strided_allocation[..., ::2]
    strided.copy_(aligned)
    vals = e4m3_values().astype(np.float32)
    for name, source in (("aligned", aligned), ("unaligned", unaligned), ("strided", strided)):
        step(f"prepare+dequant all codes ({name})")
        fields = prepare_iq3_s_fields(source)
        bits, scales = launch_dequant_iq3_s(fields, tile_n=4)
        torch.cuda.synchronize()
        actual = vals[bits.cpu().numpy()] * np.repeat(scales.cpu().numpy(), 32, axis=1)
        np.testing.assert_array_equal(actual, expected)


def test_decode_matches_oracle_and_golden(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import launch_dequant_iq3_s
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    g = np.load(GOLDEN / "decode_random.npz")
    step("dequant golden [5,3,110]")
    bits, scales = launch_dequant_iq3_s(prepare_iq3_s_fields(torch.from_numpy(g["raw"]).to(gpu)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits.cpu().numpy(), g["values"])
    np.testing.assert_array_equal(scales.cpu().numpy(), g["scales"])
    raw = make_synthetic_iq3_s(300, 12 * 256, seed=99)
    step("dequant random [300,12,110]")
    bits, scales = launch_dequant_iq3_s(prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu)))
    torch.cuda.synchronize()
    eb, es = oracle.dequant_iq3s_fp8(raw)
    np.testing.assert_array_equal(bits.cpu().numpy(), eb)
    np.testing.assert_array_equal(scales.cpu().numpy(), es)


def test_pack_from_fields_matches_prepare(gpu):
    from mambo_amd.utils.iq3_s_weight import IQ3SFields, ensure_packed, prepare_iq3_s_fields
    raw = make_synthetic_iq3_s(45, 5 * 256, seed=3)
    step("prepare + pack from SoA [45,5,110]")
    f = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu), pack=True)
    assert prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu)).packed is None  # built on first launch
    g = IQ3SFields(f.d, f.qs, f.qh, f.signs, f.scales)
    packed = ensure_packed(g)
    torch.cuda.synchronize()
    assert torch.equal(packed, f.packed)


def test_gpu_generator_matches_oracle_rows(gpu):
    from mambo_amd import _native
    blocks, rows = 32, 64
    raw = torch.empty((rows, blocks, 110), dtype=torch.uint8, device=gpu)
    step("synth iq3s rows 1000..1063")
    _native.check(_native.lib().mambo_synth_iq3s(0, blocks, 1000, rows, raw.data_ptr(),
                                                 _native.stream_handle(None)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(raw.cpu().numpy(), oracle.gen_iq3s(0, rows, blocks, row0=1000))


def test_get_iq3_table_is_the_decoders_codebook(gpu):
    """_get_iq3_table (iq3_s_fp8.py:97-102): the E4M3-encoded codebook as uint32 [512] on
    the current device, uploaded once and cached, equal to iq3_s_fp8_table(); and the
    standalone decoder emits exactly its bytes: weight 4c + j of every code c of the
    all-codes blocks is byte j of table[index c] with the weight's sign on bit 7."""
    from mambo_amd.kernels import iq3_s_fp8 as mod
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    step("_get_iq3_table on the current device")
    table = mod._get_iq3_table()
    assert table.device == gpu and table.dtype == torch.uint32 and tuple(table.shape) == (512,)
    assert mod._get_iq3_table() is table
    host = table.cpu().numpy()
    np.testing.assert_array_equal(host, mod.iq3_s_fp8_table())
    raw, code, sign = all_codes_blocks()
    step("dequant all codes against the device table")
    bits, _ = mod.launch_dequant_iq3_s(prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu)))
    torch.cuda.synchronize()
    mags = host[code].view(np.uint8).reshape(*code.shape, 4)  # byte j of each code's word
    signs = ((sign[..., None] >> np.arange(4, dtype=np.uint16)) & 1).astype(np.uint8) << 7
    expected = (mags | signs).reshape(raw.shape[0], -1)
    np.testing.assert_array_equal(bits.cpu().numpy(), expected)


def test_large_weight_kernel_args_views(gpu):
    """_large_weight_kernel_args (iq3_s_weight.py:65-77): zero-copy views qh -> uint32
    [B,N,2] and signs -> int32 [B,N*8]; d, qs and scales unchanged; the viewed bytes are
    the raw blocks' qh and sign bytes."""
    from mambo_amd.utils.iq3_s_weight import _large_weight_kernel_args, _weight_kernel_args, prepare_iq3_s_fields
    n_rows, blocks = 37, 3
    raw = make_synthetic_iq3_s(n_rows, blocks * 256, seed=0x1A6)
    step(f"prepare [{n_rows},{blocks},110] for the large-MMA views")
    fields = prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))
    d, qs, qh, signs, scales = _large_weight_kernel_args(fields)
    base = _weight_kernel_args(fields)
    assert d is base[0] and qs is base[1] and scales is base[4]
    assert qh.dtype == torch.uint32 and tuple(qh.shape) == (blocks, n_rows, 2)
    assert signs.dtype == torch.int32 and tuple(signs.shape) == (blocks, n_rows * 8)
    assert qh.data_ptr() == fields.qh.data_ptr() and signs.data_ptr() == fields.signs.data_ptr()
    torch.cuda.synchronize()
    qh_bytes = qh.cpu().view(torch.uint8).numpy().reshape(blocks, n_rows, 8)
    np.testing.assert_array_equal(qh_bytes.transpose(1, 0, 2), raw[..., 66:74])
    sign_bytes = signs.cpu().view(torch.uint8).numpy().reshape(blocks, n_rows, 32)
    np.testing.assert_array_equal(sign_bytes.transpose(1, 0, 2), raw[..., 74:106])
