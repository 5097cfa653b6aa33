"""Standalone F32/BF16 -> MXFP8 activation quantization on gfx950.

Mirror of src/python/mambo/kernels/quantize_fp8.py: ``launch_quantize_fp8`` returns
E4M3 value bytes [M, K] and one E8M0 scale byte per 32 values [M, K/32]. The kernel is
hand-written HIP (mambo_amd/csrc/quantize_mxfp8.hip) behind the C ABI; quantization
stays separate from the projection, as in the reference.
"""

from __future__ import annotations

import torch

from mambo_amd import _native

# Inert on gfx950: the kernel's launch shape is fixed (four lanes per 32-element group,
# 64 groups per workgroup, two rows per workgroup iteration) and no entry of this table
# changes it. The table is kept because the reference's launcher reads it: an
# architecture without an entry raises RuntimeError (quantize_fp8.py:60-64), and
# tile_m / tile_k_groups, given or looked up, are checked to be powers of two
# (quantize_fp8.py:73-74) and then ignored.
BEST_CONFIGS = {
    "gfx950": {
        "medium": {"tile_m": 4, "tile_k_groups": 4},
        "large": {"tile_m": 16, "tile_k_groups": 16},
    },
}
LARGE_TOKEN_THRESHOLD = 32


def _power_of_two(value: int, name: str) -> None:
    if value < 1 or value & (value - 1):
        raise ValueError(f"{name} must be a positive power of two")


def _activation_config(m: int) -> dict:
    arch = _native.device_arch()
    if arch not in BEST_CONFIGS:
        raise RuntimeError(f"FP8 activation quantizer has no tuned config for {arch}")
    return BEST_CONFIGS[arch]["large" if m >= LARGE_TOKEN_THRESHOLD else "medium"]


def launch_quantize_fp8(x: torch.Tensor, *, tile_m: int | None = None, tile_k_groups: int | None = None,
                        stream=None, out: tuple[torch.Tensor, torch.Tensor] | None = None
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """Return [M,K] E4M3 bytes and [M,K/32] E8M0 scale bytes (quantize_fp8.py:67-84).

    ``x`` is float32 (the reference's input type) or bfloat16, 2-D, K % 32 == 0, on the
    GPU. Row-strided inputs are read in place; inputs whose last dimension is not
    contiguous are copied first. ``out`` optionally supplies preallocated
    (values, scales) tensors.
    """
    if not isinstance(x, torch.Tensor) or x.ndim != 2 or x.dtype not in (torch.float32, torch.bfloat16) \
            or x.shape[1] % 32 or x.shape[0] < 1 or x.shape[1] < 32:
        raise ValueError("activation must be float32 or bfloat16 [M,K] with K divisible by 32")
    if not x.is_cuda:
        raise ValueError("activation must be a GPU tensor")
    if tile_m is None or tile_k_groups is None:
        with torch.cuda.device(x.device):
            config = _activation_config(x.shape[0])
        tile_m = config["tile_m"] if tile_m is None else tile_m
        tile_k_groups = config["tile_k_groups"] if tile_k_groups is None else tile_k_groups
    _power_of_two(tile_m, "tile_m")
    _power_of_two(tile_k_groups, "tile_k_groups")
    if x.stride(1) != 1:
        x = x.contiguous()
    m, k = x.shape
    if out is None:
        values = torch.empty((m, k), dtype=torch.uint8, device=x.device)
        scales = torch.empty((m, k // 32), dtype=torch.uint8, device=x.device)
    else:
        values, scales = out
        if values.shape != (m, k) or values.dtype != torch.uint8 or values.stride(1) != 1 \
                or scales.shape != (m, k // 32) or scales.dtype != torch.uint8 or scales.stride(1) != 1:
            raise ValueError("out must be (uint8 [M,K], uint8 [M,K/32]) with unit column stride")
    dtype = _native.DTYPE_F32 if x.dtype == torch.float32 else _native.DTYPE_BF16
    with torch.cuda.device(x.device):
        _native.check(_native.lib().mambo_quantize_mxfp8(
            x.data_ptr(), dtype, m, k, x.stride(0), values.data_ptr(), values.stride(0),
            scales.data_ptr(), scales.stride(0), _native.stream_handle(stream)), "launch_quantize_fp8")
    return values, scales
