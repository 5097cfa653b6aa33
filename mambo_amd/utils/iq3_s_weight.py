"""Persistent IQ3_S weight fields for the gfx950 kernels.

Mirrors src/python/mambo/utils/iq3_s_weight.py of the reference: the GGUF block
array u8 [N, K/256, 110] is split once, outside any timed region, into the SoA fields
the reference defines (d, qs, qh, signs, scales, each [B, N, ...]). The gfx950
projection kernels read one more private buffer, ``packed``: the same bytes permuted
into 16-row x 1-block tiles of 1760 bytes (layout in mambo_amd/csrc/mambo_common.h)
so that each lane of a wave loads its decode inputs with a few contiguous loads.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from mambo_amd import _native

IQ3_S_BLOCK_BYTES = 110
IQ3_S_BLOCK_VALUES = 256


@dataclass(frozen=True)
class IQ3SFields:
    """Byte-preserving SoA, K-block first and N rows second (iq3_s_weight.py:10-23).

    d: float16 [B,N]; qs: uint32 [B,N,16]; qh: uint16 [B,N,4];
    signs: int32 [B,N,8]; scales: uint32 [B,N]. Total: 110 bytes/block.
    packed: uint8 tile layout consumed by the projection kernels (None until built;
    launch_iq3_s_fp8_matmul builds it from the fields on first use).

    The packed tile is a cache of the SoA fields. It remembers which field tensors
    (address and in-place version) it was built from, and the launchers rebuild it when
    a field has been written in place or replaced (``dataclasses.replace``) since. A
    weight prepared with ``fields=False``, or whose fields were given up with
    ``release_soa_fields``, has placeholder fields; its packed tile is the weight itself.
    """

    d: torch.Tensor
    qs: torch.Tensor
    qh: torch.Tensor
    signs: torch.Tensor
    scales: torch.Tensor
    packed: torch.Tensor | None = None
    # fields_signature() of the SoA fields the packed tile was built from, or
    # PACKED_ONLY (the fields are placeholders)
    packed_from: tuple | None = field(default=None, repr=False, compare=False)


PACKED_ONLY = ("packed-only",)


def fields_signature(fields: IQ3SFields) -> tuple:
    """Identity of the SoA field tensors: data address (storage plus view offset) and
    in-place version counter of each (a write through any view of a tensor bumps its
    counter; ``set_`` bumps it too, and assigning ``.data`` moves the address). About
    half the host time of asking each tensor for its storage and offset, on every
    launch of a weight that keeps its fields."""
    return tuple((t.data_ptr(), t._version) for t in _weight_kernel_args(fields))


def _check_raw(iq3_weight) -> tuple[int, int]:
    if not isinstance(iq3_weight, torch.Tensor):
        raise ValueError("IQ3_S weight must be uint8 [N,K/256,110]")
    if iq3_weight.ndim != 3 or iq3_weight.dtype != torch.uint8 or iq3_weight.shape[2] != IQ3_S_BLOCK_BYTES:
        raise ValueError("IQ3_S weight must be uint8 [N,K/256,110]")
    n, blocks, _ = iq3_weight.shape
    if n < 1 or blocks < 1:
        raise ValueError("IQ3_S weight must have positive N and K")
    if not iq3_weight.is_cuda:
        raise ValueError("IQ3_S weight must be a GPU tensor")
    return int(n), int(blocks)


def packed_bytes(n: int, blocks: int) -> int:
    return int(_native.lib().mambo_iq3s_packed_bytes(n, blocks))


def prepare_iq3_s_fields(iq3_weight: torch.Tensor, *, fields: bool = True, pack: bool = False,
                         stream=None) -> IQ3SFields:
    """Split GGUF uint8 [N,B,110] blocks into SoA fields (and the tile layout) once.

    Follows prepare_iq3_s_fields (iq3_s_weight.py:25-54): any strides and any byte
    alignment of the source are accepted; every bit is preserved. By default only the
    SoA fields are built, as in the reference (110 bytes per block); the tile layout the
    projection kernels read (another 110 bytes per block) is built from them on the
    first launch and cached. ``pack=True`` builds both now, in one pass over the source.
    ``fields=False`` builds only the tile layout (the SoA tensors are then empty
    placeholders), which halves the memory of very large weights that are only
    multiplied; ``release_soa_fields`` does the same for a weight prepared with fields.
    """
    n, blocks = _check_raw(iq3_weight)
    dev = iq3_weight.device
    L = _native.lib()
    with torch.cuda.device(dev):
        packed = torch.empty(packed_bytes(n, blocks), dtype=torch.uint8, device=dev) if pack or not fields else None
        if fields:
            d = torch.empty((blocks, n), dtype=torch.float16, device=dev)
            qs = torch.empty((blocks, n, 16), dtype=torch.uint32, device=dev)
            qh = torch.empty((blocks, n, 4), dtype=torch.uint16, device=dev)
            signs = torch.empty((blocks, n, 8), dtype=torch.int32, device=dev)
            scales = torch.empty((blocks, n), dtype=torch.uint32, device=dev)
            ptrs = [d.data_ptr(), qs.data_ptr(), qh.data_ptr(), signs.data_ptr(), scales.data_ptr()]
        else:
            # zero-stride placeholders: right shapes, no memory
            d = _placeholder(torch.float16, (blocks, n), dev)
            qs = _placeholder(torch.uint32, (blocks, n, 16), dev)
            qh = _placeholder(torch.uint16, (blocks, n, 4), dev)
            signs = _placeholder(torch.int32, (blocks, n, 8), dev)
            scales = _placeholder(torch.uint32, (blocks, n), dev)
            ptrs = [None] * 5
        sn, sb, sbyte = iq3_weight.stride()
        _native.check(L.mambo_iq3s_prepare(iq3_weight.data_ptr(), n, blocks, sn, sb, sbyte, *ptrs,
                                           None if packed is None else packed.data_ptr(),
                                           _native.stream_handle(stream)),
                      "prepare_iq3_s_fields")
    result = IQ3SFields(d, qs, qh, signs, scales, packed)
    if packed is not None:
        object.__setattr__(result, "packed_from", fields_signature(result) if fields else PACKED_ONLY)
    return result


def _placeholder(dtype, shape, dev) -> torch.Tensor:
    """A zero-stride tensor of the field's dtype and shape that takes no memory."""
    return torch.zeros((), dtype=dtype, device=dev).expand(*shape)


def release_soa_fields(iq3_weight: IQ3SFields, stream=None) -> IQ3SFields:
    """Keep only the tile layout of a prepared weight: the packed tile is built (if it is
    not current), then the five SoA fields are replaced in place by zero-stride
    placeholders of the same shapes and dtypes, so their memory (110 bytes per block)
    is freed once nothing else holds them. Projections keep working and return the same
    results; reading the fields, or ``launch_dequant_iq3_s``, no longer gives the
    weight (the latter raises ValueError). For callers that only multiply: those that
    read the fields keep them by not calling this. Returns the same object."""
    ensure_packed(iq3_weight, stream)
    if iq3_weight.packed_from != PACKED_ONLY:
        dev = iq3_weight.d.device
        for name in ("d", "qs", "qh", "signs", "scales"):
            t = getattr(iq3_weight, name)
            object.__setattr__(iq3_weight, name, _placeholder(t.dtype, t.shape, dev))
        object.__setattr__(iq3_weight, "packed_from", PACKED_ONLY)
    return iq3_weight


def has_soa_fields(iq3_weight: IQ3SFields) -> bool:
    """Whether the SoA fields hold the weight (False after fields=False or
    release_soa_fields)."""
    return iq3_weight.packed_from != PACKED_ONLY


def _weight_dimensions(iq3_weight: IQ3SFields) -> tuple[int, int]:
    """Return N and the number of K blocks (iq3_s_weight.py:57-62)."""
    if not isinstance(iq3_weight, IQ3SFields):
        raise TypeError("prepare IQ3_S weights with prepare_iq3_s_fields before launch")
    blocks, n_rows = iq3_weight.d.shape
    return int(n_rows), int(blocks)


def _weight_kernel_args(iq3_weight: IQ3SFields) -> tuple[torch.Tensor, ...]:
    return (iq3_weight.d, iq3_weight.qs, iq3_weight.qh, iq3_weight.signs, iq3_weight.scales)


def _large_weight_kernel_args(iq3_weight: IQ3SFields) -> tuple[torch.Tensor, ...]:
    """Zero-copy views of the prepared fields (iq3_s_weight.py:65-77): qh as uint32
    [B,N,2], signs as int32 [B,N*8]. Kept for interface parity."""
    return (iq3_weight.d, iq3_weight.qs, iq3_weight.qh.view(torch.uint32),
            iq3_weight.signs.reshape(iq3_weight.signs.shape[0], -1), iq3_weight.scales)


def packed_is_current(iq3_weight: IQ3SFields) -> bool:
    """Whether the cached tile layout still holds the weight: it was built by
    prepare_iq3_s_fields(fields=False) (then it is the weight), or from SoA field
    tensors that are the current ones and have not been written in place since."""
    if iq3_weight.packed is None or iq3_weight.packed_from is None:
        return False
    return iq3_weight.packed_from == PACKED_ONLY or iq3_weight.packed_from == fields_signature(iq3_weight)


def ensure_packed(iq3_weight: IQ3SFields, stream=None) -> torch.Tensor:
    """Tile layout of the weight: the cached one while packed_is_current, else rebuilt
    from the current SoA fields (and cached)."""
    if packed_is_current(iq3_weight):
        return iq3_weight.packed
    n, blocks = _weight_dimensions(iq3_weight)
    for name, t in zip(("d", "qs", "qh", "signs", "scales"), _weight_kernel_args(iq3_weight)):
        if not t.is_contiguous():
            raise ValueError(f"IQ3SFields.{name} must be contiguous")
    dev = iq3_weight.d.device
    packed = torch.empty(packed_bytes(n, blocks), dtype=torch.uint8, device=dev)
    L = _native.lib()
    with torch.cuda.device(dev):
        _native.check(L.mambo_iq3s_pack(*(t.data_ptr() for t in _weight_kernel_args(iq3_weight)), n, blocks,
                                        packed.data_ptr(), _native.stream_handle(stream)), "pack")
    object.__setattr__(iq3_weight, "packed", packed)
    object.__setattr__(iq3_weight, "packed_from", fields_signature(iq3_weight))
    return packed
