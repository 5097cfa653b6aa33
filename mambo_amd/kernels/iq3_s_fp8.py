"""IQ3_S block decode and block-scaled FP8 projection on gfx950.

Mirror of src/python/mambo/kernels/iq3_s_fp8.py. The projection reads prepared IQ3_S
weights (IQ3SFields) and prequantized MXFP8 activations and decodes the IQ3_S blocks
inside the GEMM tile; the decoded weights never reach HBM. A standalone decoder serves
independent correctness checks. The kernels are hand-written HIP for gfx950
(mambo_amd/csrc/iq3s_gemm.hip, iq3s_layout.hip) behind the C ABI.

One IQ3_S block along K (256 weights, 110 bytes):

    byte  0..1   | d: FP16 base scale                 |  2 bytes
    byte  2..65  | qs: 64 low 8-bit codebook indices  | 64 bytes
    byte 66..73  | qh: 64 high index bits             |  8 bytes
    byte 74..105 | signs: one bit per weight          | 32 bytes
    byte 106..109| scales: 8 packed 4-bit values      |  4 bytes

Each 9-bit (qs, qh) index selects four magnitudes from the codebook; each group of 32
weights uses scale d * (1 + 2 * scale_nibble).
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

from mambo_amd import _native
from mambo_amd.utils.iq3_s_weight import (
    IQ3SFields,
    IQ3_S_BLOCK_BYTES,
    IQ3_S_BLOCK_VALUES,
    _weight_dimensions,
    _weight_kernel_args,
    ensure_packed,
    has_soa_fields,
    prepare_iq3_s_fields,
    release_soa_fields,
)

IQ3_S_SCALE_VALUES = 32
_IQ3_TABLES: dict[int, torch.Tensor] = {}

# Launch configurations per architecture, selected by token count as in the reference
# (iq3_s_fp8.py:49-60). Fields follow mambo_gemm_config; 0 = the library's per-shape
# default (kernel family by M, waves sized to about two residency rounds, K split only
# for small grids). Per-shape autotuned entries (tuned_gfx950.json, written by
# mambo_amd.utils.kernel_benchmark) take precedence.
BEST_CONFIGS = {
    "gfx950": {
        "medium": {"kernel": _native.GEMM_AUTO, "waves": 0, "split_k": 0},
        "large": {"kernel": _native.GEMM_AUTO, "waves": 0, "split_k": 0},
    },
}
LARGE_TOKEN_THRESHOLD = 32
TUNED_PATH = Path(__file__).resolve().parent / "tuned_gfx950.json"


@lru_cache(maxsize=1)
def _tuned_table() -> dict:
    if TUNED_PATH.exists():
        return json.loads(TUNED_PATH.read_text())
    return {}


def m_bucket(m: int) -> int:
    """Token-count bucket of the tuned table: the next power of two >= m."""
    return 1 << max(0, (int(m) - 1).bit_length())


def tuned_key(n: int, k: int, m: int) -> str:
    return f"{n}x{k}@{m_bucket(m)}"


@lru_cache(maxsize=1)
def iq3_s_table() -> np.ndarray:
    """The 512-entry IQ3_S codebook (iq3s_grid), four magnitudes per uint32."""
    out = np.zeros(512, dtype=np.uint32)
    _native.check(_native.lib().mambo_iq3s_grid(out.ctypes.data), "iq3_s_table")
    if out.shape != (512,):
        raise ValueError(f"expected 512 IQ3_S table entries, got {out.size}")
    return out


@lru_cache(maxsize=1)
def iq3_s_fp8_table() -> np.ndarray:
    """The codebook with every magnitude byte replaced by its E4M3 bits
    (iq3_s_fp8.py:77-94): the table the kernels decode with, as the library built it.
    Raises ValueError if a codebook byte is not one of the odd magnitudes 1..15, which
    are the ones with an exact E4M3 encoding."""
    grid_bytes = iq3_s_table().view(np.uint8)
    if np.any((grid_bytes & 1) == 0) or np.any(grid_bytes > 15):
        raise ValueError("IQ3_S codebook contains a magnitude without an E4M3 encoding")
    out = np.zeros(512, dtype=np.uint32)
    _native.check(_native.lib().mambo_iq3s_fp8_grid(out.ctypes.data), "iq3_s_fp8_table")
    return out


def _get_iq3_table() -> torch.Tensor:
    """FP8-encoded codebook, uint32 [512], uploaded once per device and cached
    (iq3_s_fp8.py:97-102). The kernels carry their own copy in the code object; this
    tensor is for callers that want it."""
    device = torch.cuda.current_device()
    if device not in _IQ3_TABLES:
        _IQ3_TABLES[device] = torch.from_numpy(iq3_s_fp8_table().copy()).to(f"cuda:{device}")
    return _IQ3_TABLES[device]


def _power_of_two(value: int, name: str) -> None:
    if value < 1 or value & (value - 1):
        raise ValueError(f"{name} must be a positive power of two")


def launch_dequant_iq3_s(iq3_weight: IQ3SFields, *, tile_n: int = 1, stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Return [N,K] E4M3 bit patterns and [N,K/32] original F32 scales (iq3_s_fp8.py:341-351).

    ``tile_n`` is validated (power of two) as in the reference; the gfx950 decoder's
    launch shape does not depend on it.
    """
    _power_of_two(tile_n, "tile_n")
    n_rows, blocks = _weight_dimensions(iq3_weight)
    if not has_soa_fields(iq3_weight):
        raise ValueError("the decoder reads the SoA fields; this weight holds only its tile layout "
                         "(prepared with fields=False, or after release_soa_fields)")
    fields = _weight_kernel_args(iq3_weight)
    for name, t in zip(("d", "qs", "qh", "signs", "scales"), fields):
        if not t.is_contiguous() or t.numel() == 0 and n_rows * blocks:
            raise ValueError(f"IQ3SFields.{name} must be a contiguous prepared field")
    dev = iq3_weight.d.device
    values = torch.empty((n_rows, blocks * 256), dtype=torch.uint8, device=dev)
    scales = torch.empty((n_rows, blocks * 8), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _native.check(_native.lib().mambo_iq3s_dequant(*(t.data_ptr() for t in fields), n_rows, blocks,
                                                       values.data_ptr(), scales.data_ptr(),
                                                       _native.stream_handle(stream)), "launch_dequant_iq3_s")
    return values, scales


def select_config(m: int, n: int, k: int, arch: str | None = None) -> dict:
    """Launch configuration for an [M, K] x [N, K] projection on `arch`."""
    arch = arch or _native.device_arch()
    if arch not in BEST_CONFIGS:
        raise RuntimeError(f"IQ3_S FP8 matmul has no tuned config for {arch}")
    tuned = _tuned_table().get(arch, {}).get(tuned_key(n, k, m))
    if tuned is not None:
        return dict(tuned)
    return default_config(m, arch)


def default_config(m: int, arch: str = "gfx950") -> dict:
    """The configuration used for M tokens when the tuned table has no entry."""
    return dict(BEST_CONFIGS[arch]["medium" if m < LARGE_TOKEN_THRESHOLD else "large"])


def _prepare_activations(x_values, x_scales, k: int):
    """Validate MXFP8 activations [M,K] + [M,K/32]; return them in a form the kernels
    read in place (unit column stride, 16-byte aligned rows), copying only if needed."""
    if not isinstance(x_values, torch.Tensor) or x_values.ndim != 2 or x_values.dtype != torch.uint8 \
            or x_values.shape[0] < 1 or x_values.shape[1] != k:
        raise ValueError("x_values must be uint8 [M,K]")
    m = int(x_values.shape[0])
    if not isinstance(x_scales, torch.Tensor) or tuple(x_scales.shape) != (m, k // 32) \
            or x_scales.dtype != torch.uint8:
        raise ValueError("x_scales must be uint8 [M,K/32]")
    if x_scales.device != x_values.device:
        raise ValueError("x_values and x_scales must be on the same device")
    x_values = _aligned_rows(x_values, 16)
    # the tiled kernel copies each token's 8 scale bytes of a block as two dwords
    x_scales = _aligned_rows(x_scales, 8)
    return x_values, x_scales, m


def _aligned_rows(t: torch.Tensor, align: int) -> torch.Tensor:
    """`t` itself when its rows are unit-stride and start on `align`-byte boundaries,
    else a contiguous copy (rows of K and K/32 bytes are multiples of 16 and 8)."""
    if t.stride(1) == 1 and t.stride(0) % align == 0 and t.data_ptr() % align == 0:
        return t
    return torch.empty(t.shape, dtype=t.dtype, device=t.device).copy_(t)


def _output(out, m: int, n: int, dev) -> torch.Tensor:
    if out is None:
        return torch.empty((m, n), dtype=torch.float32, device=dev)
    if tuple(out.shape) != (m, n) or out.dtype != torch.float32 or out.stride(1) != 1 or out.device != dev:
        raise ValueError("out must be float32 [M,N] with unit column stride on the activations' device")
    return out


def launch_iq3_s_fp8_matmul(x_values: torch.Tensor, x_scales: torch.Tensor, iq3_weight: IQ3SFields,
                            *, stream=None, config: dict | None = None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """Multiply prepared IQ3_S weights by prequantized MXFP8 activations (iq3_s_fp8.py:364-399).

    x_values uint8 [M,K] (E4M3), x_scales uint8 [M,K/32] (E8M0); returns float32 [M,N].
    Row-strided activations are read in place; a non-unit column stride (or a row
    stride that is not a multiple of 16 bytes) is copied first. ``config`` overrides
    the tuned launch configuration (mambo_gemm_config fields); ``out`` optionally
    supplies the float32 [M,N] output (unit column stride).
    """
    n_rows, k_blocks = _weight_dimensions(iq3_weight)
    k = k_blocks * IQ3_S_BLOCK_VALUES
    x_values, x_scales, m = _prepare_activations(x_values, x_scales, k)
    dev = x_values.device
    with torch.cuda.device(dev):
        cfg = _native.GemmConfig.from_dict(config if config is not None else select_config(m, n_rows, k))
        packed = ensure_packed(iq3_weight, stream)
        out = _output(out, m, n_rows, dev)
        _native.check(_native.lib().mambo_iq3s_fp8_matmul(
            x_values.data_ptr(), x_values.stride(0), x_scales.data_ptr(), x_scales.stride(0), m,
            packed.data_ptr(), n_rows, k_blocks, out.data_ptr(), out.stride(0), cfg,
            _native.stream_handle(stream)), "launch_iq3_s_fp8_matmul")
    return out


def launch_iq3_s_fp8_matmul_grouped(x_values: torch.Tensor, x_scales: torch.Tensor, iq3_weights,
                                    *, stream=None, config: dict | None = None, outs=None) -> list[torch.Tensor]:
    """Several projections of the same MXFP8 activations in one launch (no reference
    counterpart; the reference calls launch_iq3_s_fp8_matmul per weight,
    iq3_s_fp8.py:364-399). For projections that share an input - q/k/v, gate/up - this
    returns what one launch_iq3_s_fp8_matmul per weight returns, with one launch.

    ``iq3_weights``: 1..4 IQ3SFields with the same K. ``outs``: optional float32
    [M, N_i] outputs. ``config``: as for launch_iq3_s_fp8_matmul, defaulting to the
    tuned or library configuration for the summed N.
    """
    weights = list(iq3_weights)
    if not 1 <= len(weights) <= _native.MAX_GROUP:
        raise ValueError(f"between 1 and {_native.MAX_GROUP} weights per grouped launch")
    dims = [_weight_dimensions(w) for w in weights]
    k_blocks = dims[0][1]
    if any(b != k_blocks for _, b in dims):
        raise ValueError("grouped weights must share K")
    k = k_blocks * IQ3_S_BLOCK_VALUES
    x_values, x_scales, m = _prepare_activations(x_values, x_scales, k)
    dev = x_values.device
    if outs is not None and len(outs) != len(weights):
        raise ValueError("outs must hold one output per weight")
    n_total = sum(n for n, _ in dims)
    with torch.cuda.device(dev):
        cfg = _native.GemmConfig.from_dict(config if config is not None else select_config(m, n_total, k))
        result = [_output(None if outs is None else outs[i], m, n, dev) for i, (n, _) in enumerate(dims)]
        projections = (_native.Projection * len(weights))()
        for i, (w, (n, _)) in enumerate(zip(weights, dims)):
            projections[i] = _native.Projection(ensure_packed(w, stream).data_ptr(), n, result[i].data_ptr(),
                                                result[i].stride(0))
        _native.check(_native.lib().mambo_iq3s_fp8_matmul_grouped(
            x_values.data_ptr(), x_values.stride(0), x_scales.data_ptr(), x_scales.stride(0), m,
            projections, len(weights), k_blocks, cfg, _native.stream_handle(stream)),
            "launch_iq3_s_fp8_matmul_grouped")
    return result


def launch_iq3_s_matmul_quantize(x: torch.Tensor, iq3_weights, *, stream=None, config: dict | None = None,
                                 outs=None):
    """MXFP8 quantization of ``x`` and the projection(s) in one call (no reference
    counterpart: the reference runs launch_quantize_fp8 and then
    launch_iq3_s_fp8_matmul, quantize_fp8.py:1-4). ``x``: float32 or bfloat16 [M, K] on
    the GPU. ``iq3_weights``: one IQ3SFields (returns a tensor) or 1..4 with the same K
    (returns a list, as launch_iq3_s_fp8_matmul_grouped). For M <= 4 on the stream
    kernel every workgroup quantizes the rows into its LDS copy itself - one launch
    instead of two, results bit-identical to the two-step path under the same config;
    other shapes run the quantizer and the GEMM back to back on the stream."""
    single = isinstance(iq3_weights, IQ3SFields)
    weights = [iq3_weights] if single else list(iq3_weights)
    if not 1 <= len(weights) <= _native.MAX_GROUP:
        raise ValueError(f"between 1 and {_native.MAX_GROUP} weights per call")
    dims = [_weight_dimensions(w) for w in weights]
    k_blocks = dims[0][1]
    if any(b != k_blocks for _, b in dims):
        raise ValueError("weights must share K")
    k = k_blocks * IQ3_S_BLOCK_VALUES
    if not isinstance(x, torch.Tensor) or x.ndim != 2 or x.shape[0] < 1 or x.shape[1] != k:
        raise ValueError(f"x must be [M,{k}]")
    dtypes = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}
    if x.dtype not in dtypes:
        raise ValueError(f"x must be float32 or bfloat16, got {x.dtype}")
    if x.stride(1) != 1:
        x = x.contiguous()
    m, dev = int(x.shape[0]), x.device
    if outs is not None and len(outs) != len(weights):
        raise ValueError("outs must hold one output per weight")
    n_total = sum(n for n, _ in dims)
    with torch.cuda.device(dev):
        cfg = _native.GemmConfig.from_dict(config if config is not None else select_config(m, n_total, k))
        result = [_output(None if outs is None else outs[i], m, n, dev) for i, (n, _) in enumerate(dims)]
        projections = (_native.Projection * len(weights))()
        for i, (w, (n, _)) in enumerate(zip(weights, dims)):
            projections[i] = _native.Projection(ensure_packed(w, stream).data_ptr(), n, result[i].data_ptr(),
                                                result[i].stride(0))
        # MXFP8 buffers for shapes that quantize in a launch of their own
        xv = torch.empty((m, k), dtype=torch.uint8, device=dev)
        xs = torch.empty((m, k // 32), dtype=torch.uint8, device=dev)
        _native.check(_native.lib().mambo_iq3s_matmul_quantize_grouped(
            x.data_ptr(), dtypes[x.dtype], x.stride(0), m, projections, len(weights), k_blocks, cfg,
            xv.data_ptr(), xv.stride(0), xs.data_ptr(), xs.stride(0), _native.stream_handle(stream)),
            "launch_iq3_s_matmul_quantize")
    return result[0] if single else result


@dataclass
class ChainLaunch:
    """One launch of a chained call (launch_iq3_s_fp8_matmul_chain): 1..4 weights with the
    same K applied to the same activations. ``x``: uint8 [M, K] E4M3 values with
    ``x_scales`` uint8 [M, K/32] E8M0, or float32 / bfloat16 [M, K] rows (quantized to
    MXFP8 inside the kernel, as launch_quantize_fp8 would) - for instance the output of an
    earlier launch of the same chain. ``outs``: optional float32 [M, N_i] outputs."""

    x: torch.Tensor
    weights: list
    x_scales: torch.Tensor | None = None
    outs: list | None = field(default=None)


def new_chain_sync(device=None) -> torch.Tensor:
    """Zeroed sync words for chained calls (MAMBO_CHAIN_SYNC_WORDS int32). Calls ordered on
    one stream may share them (each call leaves them zero); calls that may overlap need
    their own."""
    return torch.zeros(_native.CHAIN_SYNC_WORDS, dtype=torch.int32, device=device or "cuda")


def chain_status(sync: torch.Tensor) -> None:
    """Raise RuntimeError if a chained call on ``sync`` had a dependency wait time out
    (synchronises with the device; clears the reported status)."""
    with torch.cuda.device(sync.device):
        _native.check(_native.lib().mambo_chain_status(sync.data_ptr()), "chain_status")


def launch_iq3_s_fp8_matmul_chain(launches, *, stream=None, waves: int = 0, sync: torch.Tensor | None = None,
                                  timeout_us: int = 0, tiles_per_workgroup: int = 0, wait_bias: int = 0) -> list:
    """Up to MAX_CHAIN launches at 1..4 tokens in one kernel launch, in order (no
    reference counterpart: the reference calls launch_iq3_s_fp8_matmul per weight,
    iq3_s_fp8.py:364-399). Returns, per launch, the list of its float32 [M, N_i] outputs:
    what launch_iq3_s_fp8_matmul_grouped returns for each launch run one after the other
    on the stream (bit-identical with the same ``waves``, 4, 8 or 16; 0 = the library's).
    Launch i reads its activations only after every output of the launches before it is
    stored, so a launch may take an earlier launch's output as its float32 input.
    ``sync``: zeroed sync words (new_chain_sync), reusable by calls ordered on one stream;
    default: fresh ones per call. ``timeout_us``, ``tiles_per_workgroup``, ``wait_bias``:
    see mambo_chain_config (wait_bias is for tests that force a timeout; check with
    chain_status)."""
    launches = list(launches)
    if not 1 <= len(launches) <= _native.MAX_CHAIN:
        raise ValueError(f"between 1 and {_native.MAX_CHAIN} launches per chained call")
    dtypes = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}
    descs = (_native.ChainLaunch * len(launches))()
    results, m, dev = [], None, None
    for i, cl in enumerate(launches):
        if not isinstance(cl, ChainLaunch):
            raise TypeError("launches must be ChainLaunch objects")
        weights = list(cl.weights)
        if not 1 <= len(weights) <= _native.MAX_GROUP:
            raise ValueError(f"launch {i}: between 1 and {_native.MAX_GROUP} weights")
        dims = [_weight_dimensions(w) for w in weights]
        k_blocks = dims[0][1]
        if any(b != k_blocks for _, b in dims):
            raise ValueError(f"launch {i}: weights must share K")
        k = k_blocks * IQ3_S_BLOCK_VALUES
        x = cl.x
        if not isinstance(x, torch.Tensor) or x.ndim != 2 or x.shape[0] < 1 or x.shape[1] != k:
            raise ValueError(f"launch {i}: x must be [M,{k}]")
        if m is None:
            m, dev = int(x.shape[0]), x.device
        if int(x.shape[0]) != m or x.device != dev:
            raise ValueError("every launch of a chain takes the same M tokens on the same device")
        desc = descs[i]
        if x.dtype == torch.uint8:
            x, xs, _ = _prepare_activations(x, cl.x_scales, k)  # rows 16- and 8-byte aligned
            desc.x_dtype, desc.xs, desc.ldxs = _native.DTYPE_MXFP8, xs.data_ptr(), xs.stride(0)
        elif x.dtype in dtypes:
            if cl.x_scales is not None:
                raise ValueError(f"launch {i}: x_scales belongs to MXFP8 (uint8) activations")
            esz = x.element_size()
            if x.stride(1) != 1 or x.data_ptr() % 16 or (x.stride(0) * esz) % 16:
                x = x.contiguous() if x.data_ptr() % 16 == 0 else x.clone()
            desc.x_dtype, desc.xs, desc.ldxs = dtypes[x.dtype], None, 0
        else:
            raise ValueError(f"launch {i}: x must be uint8 (MXFP8), float32 or bfloat16, got {x.dtype}")
        if cl.outs is not None and len(cl.outs) != len(weights):
            raise ValueError(f"launch {i}: outs must hold one output per weight")
        with torch.cuda.device(dev):
            outs = [_output(None if cl.outs is None else cl.outs[j], m, n, dev) for j, (n, _) in enumerate(dims)]
            for j, (w, (n, _)) in enumerate(zip(weights, dims)):
                desc.proj[j] = _native.Projection(ensure_packed(w, stream).data_ptr(), n, outs[j].data_ptr(),
                                                  outs[j].stride(0))
        desc.x, desc.ldx, desc.count, desc.blocks = x.data_ptr(), x.stride(0), len(weights), k_blocks
        results.append((outs, x))
    cfg = _native.ChainConfig()
    cfg.waves, cfg.tiles_per_workgroup, cfg.timeout_us, cfg.wait_bias = waves, tiles_per_workgroup, timeout_us, \
        wait_bias
    with torch.cuda.device(dev):
        if sync is None:
            sync = new_chain_sync(dev)
        if sync.dtype not in (torch.int32, torch.uint32) or sync.numel() < _native.CHAIN_SYNC_WORDS \
                or not sync.is_contiguous() or sync.device != dev:
            raise ValueError(f"sync must be {_native.CHAIN_SYNC_WORDS} contiguous int32 words on the device")
        _native.check(_native.lib().mambo_iq3s_fp8_matmul_chain(m, descs, len(launches), cfg, sync.data_ptr(),
                                                                _native.stream_handle(stream)),
                      "launch_iq3_s_fp8_matmul_chain")
    return [outs for outs, _ in results]


def gemm_search_space(m: int, n: int, k: int) -> list[dict]:
    """Candidate launch configurations for the autotuner (the analogue of the cuTile
    search spaces of iq3_s_fp8.py:416-459), as mambo_gemm_config_enumerate lists them:
    led by the library default for the token count, then the block-diagonal stream kernel
    up to 16 tokens and the dense kernel up to 128 (each re-reads every weight once per
    16- or 32-token chunk, so neither is a candidate beyond), x waves per workgroup x K
    split x weight rows (and, dense above 16 tokens, tokens) per workgroup; the tiled
    kernel's 16-token tiles for 5..64 tokens and its larger tile shapes from 32."""
    if k % IQ3_S_BLOCK_VALUES:
        raise ValueError(f"K={k} must be a multiple of {IQ3_S_BLOCK_VALUES}")
    lib = _native.lib()
    blocks = k // IQ3_S_BLOCK_VALUES
    count = lib.mambo_gemm_config_enumerate(m, n, blocks, None, 0)
    if count < 0:
        _native.check(int(count), "gemm_search_space")
    configs = (_native.GemmConfig * count)()
    _native.check(0 if lib.mambo_gemm_config_enumerate(m, n, blocks, configs, count) == count else -1,
                  "gemm_search_space")
    space = []
    for c in configs:
        if c.kernel == _native.GEMM_AUTO:
            space.append(default_config(m))
        elif c.kernel == _native.GEMM_STREAM:
            space.append({"kernel": c.kernel, "waves": c.waves, "split_k": c.split_k, "tile_n": c.tile_n})
        else:
            space.append({"kernel": c.kernel, "waves": c.waves, "split_k": c.split_k, "tile_n": c.tile_n,
                          "tile_m": c.tile_m})
    return space


def make_benchmark_cases(iq3_weight: torch.Tensor, tokens: tuple[int, ...] = (4, 128), *,
                         rotate_bytes: int = 0, max_copies: int = 64) -> list:
    """Prepare weights and MXFP8 inputs once; benchmark only the projection
    (iq3_s_fp8.py:402-465). ``iq3_weight`` is raw GGUF uint8 [N,B,110] on the GPU.
    With ``rotate_bytes`` the cases cycle over copies of the packed weight (together at
    least that many bytes, at most ``max_copies``), so that each launch streams its
    weight from HBM as the projections of a many-layer decode step do."""
    from dataclasses import replace

    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    from mambo_amd.utils.kernel_benchmark import BenchmarkCase

    fields = prepare_iq3_s_fields(iq3_weight, fields=False)
    n_rows, k_blocks = _weight_dimensions(fields)
    k = k_blocks * IQ3_S_BLOCK_VALUES
    copies = max(1, min(max_copies, -(-int(rotate_bytes) // fields.packed.numel())))
    weights = [fields] + [replace(fields, packed=fields.packed.clone()) for _ in range(copies - 1)]
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=iq3_weight.device)
    gen.manual_seed(0)

    def make_case(m: int):
        x = torch.randn((m, k), dtype=torch.float32, device=iq3_weight.device, generator=gen)
        x_values, x_scales = launch_quantize_fp8(x, stream=stream)
        out = torch.empty((m, n_rows), dtype=torch.float32, device=iq3_weight.device)
        turn = [0]

        def launch(config):
            # the current stream: the capture stream while a timing graph is recorded
            w = weights[turn[0] % copies]
            turn[0] += 1
            launch_iq3_s_fp8_matmul(x_values, x_scales, w, config=config, out=out)

        return BenchmarkCase(name=f"M={m} N={n_rows} K={k}", stream=stream, launch=launch,
                             search_space=gemm_search_space(m, n_rows, k),
                             summary_keys=("kernel", "waves", "split_k", "tile_m", "tile_n"),
                             key=tuned_key(n_rows, k, m), rotation=copies, default=default_config(m))

    return [make_case(m) for m in tokens]
