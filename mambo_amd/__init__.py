"""mambo_amd: MI355X (gfx950) fused IQ3_S x MXFP8 projection path.

Operator API (mirrors the reference's mambo.kernels / mambo.utils modules):
    mambo_amd.kernels.quantize_fp8.launch_quantize_fp8
    mambo_amd.utils.iq3_s_weight.prepare_iq3_s_fields / IQ3SFields
    mambo_amd.kernels.iq3_s_fp8.launch_dequant_iq3_s / launch_iq3_s_fp8_matmul
    mambo_amd.utils.kernel_benchmark (autotuner / benchmark CLI)
The kernels live in libmambo_hip.so (gfx950 HIP, C ABI in include/mambo_hip.h).
"""

__version__ = "0.1.0"
