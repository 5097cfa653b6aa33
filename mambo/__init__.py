"""The reference's package name for the MI355X path.

Callers written against Menooker/Mambo import the operator API under these module
paths (src/python/mambo/kernels/..., src/python/mambo/utils/...):

    mambo.kernels.quantize_fp8    -> mambo_amd.kernels.quantize_fp8
    mambo.kernels.iq3_s_fp8       -> mambo_amd.kernels.iq3_s_fp8
    mambo.utils.iq3_s_weight      -> mambo_amd.utils.iq3_s_weight
    mambo.utils.kernel_benchmark  -> mambo_amd.utils.kernel_benchmark

Each of those modules *is* the mambo_amd module (the same object in sys.modules), so
state such as BEST_CONFIGS is shared, and `python -m mambo.utils.kernel_benchmark`
runs the autotuning command.
"""

from mambo_amd import __version__  # noqa: F401
