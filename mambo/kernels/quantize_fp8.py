"""mambo.kernels.quantize_fp8 (reference module path) is mambo_amd.kernels.quantize_fp8."""

import sys

from mambo_amd.kernels.quantize_fp8 import __name__ as _impl_name

sys.modules[__name__] = sys.modules[_impl_name]
