"""mambo.utils.kernel_benchmark (reference module path) is
mambo_amd.utils.kernel_benchmark; run as a module it is the autotuning command
(`python -m mambo.utils.kernel_benchmark iq3_s_fp8 --model M.gguf --weight-name NAME`,
kernel_benchmark.py:131-145)."""

import sys

from mambo_amd.utils import kernel_benchmark as _impl

if __name__ == "__main__":
    _impl.benchmark_main()
else:
    sys.modules[__name__] = _impl
