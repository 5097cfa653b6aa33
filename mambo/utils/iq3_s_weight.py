"""mambo.utils.iq3_s_weight (reference module path) is mambo_amd.utils.iq3_s_weight."""

import sys

from mambo_amd.utils.iq3_s_weight import __name__ as _impl_name

sys.modules[__name__] = sys.modules[_impl_name]
