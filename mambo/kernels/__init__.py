"""mambo.kernels: the reference's kernel modules (see mambo/__init__.py)."""
