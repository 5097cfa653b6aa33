"""mambo.utils: the reference's utility modules (see mambo/__init__.py)."""
