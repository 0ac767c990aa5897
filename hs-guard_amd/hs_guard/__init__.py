"""HS-Guard streaming slot step on MI355X (gfx950): drop-in ``load_model`` / ``StreamingGuard``."""
__all__ = ["StreamingGuard", "load_model"]


def __getattr__(name):
    if name in __all__:
        from . import runtime
        return getattr(runtime, name)
    raise AttributeError(name)
