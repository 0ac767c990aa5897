"""HS-Guard streaming slot step on MI355X (gfx950): drop-in ``load_model`` / ``StreamingGuard`` and the
complete-message scorer ``score_messages``."""
__all__ = ["StreamingGuard", "load_model", "score_messages", "score_ids", "serialize", "encode_messages", "selfcheck"]


def __getattr__(name):
    if name in __all__:
        from . import runtime
        return getattr(runtime, name)
    raise AttributeError(name)
