"""Drop-in public API: ``load_model`` and ``StreamingGuard`` (src/hs_guard/runtime.py:92-125,148-174).

``StreamingGuard(model, metadata, max_slots).step([(slot, token_ids)], role)`` returns, per request,
``{'slot', 'cut_scores': [1 - p(safe) per submitted token], 'threshold'}`` with the reference's validation
and error messages. ``reset()`` clears every slot.
"""
from __future__ import annotations

import json
from pathlib import Path

LABELS = ("safe", "unsafe", "controversial")
MODEL_ID = "KrisLiu16/HS-Guard-v10"
# Red-line thresholds (prompt / response) and general thresholds of the released model (docs/ENGINE.md:14).
DEFAULT_THRESHOLDS = {"redline": {"user": 0.0761368871, "assistant": 0.1117895246},
                      "general": {"user": 0.5, "assistant": 0.5}}


def random_metadata(head="redline", window_tokens=512):
    """Metadata of a random-init model, shaped like the released bundle's hs_guard.json after load_model."""
    return {"format": "hs-guard-v1", "risk_labels": list(LABELS), "window_tokens": window_tokens, "head": head,
            "thresholds": dict(DEFAULT_THRESHOLDS[head])}


def load_model(model=MODEL_ID, *, revision=None, head="redline", config=None, seed=0, device="cuda"):
    """Returns (model, tokenizer, metadata) like src/hs_guard/runtime.py:92-125.

    ``model="random"`` (or a GuardConfig passed as ``config``) builds seeded random-init weights of that
    geometry on ``device`` (tokenizer None). A local bundle directory is not loadable yet, and hub names
    need a network fetch, which this build does not do: both raise."""
    if head not in ("redline", "general"):
        raise ValueError("head must be redline or general")
    import torch
    from .model import GuardConfig, GuardModel
    if config is not None or model == "random":
        if not torch.cuda.is_available():
            raise RuntimeError("HS-Guard requires an AMD Instinct GPU (HIP)")
        cfg = config or GuardConfig.baseline()
        return GuardModel.random(cfg, seed=seed, device=device), None, random_metadata(head, cfg.window_tokens)
    root = Path(str(model))
    if not root.is_dir():
        raise RuntimeError(f"{model!r} is not a local model directory and this build does not download models")
    manifest = json.loads((root / "hs_guard.json").read_text())
    if manifest.get("format") != "hs-guard-v1" or manifest.get("risk_labels") != list(LABELS):
        raise ValueError("Unsupported model format or risk-label order")
    raise NotImplementedError("loading released bundles is not implemented yet; use load_model('random')")


class StreamingGuard:
    """Callers provide stable token IDs and keep each live conversation in its own slot."""

    def __init__(self, model, metadata, max_slots=1, *, state_dtype="float32", use_graphs=True):
        if not isinstance(max_slots, int) or max_slots < 1:
            raise ValueError("max_slots must be a positive integer")
        from .engine.slot_engine import SESSION_BUCKETS, SlotStreamEngine
        buckets = tuple(x for x in SESSION_BUCKETS if x <= max_slots)
        if not buckets or buckets[-1] != max_slots:
            buckets += (max_slots,)
        self.engine = SlotStreamEngine(model, max_slots, state_dtype=state_dtype, use_graphs=use_graphs,
                                       session_buckets=buckets)
        self.metadata, self.vocab_size, self.max_slots = metadata, model.backbone.config.vocab_size, max_slots

    def reset(self):
        self.engine.reset()

    def step(self, requests, role="assistant"):
        if role not in ("user", "assistant"):
            raise ValueError("role must be user or assistant")
        slots = [s for s, _ in requests]
        if not requests or len(set(slots)) != len(slots):
            raise ValueError("Each tick requires nonempty requests and unique slots")
        for slot, ids in requests:
            if not isinstance(slot, int) or not 0 <= slot < self.max_slots:
                raise ValueError("Slot is outside the allocated range")
            if not ids or any(not isinstance(i, int) or not 0 <= i < self.vocab_size for i in ids):
                raise ValueError("Each request requires nonempty in-vocabulary integer token IDs")
        outputs = self.engine.step(requests)[role]
        tau = self.metadata["thresholds"][role]
        return [{"slot": s, "cut_scores": (1 - p[:, 0]).tolist(), "threshold": tau}
                for (s, _), p in zip(requests, outputs)]
