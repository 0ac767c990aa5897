"""Drop-in public API: ``load_model``, ``StreamingGuard`` (src/hs_guard/runtime.py:92-125,148-174) and the
complete-message scorer ``score_messages`` (runtime.py:44-51,128-145) with the stream-vs-whole self-check
(examples/demo/server.py:500-524).

``StreamingGuard(model, metadata, max_slots).step([(slot, token_ids)], role)`` returns, per request,
``{'slot', 'cut_scores': [1 - p(safe) per submitted token], 'threshold'}`` with the reference's validation
and error messages. ``reset()`` clears every slot. ``score_messages`` scores a whole conversation in one
forward; ``score_ids`` is the same on token ids (random-init models have no tokenizer).
"""
from __future__ import annotations

import hashlib
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


def sha256(path):
    """Hex SHA-256 of a file, read in 8 MiB blocks."""
    digest = hashlib.sha256()
    with Path(path).open("rb") as f:
        for block in iter(lambda: f.read(8 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def verify_model(directory):
    """The bundle check of src/hs_guard/runtime.py:19-41: hs_guard.json names format hs-guard-v1 and the risk
    labels in order, lists config.json, tokenizer.json and model.safetensors, and every listed asset is a file
    inside the bundle (or, for a hub snapshot, in its blob cache) with the listed SHA-256."""
    root = Path(directory).resolve()
    manifest = json.loads((root / "hs_guard.json").read_text())
    if manifest.get("format") != "hs-guard-v1" or manifest.get("risk_labels") != list(LABELS):
        raise ValueError("Unsupported model format or risk-label order")
    files = manifest.get("files", {})
    if not {"config.json", "tokenizer.json", "model.safetensors"}.issubset(files):
        raise ValueError("Model manifest is missing required assets")
    blobs = (root.parent.parent / "blobs").resolve() if root.parent.name == "snapshots" else None
    for name, expected in files.items():
        rel = Path(name)
        if rel.is_absolute() or ".." in rel.parts:
            raise ValueError(f"Invalid model asset: {name}")
        path = root / rel
        real = path.resolve()
        if not path.is_file() or not (real.is_relative_to(root) or (blobs is not None and real.is_relative_to(blobs))):
            raise ValueError(f"Invalid model asset: {name}")
        if sha256(path) != expected:
            raise ValueError(f"Model asset checksum mismatch: {name}")
    return manifest


def load_bundle(root, head="redline", device="cuda"):
    """(model, tokenizer, metadata) of a verified local bundle: geometry from config.json, weights from
    model.safetensors (GuardModel.from_state_dict: strict names and shapes), tokenizers.Tokenizer from
    tokenizer.json, metadata = the manifest with the chosen head's thresholds (runtime.py:92-125)."""
    if head not in ("redline", "general"):
        raise ValueError("head must be redline or general")
    from safetensors.torch import load_file
    from tokenizers import Tokenizer
    from .model import GuardConfig, GuardModel
    root = Path(root)
    manifest = verify_model(root)
    cfg = GuardConfig.from_hf(json.loads((root / "config.json").read_text()), manifest.get("window_tokens", 512))
    model = GuardModel.from_state_dict(cfg, load_file(str(root / "model.safetensors")), head=head, device=device)
    metadata = dict(manifest, head=head, thresholds=manifest["thresholds"][head])
    return model, Tokenizer.from_file(str(root / "tokenizer.json")), metadata


def load_model(model=MODEL_ID, *, revision=None, head="redline", config=None, seed=0, device="cuda"):
    """Returns (model, tokenizer, metadata) like src/hs_guard/runtime.py:92-125.

    A local bundle directory (hs_guard.json, config.json, tokenizer.json, model.safetensors) is verified and
    loaded (``load_bundle``). ``model="random"`` (or a GuardConfig passed as ``config``) builds seeded
    random-init weights of that geometry on ``device`` (tokenizer None). Hub names need a network fetch,
    which this build does not do: they raise."""
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
    verify_model(root)
    if not torch.cuda.is_available():
        raise RuntimeError("HS-Guard requires an AMD Instinct GPU (HIP)")
    return load_bundle(root, head=head, device=device)


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

    def _check(self, requests):
        """The reference's request checks and errors (src/hs_guard/runtime.py:164-171)."""
        slots = [s for s, _ in requests]
        if not requests or len(set(slots)) != len(slots):
            raise ValueError("Each tick requires nonempty requests and unique slots")
        for slot, ids in requests:
            if not isinstance(slot, int) or not 0 <= slot < self.max_slots:
                raise ValueError("Slot is outside the allocated range")
            if not ids or any(not isinstance(i, int) or not 0 <= i < self.vocab_size for i in ids):
                raise ValueError("Each request requires nonempty in-vocabulary integer token IDs")

    def step(self, requests, role="assistant"):
        if role not in ("user", "assistant"):
            raise ValueError("role must be user or assistant")
        from .engine.slot_engine import _hostpack
        eng = self.engine
        # the checks in C over the request list (Python ints only, as the reference's isinstance checks); the
        # Python checks run only when one fails, to raise the reference's error
        scan = _hostpack.scan(requests, self.max_slots, self.vocab_size, 1) if requests else None
        if scan is None:
            self._check(requests)
        tau = self.metadata["thresholds"][role]
        # 1 - p(safe) for every position at once (float32, as per row), then cut per request
        if eng.one_tick(scan):
            flat, lens = eng.step_flat(requests, scan)
            cut = (1 - flat[eng.roles.index(role), :, 0]).tolist()
            sizes = lens.tolist()
        else:
            import torch
            outputs = eng.step(requests)[role]
            cut = (1 - torch.cat(outputs)[:, 0]).tolist()
            sizes = [len(p) for p in outputs]
        records, at = [], 0
        for (s, _), k in zip(requests, sizes):
            records.append({"slot": s, "cut_scores": cut[at:at + k], "threshold": tau})
            at += k
        return records


# ------------------------------------------------------------------------------------------------------------
# Complete-message scoring
# ------------------------------------------------------------------------------------------------------------
def serialize(messages):
    """Conversation text of src/hs_guard/runtime.py:44-51: 'ROLE:\ncontent' blocks joined by blank lines."""
    if not messages or messages[-1]["role"] not in ("user", "assistant"):
        raise ValueError("The last message must have role user or assistant")
    if any(m["role"] not in ("system", "user", "assistant") or not isinstance(m["content"], str) for m in messages):
        raise ValueError("Messages require a supported role and string content")
    if not messages[-1]["content"]:
        raise ValueError("The target message is empty")
    return "\n\n".join(m["role"].upper() + ":\n" + m["content"] for m in messages)


def encode_messages(tokenizer, messages):
    """(ids, positions of the last message's tokens, its role) as src/hs_guard/runtime.py:128-133. The
    tokenizer is the bundle's (tokenizers.Tokenizer: encode(text, add_special_tokens=False) with .ids and
    .offsets); random-init models have none, so use score_ids with token ids."""
    if tokenizer is None:
        raise ValueError("This model has no tokenizer; score token ids with score_ids")
    text = serialize(messages)
    encoded = tokenizer.encode(text, add_special_tokens=False)
    start = len(text) - len(messages[-1]["content"])
    positions = [i for i, (_, end) in enumerate(encoded.offsets) if end > start]
    return encoded.ids, positions, messages[-1]["role"]


def _scorer(model):
    from .engine.whole import WholeSequenceScorer
    scorer = getattr(model, "_hsg_whole_scorer", None)
    if scorer is None:
        scorer = WholeSequenceScorer(model)
        model._hsg_whole_scorer = scorer
    return scorer


def score_ids(model, metadata, ids, positions=None, role="assistant"):
    """One whole forward over ``ids`` (hs_guard.engine.whole); the record of src/hs_guard/runtime.py:136-145
    over ``positions`` (default: every token): score = last cut for the user role, the largest for the
    assistant role, where cut = 1 - p(safe)."""
    if role not in ("user", "assistant"):
        raise ValueError("role must be user or assistant")
    vocab = model.config.vocab_size
    if not ids or any(not isinstance(i, int) or not 0 <= i < vocab for i in ids):
        raise ValueError("Each request requires nonempty in-vocabulary integer token IDs")
    positions = list(range(len(ids))) if positions is None else list(positions)
    if not positions or any(not 0 <= p < len(ids) for p in positions):
        raise ValueError("positions must be nonempty indices into ids")
    scorer = _scorer(model)
    probs = scorer.forward(ids)
    cut = (1 - probs[scorer.roles.index(role), positions, 0]).cpu()
    value = float(cut[-1] if role == "user" else cut.max())
    threshold = metadata["thresholds"][role]
    return {"role": role, "head": metadata["head"], "score": value, "threshold": threshold,
            "flagged": value > threshold}


def score_messages(model, tokenizer, metadata, messages):
    """Complete-message score of src/hs_guard/runtime.py:136-145 on this build's kernels."""
    ids, positions, role = encode_messages(tokenizer, messages)
    return score_ids(model, metadata, ids, positions, role)


def selfcheck(model, ids, piece=3, state_dtype="float32"):
    """Stream ``ids`` through a one-slot streaming engine ``piece`` tokens per tick and compare every position's
    class probabilities (both roles) with one whole forward, as examples/demo/server.py:500-524 does for its
    readiness check (which fails above 0.05)."""
    from .engine.slot_engine import SlotStreamEngine
    if piece < 1:
        raise ValueError("piece must be positive")
    whole = _scorer(model).forward(ids).cpu().numpy()
    eng = SlotStreamEngine(model, 1, state_dtype=state_dtype)
    streamed = {r: [] for r in eng.roles}
    for a in range(0, len(ids), piece):
        out = eng.step([(0, list(ids[a:a + piece]))])
        for r in eng.roles:
            streamed[r].append(out[r][0])
    import numpy as np
    diff = 0.0
    for i, r in enumerate(eng.roles):
        got = np.concatenate(streamed[r])
        diff = max(diff, float(np.abs(got - whole[i]).max()))
    return {"tokens": len(ids), "stream_positions": sum(len(x) for x in streamed[eng.roles[0]]),
            "max_prob_diff_stream_vs_whole": round(diff, 5)}
