"""Integer bookkeeping of the streaming step (test infrastructure only).

* ``pack_inputs`` restates ``src/hs_guard/engine/slot_engine_v7.py:7-25``: one int64 buffer
  ``[ids nb*lb | lens nb | slots nb | starts nb]``, ids right-padded with 0, padded rows pointing at the
  scratch slot ``max_slots`` with start 0. Pinned by the reference's own known-answer vector
  (``tests/test_contract.py:14-18``), restated in ``tests/test_oracle_pack.py``.
* ``ring_columns`` / ``ring_pos_update`` restate ``slot_engine_v8.py:41,57`` (``ring_col = pos % W`` for
  valid tokens, the scratch column ``W`` otherwise; after all layers ``ring_pos[slot, col] = pos`` or -1).
  Pinned by brute force against a dictionary model of the window in ``tests/test_oracle_pack.py``.
* ``bucket`` restates ``bucketed_engine.py:12-16``.
"""
import numpy as np


def bucket(value, choices):
    for choice in choices:
        if value <= choice:
            return choice
    raise ValueError(f"{value} exceeds the largest bucket {choices[-1]}")


def pack_inputs(chunks, slots, nb, lb, length, max_slots, out):
    n = len(chunks)
    lens = np.array([len(c) for c in chunks], dtype=np.int64)
    ids = out[:nb * lb].reshape(nb, lb)
    ids[:] = 0
    for row, chunk in enumerate(chunks):
        ids[row, :len(chunk)] = np.asarray(chunk, dtype=np.int64)
    o = nb * lb
    out[o:o + nb] = 0
    out[o:o + n] = lens
    out[o + nb:o + 2 * nb] = max_slots
    out[o + nb:o + nb + n] = np.asarray(slots, dtype=np.int64)
    out[o + 2 * nb:o + 3 * nb] = 0
    out[o + 2 * nb:o + 2 * nb + n] = np.asarray(length, dtype=np.int64)[np.asarray(slots, dtype=np.int64)]
    return lens


def ring_columns(starts, lens, lb, window):
    """[nb, lb] ring column of each (row, step): pos % W for valid steps, W (scratch) otherwise."""
    steps = np.arange(lb)[None, :]
    pos = np.asarray(starts, dtype=np.int64)[:, None] + steps
    valid = steps < np.asarray(lens, dtype=np.int64)[:, None]
    return np.where(valid, pos % window, window), pos, valid


def ring_pos_update(ring_pos, slots, starts, lens, lb, window):
    """Apply ``ring_pos[slots[:, None], ring_col] = where(valid, pos, -1)`` in place (row order)."""
    cols, pos, valid = ring_columns(starts, lens, lb, window)
    for r, s in enumerate(np.asarray(slots, dtype=np.int64)):
        for t in range(lb):
            ring_pos[s, cols[r, t]] = pos[r, t] if valid[r, t] else -1
    return ring_pos
