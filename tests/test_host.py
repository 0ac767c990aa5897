"""Host-side logic without a GPU: packed tick layout, buckets, StreamingGuard validation (fake engine)."""
import numpy as np
import pytest

from oracle import pack as opack


def test_pack_ticks_matches_padded_layout():
    """The packed layout carries the same ids, lens, slots and starts as pack_inputs' padded layout (the
    reference's contract, slot_engine_v7.py:7-25), and pos = start + step for every real token."""
    from hs_guard.engine.slot_engine import pack_ticks
    rng = np.random.default_rng(0)
    for _ in range(50):
        max_slots = 9
        n = int(rng.integers(1, 7))
        slots = rng.permutation(max_slots)[:n]
        chunks = [rng.integers(0, 100, int(rng.integers(1, 9))).tolist() for _ in range(n)]
        length = rng.integers(0, 1000, max_slots)
        nb = n + int(rng.integers(0, 3))
        total = sum(map(len, chunks))
        tb = total + int(rng.integers(0, 5))
        out = np.full(2 * tb + 4 * nb, -7, dtype=np.int64)
        lens, offsets = pack_ticks(chunks, slots, length, nb, tb, max_slots, out)
        lb = max(map(len, chunks))
        ref = np.empty(nb * lb + 3 * nb, dtype=np.int64)
        ref_lens = opack.pack_inputs(chunks, slots, nb, lb, length, max_slots, ref)
        np.testing.assert_array_equal(lens, ref_lens)
        ids, pos = out[:tb], out[tb:2 * tb]
        offs, lns, sls, sts = (out[2 * tb + i * nb:2 * tb + (i + 1) * nb] for i in range(4))
        np.testing.assert_array_equal(lns, ref[nb * lb:nb * lb + nb])
        np.testing.assert_array_equal(sls, ref[nb * lb + nb:nb * lb + 2 * nb])
        np.testing.assert_array_equal(sts, ref[nb * lb + 2 * nb:])
        ref_ids = ref[:nb * lb].reshape(nb, lb)
        for r in range(n):
            np.testing.assert_array_equal(ids[offs[r]:offs[r] + lns[r]], ref_ids[r, :lns[r]])
            np.testing.assert_array_equal(pos[offs[r]:offs[r] + lns[r]], sts[r] + np.arange(lns[r]))
        assert (offs[n:] == total).all() and (ids[total:] == 0).all()


def test_buckets():
    from hs_guard.engine.slot_engine import bucket, token_buckets
    tb = token_buckets(352 * 64)
    assert tb[0] == 1 and tb[-1] == 352 * 64 and list(tb) == sorted(set(tb))
    assert bucket(1470, tb) == 1536 and bucket(1, tb) == 1 and bucket(352, tb) == 352
    with pytest.raises(ValueError):
        bucket(352 * 64 + 1, tb)


class _FakeEngine:
    """The reference's fake-backend pattern (examples/demo/test_batching.py:7-27): scores from an integer
    recurrence instead of a GPU."""

    roles = ("user", "assistant")

    def __init__(self, one_tick=True):
        import torch
        self.torch = torch
        self.calls = []
        self.max_rows, self.max_tick_tokens, self.native = 4, 64, one_tick

    def step(self, requests):
        self.calls.append(requests)
        out = []
        for slot, ids in requests:
            p = self.torch.zeros(len(ids), 3)
            p[:, 0] = self.torch.tensor([(7 * slot + i) % 10 / 10 for i in ids])
            out.append(p)
        return {"user": out, "assistant": out}

    def one_tick(self, scan):
        return self.native and scan is not None and scan[0] <= self.max_rows and scan[2] <= self.max_tick_tokens

    def step_flat(self, requests, scan):
        out = self.step(requests)
        flat = np.stack([self.torch.cat(out[r]).numpy() for r in self.roles])
        return flat, np.array([len(ids) for _, ids in requests], dtype=np.int64)

    def reset(self):
        self.calls.append("reset")


def _guard(one_tick=True):
    from hs_guard.runtime import StreamingGuard, random_metadata
    g = StreamingGuard.__new__(StreamingGuard)
    g.engine, g.metadata, g.vocab_size, g.max_slots = _FakeEngine(one_tick), random_metadata(), 100, 4
    return g


def test_streaming_guard_validation_matches_reference_messages():
    """Same ValueError conditions and messages as src/hs_guard/runtime.py:151-171."""
    from hs_guard.runtime import StreamingGuard
    g = _guard()
    cases = [(([(0, [1])], "system"), "role must be user or assistant"),
             (([], "user"), "Each tick requires nonempty requests and unique slots"),
             (([(1, [1]), (1, [2])], "user"), "Each tick requires nonempty requests and unique slots"),
             (([(4, [1])], "user"), "Slot is outside the allocated range"),
             (([(-1, [1])], "user"), "Slot is outside the allocated range"),
             (([(True, [1])], "user"), None),   # bool is an int in Python, as in the reference
             (([(0, [])], "user"), "Each request requires nonempty in-vocabulary integer token IDs"),
             (([(0, [100])], "user"), "Each request requires nonempty in-vocabulary integer token IDs"),
             (([(0, [1.0])], "user"), "Each request requires nonempty in-vocabulary integer token IDs"),
             # numpy integers are not ints to the reference's isinstance checks
             (([(0, [np.int64(1)])], "user"), "Each request requires nonempty in-vocabulary integer token IDs"),
             (([(np.int64(0), [1])], "user"), "Slot is outside the allocated range"),
             (([(0, [True, 2])], "user"), None)]
    for one_tick in (True, False):   # the native checks and the Python ones
        g = _guard(one_tick)
        for (req, role), msg in cases:
            if msg is None:
                g.step(req, role=role)
                continue
            with pytest.raises(ValueError, match=msg):
                g.step(req, role=role)
    for bad in (0, -1, 1.5, "2"):
        with pytest.raises(ValueError, match="max_slots must be a positive integer"):
            StreamingGuard(None, {}, max_slots=bad)


def test_streaming_guard_cut_scores():
    """Records through the one-tick native route equal those through engine.step, bit for bit (1 - p in float32)."""
    g = _guard()
    out = g.step([(2, [3, 4]), (0, [9])], role="assistant")
    assert out[0]["slot"] == 2 and out[1]["slot"] == 0
    np.testing.assert_allclose(out[0]["cut_scores"], [1 - 0.7, 1 - 0.8], rtol=1e-6)
    np.testing.assert_allclose(out[1]["cut_scores"], [1 - 0.9], rtol=1e-6)
    assert out[0]["threshold"] == pytest.approx(0.1117895246)
    assert _guard(False).step([(2, [3, 4]), (0, [9])], role="assistant") == out
    g.reset()
    assert g.engine.calls[-1] == "reset"


def test_load_model_offline_behaviour(tmp_path):
    from hs_guard.runtime import load_model
    with pytest.raises(ValueError):
        load_model("random", head="other")
    with pytest.raises(RuntimeError, match="does not download"):
        load_model("KrisLiu16/HS-Guard-v10")
    (tmp_path / "hs_guard.json").write_text('{"format": "other"}')
    with pytest.raises(ValueError, match="Unsupported model format"):
        load_model(str(tmp_path))


def test_serialize_and_encode_messages():
    """serialize / encode_messages (src/hs_guard/runtime.py:44-51,128-133): 'ROLE:\\ncontent' blocks joined by a
    blank line; positions are the tokens ending inside the last message; the reference's ValueErrors."""
    import pytest
    from hs_guard.runtime import encode_messages, serialize
    msgs = [{"role": "system", "content": "be nice"}, {"role": "user", "content": "hi there"},
            {"role": "assistant", "content": "hello"}]
    text = serialize(msgs)
    assert text == "SYSTEM:\nbe nice\n\nUSER:\nhi there\n\nASSISTANT:\nhello"

    class Tok:   # whitespace-and-newline tokenizer with character offsets, like tokenizers.Encoding
        def encode(self, text, add_special_tokens=False):
            import re
            spans = [(m.start(), m.end()) for m in re.finditer(r"\S+", text)]
            return type("E", (), {"ids": list(range(len(spans))), "offsets": spans})()
    ids, positions, role = encode_messages(Tok(), msgs)
    assert role == "assistant" and len(ids) == 8 and positions == [7]      # only "hello" ends after its start
    ids, positions, role = encode_messages(Tok(), msgs[:2])
    assert role == "user" and positions == [4, 5]                          # 'hi', 'there'
    for bad, msg in (([], "The last message must have role user or assistant"),
                     ([{"role": "system", "content": "x"}], "The last message must have role user or assistant"),
                     ([{"role": "tool", "content": "x"}, {"role": "user", "content": "y"}],
                      "Messages require a supported role and string content"),
                     ([{"role": "user", "content": ""}], "The target message is empty")):
        with pytest.raises(ValueError, match=msg):
            serialize(bad)
    with pytest.raises(ValueError, match="no tokenizer"):
        encode_messages(None, msgs)


def test_request_order_gathers_rows():
    """The engine's tick outputs are packed longest row first; request_order puts them back in request order
    (row r at sum(lens[:r])) exactly as slicing each row out of the packed outputs would."""
    from hs_guard.engine.slot_engine import request_order
    rng = np.random.default_rng(5)
    lens = rng.integers(1, 40, 37)
    order = np.argsort(-lens, kind="stable")
    packed_off = np.concatenate([[0], np.cumsum(lens[order])[:-1]])
    offsets = np.empty(len(lens), dtype=np.int64)
    offsets[order] = packed_off
    flat = rng.random((2, int(lens.sum()) + 5, 3)).astype(np.float32)   # 5 padding positions at the end
    got = request_order(flat, lens, offsets)
    want = np.concatenate([flat[:, o:o + n] for o, n in zip(offsets, lens)], axis=1)
    assert got.shape == want.shape and np.array_equal(got, want)
    one = request_order(flat, lens[:1], offsets[:1])
    assert np.array_equal(one, flat[:, offsets[0]:offsets[0] + lens[0]])


def test_padded_rows_scatters_each_request():
    """step_packed's [R, n, lb, 3] layout: request r's outputs (packed at offsets[r], rows packed longest first)
    at [:, r, :lens[r]], zeros after; the same as copying each row out on its own."""
    from hs_guard.engine.slot_engine import padded_rows
    rng = np.random.default_rng(6)
    lens = rng.integers(1, 65, 41)
    order = np.argsort(-lens, kind="stable")
    packed_off = np.concatenate([[0], np.cumsum(lens[order])[:-1]])
    offsets = np.empty(len(lens), dtype=np.int64)
    offsets[order] = packed_off
    flat = rng.random((2, int(lens.sum()) + 3, 3)).astype(np.float32)
    got = padded_rows(flat, lens, offsets, 64)
    want = np.zeros((2, len(lens), 64, 3), dtype=np.float32)
    for r, (o, n) in enumerate(zip(offsets, lens)):
        want[:, r, :n] = flat[:, o:o + n]
    assert got.shape == want.shape and np.array_equal(got, want)
    one = padded_rows(flat, lens[:1], offsets[:1], 64)
    assert np.array_equal(one[:, 0, :lens[0]], flat[:, offsets[0]:offsets[0] + lens[0]])
    assert not one[:, 0, lens[0]:].any()


def test_native_host_packing_matches_numpy_route():
    """hs_guard._hostpack (the packing step_packed and step run) against the numpy route it replaces: pack_ticks
    with the rows longest first (stable), padded_rows and request_order, bit for bit, on random config-5-like ticks with ties, ids given
    as lists, tuples and numpy integers; and scan's verdicts against the engine's request checks."""
    import numpy as np

    from hs_guard import _hostpack
    from hs_guard.engine.slot_engine import pack_ticks, padded_rows, request_order

    rng = np.random.default_rng(3)
    max_slots = 40
    for trial in range(30):
        n = int(rng.integers(1, max_slots + 1))
        slots = rng.permutation(max_slots)[:n]
        lens = np.where(rng.random(n) < 0.7, 1, rng.integers(1, 65, n))
        chunks = [list(map(int, rng.integers(0, 151936, int(l)))) for l in lens]
        reqs = []
        for i, (s, c) in enumerate(zip(slots, chunks)):
            ids = c if i % 3 == 0 else tuple(c) if i % 3 == 1 else [np.int64(x) for x in c]
            reqs.append((int(s) if i % 2 else np.int64(s), ids))
        length = rng.integers(0, 9000, max_slots).astype(np.int64)
        total = int(lens.sum())
        assert _hostpack.scan(reqs, max_slots, 151936) == (n, total, int(lens.max()))
        nb, tb = n + int(rng.integers(0, 5)), total + int(rng.integers(0, 40))
        ref = np.full(2 * tb + 4 * nb, -7, dtype=np.int64)
        order = np.argsort(-lens, kind="stable")
        lens_p, offs_p = pack_ticks([chunks[r] for r in order], slots[order], length, nb, tb, max_slots, ref)
        got = np.full(2 * tb + 4 * nb, -7, dtype=np.int64)
        g_lens, g_offs, g_slots = (np.empty(n, dtype=np.int64) for _ in range(3))
        _hostpack.fill(reqs, length, nb, tb, max_slots, 151936, got, g_lens, g_offs, g_slots)
        np.testing.assert_array_equal(got, ref)
        np.testing.assert_array_equal(g_lens, lens)
        np.testing.assert_array_equal(g_slots, slots)
        offs = np.empty(n, dtype=np.int64)
        offs[order] = offs_p
        np.testing.assert_array_equal(g_offs, offs)
        flat = rng.standard_normal((2, tb, 3)).astype(np.float32)
        for lb in (64, int(lens.max())):
            want = padded_rows(flat[:, :total].copy(), lens, offs, lb)
            out = np.full((2, n, lb, 3), np.nan, dtype=np.float32)
            _hostpack.scatter_padded(flat, 2, tb, g_lens, g_offs, lb, out)
            np.testing.assert_array_equal(out, want)
        want = request_order(flat, lens, offs)
        got_o = np.full((2, total, 3), np.nan, dtype=np.float32)
        _hostpack.gather_rows(flat, 2, tb, g_lens, g_offs, got_o)
        np.testing.assert_array_equal(got_o, want)
    # requests the engine's checks reject (or that the native route leaves to the numpy route): scan says None
    ok = [(0, [1, 2]), (3, [np.int32(9)])]
    assert _hostpack.scan(ok, 4, 10) == (2, 3, 2)
    for bad in ([(0, [1]), (0, [2])], [(4, [1])], [(-1, [1])], [(1, [])], [(1.0, [2])], [(1, (x for x in [2]))],
                [(0, [1, 10])], [(0, [-1])], [(0, [np.int64(10)])], [(0, [2.0])], [(0, [np.float32(2)])],
                [(2, [3]), (0, [1 << 40])]):
        assert _hostpack.scan(bad, 4, 10) is None, bad
        assert _hostpack.scan(bad, 4, 10, 1) is None, bad
    # strict: Python ints only (bool included), as the reference's isinstance(x, int) checks
    assert _hostpack.scan([(0, [1, True]), (True, [2])], 4, 10, 1) == (2, 3, 2)
    for bad in ([(0, [np.int32(9)])], [(np.int64(0), [1])]):
        assert _hostpack.scan(bad, 4, 10) is not None and _hostpack.scan(bad, 4, 10, 1) is None, bad
    # fill refuses an out-of-vocabulary id itself (the docs/ENGINE.md:9 contract), before the tick could run
    out, l3 = np.zeros(2 * 8 + 4 * 2, np.int64), np.zeros(2, np.int64)
    with pytest.raises(ValueError, match="in-vocabulary"):
        _hostpack.fill([(0, [1, 2]), (1, [10])], np.zeros(4, np.int64), 2, 8, 4, 10, out, l3, l3.copy(), l3.copy())
    with pytest.raises(ValueError):
        _hostpack.scatter_padded(np.zeros((2, 4, 3), np.float32), 2, 4, np.array([3], np.int64),
                                 np.array([2], np.int64), 4, np.zeros((2, 1, 4, 3), np.float32))
