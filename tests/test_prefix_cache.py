"""Prefix cache bookkeeping, the PRGPFXS1 file size and the model fingerprint,
on the host (no GPU).

Reference tests restated here (a cache created without a model keeps the
same tokens and accounting, so these need no device):
  prefix_state_cache.zig:807-935 (exact-prefix entries, LRU eviction,
  descendants after branch removal, shifted match after extend + evict, pinned
  entries) and :1166-1201 (token-level hit ratio);
  prefix_persist.zig:441-470 (fingerprint tracks content) and :472-484
  (expected file bytes for 16,153 tokens).
The Wyhash behind the fingerprint is pinned by the published test vectors of
std.hash.Wyhash (seeds 0..6 over the classic message set).
"""
import struct

import numpy as np
import pytest

from peregrine_amd.model import ModelConfig
from peregrine_amd.prefix import PrefixCache, default_path, file_bytes, model_fingerprint, wyhash

MAGIC = 0x3153584650475250  # "PRGPFXS1" little-endian
VERSION = 3


def test_prgpfxs1_magic_spells_the_name():
    assert struct.pack("<Q", MAGIC) == b"PRGPFXS1"


@pytest.mark.parametrize("seed,msg,want", [
    (0, b"", 0x409638ee2bde459),
    (1, b"a", 0xa8412d091b5fe0a9),
    (2, b"abc", 0x32dd92e4b2915153),
    (3, b"message digest", 0x8619124089a3a16b),
    (4, b"abcdefghijklmnopqrstuvwxyz", 0x7a43afb61d7f5f40),
    (5, b"ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789", 0xff42329b90e50d58),
    (6, b"1234567890" * 8, 0xc39cab13b115aad3),
])
def test_wyhash_vectors(seed, msg, want):
    assert wyhash(msg, seed) == want


def _model_dir(d, config: bytes, shards: dict):
    (d / "config.json").write_bytes(config)
    for name, data in shards.items():
        (d / name).write_bytes(data)
    return d


@pytest.mark.parametrize("sizes", [(0,), (5,), (16,), (17, 3), (48, 1), (49, 47, 48), (200, 4 * 2**20 + 77)])
def test_fingerprint_is_one_stream(tmp_path, sizes):
    """The streamed fingerprint equals one Wyhash over config ‖ name ‖ bytes
    ‖ ... in sorted name order, whatever the file and read-chunk boundaries."""
    rng = np.random.default_rng(len(sizes))
    config = b'{"a":1}'
    shards = {f"model-{k:05d}.safetensors": rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()
              for k, n in enumerate(sizes)}
    _model_dir(tmp_path, config, shards)
    (tmp_path / "notes.txt").write_bytes(b"ignored")
    (tmp_path / "tokenizer.json").write_bytes(b"ignored")
    stream = config + b"".join(n.encode() + shards[n] for n in sorted(shards))
    assert model_fingerprint(tmp_path) == wyhash(stream, MAGIC ^ VERSION)


def test_fingerprint_tracks_content_not_path(tmp_path):
    """prefix_persist.zig:441-470."""
    d = _model_dir(tmp_path, b'{"a":1}', {"model-00001.safetensors": b"weights-v1"})
    first = model_fingerprint(d)
    assert model_fingerprint(d) == first
    (d / "model-00001.safetensors").write_bytes(b"weights-v2")  # same size
    same_size = model_fingerprint(d)
    assert same_size != first
    (d / "model-00001.safetensors").write_bytes(b"weights-v2-longer")
    reshard = model_fingerprint(d)
    assert reshard != same_size
    (d / "config.json").write_bytes(b'{"a":2}')
    assert model_fingerprint(d) != reshard


def test_fingerprint_needs_config(tmp_path):
    from peregrine_amd._lib import PrgError

    with pytest.raises(PrgError) as e:
        model_fingerprint(tmp_path)
    assert e.value.code == 8


def test_expected_file_bytes_9b():
    """prefix_persist.zig:472-484: 24 linear + 8 full layers, 16,153 tokens."""
    T = 16_153
    conv, recur = 3 * 8192 * 4, 32 * 128 * 128 * 4
    kv = 4 * T * 256 * 2
    want = 48 + T * 4 + 24 * (conv + recur) + 8 * 2 * kv + T * 4096 * 2
    assert file_bytes(ModelConfig(), T) == want
    small = ModelConfig(num_layers=6, hidden=1024, intermediate=2048, vocab=4096)  # layers 3 full, rest linear
    assert file_bytes(small, 10) == 48 + 40 + 5 * (conv + recur) + 1 * 2 * (4 * 10 * 256 * 2) + 10 * 1024 * 2


def test_default_path(monkeypatch):
    monkeypatch.setenv("HOME", "/home/someone")
    assert default_path() == "/home/someone/.cache/peregrine/qwen35-9b-q4-prefix-state.bin"


def _add(cache, tokens, pinned, next_token):
    """addTestEntry (prefix_state_cache.zig:788-805)."""
    m = cache.start_direct(tokens, pinned)
    cache.finish_direct(m, next_token)
    return m


def test_keeps_multiple_exact_prefix_entries():
    c = PrefixCache(None, 12, 4)
    _add(c, [1, 2, 3], False, 10)
    _add(c, [1, 2, 3, 4], False, 11)
    _add(c, [9, 8], False, 12)
    s = c.stats()
    assert (c.entry_count(), s["resident_tokens"], s["reserved_tokens"]) == (3, 9, 12)
    longest = c.find([1, 2, 3, 4, 5])
    assert longest.len == 4
    assert c.cached_next_token(longest) == (11, True)
    assert c.find([1, 2, 9]) is None
    assert c.contains([1, 2, 3, 4, 5], 3)


def test_evicts_least_recently_used_unpinned():
    c = PrefixCache(None, 8, 4)
    first = _add(c, [1, 2, 3], False, 10)
    _add(c, [4, 5, 6], False, 11)
    c.touch(first)
    _add(c, [7, 8, 9], False, 12)
    s = c.stats()
    assert (c.entry_count(), s["resident_tokens"], s["reserved_tokens"], s["evictions"]) == (2, 6, 8, 1)
    assert c.find([1, 2, 3, 0]) is not None
    assert c.find([4, 5, 6, 0]) is None
    assert c.find([7, 8, 9, 0]) is not None


def test_descendants_survive_branch_removal():
    c = PrefixCache(None, 8, 4)
    shorter = _add(c, [1, 2, 3], False, 10)
    _add(c, [1, 2, 3, 4], False, 11)
    c.remove(shorter.index)
    assert c.entry_count() == 1 and c.stats()["resident_tokens"] == 4
    assert c.find([1, 2, 3, 0]) is None
    assert not c.contains([1, 2, 3, 4, 5], 3)
    assert c.contains([1, 2, 3, 4, 5], 4)
    longest = c.find([1, 2, 3, 4, 5])
    assert longest.len == 4 and c.cached_next_token(longest) == (11, True)


def test_shifted_match_after_extending_and_evicting():
    c = PrefixCache(None, 5, 2)
    _add(c, [9, 9], False, 10)
    reuse = _add(c, [1, 2, 3], False, 11)
    assert reuse.index == 1
    stored = c.store([1, 2, 3, 4, 5], None, reuse=reuse, next_token=12)
    assert (stored.index, stored.len) == (0, 5)
    assert c.entry_count() == 1 and c.stats()["evictions"] == 1
    assert c.find([9, 9, 0]) is None
    m = c.find([1, 2, 3, 4, 5, 6])
    assert (m.index, m.len) == (stored.index, stored.len)
    assert c.cached_next_token(m) == (12, True)
    # the old, shorter key no longer matches on its own
    assert c.find([1, 2, 3, 7]) is None


def test_pinned_entries_survive_eviction():
    c = PrefixCache(None, 8, 4)
    _add(c, [1, 2, 3], True, 10)
    _add(c, [4, 5, 6], False, 11)
    _add(c, [7, 8, 9], False, 12)
    s = c.stats()
    assert (c.entry_count(), s["resident_tokens"], s["reserved_tokens"], c.pinned_count()) == (2, 6, 8, 1)
    assert c.find([1, 2, 3, 0]) is not None
    assert c.find([4, 5, 6, 0]) is None
    assert c.find([7, 8, 9, 0]) is not None


def test_budget_exhausted_by_pinned_entries():
    from peregrine_amd._lib import PrgError

    c = PrefixCache(None, 8, 4)
    _add(c, [1, 2, 3], True, 10)
    _add(c, [4, 5, 6], True, 11)
    with pytest.raises(PrgError) as e:
        _add(c, [7, 8, 9], False, 12)
    assert e.value.code == 5
    with pytest.raises(PrgError):
        c.start_direct(list(range(9)))  # longer than the whole budget


def test_stats_token_hit_ratio():
    c = PrefixCache(None, 4096, 1600)
    c.record_miss()
    c.record_computed(1000)
    m = c.start_direct([1] * 1000)
    c.finish_direct(m, 5)
    c.record_hit(800)
    c.record_computed(400)
    c.record_hit(1000)
    c.record_computed(0)
    s = c.stats()
    assert (s["hits"], s["misses"], s["hit_tokens"], s["computed_tokens"]) == (2, 1, 1800, 1400)
    assert abs(s["hit_tokens"] / (s["hit_tokens"] + s["computed_tokens"]) - 0.5625) < 1e-9


def test_exact_store_replaces_and_touch_activates():
    c = PrefixCache(None, 16, 4)
    a = _add(c, [1, 2, 3], False, 10)
    _add(c, [5, 6], False, 11)
    again = c.store([1, 2, 3], None, next_token=99, pinned=True)
    assert again.index == a.index and c.entry_count() == 2
    assert c.cached_next_token(again) == (99, True)
    assert c.entry_info(again.index)["pinned"]
    assert c.active_tokens() == 3
    np.testing.assert_array_equal(c.entry_tokens(again.index), [1, 2, 3])
    no_next = c.store([5, 6], None)
    assert c.cached_next_token(no_next) == (11, False)


def test_state_calls_need_a_model():
    from peregrine_amd._lib import PrgError

    c = PrefixCache(None, 16, 4)
    m = _add(c, [1, 2], False, 3)
    with pytest.raises(PrgError):
        c.entry_state_handle(m.index)
    with pytest.raises(PrgError):
        c.save("/tmp/never-written.bin", 1)


def test_index_matches_brute_force_under_random_operations():
    """The hash-and-length index against a brute-force scan of the live
    entries: longest cached prefix, exact containment, creation-order
    numbering across removals and evictions, and the budget invariant."""
    rng = np.random.default_rng(0)
    c = PrefixCache(None, 64, 4)
    for step in range(400):
        op = rng.integers(0, 10)
        if op < 6:  # cache a prefix drawn from a small alphabet (shared prefixes, repeats)
            n = int(rng.integers(1, 9))
            toks = rng.integers(0, 3, size=n).tolist()
            try:
                _add(c, toks, bool(rng.integers(0, 8) == 0), int(rng.integers(0, 100)))
            except Exception:
                pass  # budget exhausted by pinned entries
        elif op < 8 and c.entry_count():
            c.remove(int(rng.integers(0, c.entry_count())))
        live = [c.entry_tokens(i).tolist() for i in range(c.entry_count())]
        assert len({tuple(t) for t in live}) == len(live), "one entry per exact prefix"
        s = c.stats()
        assert s["reserved_tokens"] <= 64
        assert s["resident_tokens"] == sum(len(t) for t in live)
        prompt = rng.integers(0, 3, size=int(rng.integers(0, 12))).tolist()
        best = max((i for i, t in enumerate(live) if t == prompt[:len(t)]), key=lambda i: len(live[i]), default=None)
        m = c.find(prompt)
        if best is None:
            assert m is None
        else:
            assert m is not None and (m.index, m.len) == (best, len(live[best])), step
        for k in range(len(prompt) + 1):
            assert c.contains(prompt, k) == (k == 0 or prompt[:k] in live)
