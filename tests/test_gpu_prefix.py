"""Prefix reuse on the GPU: state copies, prefill on top of a restored prefix,
the prefix cache with device states, and the PRGPFXS1 v3 file.

Reference: ModelState.copyPrefixFrom (src/model/state.zig:124-180), the
prefix-hit prefill (model.zig:940-1060), Cache.storePrefixFromWork and the
hidden-row tests (src/server/prefix_state_cache.zig:563-648, 935-1070), and
save / load (src/server/prefix_persist.zig:253-412, tests :486-639).

The bar is bit-exactness: a prompt prefilled in one pass and the same prompt
prefilled as a cached prefix plus a continuation run the same kernels over
the same rows (the chunked prefill is bit-exact across chunk boundaries), so
next tokens, decoded tokens, GDN states and K/V must be identical.
"""
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL = dict(num_layers=4, hidden=1024, intermediate=2048, vocab=4096)
HDR = struct.Struct("<QIIQQIII4x")  # the 48-byte PRGPFXS1 header
MAGIC = 0x3153584650475250


@pytest.fixture(scope="module")
def model(gpu):
    from peregrine_amd.model import DeviceModel, ModelConfig

    m = DeviceModel(ModelConfig(**SMALL), seed=7)
    yield m
    m.close()


@pytest.fixture(scope="module")
def prompt():
    return np.random.default_rng(12).integers(0, SMALL["vocab"], size=48).astype(np.uint32)


@pytest.fixture(scope="module")
def full_run(model, prompt):
    """One-pass prefill of the whole prompt, then 10 decode steps."""
    from peregrine_amd.model import ModelState

    st = ModelState(model, 128)
    nxt = st.prefill(prompt)
    snap = snapshot(model, st, len(prompt))
    toks, _ = st.decode(10)
    st.close()
    return nxt, toks, snap


def state_tensors(handle, model, n):
    """GDN states and K/V [0, n) of a state handle, compacted."""
    from peregrine_amd._lib import lib
    from peregrine_amd.model import _d2h, _tensor

    stride = int(lib.prg_model_state_stride(handle))
    out = {}
    for i in range(model.cfg.num_layers):
        if model.cfg.is_linear(i):
            for k in ("conv", "recur"):
                p, nb = _tensor("prg_model_state_tensor", handle, f"layers.{i}.{k}", None)
                out[f"{i}.{k}"] = _d2h(p, nb, np.float32)
        else:
            p, nb = _tensor("prg_model_state_tensor", handle, f"layers.{i}.cache_k", None)
            out[f"{i}.k"] = _d2h(p, nb, np.uint16).reshape(4, stride, 256)[:, :n].copy()
            p, nb = _tensor("prg_model_state_tensor", handle, f"layers.{i}.cache_v", None)
            out[f"{i}.v"] = _d2h(p, nb, np.uint16).reshape(4, 256, stride)[:, :, :n].copy()
    return out


def snapshot(model, st, n):
    return state_tensors(st.handle, model, n)


def assert_same_state(a, b, what):
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), f"{what}: {k} differs"


def test_copy_prefix_between_strides(model, prompt):
    from peregrine_amd.model import ModelState

    a, b = ModelState(model, 100), ModelState(model, 300)
    assert (a.stride, b.stride) == (256, 512)
    a.prefill(prompt[:40])
    b.copy_prefix_from(a, 40)
    assert_same_state(snapshot(model, a, 40), snapshot(model, b, 40), "copy_prefix")
    from peregrine_amd._lib import PrgError

    with pytest.raises(PrgError) as e:
        b.copy_prefix_from(a, 101)  # past a's capacity (state.zig:125)
    assert e.value.code == 5
    a.close()
    b.close()


def test_prefill_from_equals_one_pass(model, prompt, full_run):
    from peregrine_amd.model import ModelState

    nxt, toks, snap = full_run
    st = ModelState(model, 128)
    st.prefill(prompt[:20])
    assert st.prefill_from(prompt, 20) == nxt
    assert_same_state(snap, snapshot(model, st, len(prompt)), "prefill_from")
    got, _ = st.decode(10)
    np.testing.assert_array_equal(got, toks)
    st.close()


def test_cache_restore_then_continue(model, prompt, full_run):
    """Store a 24-token prefix from a work state, restore it into a fresh state
    and prefill the rest: identical to the one-pass run."""
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    nxt, toks, snap = full_run
    cache = PrefixCache(model, 4096, 256)
    w1 = ModelState(model, 128)
    n24 = w1.prefill(prompt[:24])
    m = cache.store(prompt[:24], w1, next_token=n24)
    assert (m.len, cache.entry_count()) == (24, 1)
    assert cache.entry_info(m.index)["capacity"] == 256  # max(24, min(4096, 256))
    hit = cache.find(prompt)
    assert (hit.index, hit.len) == (m.index, 24)
    assert cache.cached_next_token(hit) == (n24, True)
    w2 = ModelState(model, 128)
    cache.restore(hit, w2)
    assert w2.prefill_from(prompt, 24) == nxt
    assert_same_state(snap, snapshot(model, w2, len(prompt)), "restore + prefill_from")
    got, _ = w2.decode(10)
    np.testing.assert_array_equal(got, toks)
    # the entry's own state still holds exactly the 24-token prefix
    assert_same_state(snapshot(model, w1, 24), state_tensors(cache.entry_state_handle(m.index), model, 24), "entry")
    for s in (w1, w2):
        s.close()
    cache.close()


def test_decode_with_prefix_bookkeeping(model, prompt, full_run):
    """decodeFromPrefixCache (decode_loop.zig:96-160) on a prefix-cache hit:
    restore the 24-token entry, prefill the rest of the prompt, then step with
    the reference's bookkeeping (cache_pos = logical_pos - prefix_len,
    rope_pos = logical_pos, seq_len = logical_pos + 1) through
    prg_model_forward_next_token_prefixed: the same tokens as the one-pass
    greedy run, and a seq_len that does not match is rejected."""
    from peregrine_amd._lib import PrgError
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    nxt, toks, _ = full_run
    cache = PrefixCache(model, 4096, 256)
    w1 = ModelState(model, 128)
    m = cache.store(prompt[:24], w1, next_token=w1.prefill(prompt[:24]))
    w2 = ModelState(model, 128)
    cache.restore(cache.find(prompt), w2)
    prefix_len, prompt_len = m.len, len(prompt)
    current = w2.prefill_from(prompt, prefix_len)
    assert current == nxt
    got = []
    for n in range(1, 11):  # n tokens emitted so far
        logical_pos = prompt_len + n - 1
        current = w2.forward_next_token_prefixed(current, logical_pos - prefix_len, prefix_len, rope_pos=logical_pos,
                                                 seq_len=logical_pos + 1)
        got.append(current)
    np.testing.assert_array_equal(np.array(got, np.uint32), toks)
    with pytest.raises(PrgError) as e:
        w2.forward_next_token_prefixed(current, 40, prefix_len, seq_len=40 + 1)
    assert e.value.code == 1
    for s in (w1, w2):
        s.close()
    cache.close()


def test_store_with_reuse_extends_entry(model, prompt, full_run):
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    nxt, toks, snap = full_run
    cache = PrefixCache(model, 4096, 16)
    w1 = ModelState(model, 128)
    m = cache.store(prompt[:16], w1, next_token=w1.prefill(prompt[:16]))
    assert cache.entry_info(m.index)["capacity"] == 16
    w2 = ModelState(model, 128)
    cache.restore(m, w2)
    n40 = w2.prefill_from(prompt[:40], 16)
    m40 = cache.store(prompt[:40], w2, reuse=m, next_token=n40)
    # re-keyed in place and grown: one entry, 40 tokens, capacity 40
    assert cache.entry_count() == 1 and m40.index == m.index
    assert cache.entry_info(m40.index)["capacity"] == 40
    assert cache.find(prompt[:20]) is None
    hit = cache.find(prompt)
    assert hit.len == 40
    w3 = ModelState(model, 128)
    cache.restore(hit, w3)
    assert w3.prefill_from(prompt, 40) == nxt
    assert_same_state(snap, snapshot(model, w3, len(prompt)), "extended entry")
    got, _ = w3.decode(10)
    np.testing.assert_array_equal(got, toks)
    for s in (w1, w2, w3):
        s.close()
    cache.close()


def _parse_file(raw: bytes, cfg, T):
    """PRGPFXS1 v3 read independently of the library (prefix_persist.zig:44-80)."""
    h = HDR.unpack_from(raw, 0)
    off = HDR.size
    toks = np.frombuffer(raw, np.uint32, T, off)
    off += 4 * T
    layers = {}
    for i in range(cfg.num_layers):
        if cfg.is_linear(i):
            layers[f"{i}.conv"] = np.frombuffer(raw, np.float32, 3 * 8192, off)
            off += 3 * 8192 * 4
            layers[f"{i}.recur"] = np.frombuffer(raw, np.float32, 32 * 128 * 128, off)
            off += 32 * 128 * 128 * 4
        else:
            layers[f"{i}.k"] = np.frombuffer(raw, np.uint16, 4 * T * 256, off).reshape(4, T, 256)
            off += 4 * T * 256 * 2
            layers[f"{i}.v"] = np.frombuffer(raw, np.uint16, 4 * 256 * T, off).reshape(4, 256, T)
            off += 4 * 256 * T * 2
    hidden = np.frombuffer(raw, np.uint16, T * cfg.hidden, off)
    off += T * cfg.hidden * 2
    assert off == len(raw)
    return h, toks, layers, hidden


def test_persist_round_trip(model, prompt, full_run, tmp_path):
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache, file_bytes

    nxt, toks, snap = full_run
    fp = 0x1234_5678_9ABC_DEF0
    src = PrefixCache(model, 4096, 64)
    w1 = ModelState(model, 128)
    n24 = w1.prefill(prompt[:24])
    src.store(prompt[:24], w1, next_token=n24)
    path = tmp_path / "cache" / "prefix-state.bin"  # parent directories are created
    src.save(path, fp)
    raw = path.read_bytes()
    assert len(raw) == file_bytes(model.cfg, 24)
    h, ftoks, layers, hidden = _parse_file(raw, model.cfg, 24)
    assert h == (MAGIC, 3, 0, fp, 24, n24, 1, 0)
    np.testing.assert_array_equal(ftoks, prompt[:24])
    assert_same_state(snapshot(model, w1, 24), layers, "file sections")
    assert not hidden.any()  # no hidden tracking: zero-filled, hidden_valid 0

    dst = PrefixCache(model, 4096, 64)
    dst.start_direct([7, 7, 7])  # replaced by the load
    assert dst.load(path, fp) == 24
    assert dst.entry_count() == 1 and dst.pinned_count() == 1 and dst.active_tokens() == 24
    hit = dst.find(prompt)
    assert hit.len == 24 and dst.cached_next_token(hit) == (n24, True)
    w2 = ModelState(model, 128)
    dst.restore(hit, w2)
    assert w2.prefill_from(prompt, 24) == nxt
    got, _ = w2.decode(10)
    np.testing.assert_array_equal(got, toks)

    # rejected files leave the cache as it was (prefix_persist.zig:612-621)
    assert dst.load(path, fp + 1) == 0
    assert dst.entry_count() == 1 and dst.active_tokens() == 24
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 32, SMALL["vocab"])  # next token outside the vocab
    (tmp_path / "vocab.bin").write_bytes(bad)
    assert dst.load(tmp_path / "vocab.bin", fp) == 0
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 8, 2)  # version 2
    (tmp_path / "v2.bin").write_bytes(bad)
    assert dst.load(tmp_path / "v2.bin", fp) == 0
    (tmp_path / "short.bin").write_bytes(raw[:-2])
    assert dst.load(tmp_path / "short.bin", fp) == 0
    assert dst.load(tmp_path / "absent.bin", fp) == 0
    assert dst.entry_count() == 1 and dst.active_tokens() == 24
    for s in (w1, w2):
        s.close()
    src.close()
    dst.close()


def _rows(n, cols, byte):
    from peregrine_amd.device import DeviceArray

    return DeviceArray.from_numpy(np.full((n, cols), byte * 0x0101, np.uint16))


def _hidden(cache, m, n, cols):
    from peregrine_amd.model import _d2h

    p, valid = cache.entry_hidden(m)
    return (_d2h(p, n * cols * 2, np.uint16).reshape(n, cols) if p else None), valid


def test_hidden_rows_fresh_entry(model):
    """prefix_state_cache.zig:936-966."""
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    H = SMALL["hidden"]
    c = PrefixCache(model, 8, 4)
    c.enable_hidden()
    w = ModelState(model, 4)
    rows = _rows(3, H, 0xAB)
    m = c.store([1, 2, 3], w, work_hidden=rows.ptr)
    got, valid = _hidden(c, m, 3, H)
    assert valid and (got == 0xABAB).all()
    w.close()
    c.close()


def test_hidden_rows_reuse_extends_validity(model):
    """prefix_state_cache.zig:968-1019: reused rows keep their bytes, the
    suffix comes from the work buffer at its base row."""
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    H = SMALL["hidden"]
    c = PrefixCache(model, 16, 4)
    c.enable_hidden()
    w = ModelState(model, 8)
    ra = _rows(3, H, 0x11)  # held until the copy is done
    a = c.store([1, 2, 3], w, work_hidden=ra.ptr)
    assert c.entry_hidden(a)[1]
    hb = np.zeros((5, H), np.uint16)
    hb[3:5] = 0x2222
    from peregrine_amd.device import DeviceArray

    buf = DeviceArray.from_numpy(hb)
    b = c.store([1, 2, 3, 4, 5], w, reuse=a, work_hidden=buf.ptr, hidden_base_rows=3)
    got, valid = _hidden(c, b, 5, H)
    assert valid
    assert (got[:3] == 0x1111).all() and (got[3:] == 0x2222).all()
    # extending again without hidden rows clears validity (:1021-1068)
    d = c.store([1, 2, 3, 4, 5, 6], w, reuse=b)
    assert not c.entry_hidden(d)[1]
    w.close()
    c.close()


def test_hidden_rows_persist(model, tmp_path):
    """prefix_persist.zig:540-639: hidden rows survive a round trip; a file
    written without them loads with hidden_valid clear."""
    from peregrine_amd.model import ModelState
    from peregrine_amd.prefix import PrefixCache

    H = SMALL["hidden"]
    src = PrefixCache(model, 64, 16)
    src.enable_hidden()
    w = ModelState(model, 16)
    rows = np.random.default_rng(2).integers(0, 2**16, size=(5, H), dtype=np.uint16)
    from peregrine_amd.device import DeviceArray

    buf = DeviceArray.from_numpy(rows)
    src.store([10, 11, 12, 13, 14], w, work_hidden=buf.ptr, next_token=777)
    src.save(tmp_path / "h.bin", 5)
    dst = PrefixCache(model, 64, 16)
    dst.enable_hidden()
    assert dst.load(tmp_path / "h.bin", 5) == 5
    m = dst.find([10, 11, 12, 13, 14])
    got, valid = _hidden(dst, m, 5, H)
    assert valid and np.array_equal(got, rows)

    plain = PrefixCache(model, 64, 16)
    plain.store([1, 2, 3, 4], w, next_token=99)
    plain.save(tmp_path / "plain.bin", 5)
    assert dst.load(tmp_path / "plain.bin", 5) == 4
    m = dst.find([1, 2, 3, 4])
    p, valid = dst.entry_hidden(m)
    assert p and not valid
    w.close()
    for c in (src, dst, plain):
        c.close()
