"""Long prompts through the layer-major chunked prefill at the full 9B shape
(DeviceModel.prefillLayerMajor*, src/model/model.zig:829-1093;
prefill.zig:38-196; KV stride rule state.zig:11-32).

Chunking must not change a single bit: every projection is row-independent,
the attention of chunk c reads the cache that chunks < c wrote (masked
columns contribute exact zeros), and the GDN / conv states carry across
chunk boundaries with the same arithmetic. So prompts ingested with
different chunk sizes must leave identical tokens and states. The chunk size
is capped per state through PEREGRINE_PREFILL_CHUNK (read when the state's
prefill workspace is created).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def m9b(gpu):
    from peregrine_amd.model import QWEN35_9B, DeviceModel

    m = DeviceModel(QWEN35_9B, seed=7)
    yield m
    m.close()


def _state(m, max_seq, chunk, monkeypatch):
    from peregrine_amd.model import ModelState

    if chunk is None:
        monkeypatch.delenv("PEREGRINE_PREFILL_CHUNK", raising=False)
    else:
        monkeypatch.setenv("PEREGRINE_PREFILL_CHUNK", str(chunk))
    return ModelState(m, max_seq=max_seq)


def _same_states(a, b, m, upto):
    cfg = m.cfg
    for i in range(cfg.num_layers):
        if cfg.is_linear(i):
            for n in ("recur", "conv"):
                assert np.array_equal(a.read(f"layers.{i}.{n}", np.uint32), b.read(f"layers.{i}.{n}", np.uint32)), \
                    f"layer {i} {n}"
        else:
            for n in ("cache_k", "cache_v"):
                ga = a.read(f"layers.{i}.{n}", np.uint16).reshape(4, -1)
                gb = b.read(f"layers.{i}.{n}", np.uint16).reshape(4, -1)
                assert np.array_equal(ga, gb), f"layer {i} {n}"


def _compare(m, prompt, max_seq, chunks, monkeypatch, decode_steps=4):
    states = [_state(m, max_seq, c, monkeypatch) for c in chunks]
    firsts = []
    for c, st in zip(chunks, states):
        print(f"[long-prefill] {len(prompt)} tokens, chunk cap {c}, stride {st.stride}", flush=True)
        firsts.append(st.prefill(prompt))
    assert len(set(firsts)) == 1, firsts
    for st in states[1:]:
        _same_states(states[0], st, m, len(prompt))
    toks = [st.decode(decode_steps)[0] for st in states]
    for t in toks[1:]:
        np.testing.assert_array_equal(toks[0], t)
    for st in states:
        st.close()


def test_1600_tokens_one_chunk_equals_two(m9b, monkeypatch):
    prompt = np.random.default_rng(0).integers(0, 248320, size=1600).astype(np.uint32)
    _compare(m9b, prompt, 2048, [None, 800], monkeypatch)


def test_4096_tokens_default_chunks_equal_1024(m9b, monkeypatch):
    prompt = np.random.default_rng(1).integers(0, 248320, size=4096).astype(np.uint32)
    _compare(m9b, prompt, 4200, [None, 1024], monkeypatch)


def test_long_context_stride_and_score_block_shrink(m9b, monkeypatch):
    """max_seq 16000: the KV stride is aligned to 64 rather than 256
    (state.zig:11-32), and the 2048-token chunk at position 8192 needs
    16 * 2048 * 10240 bf16 scores, more than the 512 MiB score block, so it
    is halved. Same tokens and states as 512-token chunks."""
    from peregrine_amd.model import ModelState

    st = ModelState(m9b, max_seq=16000)
    assert st.stride == 16000
    st.close()
    assert ModelState(m9b, max_seq=15000).stride == 15104  # below 16000: aligned to 256
    prompt = np.random.default_rng(2).integers(0, 248320, size=9000).astype(np.uint32)
    _compare(m9b, prompt, 16000, [None, 512], monkeypatch)


def test_prepared_dense_prefill_is_identical(m9b, monkeypatch):
    """The prepared dense route (prg_model_prepare_dense; the reference's
    prepared dense RHS, block_attn.zig:143-215) stages bf16 copies of the
    weights that hold exactly the values the Q4 GEMM dequantises per tile, so
    a 1600-token prefill leaves the same next token, GDN states and KV caches
    bit for bit, and the same decoded tokens. Runs last in this module: the
    shared model keeps its dense copies afterwards."""
    import time

    from peregrine_amd.device import synchronize

    prompt = np.random.default_rng(5).integers(0, 248320, size=1600).astype(np.uint32)
    a = _state(m9b, 2048, None, monkeypatch)
    b = _state(m9b, 2048, None, monkeypatch)
    a.prefill(prompt)  # warm
    synchronize()
    t0 = time.perf_counter()
    fa = a.prefill(prompt)
    synchronize()
    t1 = time.perf_counter()
    nbytes = m9b.prepare_dense()
    assert nbytes > 13 * 10**9  # every prompt GEMM weight as bf16 (13.8 GB at the 9B shape)
    b.prefill(prompt)
    synchronize()
    t2 = time.perf_counter()
    fb = b.prefill(prompt)
    synchronize()
    t3 = time.perf_counter()
    print(f"[dense] 1600-token prefill {1e3 * (t1 - t0):.1f} ms Q4 -> {1e3 * (t3 - t2):.1f} ms dense "
          f"({nbytes / 2**30:.1f} GiB prepared)", flush=True)
    assert fa == fb
    _same_states(a, b, m9b, len(prompt))
    np.testing.assert_array_equal(a.decode(4)[0], b.decode(4)[0])
    a.close()
    b.close()


@pytest.mark.parametrize("T", [100, 700, 1600])
def test_dma_gemms_match_the_q4_kernel(m9b, monkeypatch, T):
    """The prompt GEMM with direct-to-LDS copies (gemm_dma_kernel: 256- or
    320-row tiles, SiLU-pair and multi-segment store epilogues, taken for the
    dense gate / up, GDN in_proj and attention q / k / v GEMMs when it costs
    fewer rounds) issues, per output element, the matrix instructions of
    gemm_q4_kernel in the same k order. Forced to each kernel in turn
    (PEREGRINE_GEMM_DMA = 0 / 256 / 320, read per launch), prompts of 100 /
    700 / 1600 tokens (one partial row tile; several with a partial last one;
    1600 = 5 x 320) leave the same next token, GDN states and KV caches bit
    for bit."""
    m9b.prepare_dense()
    prompt = np.random.default_rng(11 + T).integers(0, 248320, size=T).astype(np.uint32)
    states, firsts = [], []
    for pick in ("0", "256", "320"):
        st = _state(m9b, 2048, None, monkeypatch)
        monkeypatch.setenv("PEREGRINE_GEMM_DMA", pick)
        firsts.append(st.prefill(prompt))
        states.append(st)
    monkeypatch.delenv("PEREGRINE_GEMM_DMA")
    assert len(set(firsts)) == 1, firsts
    for st in states[1:]:
        _same_states(states[0], st, m9b, T)
    for st in states:
        st.close()
