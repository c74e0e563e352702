"""The allocation-free decode attention (prg_attn_decode_noalloc_bf16) against
the workspace entry point it mirrors (prg_attn_decode_bf16), through the C
ABI: bit-identical outputs on two calls in a row, the second with a smaller
cache and context (the library-owned partials keep the first call's
contents, which the second must not read), and a clear error for a cache
beyond its capacity."""
import numpy as np
import pytest

from peregrine_amd.synth import random_bf16

pytestmark = pytest.mark.gpu


def _case(rng, stride, L):
    from peregrine_amd.device import DeviceArray

    q = random_bf16(rng, (16 * 256,))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    gate = random_bf16(rng, (16 * 256,))
    return [DeviceArray.from_numpy(a) for a in (q, kc, vc, gate)]


def test_noalloc_attention_matches_workspace_entry(gpu):
    from peregrine_amd import ops
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(0)
    for stride, L in ((131072, 100000), (2048, 700)):  # 128 splits, then 64
        print(f"[no-alloc] stride {stride} seq_len {L}", flush=True)
        q, kc, vc, gate = _case(rng, stride, L)
        ref = DeviceArray((16 * 256,), np.uint16)
        part = DeviceArray((ops.attn_partials_bytes(stride) // 4,), np.float32)
        ops.attn_decode(q, kc, vc, gate, ref, part, stride, L)
        got = DeviceArray((16 * 256,), np.uint16)
        ops.attn_decode_noalloc(q, kc, vc, gate, got, stride, L)
        np.testing.assert_array_equal(got.numpy(), ref.numpy())


def test_noalloc_attention_rejects_a_cache_beyond_capacity(gpu):
    from peregrine_amd import ops
    from peregrine_amd._lib import PrgError
    from peregrine_amd.device import DeviceArray

    z = DeviceArray((16 * 256,), np.uint16)
    with pytest.raises(PrgError) as e:
        ops.attn_decode_noalloc(z, z, z, z, z, 1 << 20, 1)  # 1024 splits > 256
    assert "splits" in str(e.value)
