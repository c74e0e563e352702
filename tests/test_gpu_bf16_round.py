"""GPU f32 -> bf16 rounding (prg_f32_to_bf16: the conversion every kernel of
the library applies, one v_cvt_pk_bf16_f32) against the oracle's orc_f2bf
(round to nearest even; NaN -> (u >> 16) | 0x40), bit for bit, on every
special class (signed zeros, denormals, the largest finite values and their
rounding to infinity, infinities, NaNs with sign and payload bits), on ties
and near-ties of the rounding for both parities of the kept bit, and on
random bit patterns. The reference's shaders round the same way where they
write bfloat(f) (e.g. shaders/attention.metal:210).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _patterns():
    rng = np.random.default_rng(2024)
    special = np.array([
        0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007FFFFF, 0x00800000, 0x00008000, 0x00018000,
        0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0xFF7FFFFF, 0xFF7F8000, 0x7F800000, 0xFF800000,
        0x7F800001, 0x7FC00000, 0xFFC00001, 0x7FFFFFFF, 0xFFFFFFFF, 0x7FA00000, 0xFF812345,
        0x3F800000, 0xBF800000, 0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001,
    ], dtype=np.uint32)
    hi = rng.integers(0, 1 << 16, size=2000, dtype=np.uint32)
    lows = np.array([0x0000, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    ties = ((hi[:, None] << 16) | lows[None, :]).reshape(-1)
    rand = rng.integers(0, 1 << 32, size=100_000, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([special, ties, rand])


def test_f32_to_bf16_matches_oracle(gpu, orc):
    from peregrine_amd._lib import call
    from peregrine_amd.device import DeviceArray, ptr

    bits = _patterns()
    x = DeviceArray.from_numpy(bits.view(np.float32))
    y = DeviceArray((bits.size,), np.uint16)
    call("prg_f32_to_bf16", None, ptr(x), ptr(y), bits.size)
    got = y.numpy()
    want = orc.f2bf(bits.view(np.float32))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
