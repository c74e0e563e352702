"""The library GEMM comparison (peregrine_amd/gemm_baseline.py) times the
shapes the 1600-token ingest runs: checked here against the model's
dimensions (BASELINE's 9B shape, src/model/config.zig) so that the
comparison cannot drift from the prompt GEMMs it stands beside."""
import pytest

from peregrine_amd import gemm_baseline
from peregrine_amd.model import ModelConfig


def test_shapes_are_the_prompt_gemms():
    c = ModelConfig()
    key_heads, key_dim, val_heads, val_dim = 16, 128, 32, 128  # GDN: 16 q/k heads, 32 v heads, 128 wide
    q_heads, kv_heads, head_dim = 16, 4, 256                   # attention: q | gate, k, v
    conv = 2 * key_heads * key_dim + val_heads * val_dim       # q, k, v rows through the conv1d
    want = {
        "gate_up": (2 * c.intermediate, c.hidden),
        "down": (c.hidden, c.intermediate),
        "in_proj": (conv + val_heads * val_dim + 2 * val_heads, c.hidden),  # + z + a + b
        "attn_qkv": (2 * q_heads * head_dim + 2 * kv_heads * head_dim, c.hidden),
        "out_proj": (c.hidden, c.hidden),
    }
    got = {name: (N, K) for name, M, N, K in gemm_baseline.SHAPES}
    assert got == want
    assert {M for _, M, _, _ in gemm_baseline.SHAPES} == {1600}


def test_needs_a_gpu():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError):
        gemm_baseline.library_gemms()
