"""Model upload from a safetensors checkpoint (prg_model_load) on the GPU.

Reference: DeviceModel.upload (src/model/model.zig:580-658), DecoderLayer.upload
(decoder_layer.zig:376-412), LinearAttentionBlock.upload (block_linear.zig:155-173),
FullAttentionBlock.upload (block_attn.zig:235-248), MlpBlock.upload
(block_mlp.zig:116-122), Q4Linear.upload (linear_q4.zig:28-63, 261-268),
Drafter.upload / detectRoot (mtp.zig:86-96, 347-355).

A random model is written out tensor by tensor with the test's own
safetensors writer and loaded back: every device tensor must come back bit for
bit, and the loaded model must decode exactly as the original and as the
oracle does.
"""
import numpy as np
import pytest

from helpers import qwen35_config, write_checkpoint

pytestmark = pytest.mark.gpu

SMALL = dict(num_layers=4, hidden=1024, intermediate=2048, vocab=4096)
NP = {"U32": np.uint32, "BF16": np.uint16, "F32": np.float32}
ROOT = "language_model.model"


def reference_names(cfg) -> dict:
    """Tensor names and checkpoint shapes the reference's upload code reads,
    spelled out from the files cited above (q4 linear: weight [out, in/8] u32,
    scales / biases [out, in/64] bf16)."""
    out = {}

    def q4(base, n, k):
        out[base + ".weight"] = ("U32", (n, k // 8))
        out[base + ".scales"] = ("BF16", (n, k // 64))
        out[base + ".biases"] = ("BF16", (n, k // 64))

    def full_layer(p):
        a = p + ".self_attn"
        q4(a + ".q_proj", 2 * 16 * 256, cfg.hidden)
        q4(a + ".k_proj", 4 * 256, cfg.hidden)
        q4(a + ".v_proj", 4 * 256, cfg.hidden)
        q4(a + ".o_proj", cfg.hidden, 16 * 256)
        out[a + ".q_norm.weight"] = ("BF16", (256,))
        out[a + ".k_norm.weight"] = ("BF16", (256,))

    def common(p):
        out[p + ".input_layernorm.weight"] = ("BF16", (cfg.hidden,))
        out[p + ".post_attention_layernorm.weight"] = ("BF16", (cfg.hidden,))
        q4(p + ".mlp.gate_proj", cfg.intermediate, cfg.hidden)
        q4(p + ".mlp.up_proj", cfg.intermediate, cfg.hidden)
        q4(p + ".mlp.down_proj", cfg.hidden, cfg.intermediate)

    q4(ROOT + ".embed_tokens", cfg.vocab, cfg.hidden)
    for i in range(cfg.num_layers):
        p = f"{ROOT}.layers.{i}"
        common(p)
        if cfg.is_linear(i):
            a = p + ".linear_attn"
            q4(a + ".in_proj_qkv", 8192, cfg.hidden)
            q4(a + ".in_proj_z", 4096, cfg.hidden)
            q4(a + ".in_proj_a", 32, cfg.hidden)
            q4(a + ".in_proj_b", 32, cfg.hidden)
            q4(a + ".out_proj", cfg.hidden, 4096)
            out[a + ".conv1d.weight"] = ("BF16", (8192, 4, 1))
            out[a + ".A_log"] = ("F32", (32,))
            out[a + ".dt_bias"] = ("BF16", (32,))
            out[a + ".norm.weight"] = ("BF16", (128,))
        else:
            full_layer(p)
    out[ROOT + ".norm.weight"] = ("BF16", (cfg.hidden,))
    q4("language_model.lm_head", cfg.vocab, cfg.hidden)
    if cfg.mtp_layers:
        q4("mtp.fc", cfg.hidden, 2 * cfg.hidden)
        full_layer("mtp.layers.0")
        common("mtp.layers.0")
        for n in ("mtp.norm.weight", "mtp.pre_fc_norm_embedding.weight", "mtp.pre_fc_norm_hidden.weight"):
            out[n] = ("BF16", (cfg.hidden,))
    return out


def dump(m) -> dict:
    """{name: (dtype, shape, host array)} of every device tensor."""
    out = {}
    for n in m.tensor_names():
        dt, shape = m.tensor_info(n)
        out[n] = (dt, shape, m.read(n, NP[dt]).reshape(shape))
    return out


def split(tensors, mtp_root="mtp."):
    target = {n: t for n, t in tensors.items() if not n.startswith("mtp.")}
    mtp = {mtp_root + n[4:]: t for n, t in tensors.items() if n.startswith("mtp.")}
    return target, mtp


@pytest.fixture(scope="module")
def source(gpu, tmp_path_factory):
    from peregrine_amd.model import DeviceModel, ModelConfig

    cfg = ModelConfig(**SMALL, mtp_layers=1)
    m = DeviceModel(cfg, seed=11)
    tensors = dump(m)
    d = tmp_path_factory.mktemp("ckpt")
    target, mtp = split(tensors)
    write_checkpoint(d / "target", target, n_shards=3,
                     config=qwen35_config(hidden=1024, intermediate=2048, layers=4, vocab=4096))
    write_checkpoint(d / "mtp", mtp, n_shards=1)
    print(f"[ckpt] {len(tensors)} tensors, {m.weight_bytes / 2**20:.1f} MiB", flush=True)
    yield cfg, m, tensors, d
    m.close()


def test_tensor_names_and_shapes_are_the_references(source):
    cfg, m, tensors, _ = source
    ref = reference_names(cfg)
    assert set(tensors) == set(ref)
    for n, (dt, shape) in ref.items():
        assert (tensors[n][0], tuple(tensors[n][1])) == (dt, shape), n


def test_load_round_trip_bit_exact_and_same_tokens(source):
    from peregrine_amd.checkpoint import read_config
    from peregrine_amd.model import DeviceModel, ModelState

    cfg, m, tensors, d = source
    rc = read_config(d / "target")
    assert (rc.num_layers, rc.hidden, rc.intermediate, rc.vocab) == (4, 1024, 2048, 4096)
    rc.mtp_layers = 1
    loaded = DeviceModel.load(rc, d / "target", d / "mtp")
    try:
        for n, (dt, shape, a) in tensors.items():
            got = loaded.read(n, NP[dt]).reshape(shape)
            assert np.array_equal(got.view(np.uint8), a.view(np.uint8)), n
        prompt = np.random.default_rng(3).integers(0, cfg.vocab, size=24).astype(np.uint32)
        s0, s1 = ModelState(m, 64), ModelState(loaded, 64)
        p0, _ = s0.generate(prompt, 0, teacher_force=True)
        p1, _ = s1.generate(prompt, 0, teacher_force=True)
        np.testing.assert_array_equal(p0, p1)
        g0, _ = s0.generate(prompt, 16)
        g1, _ = s1.generate(prompt, 16)
        np.testing.assert_array_equal(g0, g1)
        t0 = s0.generate_speculative(prompt, 12)[0]
        t1 = s1.generate_speculative(prompt, 12)[0]
        np.testing.assert_array_equal(t0, t1)
        s0.close()
        s1.close()
    finally:
        loaded.close()


def test_loaded_model_matches_oracle(source):
    """The uploaded weights drive the same decode as the oracle's restatement
    of the reference composition (decisive steps only, as in the model tests)."""
    from oracle.model import OracleModel
    from peregrine_amd.model import DeviceModel, ModelConfig, ModelState

    cfg, _, _, d = source
    loaded = DeviceModel.load(ModelConfig(**SMALL, mtp_layers=1), d / "target", d / "mtp")
    try:
        st = ModelState(loaded, 32)
        prompt = np.random.default_rng(4).integers(0, cfg.vocab, size=12).astype(np.uint32)
        preds, _ = st.generate(prompt, 0, teacher_force=True)
        ref, logits = OracleModel(loaded, 32).teacher_forced(prompt, want_logits=True)
        checked = 0
        for n in range(len(prompt)):
            srt = np.sort(logits[n])
            ulp = 2.0 ** (np.floor(np.log2(max(abs(float(srt[-1])), 1e-30))) - 7)
            if srt[-1] - srt[-2] > 4 * ulp:
                checked += 1
                assert preds[n] == ref[n], n
        assert checked >= len(prompt) // 2
        st.close()
    finally:
        loaded.close()


@pytest.mark.parametrize("root", ["", "language_model.mtp.", "model.mtp."])
def test_mtp_root_detection(source, tmp_path, root):
    """detectRoot (mtp.zig:347-355) tries "", "mtp.", "language_model.mtp.",
    "model.mtp." for fc.weight."""
    from peregrine_amd.model import DeviceModel, ModelConfig

    _, _, tensors, d = source
    _, mtp = split(tensors, root)
    write_checkpoint(tmp_path, mtp, n_shards=1)
    loaded = DeviceModel.load(ModelConfig(**SMALL, mtp_layers=1), d / "target", tmp_path)
    try:
        for n in ("mtp.fc.weight", "mtp.layers.0.self_attn.q_norm.weight", "mtp.norm.weight"):
            dt, shape, a = tensors[n]
            assert np.array_equal(loaded.read(n, NP[dt]).reshape(shape), a), n
    finally:
        loaded.close()


def test_bf16_a_log_is_widened(source, tmp_path):
    from peregrine_amd.model import DeviceModel, ModelConfig
    from peregrine_amd.synth import bf16_to_f32, f32_to_bf16

    _, _, tensors, _ = source
    target, _ = split(tensors)
    name = f"{ROOT}.layers.0.linear_attn.A_log"
    a16 = f32_to_bf16(target[name][2])
    target = dict(target)
    target[name] = ("BF16", (32,), a16)
    write_checkpoint(tmp_path, target, n_shards=2)
    loaded = DeviceModel.load(ModelConfig(**SMALL), tmp_path)
    try:
        np.testing.assert_array_equal(loaded.read(name, np.float32), bf16_to_f32(a16))
    finally:
        loaded.close()


def _load_err(tmp_path, target, mtp_dir=None, cfg=None):
    from peregrine_amd._lib import PrgError
    from peregrine_amd.model import DeviceModel, ModelConfig

    write_checkpoint(tmp_path, target, n_shards=2)
    with pytest.raises(PrgError) as e:
        DeviceModel.load(cfg or ModelConfig(**SMALL), tmp_path, mtp_dir)
    return e.value


def test_load_errors(source, tmp_path):
    _, _, tensors, d = source
    target, _ = split(tensors)
    w = f"{ROOT}.layers.3.self_attn.k_proj.weight"

    missing = {n: t for n, t in target.items() if n != w}
    e = _load_err(tmp_path / "a", missing)
    assert e.code == 8 and "TensorNotFound" in str(e) and w in str(e)

    bad_shape = dict(target)
    dt, (n_, k8), arr = target[w]
    bad_shape[w] = (dt, (n_ // 2, k8 * 2), arr)
    e = _load_err(tmp_path / "b", bad_shape)
    assert e.code == 9 and "InvalidTensorShape" in str(e)

    flat = dict(target)
    flat[w] = (dt, (n_ * k8,), arr)  # a q4 weight must be 2-D (linear_q4.zig:262)
    e = _load_err(tmp_path / "c", flat)
    assert e.code == 10 and "UnsupportedQuantization" in str(e)

    bad_dtype = dict(target)
    nw = f"{ROOT}.norm.weight"
    bad_dtype[nw] = ("F16", target[nw][1], target[nw][2])
    e = _load_err(tmp_path / "d", bad_dtype)
    assert e.code == 9 and "dtype" in str(e)

    from peregrine_amd.model import ModelConfig

    wrong_vocab = ModelConfig(**{**SMALL, "vocab": 2048})
    e = _load_err(tmp_path / "e", target, cfg=wrong_vocab)
    assert e.code == 9 and "InvalidTensorShape" in str(e)

    from peregrine_amd._lib import PrgError
    from peregrine_amd.model import DeviceModel

    with pytest.raises(PrgError) as ei:
        DeviceModel.load(ModelConfig(**SMALL), d / "target", d / "mtp")  # mtp_dir without mtp_layers
    assert ei.value.code == 1


def test_short_tensor_bytes_rejected(source, tmp_path):
    """A header whose data_offsets disagree with dtype x shape is refused
    before any byte is copied."""
    _, _, tensors, _ = source
    target, _ = split(tensors)
    nw = f"{ROOT}.norm.weight"
    target = dict(target)
    dt, shape, a = target[nw]
    target[nw] = (dt, shape, a.tobytes()[:-2])
    e = _load_err(tmp_path, target)
    assert e.code == 9 and "MalformedHeader" in str(e)
