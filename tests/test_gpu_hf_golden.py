"""The HIP model against the transformers float reference (GPU).

The seeded host model of tests/hostmodel.py is written as an MLX checkpoint,
uploaded with prg_model_load, and driven through the C ABI. Its greedy tokens
(teacher-forced decode, the layer-major prefill, and the MTP drafter fed the
fixture's hidden rows) must equal the fixture's top-1 wherever the fixture's
top-2 margin exceeds 4 bf16 ulps of its top logit. The fixture,
tests/golden/hf_v1.npz, comes from transformers' Qwen3.5 text model in
float64 (tests/golden/make_hf_golden.py; CPU only, not imported here), so
this check does not pass through the oracle.
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import qwen35_config, write_checkpoint
from hostmodel import HostModel
from peregrine_amd.model import ModelConfig
from peregrine_amd.synth import f32_to_bf16

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "hf_v1.npz"


def decisive(ref_logits) -> bool:
    s = np.sort(np.asarray(ref_logits, np.float64))
    guard = 4 * 2.0 ** (np.floor(np.log2(max(abs(s[-1]), 1e-30))) - 7)
    return bool(s[-1] - s[-2] > guard)


@pytest.fixture(scope="module")
def loaded(gpu, tmp_path_factory):
    from peregrine_amd.model import DeviceModel

    z = np.load(FIXTURE, allow_pickle=False)
    c = [int(v) for v in z["config"]]
    cfg = ModelConfig(num_layers=c[0], hidden=c[1], intermediate=c[2], vocab=c[3], mtp_layers=c[4])
    hm = HostModel(cfg, int(z["seed"]))
    assert hm.digest() == str(z["digest"])
    d = tmp_path_factory.mktemp("hf_ckpt")
    t = hm.tensors()
    write_checkpoint(d / "target", {n: v for n, v in t.items() if not n.startswith("mtp.")}, n_shards=2,
                     config=qwen35_config(hidden=cfg.hidden, intermediate=cfg.intermediate,
                                          layers=cfg.num_layers, vocab=cfg.vocab))
    write_checkpoint(d / "mtp", {n: v for n, v in t.items() if n.startswith("mtp.")}, n_shards=1)
    m = DeviceModel.load(cfg, d / "target", d / "mtp")
    print(f"[hf] loaded {len(t)} tensors", flush=True)
    yield m, z
    m.close()


def test_teacher_forced_tokens_match_transformers(loaded):
    from peregrine_amd.model import ModelState

    m, z = loaded
    st = ModelState(m, 64)
    preds, _ = st.generate(z["prompt"], 0, teacher_force=True)
    st.close()
    dec = [n for n in range(len(z["prompt"])) if decisive(z["logits"][n])]
    assert len(dec) >= 20
    bad = [(n, int(preds[n]), int(np.argmax(z["logits"][n]))) for n in dec if preds[n] != np.argmax(z["logits"][n])]
    assert not bad, bad


def test_prefill_next_token_matches_transformers(loaded):
    from peregrine_amd.model import ModelState

    m, z = loaded
    for cut in (8, 17, len(z["prompt"])):
        if not decisive(z["logits"][cut - 1]):
            continue
        st = ModelState(m, 64)
        assert st.prefill(z["prompt"][:cut]) == int(np.argmax(z["logits"][cut - 1])), cut
        st.close()


def test_drafter_tokens_match_transformers_parts(loaded):
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.model import ModelState

    m, z = loaded
    p, hid, ref = z["prompt"], f32_to_bf16(z["hidden"]), z["draft_logits"]
    st = ModelState(m, 64)
    split = 12
    st.mtp_prefill(p[1:split + 1], DeviceArray.from_numpy(np.ascontiguousarray(hid[:split])), 0)
    checked = 0
    for j in range(split, len(p) - 1):
        d = st.mtp_draft(int(p[j + 1]), DeviceArray.from_numpy(np.ascontiguousarray(hid[j])), j)
        if decisive(ref[j]):
            checked += 1
            assert d == int(np.argmax(ref[j])), j
    st.close()
    assert checked >= 8
