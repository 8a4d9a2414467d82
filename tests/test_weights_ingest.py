"""Checkpoint ingest on the CPU: HF's packed ternary layout, the reference's
key conversion, safetensors snapshots (bf16 latents and HF pre-packed) and
the npz round trip (utils/weights.py:19-246; transformers
integrations/bitnet.py:17-119 for the packed layout)."""

import os

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt.config import BitNetMiniConfig
from bitnet_tt.utils.quantization import weight_quant_ternary
from bitnet_tt.utils.weights import (
    TernaryWeight,
    convert_hf_state_dict,
    get_layer_weights,
    load_bitnet_weights,
    load_numpy_weights,
    pack_hf_ternary,
    save_numpy_weights,
    unpack_hf_ternary,
)


def test_unpack_hf_known_answer():
    """The worked example of HF's unpack_weights docstring
    (integrations/bitnet.py:76-100): two packed rows -> eight ternary rows."""
    packed = np.array([[0b10100001, 0b00011000], [0b10010000, 0b00001010]], dtype=np.uint8)
    expect = np.array([[0, -1], [-1, 1], [-1, 1], [-1, 1], [1, 0], [0, -1], [1, -1], [1, -1]], dtype=np.int8)
    assert np.array_equal(unpack_hf_ternary(packed), expect)
    assert np.array_equal(pack_hf_ternary(expect), packed)


def test_every_byte_code():
    """All 81 ternary 4-tuples of a one-column matrix: each packs to the byte
    sum((w_i + 1) << 2i) and unpacks back; the 175 bytes holding a 3 code are
    rejected."""
    vals = (-1, 0, 1)
    seen = set()
    for a in vals:
        for b in vals:
            for c in vals:
                for d in vals:
                    col = np.array([[a], [b], [c], [d]], dtype=np.int8)
                    byte = int(pack_hf_ternary(col)[0, 0])
                    assert byte == (a + 1) | (b + 1) << 2 | (c + 1) << 4 | (d + 1) << 6
                    assert np.array_equal(unpack_hf_ternary(np.array([[byte]], dtype=np.uint8)), col)
                    seen.add(byte)
    assert len(seen) == 81
    for byte in set(range(256)) - seen:
        with pytest.raises(ValueError):
            unpack_hf_ternary(np.array([byte], dtype=np.uint8))


@pytest.mark.parametrize("shape", [(8, 5), (64, 96), (12,), (10, 3)])
def test_pack_matches_transformers_pack_weights(shape):
    """Against transformers' own pack_weights (a library routine, not the
    reference), including an out dimension that is not a multiple of 4."""
    from transformers.integrations.bitnet import pack_weights

    rng = np.random.default_rng(sum(shape))
    q = rng.integers(-1, 2, size=shape).astype(np.int8)
    ref = pack_weights(torch.from_numpy(q.astype(np.int32))).numpy()
    assert np.array_equal(pack_hf_ternary(q), ref)
    back = unpack_hf_ternary(ref)
    assert np.array_equal(back[: shape[0]], q)
    assert np.all(back[shape[0]:] == -1)  # rows past `out` unpack from zero bits


def test_convert_keys_and_layer_split():
    sd = {
        "model.embed_tokens.weight": 1,
        "model.norm.weight": 2,
        "lm_head.weight": 3,
        "model.layers.0.self_attn.q_proj.weight": 4,
        "model.layers.0.mlp.ffn_sub_norm.weight": 5,
        "model.layers.11.self_attn.q_proj.weight_scale": 6,
        "extra.thing": 7,
    }
    c = convert_hf_state_dict(sd)
    assert c == {
        "embed_tokens.weight": 1,
        "norm.weight": 2,
        "lm_head.weight": 3,
        "layers.0.self_attn.q_proj.weight": 4,
        "layers.0.mlp.ffn_sub_norm.weight": 5,
        "layers.11.self_attn.q_proj.weight_scale": 6,
        "extra.thing": 7,
    }
    assert get_layer_weights(c, 0) == {"self_attn.q_proj.weight": 4, "mlp.ffn_sub_norm.weight": 5}
    assert get_layer_weights(c, 1) == {}


@pytest.mark.parametrize("packed", [False, True])
def test_safetensors_snapshot(tmp_path, packed):
    cfg = BitNetMiniConfig(num_layers=2)
    expect = H.write_hf_snapshot(str(tmp_path), cfg, seed=5, packed=packed)
    sd, got_cfg = load_bitnet_weights(str(tmp_path))
    assert (got_cfg.hidden_size, got_cfg.num_layers, got_cfg.intermediate_size) == (256, 2, 512)
    assert (got_cfg.num_attention_heads, got_cfg.num_key_value_heads, got_cfg.rms_norm_eps) == (4, 2, cfg.rms_norm_eps)
    assert "embed_tokens.weight" in sd and "norm.weight" in sd
    assert not any(k.endswith("weight_scale") for k in sd)
    for hf_key, ref in expect.items():
        key = hf_key[len("model."):]
        got = sd[key]
        if packed and isinstance(ref, tuple):
            assert isinstance(got, TernaryWeight)
            assert np.array_equal(got.q, ref[0])
            assert got.scale == float(ref[1])
        else:
            assert got.dtype == np.float32 and np.array_equal(got, ref)
    if not packed:  # the latent path quantises exactly as the reference does
        w = sd["layers.1.mlp.down_proj.weight"]
        q, s = weight_quant_ternary(w)
        assert q.dtype == np.int8 and np.float32(s) == s


def test_npz_round_trip(tmp_path):
    sd = {"layers.0.x.weight": np.arange(6, dtype=np.float32).reshape(2, 3),
          "layers.0.q_proj.weight": TernaryWeight(np.array([[1, 0, -1]], dtype=np.int8), 0.0123)}
    p = os.path.join(str(tmp_path), "w.npz")
    save_numpy_weights(sd, p)
    back = load_numpy_weights(p)
    assert set(back) == set(sd)
    assert np.array_equal(back["layers.0.x.weight"], sd["layers.0.x.weight"])
    t = back["layers.0.q_proj.weight"]
    assert isinstance(t, TernaryWeight) and np.array_equal(t.q, sd["layers.0.q_proj.weight"].q)
    assert t.scale == float(np.float32(0.0123))


def test_missing_snapshot_is_an_error(monkeypatch, tmp_path):
    monkeypatch.setenv("HF_HUB_OFFLINE", "1")
    with pytest.raises(FileNotFoundError):
        load_bitnet_weights("no-such-org/no-such-model", cache_dir=str(tmp_path))
    os.makedirs(os.path.join(str(tmp_path), "empty"))
    with open(os.path.join(str(tmp_path), "empty", "config.json"), "w") as f:
        f.write("{}")
    with pytest.raises(FileNotFoundError):
        load_bitnet_weights(os.path.join(str(tmp_path), "empty"))


def test_bad_weight_scale_rejected(tmp_path):
    from safetensors.torch import save_file

    save_file({"model.layers.0.self_attn.q_proj.weight": torch.zeros((1, 4), dtype=torch.uint8),
               "model.layers.0.self_attn.q_proj.weight_scale": torch.zeros(1, dtype=torch.bfloat16)},
              os.path.join(str(tmp_path), "m.safetensors"))
    with open(os.path.join(str(tmp_path), "config.json"), "w") as f:
        f.write("{}")
    with pytest.raises(ValueError, match="weight_scale"):
        load_bitnet_weights(str(tmp_path))
