"""Checkpoint ingest: HF safetensors -> state dict -> the decode step's device
weights (API of bitnet-tt's ``src/bitnet_tt/utils/weights.py``).

``load_bitnet_weights`` reads a local HF snapshot (``config.json`` plus
``*.safetensors``) into float32 numpy arrays under the reference's keys
(utils/weights.py:19-84, key map :87-155).  The reference downloads the
snapshot first; this environment has no network, so a model id resolves only
through an existing directory or the local HF cache.

Two checkpoint kinds are read:

* the bf16 latent checkpoint the reference loads
  (``microsoft/bitnet-b1.58-2B-4T-bf16``): every BitLinear weight is a float
  (out, in) matrix, quantised later by the absmean rule
  (quantization.py:15-57);
* HF's pre-packed checkpoint (``microsoft/bitnet-b1.58-2B-4T``): each BitLinear
  weight is uint8 (out/4, in) holding four 2-bit codes w+1 per byte, stacked
  along out in blocks of out/4 rows, with a ``weight_scale`` that multiplies
  the latent weight before rounding (transformers integrations/bitnet.py:
  17-119, 139-143, 200-205).  Such a pair becomes a :class:`TernaryWeight`
  (ternary int8 (out, in) and the dequantisation scale 1/weight_scale).

``load_weights_to_model`` / ``BitLinearDecodeStep.from_state_dict`` then
quantise on the device (or take the ternary codes as they are) and pack into
the GEMM's device layout.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Any

import numpy as np

from ..config import BitNet2B4TConfig, BitNetConfig

VALUES_PER_ITEM = 4  # 2-bit codes per uint8 in HF's packed format

# reference key map (utils/weights.py:104-132)
_KEY_MAPPING = {
    "model.embed_tokens.weight": "embed_tokens.weight",
    "model.norm.weight": "norm.weight",
    "lm_head.weight": "lm_head.weight",
}
_LAYER_MAPPING = {
    name: name
    for name in (
        "input_layernorm.weight",
        "post_attention_layernorm.weight",
        "self_attn.q_proj.weight",
        "self_attn.k_proj.weight",
        "self_attn.v_proj.weight",
        "self_attn.o_proj.weight",
        "mlp.gate_proj.weight",
        "mlp.up_proj.weight",
        "mlp.down_proj.weight",
        "self_attn.attn_sub_norm.weight",
        "mlp.ffn_sub_norm.weight",
        "self_attn.q_proj.input_norm.weight",
        "self_attn.k_proj.input_norm.weight",
        "self_attn.v_proj.input_norm.weight",
        "self_attn.o_proj.input_norm.weight",
        "mlp.gate_proj.input_norm.weight",
        "mlp.up_proj.input_norm.weight",
        "mlp.down_proj.input_norm.weight",
    )
}

BITLINEAR_KEYS = (
    "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
    "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj",
)


@dataclass
class TernaryWeight:
    """An already-quantised BitLinear weight: ``q`` int8 (out, in) in {-1, 0, +1}
    and ``scale`` with latent ~= q * scale (the reference's ``weight_scale``)."""

    q: np.ndarray
    scale: float

    @property
    def shape(self):
        return self.q.shape


# ---------------------------------------------------------------- HF packing --
def unpack_hf_ternary(packed: np.ndarray) -> np.ndarray:
    """uint8 (rows, ...) -> int8 (4*rows, ...): row i*rows + r of the result is
    bits 2i..2i+1 of packed row r, minus 1 (integrations/bitnet.py:52-119)."""
    p = np.asarray(packed)
    if p.dtype != np.uint8:
        raise TypeError(f"packed ternary weights are uint8, got {p.dtype}")
    shifts = (2 * np.arange(VALUES_PER_ITEM, dtype=np.uint8)).reshape((VALUES_PER_ITEM,) + (1,) * p.ndim)
    codes = (p[None, ...] >> shifts) & np.uint8(3)
    if np.any(codes == 3):
        raise ValueError("packed ternary weight holds the unused 2-bit code 3")
    return (codes.astype(np.int8) - 1).reshape((VALUES_PER_ITEM * p.shape[0],) + p.shape[1:])


def pack_hf_ternary(q: np.ndarray) -> np.ndarray:
    """int8 ternary (out, ...) -> HF's uint8 (ceil(out/4), ...) layout
    (integrations/bitnet.py:17-49): block i of ceil(out/4) rows goes to bits
    2i..2i+1 as the code w+1; rows past ``out`` stay 0 bits."""
    w = np.asarray(q)
    if not np.all(np.isin(w, (-1, 0, 1))):
        raise ValueError("pack_hf_ternary expects values in {-1, 0, +1}")
    rows = (w.shape[0] + VALUES_PER_ITEM - 1) // VALUES_PER_ITEM
    out = np.zeros((rows,) + w.shape[1:], dtype=np.uint8)
    codes = (w.astype(np.int16) + 1).astype(np.uint8)
    for i in range(VALUES_PER_ITEM):
        blk = codes[i * rows:(i + 1) * rows]
        out[: blk.shape[0]] |= blk << np.uint8(2 * i)
    return out


# ------------------------------------------------------------------ loading --
def _resolve_snapshot(model_id: str, cache_dir: str | None) -> str:
    if os.path.isdir(model_id):
        return model_id
    try:
        from huggingface_hub import snapshot_download
    except ImportError as e:  # pragma: no cover - huggingface_hub is installed here
        raise FileNotFoundError(f"{model_id!r} is not a directory and huggingface_hub is missing") from e
    try:
        return snapshot_download(model_id, cache_dir=cache_dir, allow_patterns=["*.safetensors", "config.json"],
                                 local_files_only=True)
    except Exception as e:
        raise FileNotFoundError(
            f"{model_id!r}: no local snapshot (pass a directory holding config.json and *.safetensors; "
            "nothing is downloaded)"
        ) from e


def config_from_hf(hf_config: dict) -> BitNetConfig:
    """Our config from an HF ``config.json`` dict (utils/weights.py:56-67)."""
    return BitNet2B4TConfig(
        hidden_size=hf_config.get("hidden_size", 2560),
        num_layers=hf_config.get("num_hidden_layers", 30),
        num_attention_heads=hf_config.get("num_attention_heads", 20),
        num_key_value_heads=hf_config.get("num_key_value_heads", 5),
        intermediate_size=hf_config.get("intermediate_size", 6912),
        vocab_size=hf_config.get("vocab_size", 128256),
        max_position_embeddings=hf_config.get("max_position_embeddings", 4096),
        rms_norm_eps=hf_config.get("rms_norm_eps", 1e-6),
        rope_theta=hf_config.get("rope_theta", 500000.0),
    )


def _fold_packed(state: dict[str, Any]) -> dict[str, Any]:
    """Replace every (uint8 ``X.weight``, ``X.weight_scale``) pair by a
    TernaryWeight under ``X.weight``."""
    out = dict(state)
    for key in list(state):
        if not key.endswith(".weight_scale"):
            continue
        wkey = key[: -len("_scale")]
        w = state.get(wkey)
        if w is None or np.asarray(w).dtype != np.uint8:
            continue
        s = float(np.asarray(state[key], dtype=np.float32).reshape(-1)[0])
        if not np.isfinite(s) or s <= 0.0:
            raise ValueError(f"{key}: weight_scale must be positive, got {s}")
        out[wkey] = TernaryWeight(unpack_hf_ternary(w), float(np.float32(1.0) / np.float32(s)))
        del out[key]
    return out


def load_bitnet_weights(
    model_id: str = "microsoft/bitnet-b1.58-2B-4T-bf16",
    cache_dir: str | None = None,
) -> tuple[dict[str, Any], BitNetConfig]:
    """(state dict under the reference's keys, config) of a local HF snapshot
    (utils/weights.py:19-84).  Float tensors become float32 numpy arrays (bf16
    widened exactly); packed uint8 BitLinear weights become TernaryWeight."""
    import torch
    from safetensors import safe_open

    path = _resolve_snapshot(model_id, cache_dir)
    with open(os.path.join(path, "config.json")) as f:
        config = config_from_hf(json.load(f))
    state: dict[str, Any] = {}
    files = sorted(fn for fn in os.listdir(path) if fn.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"{path}: no *.safetensors files")
    for fn in files:
        with safe_open(os.path.join(path, fn), framework="pt") as f:
            for key in f.keys():
                t = f.get_tensor(key)
                if t.dtype in (torch.bfloat16, torch.float16):
                    t = t.float()
                state[key] = t.numpy()
    return convert_hf_state_dict(_fold_packed(state)), config


def convert_hf_state_dict(hf_state_dict: dict[str, Any]) -> dict[str, Any]:
    """HF keys -> the reference's keys (utils/weights.py:87-155): top-level
    names mapped, ``model.layers.<i>.<rest>`` -> ``layers.<i>.<rest>``, other
    keys kept."""
    converted: dict[str, Any] = {}
    for hf_key, tensor in hf_state_dict.items():
        if hf_key in _KEY_MAPPING:
            converted[_KEY_MAPPING[hf_key]] = tensor
        elif hf_key.startswith("model.layers."):
            parts = hf_key.split(".")
            rest = ".".join(parts[3:])
            converted[f"layers.{parts[2]}.{_LAYER_MAPPING.get(rest, rest)}"] = tensor
        else:
            converted[hf_key] = tensor
    return converted


def get_layer_weights(state_dict: dict[str, Any], layer_idx: int) -> dict[str, Any]:
    """Entries of one layer with the ``layers.<i>.`` prefix removed
    (utils/weights.py:158-181)."""
    prefix = f"layers.{layer_idx}."
    return {k[len(prefix):]: v for k, v in state_dict.items() if k.startswith(prefix)}


def save_numpy_weights(state_dict: dict[str, Any], output_path: str) -> None:
    """npz of the state dict (utils/weights.py:184-196); a TernaryWeight is
    stored as ``<key>.ternary`` (int8) plus ``<key>.ternary_scale``."""
    arrays = {}
    for k, v in state_dict.items():
        if isinstance(v, TernaryWeight):
            arrays[k + ".ternary"] = v.q
            arrays[k + ".ternary_scale"] = np.float32(v.scale)
        else:
            arrays[k] = np.asarray(v)
    np.savez_compressed(output_path, **arrays)


def load_numpy_weights(input_path: str) -> dict[str, Any]:
    """Inverse of :func:`save_numpy_weights` (utils/weights.py:199-211); no
    pickled objects are accepted."""
    out: dict[str, Any] = {}
    with np.load(input_path, allow_pickle=False) as data:
        names = set(data.files)
        for k in data.files:
            if k.endswith(".ternary_scale"):
                continue
            if k.endswith(".ternary") and k + "_scale" in names:
                out[k[: -len(".ternary")]] = TernaryWeight(data[k], float(data[k + "_scale"]))
            else:
                out[k] = data[k]
    return out


def load_weights_to_model(model: Any, state_dict: dict[str, Any]) -> None:
    """Per-layer weights into a model with ``load_layer_weights(i, weights)``
    (utils/weights.py:214-246).  Embedding, final norm and LM head are not on
    the BitLinear path and are ignored here."""
    for layer_idx in range(len(model.layers)):
        lw = get_layer_weights(state_dict, layer_idx)
        if lw:
            model.load_layer_weights(layer_idx, lw)
