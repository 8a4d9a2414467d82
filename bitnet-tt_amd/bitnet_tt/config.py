"""BitNet model dimensions used by the BitLinear path.

The numbers of ``src/bitnet_tt/config.py:13-48`` (BitNet b1.58 2B-4T): hidden
2560, 30 layers, 20 query heads / 5 key-value heads of 128, FFN 6912, RMSNorm
eps 1e-5, RoPE theta 5e5.  Tenstorrent compute-kernel settings of the
reference have no counterpart here.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class BitNetConfig:
    hidden_size: int = 2560
    num_layers: int = 30
    num_attention_heads: int = 20
    num_key_value_heads: int = 5
    intermediate_size: int = 6912
    vocab_size: int = 128256
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    weight_bits: int = 2
    activation_bits: int = 8
    hidden_act: str = "relu2"

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def num_kv_heads(self) -> int:
        return self.num_key_value_heads

    @property
    def qkv_dim(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim


@dataclass
class BitNet2B4TConfig(BitNetConfig):
    pass


@dataclass
class BitNetMiniConfig(BitNetConfig):
    """Small model for tests (src/bitnet_tt/config.py:130-147)."""

    hidden_size: int = 256
    num_layers: int = 4
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    intermediate_size: int = 512
    vocab_size: int = 1000
    max_position_embeddings: int = 512


def get_config(model_name: str = "mini") -> BitNetConfig:
    """One of "mini", "2b4t" or "base" (src/bitnet_tt/config.py:174-193)."""
    configs = {"mini": BitNetMiniConfig, "2b4t": BitNet2B4TConfig, "base": BitNetConfig}
    if model_name not in configs:
        raise ValueError(f"Unknown model: {model_name}. Choose from {list(configs.keys())}")
    return configs[model_name]()
