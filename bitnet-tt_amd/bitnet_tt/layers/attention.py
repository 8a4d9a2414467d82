"""The BitLinear side of attention: the fused Q|K|V projection with its RMSNorm
prologue, and the o_proj projection (API pieces of bitnet-tt's
``src/bitnet_tt/layers/attention.py``).

The attention core (RoPE, KV cache, SDPA) is not part of this package.

Fused QKV: q, k and v are quantised separately (three absmean scales), the
Q and K column blocks are optionally permuted from HF half-split to
adjacent-pair RoPE order, and the three are concatenated along N
(attention.py:462-506).  One launch computes
``RMSNorm(input_layernorm) -> int8 quant -> [Q|K|V] GEMM`` exactly as the
decode loop's ``ternary_matmul(hidden, qkv, norm_weight=..., norm_epsilon=...)``
(inference/generator_batch32.py:718-727).  By default the epilogue applies
q_s, k_s, v_s to their column segments; ``apply_scales=False`` reproduces the
reference's folding (scale 1.0 here, q_s*k_s into the SDPA scale and v_s
absorbed by attn_sub_norm, attention.py:817-839).
"""

from __future__ import annotations

import numpy as np

from .bitlinear import Linear, quantize_and_transpose_weight


def _permute_halfsplit_to_adjacent(weight_t: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """Per head, new column 2k = old column k and 2k+1 = old k + head_dim/2
    (attention.py:462-478)."""
    half = head_dim // 2
    perm = np.empty(head_dim, dtype=np.intp)
    perm[0::2] = np.arange(half)
    perm[1::2] = np.arange(half) + half
    k = weight_t.shape[0]
    return weight_t.reshape(k, num_heads, head_dim)[:, :, perm].reshape(k, num_heads * head_dim).copy()


def build_fused_qkv_weight(q_weight, k_weight, v_weight, num_heads: int = 0, num_kv_heads: int = 0,
                           head_dim: int = 0, permute_for_rope: bool = False):
    """(hidden, q+k+v) ternary matrix and the three scales (attention.py:481-506)."""
    q_t, q_scale = quantize_and_transpose_weight(q_weight)
    k_t, k_scale = quantize_and_transpose_weight(k_weight)
    v_t, v_scale = quantize_and_transpose_weight(v_weight)
    if permute_for_rope and head_dim > 0:
        q_t = _permute_halfsplit_to_adjacent(q_t, num_heads, head_dim)
        k_t = _permute_halfsplit_to_adjacent(k_t, num_kv_heads, head_dim)
    fused = np.concatenate([q_t, k_t, v_t], axis=1)
    return fused, q_scale, k_scale, v_scale


class QKVProjection:
    """Fused RMSNorm -> Q|K|V BitLinear plus o_proj (attention.py:776-839)."""

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int, device=None,
                 weight_dtype: str = "packed_ternary", use_fused_rope: bool = False) -> None:
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.device = device
        self.use_fused_rope = use_fused_rope
        self.q_dim = num_heads * head_dim
        self.kv_dim = num_kv_heads * head_dim
        self._qkv_dim = self.q_dim + 2 * self.kv_dim
        self.qkv = Linear(hidden_size, self._qkv_dim, device, weight_dtype=weight_dtype)
        self.o_proj = Linear(self.q_dim, hidden_size, device, weight_dtype=weight_dtype)
        self._qkv_scales = (1.0, 1.0, 1.0)

    def load_weights(self, q_weight, k_weight, v_weight, o_weight=None, apply_scales: bool = True) -> None:
        fused, q_s, k_s, v_s = build_fused_qkv_weight(
            q_weight, k_weight, v_weight, num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim, permute_for_rope=self.use_fused_rope,
        )
        self._qkv_scales = (float(q_s), float(k_s), float(v_s))
        ends = (self.q_dim, self.q_dim + self.kv_dim, self._qkv_dim)
        scales = self._qkv_scales if apply_scales else (1.0, 1.0, 1.0)
        self.qkv.load_pretransposed_weight(fused, segment_scales=scales, segment_ends=ends)
        if o_weight is not None:
            self.o_proj.load_weights(o_weight)

    @property
    def qkv_fused_weight(self):
        return self.qkv.weight

    def __call__(self, hidden, norm_weight=None, norm_epsilon: float | None = None):
        """bf16 [..., hidden] -> bf16 [..., q+k+v]."""
        return self.qkv(hidden, norm_weight=norm_weight, norm_epsilon=norm_epsilon)
