"""Gated squared-ReLU feed-forward block on gfx950 (API of bitnet-tt's
``src/bitnet_tt/layers/ffn.py``).

    gate||up = BitLinear(x)                     one launch, K=hidden, N=2*F
    h        = relu(gate)^2 * up                in that launch's epilogue
    out      = BitLinear_down(ffn_sub_norm(h))  one launch, the sub-norm and the
                                                int8 quantiser are its prologue

Gate and up keep their own absmean scales (separately quantised,
ffn.py:22-34) and the epilogue applies them per column segment, which is the
HF BitNet arithmetic.  The reference instead runs gate||up with scale 1.0 and
lets ffn_sub_norm absorb the positive factor s_gate^2*s_up (ffn.py:153-158);
the two agree up to the eps inside the sub-norm.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

from .bitlinear import Linear, RMSNorm, quantize_and_transpose_weight


def build_fused_gate_up_weight(gate_weight, up_weight) -> tuple[np.ndarray, float, float]:
    """Pre-transposed ternary (hidden, 2F) gate||up matrix plus the two scales
    (ffn.py:22-34)."""
    gate_weight_t, gate_scale = quantize_and_transpose_weight(gate_weight)
    up_weight_t, up_scale = quantize_and_transpose_weight(up_weight)
    fused = np.concatenate([gate_weight_t, up_weight_t], axis=1)
    return fused, gate_scale, up_scale


class FeedForward:
    """ffn.py:37-183 with the launches fused as described in the module doc."""

    def __init__(self, hidden_size: int, intermediate_size: int, device=None, eps: float = 1e-5,
                 model_config: Optional[dict] = None, use_lofi: bool = False,
                 weight_dtype: str = "packed_ternary") -> None:
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.device = device
        self.eps = eps
        self.model_config = model_config or {}
        self.use_lofi = use_lofi
        fidelity = "lofi" if use_lofi else "hifi2"
        self.gate_up_proj = Linear(hidden_size, intermediate_size * 2, device, compute_fidelity=fidelity,
                                   weight_dtype=weight_dtype)
        self.gate_up_proj.epilogue = "relu2_mul"
        self.down_proj = Linear(intermediate_size, hidden_size, device, compute_fidelity=fidelity,
                                weight_dtype=weight_dtype)
        self.ffn_sub_norm = RMSNorm(intermediate_size, device, eps)
        self._gate_scale = 1.0
        self._up_scale = 1.0

    def load_weights(self, gate_weight, up_weight, down_weight, ffn_sub_norm_weight=None) -> None:
        """ffn.py:104-127."""
        fused, self._gate_scale, self._up_scale = build_fused_gate_up_weight(gate_weight, up_weight)
        f = self.intermediate_size
        self.gate_up_proj.load_pretransposed_weight(
            fused, segment_scales=(self._gate_scale, self._up_scale), segment_ends=(f, 2 * f)
        )
        self.down_proj.load_weights(down_weight)
        if ffn_sub_norm_weight is None:
            ffn_sub_norm_weight = np.ones(f, dtype=np.float32)
        self.ffn_sub_norm.load_weights(ffn_sub_norm_weight)

    def __call__(self, x, mode: str = "prefill", norm_weight=None, norm_epsilon: float | None = None,
                 residual=None, out=None):
        """x bf16 [..., hidden] -> bf16 [..., hidden] (ffn.py:129-183).

        ``norm_weight``/``norm_epsilon`` optionally fuse the block's input
        RMSNorm (post_attention_layernorm) into the gate||up prologue;
        ``residual`` (and ``out``) fuse the block's residual add into the
        down projection.  ``mode`` is accepted for API compatibility: decode and
        prefill differ only in the kernel the library picks for M."""
        h = self.gate_up_proj(x, norm_weight=norm_weight, norm_epsilon=norm_epsilon)
        return self.down_proj(h, norm_weight=self.ffn_sub_norm.weight, norm_epsilon=self.ffn_sub_norm.eps,
                              residual=residual, out=out)
