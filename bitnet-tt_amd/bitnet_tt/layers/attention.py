"""The BitLinear side of attention: the fused Q|K|V projection with its RMSNorm
prologue, and the o_proj projection (API pieces of bitnet-tt's
``src/bitnet_tt/layers/attention.py``).

``DecodeAttention`` is the decode attention between the QKV projection and
o_proj (attention.py:1040-1262): RoPE, KV-cache update and SDPA over the
cached positions, one gfx950 launch per layer.

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


class KVCache:
    """Pre-allocated per-layer cache (attention.py KVCache): key_cache and
    value_cache [batch, kv_heads, max_seq_len, head_dim] bf16."""

    def __init__(self, batch: int, num_kv_heads: int, max_seq_len: int, head_dim: int, device) -> None:
        import torch

        shape = (batch, num_kv_heads, max_seq_len, head_dim)
        self.key_cache = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.value_cache = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.seq_len_cached = 0


class DecodeAttention:
    """Decode attention of one layer (attention.py:1040-1262):

    q, k, v = split(qkv); q, k = RoPE(q, k; pos); cache[pos] = k, v;
    out = concat_h softmax(scale * q_h K^T) V over positions [0, pos]

    ``use_fused_rope`` selects the reference's adjacent-pair RoPE (for Q/K
    weights permuted as ``build_fused_qkv_weight(permute_for_rope=True)``
    does); otherwise HF's half-split RoPE on unpermuted weights.  ``scale``
    defaults to 1/sqrt(head_dim); with the QKV scales folded out of the
    projection it is that times q_scale * k_scale (attention.py:817-839)."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int, max_seq_len: int, device=None,
                 rope_theta: float = 500000.0, use_fused_rope: bool = False, scale: float | None = None) -> None:
        import math

        import torch

        from ..utils.rope import rope_tables

        if head_dim != 128 or num_heads % num_kv_heads or num_heads // num_kv_heads > 4:
            raise ValueError("the decode-attention kernel takes head_dim 128 and up to 4 query heads per KV head")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.use_fused_rope = use_fused_rope
        self.scale = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
        cos, sin = rope_tables(head_dim, max_seq_len, rope_theta)
        self.rope_cos = torch.from_numpy(cos).to(self.device)
        self.rope_sin = torch.from_numpy(sin).to(self.device)

    def new_cache(self, batch: int) -> KVCache:
        return KVCache(batch, self.num_kv_heads, self.max_seq_len, self.head_dim, self.device)

    def __call__(self, qkv, kv_cache: KVCache, pos, out=None):
        """qkv bf16 [B, (H + 2 Hkv) D]; pos int32 [B] on the device (each user's
        new position; a device tensor so a captured graph can advance it);
        returns bf16 [B, H D] (written into ``out`` when given)."""
        import torch

        from .. import _native as N

        B = qkv.shape[0]
        H, Hkv, D, S = self.num_heads, self.num_kv_heads, self.head_dim, self.max_seq_len
        N.require_cuda(qkv, "qkv")
        N.require_cuda(pos, "pos")
        if qkv.dtype != torch.bfloat16 or tuple(qkv.shape) != (B, (H + 2 * Hkv) * D):
            raise ValueError(f"qkv must be bf16 [B, {(H + 2 * Hkv) * D}]")
        if pos.dtype != torch.int32 or pos.numel() != B:
            raise ValueError("pos must be int32 [B]")
        if tuple(kv_cache.key_cache.shape) != (B, Hkv, S, D):
            raise ValueError("cache shape does not match")
        if out is None:
            out = torch.empty((B, H * D), dtype=torch.bfloat16, device=qkv.device)
        L = N.lib()
        nbytes = int(L.btl_decode_attention_workspace_bytes(B, H, Hkv, S))
        if torch.cuda.is_current_stream_capturing() and not N.has_workspace(qkv.device, nbytes, "attention"):
            raise RuntimeError("run one eager attention call on this stream before capturing it in a graph")
        ws = N.workspace(qkv.device, nbytes, kind="attention",
                         error_offset=int(L.btl_decode_attention_error_offset(B, Hkv)))
        N.check(
            L.btl_decode_attention(N.ptr(qkv), B, H, Hkv, D, S, N.ptr(pos), N.ptr(self.rope_cos), N.ptr(self.rope_sin),
                                   int(self.use_fused_rope), float(self.scale), N.ptr(kv_cache.key_cache),
                                   N.ptr(kv_cache.value_cache), N.ptr(out), N.ptr(ws), ws.numel(),
                                   N.stream_of(qkv.device)),
            "btl_decode_attention",
        )
        return out

    def check(self) -> None:
        """Raise RuntimeError if a call since the last check met a position
        outside [0, max_seq_len) (or any other launch on the device reported
        a timed-out wait); synchronises the device."""
        from .. import _native as N

        N.check_errors(self.device)

    def error_word(self, device=None, B: int = 32) -> int:
        """Non-zero once a position outside [0, max_seq_len) reached a call on
        the current stream."""
        from .. import _native as N

        L = N.lib()
        ws = N.workspace(self.device if device is None else device, 0, kind="attention")
        off = int(L.btl_decode_attention_error_offset(B, self.num_kv_heads))
        return int(ws[off:off + 4].view(__import__("torch").int32).item())
