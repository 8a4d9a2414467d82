"""Rotary position tables (API of bitnet-tt's ``src/bitnet_tt/utils/rope.py``).

Frequencies are computed in float32 exactly as the reference does
(utils/rope.py:7-23): ``freq_i = 1 / theta ** (2i / dim)``, angle = position x
freq_i, cos/sin in float32.
"""

from __future__ import annotations

import numpy as np


def precompute_freqs_cis(dim: int, max_seq_len: int, theta: float = 10000.0):
    """(cos, sin), each [1, 1, max_seq_len, dim] float32 in the interleaved
    format [f0, f0, f1, f1, ...] of adjacent-pair RoPE (utils/rope.py:7-23)."""
    freqs = 1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    positions = np.arange(max_seq_len, dtype=np.float32)
    emb = np.repeat(np.outer(positions, freqs), 2, axis=-1)
    cos = np.cos(emb).astype(np.float32).reshape(1, 1, max_seq_len, dim)
    sin = np.sin(emb).astype(np.float32).reshape(1, 1, max_seq_len, dim)
    return cos, sin


def rope_tables(dim: int, max_seq_len: int, theta: float = 10000.0):
    """(cos, sin), each [max_seq_len, dim/2] float32: one value per position and
    frequency (the same numbers as precompute_freqs_cis, not repeated); the
    decode-attention kernel reads these."""
    cos, sin = precompute_freqs_cis(dim, max_seq_len, theta)
    return np.ascontiguousarray(cos[0, 0, :, 0::2]), np.ascontiguousarray(sin[0, 0, :, 0::2])
