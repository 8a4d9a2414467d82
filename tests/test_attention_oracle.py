"""CPU pins of the decode-attention restatement (attention.py:1040-1262,
utils/rope.py:7-23) against library routines and closed forms."""

import numpy as np
import pytest
import torch

from bitnet_tt.utils.rope import precompute_freqs_cis, rope_tables


def test_rope_tables_are_the_reference_frequencies(orc):
    cos, sin = precompute_freqs_cis(128, 64, 500000.0)
    c2, s2 = rope_tables(128, 64, 500000.0)
    assert np.array_equal(c2, cos[0, 0, :, 0::2]) and np.array_equal(c2, cos[0, 0, :, 1::2])
    oc, os_ = orc.rope_tables(128, 64, 500000.0)
    assert np.array_equal(oc, c2) and np.array_equal(os_, s2)
    assert np.all(c2[0] == 1.0) and np.all(s2[0] == 0.0)  # position 0: no rotation


def test_halfsplit_rope_matches_transformers(orc):
    """rotate_half form against transformers' apply_rotary_pos_emb (float64)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    rng = np.random.default_rng(1)
    D, P = 128, 37
    q = rng.standard_normal((3, D))
    k = rng.standard_normal((3, D))
    c, s = orc.rope_tables(D, P + 1, 500000.0)
    c64, s64 = c[P].astype(np.float64), s[P].astype(np.float64)
    cos_full = torch.from_numpy(np.concatenate([c64, c64]))[None, None]
    sin_full = torch.from_numpy(np.concatenate([s64, s64]))[None, None]
    qe, ke = apply_rotary_pos_emb(torch.from_numpy(q)[None], torch.from_numpy(k)[None], cos_full, sin_full)
    assert np.allclose(orc.rope_rotate(q, c64, s64, adjacent=False), qe[0].numpy(), rtol=0, atol=1e-12)
    assert np.allclose(orc.rope_rotate(k, c64, s64, adjacent=False), ke[0].numpy(), rtol=0, atol=1e-12)


def test_adjacent_rope_is_permuted_halfsplit(orc):
    """Adjacent-pair RoPE on the permuted head (attention.py:462-478) equals the
    permuted half-split RoPE."""
    rng = np.random.default_rng(2)
    D = 128
    x = rng.standard_normal((4, D))
    c, s = orc.rope_tables(D, 100, 500000.0)
    c, s = c[99].astype(np.float64), s[99].astype(np.float64)
    perm = np.empty(D, dtype=np.intp)
    perm[0::2] = np.arange(D // 2)
    perm[1::2] = np.arange(D // 2) + D // 2
    assert np.allclose(orc.rope_rotate(x[:, perm], c, s, True), orc.rope_rotate(x, c, s, False)[:, perm], atol=1e-12)


@pytest.mark.parametrize("adjacent", [False, True])
def test_rope_relative_position_invariant(orc, adjacent):
    """<R(p) q, R(p') k> depends only on p - p' (rotations); a wrong sign or
    pairing breaks it."""
    rng = np.random.default_rng(3)
    D = 128
    q, k = rng.standard_normal(D), rng.standard_normal(D)
    ang = np.outer(np.arange(64), 1.0 / (500000.0 ** (np.arange(0, D, 2) / D)))
    c, s = np.cos(ang), np.sin(ang)
    dots = lambda p1, p2: orc.rope_rotate(q, c[p1], s[p1], adjacent) @ orc.rope_rotate(k, c[p2], s[p2], adjacent)
    assert np.isclose(dots(10, 3), dots(30, 23), atol=1e-9)
    assert np.isclose(dots(5, 5), q @ k, atol=1e-9)


def test_attention_restatement_matches_torch_sdpa(orc):
    """GQA decode attention against torch's scaled_dot_product_attention
    (float64), with the cache rows at the new positions replaced."""
    rng = np.random.default_rng(4)
    B, H, Hkv, D, S = 3, 8, 2, 128, 40
    pos = np.array([0, 17, 39])
    qkv = orc.f32_to_bf16(rng.standard_normal((B, (H + 2 * Hkv) * D)).astype(np.float32))
    kc = orc.f32_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    vc = orc.f32_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    cos, sin = orc.rope_tables(D, S, 500000.0)
    scale = 1.0 / np.sqrt(D)
    out, kc2, vc2 = orc.decode_attention(qkv, kc, vc, pos, H, Hkv, cos, sin, False, scale)
    for b in range(B):
        p = pos[b]
        q = orc.bf16_to_f32(qkv[b, :H * D]).astype(np.float64).reshape(H, D)
        qr = orc.bf16_to_f32(orc.f32_to_bf16(orc.rope_rotate(q, cos[p].astype(np.float64), sin[p].astype(np.float64),
                                                             False).astype(np.float32))).astype(np.float64)
        K = torch.from_numpy(orc.bf16_to_f32(kc2[b, :, :p + 1]).astype(np.float64)).repeat_interleave(H // Hkv, 0)
        V = torch.from_numpy(orc.bf16_to_f32(vc2[b, :, :p + 1]).astype(np.float64)).repeat_interleave(H // Hkv, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(qr)[:, None], K, V, scale=scale)
        assert np.allclose(out[b].reshape(H, D), ref[:, 0].numpy(), atol=1e-12)
        assert np.array_equal(vc2[b, :, p], qkv[b, (H + Hkv) * D:].reshape(Hkv, D))
    assert np.array_equal(np.delete(kc2[0], 0, axis=1), np.delete(kc[0], 0, axis=1))  # other rows untouched
