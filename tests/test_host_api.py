"""Host-side API of bitnet_tt against the oracle (CPU only).

The numpy functions of ``bitnet_tt.kernels.pack`` / ``bitnet_tt.utils.quantization``
and the fused-weight builders must give the reference's bytes and values; the
reference tests' own cases are restated here (tests/test_ternary_kernel.py,
tests/test_bitlinear.py, tests/test_model.py, tests/test_ffn_fused.py,
tests/test_projection_fusion.py of bitnet-tt).
"""

import numpy as np
import pytest

from bitnet_tt import config as cfg
from bitnet_tt.kernels import pack as P
from bitnet_tt.layers.attention import _permute_halfsplit_to_adjacent, build_fused_qkv_weight
from bitnet_tt.layers.bitlinear import quantize_and_transpose_weight
from bitnet_tt.layers.ffn import build_fused_gate_up_weight
from bitnet_tt.utils import quantization as Q


def test_codes_and_bytes(orc, known):
    v = np.array(known["encode_values"]["values"], np.int8)
    assert P._encode_ternary(v).tolist() == known["encode_values"]["codes"]
    assert P._decode_ternary(np.array(known["decode_values"]["codes"], np.uint8)).tolist() == known["decode_values"]["values"]
    assert P._decode_ternary(np.array([3], np.uint8)).tolist() == [0]
    k = known["pack_single_byte"]
    assert P._pack_4_to_byte(np.array(k["codes"], np.uint8))[0] == k["byte"]
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 4, 4096).astype(np.uint8)
    assert np.array_equal(P._pack_4_to_byte(codes), orc.pack_4_to_byte(codes))
    assert np.array_equal(P._unpack_byte_to_4(P._pack_4_to_byte(codes)), codes)
    assert P.PACKED_TILE_BYTES == 256 and P.TILE_ELEMENTS == 1024


def test_faces(orc, known):
    tile = (np.arange(1024) % 100).astype(np.int8).reshape(32, 32)
    assert np.array_equal(P._tile_to_faces(tile), orc.tile_to_faces(tile))
    assert np.array_equal(P._faces_to_tile(P._tile_to_faces(tile)), tile)
    t = np.zeros((32, 32), np.int8)
    for r, c, v in known["face_ordering"]["marks"]:
        t[r, c] = v
    f = P._tile_to_faces(t)
    for idx, v in known["face_ordering"]["expect"]:
        assert f[idx] == v


@pytest.mark.parametrize("out_f,in_f", [(64, 128), (50, 100), (96, 64), (33, 65), (32, 2560)])
def test_pack_tilized_bit_exact(orc, out_f, in_f):
    rng = np.random.default_rng(out_f * 1000 + in_f)
    q = rng.choice([-1, 0, 1], size=(out_f, in_f)).astype(np.int8)
    packed, sc = P.pack_ternary_tilized(q, 0.125)
    ref, ref_sc = orc.pack_ternary_tilized(q, 0.125)
    assert np.array_equal(packed, ref)
    assert np.array_equal(sc, ref_sc)
    un = P.unpack_ternary_tilized(packed, sc, in_f, out_f)
    assert np.array_equal(un, orc.unpack_ternary_tilized(packed, sc, in_f, out_f))
    np.testing.assert_allclose(un, q.T.astype(np.float32) * 0.125)


def test_tile_counts(known):
    for in_f, out_f, tiles in known["tile_counts"]["cases"]:
        assert P.packed_tile_count(in_f, out_f) == tiles
        assert P.packed_dram_bytes(in_f, out_f) == 256 * tiles


def test_quantization_matches_oracle(orc, known):
    rng = np.random.default_rng(3)
    for shape in [(64, 128), (300, 301), (2560, 640)]:
        w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        q, s = Q.weight_quant_ternary(w)
        oq, os_ = orc.weight_quant_ternary(w)
        assert s == os_ and np.array_equal(q, oq)
        assert Q.compute_weight_scale(w) == os_
    x = rng.standard_normal((2, 16, 256)).astype(np.float32)
    q, s = Q.activation_quant_absmax(x)
    oq, os_, _, _ = orc.act_quant_absmax(x)
    assert np.array_equal(q, oq) and np.array_equal(s, os_) and s.shape == (2, 16, 1)
    k = known["act_scale_known"]
    x = np.zeros(k["shape"], np.float32)
    x[0, 0, 0] = k["x000"]
    assert np.allclose(Q.activation_quant_absmax(x)[1], k["scale"], atol=k["atol"])
    w = np.array(known["weight_sign"]["weight"], np.float32)
    q, _ = Q.weight_quant_ternary(w)
    assert q[0, 0] == 1 and q[0, 1] == -1
    assert np.all(Q.weight_quant_ternary(np.zeros((4, 8), np.float32))[0] == 0)


def test_reconstruction_bounds():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((64, 128)).astype(np.float32)
    q, s = Q.weight_quant_ternary(w)
    assert np.corrcoef(w.ravel(), (q * s).ravel())[0, 1] > 0.5
    np.testing.assert_array_equal(Q.dequantize_weight(q, s), q.astype(np.float32) * float(s))
    x = rng.standard_normal((2, 16, 256)).astype(np.float32)
    xq, sc = Q.activation_quant_absmax(x)
    step = np.max(np.abs(x), axis=-1, keepdims=True) / 127.0
    assert np.max(np.abs(x - xq / sc)) <= np.max(step) + 1e-5


def test_flat_pack_roundtrip():
    rng = np.random.default_rng(5)
    q = rng.choice([-1, 0, 1], size=(7, 13)).astype(np.int8)
    p = Q.pack_ternary_weights(q)
    assert p.size == (91 + 3) // 4
    # -1 -> 0b00, 0 -> 0b01, +1 -> 0b10, first in the top bits (quantization.py:111-138)
    assert Q.pack_ternary_weights(np.array([-1, 0, 1, 0], np.int8)).tolist() == [0b00_01_10_01]
    assert np.array_equal(Q.unpack_ternary_weights(p, q.shape), q)


def test_fused_builders(known):
    k = known["fused_gate_up_builder"]
    gate, up = np.array(k["gate"], np.float32), np.array(k["up"], np.float32)
    fused, gs, us = build_fused_gate_up_weight(gate, up)
    assert fused.shape == tuple(k["fused_shape"])
    g_t, g_s = quantize_and_transpose_weight(gate)
    u_t, u_s = quantize_and_transpose_weight(up)
    assert (gs, us) == (g_s, u_s)
    np.testing.assert_array_equal(fused[:, :2], g_t)
    np.testing.assert_array_equal(fused[:, 2:], u_t)
    # closed form: mean|gate| = 3.2/6; gate/s = [2.25,-1.5,.1875; -1.3125,.75,0]
    np.testing.assert_array_equal(g_t, np.array([[1, -1], [-1, 1], [0, 0]], np.float32))
    k = known["fused_qkv_builder"]
    q, kk, v = (np.array(k[n], np.float32) for n in ("q", "k", "v"))
    fused, qs, ks, vs = build_fused_qkv_weight(q, kk, v)
    assert fused.shape == tuple(k["fused_shape"])
    np.testing.assert_array_equal(fused[:, :2], quantize_and_transpose_weight(q)[0])
    np.testing.assert_array_equal(fused[:, 2:3], quantize_and_transpose_weight(kk)[0])
    np.testing.assert_array_equal(fused[:, 3:], quantize_and_transpose_weight(v)[0])


def test_rope_permutation(orc):
    rng = np.random.default_rng(6)
    w = rng.standard_normal((8, 3 * 16)).astype(np.float32)
    assert np.array_equal(_permute_halfsplit_to_adjacent(w, 3, 16), orc.permute_halfsplit_to_adjacent(w, 3, 16))
    p = _permute_halfsplit_to_adjacent(np.arange(16, dtype=np.float32)[None, :], 1, 16)
    assert p[0].tolist() == [0, 8, 1, 9, 2, 10, 3, 11, 4, 12, 5, 13, 6, 14, 7, 15]


def test_config_dims(known):
    k = known["bitnet_2b_dims"]
    c = cfg.get_config("2b4t")
    for name in ("hidden_size", "num_layers", "num_attention_heads", "num_key_value_heads", "intermediate_size",
                 "rms_norm_eps", "rope_theta", "head_dim"):
        assert getattr(c, name) == k[name]
    assert c.qkv_dim == 3840
    m = cfg.get_config("mini")
    assert (m.hidden_size, m.num_layers, m.num_attention_heads) == (256, 4, 4)
    with pytest.raises(ValueError):
        cfg.get_config("nope")
