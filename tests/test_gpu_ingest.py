"""GPU side of checkpoint ingest: an HF snapshot (bf16 latents, or HF's
pre-packed uint8 ternary weights) -> BitLinearDecodeStep device weights.

The device codes must equal those of the reference's host quantisation
(numpy absmean, quantization.py:15-57) packed through the tested tile path,
for both checkpoint kinds, and a decode step from the loaded weights must give
the oracle chain's bits (utils/weights.py:19-246; attention.py:481-506;
ffn.py:22-34)."""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt.config import BitNet2B4TConfig, BitNetMiniConfig
from bitnet_tt.decode import BitLinearDecodeStep
from bitnet_tt.layers.bitlinear import pack_for_device
from bitnet_tt.utils.quantization import weight_quant_ternary
from bitnet_tt.utils.weights import load_bitnet_weights, load_weights_to_model
from test_gpu_layers import oracle_layer

pytestmark = pytest.mark.gpu

FUSED = {"qkv": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), "o_proj": ("self_attn.o_proj",),
         "gate_up": ("mlp.gate_proj", "mlp.up_proj"), "down": ("mlp.down_proj",)}


def expected_weight(sd, i, names):
    """Host (numpy) quantisation of the latents, packed by the tile path."""
    qs, scales, ends, total = [], [], [], 0
    for n in names:
        q, s = weight_quant_ternary(sd[f"layers.{i}.{n}.weight"])
        qs.append(q)
        scales.append(float(s))
        total += q.shape[0]
        ends.append(total)
    return pack_for_device(np.concatenate(qs), H.dev(), tuple(scales), tuple(ends))


def test_latent_snapshot_weights_and_step(tmp_path, orc):
    cfg = BitNetMiniConfig(num_layers=2)
    print("mini snapshot, bf16 latents, 2 layers", flush=True)
    H.write_hf_snapshot(str(tmp_path), cfg, seed=11)
    sd, cfg2 = load_bitnet_weights(str(tmp_path))
    step = BitLinearDecodeStep.from_state_dict(cfg2, sd, H.dev())
    assert len(step.layers) == 2
    for i, lw in enumerate(step.layers):
        for kind, names in FUSED.items():
            got, exp = getattr(lw, kind), expected_weight(sd, i, names)
            assert torch.equal(got.data, exp.data), f"layer {i} {kind} codes"
            assert got.segment_scales == exp.segment_scales and got.segment_ends == exp.segment_ends
        g = sd[f"layers.{i}.mlp.ffn_sub_norm.weight"]
        assert np.array_equal(lw.ffn_sub_norm.float().cpu().numpy(), g)
    step.alloc_buffers(seed=12)
    hid, attn = H.bits_of(step.hidden), H.bits_of(step.attn_out)
    step.step()
    torch.cuda.synchronize()
    for i in range(2):
        hid, qkv = oracle_layer(orc, step, i, hid, attn)
    assert np.array_equal(H.bits_of(step.hidden), hid)
    assert np.array_equal(H.bits_of(step.qkv_out), qkv)


def test_packed_snapshot_matches_latent(tmp_path):
    """HF's pre-packed checkpoint of the same latents loads to the same device
    codes; its scales are 1/weight_scale (weight_scale stored in bf16)."""
    cfg = BitNetMiniConfig(num_layers=2)
    print("mini snapshot, latent vs HF pre-packed", flush=True)
    H.write_hf_snapshot(str(tmp_path / "lat"), cfg, seed=13)
    expect = H.write_hf_snapshot(str(tmp_path / "pk"), cfg, seed=13, packed=True)
    a = BitLinearDecodeStep.from_state_dict(cfg, load_bitnet_weights(str(tmp_path / "lat"))[0], H.dev())
    sd_p, _ = load_bitnet_weights(str(tmp_path / "pk"))
    b = BitLinearDecodeStep(cfg, H.dev())
    b.layers = [None, None]
    load_weights_to_model(b, sd_p)
    for i in range(2):
        for kind, names in FUSED.items():
            wa, wb = getattr(a.layers[i], kind), getattr(b.layers[i], kind)
            assert torch.equal(wa.data, wb.data), f"layer {i} {kind} codes"
            exp = tuple(float(expect[f"model.layers.{i}.{n}.weight"][1]) for n in names)
            assert wb.segment_scales == exp
            for sa, sb in zip(wa.segment_scales, wb.segment_scales):
                assert abs(sa - sb) <= 4e-3 * sa  # bf16 rounding of 1/scale
    b.alloc_buffers(seed=14)
    b.step()
    torch.cuda.synchronize()
    assert torch.isfinite(b.hidden.float()).all()


def test_2b_layer_from_snapshot(tmp_path):
    """One layer at the 2B shapes (2560 / 3840 / 2x6912 / 6912) through the
    safetensors path: device codes equal the host quantisation."""
    cfg = BitNet2B4TConfig(num_layers=1)
    print("2B shapes, one-layer snapshot", flush=True)
    H.write_hf_snapshot(str(tmp_path), cfg, seed=15, embed=False)
    sd, cfg2 = load_bitnet_weights(str(tmp_path))
    step = BitLinearDecodeStep.from_state_dict(cfg2, sd, H.dev())
    for kind, names in FUSED.items():
        assert torch.equal(getattr(step.layers[0], kind).data, expected_weight(sd, 0, names).data), kind
    assert step.ternary_split is not None and abs(sum(step.ternary_split) - 1.0) < 1e-9
