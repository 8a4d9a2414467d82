"""GPU parity of the persistent decode-layer launch (btl_decode_layer).

One launch covers a layer's o_proj, gate||up (relu^2*up), down and the next
layer's fused RMSNorm->QKV (generator_batch32.py:718-761).  It must give the
same bits as the per-BitLinear launches (btl_bitlinear_fused, themselves
pinned to the oracle) and as the oracle directly: hidden state, FFN
intermediate and QKV output, for full and partial batches, the last layer
(no QKV), repeated launches (the per-workgroup launch counters) and graph
replays.
"""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N
from bitnet_tt.config import BitNet2B4TConfig, BitNetMiniConfig
from bitnet_tt.decode import BitLinearDecodeStep
from test_gpu_layers import oracle_layer

pytestmark = pytest.mark.gpu


def both_paths(step):
    """(per-call, layer-kernel) results of one step from the same start."""
    outs = []
    for run in (step.step_per_call, step.step_layers):
        step.reset_hidden()
        step.qkv_out.zero_()
        step.ffn_h.zero_()
        run()
        torch.cuda.synchronize()
        outs.append((H.bits_of(step.hidden), H.bits_of(step.qkv_out), H.bits_of(step.ffn_h)))
    return outs


@pytest.mark.parametrize("batch", [32, 17, 5, 1])
def test_mini_layer_kernel_matches_per_call(batch):
    cfg = BitNetMiniConfig(num_layers=3)
    print(f"mini, 3 layers, batch {batch}", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=21, batch=batch).alloc_buffers(seed=22)
    ref, got = both_paths(step)
    for name, a, b in zip(("hidden", "qkv_out", "ffn_h"), ref, got):
        assert np.array_equal(a, b), f"{name} differs (batch {batch})"
    assert step.layer_error_word() == 0


def test_2b_layer_kernel_matches_per_call():
    cfg = BitNet2B4TConfig()
    print("2B shapes, 3 layers, batch 32", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=31, num_layers=3).alloc_buffers(seed=32)
    ref, got = both_paths(step)
    for name, a, b in zip(("hidden", "qkv_out", "ffn_h"), ref, got):
        assert np.array_equal(a, b), f"{name} differs"
    assert step.layer_error_word() == 0


def test_2b_layer_launch_against_oracle(orc):
    """Layer 0's o_proj/gate_up/down and layer 1's QKV in one launch, against
    the oracle chain."""
    cfg = BitNet2B4TConfig()
    print("2B shapes, one layer launch vs oracle", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=41, num_layers=2).alloc_buffers(seed=42)
    hid0, attn = H.bits_of(step.hidden), H.bits_of(step.attn_out)
    step.decode_layer(0, step.hidden, step.attn_out, step.qkv_out, step.ffn_h)
    torch.cuda.synchronize()
    ref_h, _ = oracle_layer(orc, step, 0, hid0, attn)  # its qkv is layer 0's, not computed here
    assert np.array_equal(H.bits_of(step.hidden), ref_h)
    w1 = step.layers[1]

    def wkn(pw):
        return orc.devlayout_decode(pw.data.cpu().numpy().view(np.uint32), pw.in_features, pw.out_features)

    ref_qkv = orc.bitlinear(ref_h, wkn(w1.qkv), list(w1.qkv.segment_scales), list(w1.qkv.segment_ends),
                            gamma_bf16=H.bits_of(w1.input_layernorm), norm_eps=step.eps)["out"]
    assert np.array_equal(H.bits_of(step.qkv_out), ref_qkv)
    assert step.layer_error_word() == 0


def test_last_layer_leaves_qkv_untouched():
    cfg = BitNetMiniConfig(num_layers=1)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=51).alloc_buffers(seed=52)
    step.qkv_out.fill_(1.5)
    step.decode_layer(0, step.hidden, step.attn_out, step.qkv_out, step.ffn_h)
    torch.cuda.synchronize()
    assert bool((step.qkv_out == 1.5).all())
    assert torch.isfinite(step.hidden.float()).all()


def test_repeated_launches_and_graph_replays():
    """Launch counters advance per launch: 12 eager steps, then graph replays
    with eager work in between, all give the first step's bits."""
    cfg = BitNet2B4TConfig()
    print("2B shapes, 2 layers: 12 eager steps + 4 graph replays", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=61, num_layers=2).alloc_buffers(seed=62)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step.reset_hidden()
        step.step_layers()
        torch.cuda.synchronize()
        first = H.bits_of(step.hidden)
        for _ in range(11):
            step.reset_hidden()
            step.step_layers()
        torch.cuda.synchronize()
        assert np.array_equal(H.bits_of(step.hidden), first)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step.step_layers()
    for rep in range(4):
        with torch.cuda.stream(s):
            step.reset_hidden()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(H.bits_of(step.hidden), first), f"replay {rep} differs"
        _ = torch.ones(1024, device=H.dev()).sum().item()
    with torch.cuda.stream(s):
        assert step.layer_error_word() == 0


def test_capture_without_warm_up_is_refused():
    cfg = BitNetMiniConfig(num_layers=1)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=71).alloc_buffers(seed=72)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="eager decode step"):
        with torch.cuda.graph(g, stream=s):
            step.decode_layer(0, step.hidden, step.attn_out, step.qkv_out, step.ffn_h)
    torch.cuda.synchronize()
    assert N.lib().btl_version() == 101
