"""GPU parity of the decode attention (attention.py:1040-1262) against the
oracle: the new cache rows (rotated k within one bf16 ulp -- the kernel rotates
in fp32, the oracle in fp64 --, v exact), untouched rows elsewhere, and the
output within 2^-7 relative plus 1e-3 of the row's largest value (bf16
operands and output, fp32 accumulation, the exp of the hardware)."""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N
from bitnet_tt.layers.attention import DecodeAttention

pytestmark = pytest.mark.gpu


def run(orc, B, Hq, Hkv, S, pos, adjacent, seed, scale=None):
    rng = np.random.default_rng(seed)
    D = 128
    qkv = orc.f32_to_bf16(rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float32))
    kc = orc.f32_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    vc = orc.f32_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    att = DecodeAttention(Hq, Hkv, D, S, H.dev(), rope_theta=500000.0, use_fused_rope=adjacent, scale=scale)
    cache = att.new_cache(B)
    cache.key_cache.copy_(H.to_dev_bf16(kc).view(B, Hkv, S, D))
    cache.value_cache.copy_(H.to_dev_bf16(vc).view(B, Hkv, S, D))
    out = att(H.to_dev_bf16(qkv), cache, torch.tensor(pos, dtype=torch.int32, device=H.dev()))
    torch.cuda.synchronize()
    cos, sin = orc.rope_tables(D, S, 500000.0)
    ref, kc2, vc2 = orc.decode_attention(qkv, kc, vc, np.asarray(pos), Hq, Hkv, cos, sin, adjacent, att.scale)
    return att, cache, H.bits_of(out).astype(np.uint16), ref, kc, vc, kc2, vc2


def check(orc, got_bits, ref, cache, kc2, vc2):
    got = orc.bf16_to_f32(got_bits.view(np.uint16)).astype(np.float64)
    tol = 2.0 ** -7 * np.abs(ref) + 1e-3 * np.abs(ref).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - ref) <= tol), np.max(np.abs(got - ref) - tol)
    kgot = H.bits_of(cache.key_cache).reshape(kc2.shape).astype(np.int32)
    assert np.all(np.abs(kgot - kc2.astype(np.int32)) <= 1)  # 1 bf16 ulp (same sign here)
    assert np.array_equal(H.bits_of(cache.value_cache).reshape(vc2.shape), vc2)


@pytest.mark.parametrize("adjacent", [False, True])
@pytest.mark.parametrize("B,Hq,Hkv,S,pos", [(3, 4, 1, 256, [0, 130, 255]), (2, 4, 2, 128, [5, 127]),
                                           (4, 2, 2, 384, [383, 0, 129, 256]), (1, 1, 1, 64, [63])])
def test_small_shapes(orc, B, Hq, Hkv, S, pos, adjacent):
    print(f"attention B={B} H={Hq} Hkv={Hkv} S={S} adjacent={adjacent}", flush=True)
    att, cache, out, ref, kc, vc, kc2, vc2 = run(orc, B, Hq, Hkv, S, pos, adjacent, seed=B * 31 + S)
    check(orc, out, ref, cache, kc2, vc2)


@pytest.mark.parametrize("full", [True, False])
def test_2b_shape(orc, full):
    """32 users, 20 query / 5 key-value heads, context 512 (4 chunks per
    user and head group): every user at the last position, or at spread
    positions."""
    B, Hq, Hkv, S = 32, 20, 5, 512
    pos = [511] * B if full else list(np.random.default_rng(9).integers(0, S, size=B))
    print(f"attention 2B shape full={full}", flush=True)
    att, cache, out, ref, kc, vc, kc2, vc2 = run(orc, B, Hq, Hkv, S, pos, True, seed=77 + full)
    check(orc, out, ref, cache, kc2, vc2)


def test_graph_replay_advances_position(orc):
    """A captured call reads the position from the device: replays after an
    increment of pos write the next cache rows and match the eager results."""
    B, Hq, Hkv, S, D = 4, 4, 1, 256, 128
    rng = np.random.default_rng(5)
    att = DecodeAttention(Hq, Hkv, D, S, H.dev())
    cache = att.new_cache(B)
    qkv = H.to_dev_bf16(orc.f32_to_bf16(rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float32)))
    pos = torch.zeros(B, dtype=torch.int32, device=H.dev())
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=H.dev())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    eager = []
    with torch.cuda.stream(s):
        for t in range(3):
            pos.fill_(t)
            att(qkv, cache, pos, out=out)
            eager.append(H.bits_of(out).copy())
    torch.cuda.synchronize()
    k_eager = H.bits_of(cache.key_cache).copy()
    cache.key_cache.zero_()
    cache.value_cache.zero_()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        att(qkv, cache, pos, out=out)
    for t in range(3):
        with torch.cuda.stream(s):
            pos.fill_(t)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(H.bits_of(out), eager[t]), f"replay {t}"
    assert np.array_equal(H.bits_of(cache.key_cache), k_eager)
    with torch.cuda.stream(s):
        assert att.error_word(B=B) == 0


def test_position_out_of_range_is_flagged(orc):
    B, Hq, Hkv, S, D = 2, 4, 1, 128, 128
    att = DecodeAttention(Hq, Hkv, D, S, H.dev())
    cache = att.new_cache(B)
    qkv = torch.ones((B, (Hq + 2 * Hkv) * D), dtype=torch.bfloat16, device=H.dev())
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = att(qkv, cache, torch.tensor([3, S], dtype=torch.int32, device=H.dev()))
        torch.cuda.synchronize()
        assert att.error_word(B=B) != 0
    # check() surfaces the sticky word as RuntimeError and resets the workspace
    with pytest.raises(RuntimeError, match="error word"):
        att.check()
    with torch.cuda.stream(s):
        assert att.error_word(B=B) == 0
    att.check()
    assert torch.all(out[1] == 0) and torch.isfinite(out[0].float()).all()
    assert not cache.key_cache[1].any()  # nothing written for the bad row


def test_full_layer_chain(orc):
    """One mini layer through step_full: QKV (bit-exact), attention (oracle
    tolerance), then o_proj, gate||up and down from the kernel's attention
    output (bit-exact), and the cache rows at the position."""
    from bitnet_tt.config import BitNetMiniConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    cfg = BitNetMiniConfig(num_layers=1, num_attention_heads=4, num_key_value_heads=1, hidden_size=512,
                           intermediate_size=512)
    print("mini layer with attention", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=81, batch=8).alloc_buffers(seed=82)
    step.alloc_attention(max_seq_len=256, pos=200)
    kc0 = H.bits_of(step.kv[0].key_cache).reshape(8, 1, 256, 128).copy()
    vc0 = H.bits_of(step.kv[0].value_cache).reshape(8, 1, 256, 128).copy()
    hid = H.bits_of(step.hidden).copy()
    step.step_full()
    torch.cuda.synchronize()
    w = step.layers[0]

    def wkn(pw):
        return orc.devlayout_decode(pw.data.cpu().numpy().view(np.uint32), pw.in_features, pw.out_features)

    qkv = orc.bitlinear(hid, wkn(w.qkv), list(w.qkv.segment_scales), list(w.qkv.segment_ends),
                        gamma_bf16=H.bits_of(w.input_layernorm), norm_eps=step.eps)["out"]
    assert np.array_equal(H.bits_of(step.qkv_out), qkv)
    cos, sin = orc.rope_tables(128, 256, cfg.rope_theta)
    ref, kc2, vc2 = orc.decode_attention(qkv, kc0, vc0, np.full(8, 200), 4, 1, cos, sin, False, step.attention.scale)
    attn = H.bits_of(step.attn_out)
    check(orc, attn, ref, step.kv[0], kc2, vc2)
    h = orc.bitlinear(attn, wkn(w.o_proj), list(w.o_proj.segment_scales), gamma_bf16=H.bits_of(w.attn_sub_norm),
                      norm_eps=step.eps, residual_bf16=hid)["out"]
    r = orc.gate_up_relu2(h, wkn(w.gate_up), w.gate_up.segment_scales[0], w.gate_up.segment_scales[1],
                          gamma_bf16=H.bits_of(w.post_attention_layernorm), norm_eps=step.eps)
    h = orc.bitlinear(r["h"], wkn(w.down), list(w.down.segment_scales), gamma_bf16=H.bits_of(w.ffn_sub_norm),
                      norm_eps=step.eps, residual_bf16=h)["out"]
    assert np.array_equal(H.bits_of(step.hidden), h)


def _full_state(step):
    return (step.hidden.clone(), [(kv.key_cache.clone(), kv.value_cache.clone()) for kv in step.kv])


def _restore(step, state):
    hid, caches = state
    step.hidden.copy_(hid)
    for kv, (k, v) in zip(step.kv, caches):
        kv.key_cache.copy_(k)
        kv.value_cache.copy_(v)
    torch.cuda.synchronize()


def _outputs(step):
    torch.cuda.synchronize()
    return {"hidden": H.bits_of(step.hidden).copy(), "qkv": H.bits_of(step.qkv_out).copy(),
            "attn": H.bits_of(step.attn_out).copy(), "ffn_h": H.bits_of(step.ffn_h).copy(),
            "k": [H.bits_of(kv.key_cache).copy() for kv in step.kv],
            "v": [H.bits_of(kv.value_cache).copy() for kv in step.kv]}


def _compare(a, b, what):
    for key in ("hidden", "qkv", "attn", "ffn_h"):
        bad = int((a[key] != b[key]).sum())
        assert bad == 0, f"{what}: {key} differs in {bad} of {a[key].size} values"
    for i, (ka, kb, va, vb) in enumerate(zip(a["k"], b["k"], a["v"], b["v"])):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"{what}: layer {i} cache differs"


@pytest.mark.parametrize("layers,batch,pos", [(2, 8, 200), (3, 5, None)])
def test_persistent_full_step_matches_step_full_mini(orc, layers, batch, pos):
    """The one-launch step with the decode attention (btl_decode_step_full)
    against step_full (QKV, attention and the other BitLinears as separate
    launches, each pinned to the oracle elsewhere): hidden, the last layer's
    qkv / attention / FFN rows and every layer's cache, bit for bit; spread
    positions per user in the second case."""
    from bitnet_tt.config import BitNetMiniConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    cfg = BitNetMiniConfig(num_layers=layers, num_attention_heads=4, num_key_value_heads=1, hidden_size=512,
                           intermediate_size=512)
    print(f"persistent full step mini layers={layers} batch={batch} pos={pos}", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=91 + layers, batch=batch).alloc_buffers(seed=92)
    step.alloc_attention(max_seq_len=256, pos=pos if pos is not None else 0)
    if pos is None:
        step.pos.copy_(torch.from_numpy(np.random.default_rng(3).integers(0, 256, batch).astype(np.int32)))
    state = _full_state(step)
    step.step_full()
    step.check()
    ref = _outputs(step)
    _restore(step, state)
    step.step_persistent_full()
    step.check()
    _compare(_outputs(step), ref, "persistent full step")


def test_persistent_full_step_attention_on_qkv_units(orc):
    """More attention items than GEMM units without QKV work (26 users x 8
    key-value heads = 208 items; 64 QKV units of 224), so that units 16-63
    run a QKV unit and then an attention item in each layer: the one-launch
    step against step_full, bit for bit."""
    from bitnet_tt.config import BitNetMiniConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    cfg = BitNetMiniConfig(num_layers=2, num_attention_heads=16, num_key_value_heads=8, hidden_size=2048,
                           intermediate_size=512)
    print("persistent full step, attention on QKV units: batch 26, 8 kv heads", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=97, batch=26).alloc_buffers(seed=98)
    step.alloc_attention(max_seq_len=128, pos=0)
    step.pos.copy_(torch.from_numpy(np.random.default_rng(5).integers(0, 128, 26).astype(np.int32)))
    state = _full_state(step)
    step.step_full()
    step.check()
    ref = _outputs(step)
    _restore(step, state)
    step.step_persistent_full()
    step.check()
    _compare(_outputs(step), ref, "persistent full step, attention on QKV units")


def test_persistent_full_step_2b_layer_against_oracle(orc):
    """One 2B layer (20 query / 5 key-value heads, batch 32, every user at
    position 511 of a 512 context) through the one-launch step with the
    attention, against the oracle: QKV bit-exact, the attention within the
    oracle tolerance (with the new cache rows), and o_proj, gate||up and down
    from the kernel's attention output bit-exact."""
    from bitnet_tt.config import BitNet2B4TConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    cfg = BitNet2B4TConfig()
    print("persistent full step, one 2B layer against the oracle", flush=True)
    step = BitLinearDecodeStep.random_init(cfg, H.dev(), seed=99, num_layers=1).alloc_buffers(seed=100)
    step.alloc_attention(max_seq_len=512)
    B, Hq, Hkv, S = 32, cfg.num_attention_heads, cfg.num_key_value_heads, 512
    kc0 = H.bits_of(step.kv[0].key_cache).reshape(B, Hkv, S, 128).copy()
    vc0 = H.bits_of(step.kv[0].value_cache).reshape(B, Hkv, S, 128).copy()
    hid = H.bits_of(step.hidden).copy()
    pos = step.pos.cpu().numpy().astype(np.int64)
    step.step_persistent_full()
    step.check()
    w = step.layers[0]

    def wkn(pw):
        return orc.devlayout_decode(pw.data.cpu().numpy().view(np.uint32), pw.in_features, pw.out_features)

    qkv = orc.bitlinear(hid, wkn(w.qkv), list(w.qkv.segment_scales), list(w.qkv.segment_ends),
                        gamma_bf16=H.bits_of(w.input_layernorm), norm_eps=step.eps)["out"]
    assert np.array_equal(H.bits_of(step.qkv_out), qkv)
    cos, sin = orc.rope_tables(128, S, cfg.rope_theta)
    ref, kc2, vc2 = orc.decode_attention(qkv, kc0, vc0, pos, Hq, Hkv, cos, sin, False, step.attention.scale)
    attn = H.bits_of(step.attn_out)
    check(orc, attn, ref, step.kv[0], kc2, vc2)
    h = orc.bitlinear(attn, wkn(w.o_proj), list(w.o_proj.segment_scales), gamma_bf16=H.bits_of(w.attn_sub_norm),
                      norm_eps=step.eps, residual_bf16=hid)["out"]
    r = orc.gate_up_relu2(h, wkn(w.gate_up), w.gate_up.segment_scales[0], w.gate_up.segment_scales[1],
                          gamma_bf16=H.bits_of(w.post_attention_layernorm), norm_eps=step.eps)
    assert np.array_equal(H.bits_of(step.ffn_h), r["h"])
    h = orc.bitlinear(r["h"], wkn(w.down), list(w.down.segment_scales), gamma_bf16=H.bits_of(w.ffn_sub_norm),
                      norm_eps=step.eps, residual_bf16=h)["out"]
    assert np.array_equal(H.bits_of(step.hidden), h)


def test_persistent_full_step_matches_step_full_2b(orc):
    """The 2B model (30 layers, 20 query / 5 key-value heads, batch 32, every
    user at position 511 of a 512 context), the one-launch step with
    attention against step_full, bit for bit; then graph replays of the
    one-launch step from the same state give the same bits again (three
    compared in full, 100 more on the hidden state), and once more with every
    GEMM unit forced onto the sentinel check's re-read path."""
    from bitnet_tt.config import BitNet2B4TConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    print("persistent full step 2B", flush=True)
    step = BitLinearDecodeStep.random_init(BitNet2B4TConfig(), H.dev(), seed=95).alloc_buffers(seed=96)
    step.alloc_attention(max_seq_len=512)
    state = _full_state(step)
    step.step_full()
    step.check()
    ref = _outputs(step)
    _restore(step, state)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step.step_persistent_full()
    s.synchronize()
    step.check()
    _compare(_outputs(step), ref, "persistent full step")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step.step_persistent_full()
    for rep in range(3):
        _restore(step, state)
        g.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1024, device=H.dev()).sum().item()  # eager work between replays
        _compare(_outputs(step), ref, f"graph replay {rep}")
    step.check()
    # 100 more replays, the hidden state compared on the device: the hand-offs
    # of the attention units (QKV words in, attention words out) every layer
    ref_h = torch.from_numpy(ref["hidden"].view(np.int16)).to(H.dev())
    bad = []
    for rep in range(100):
        _restore(step, state)
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(step.hidden.view(torch.int16), ref_h):
            bad.append(rep)
    step.check()
    assert not bad, f"replays {bad[:10]} differ"
    # Every GEMM unit on the sentinel check's rare path (it waits for its
    # operand pieces, reads them and its weights again and redoes its MFMAs),
    # forced through the step workspace's test word: the attention instance's
    # own register allocation of that path gives the same bits.
    key = next(k for k in N._workspaces if k[0] == "step" and k[2] == s.cuda_stream)
    ws = N._workspaces[key]
    off = int(N.lib().btl_decode_step_error_offset()) + 64
    ws[off:off + 4] = torch.tensor([1, 0, 0, 0], dtype=torch.uint8, device=ws.device)
    try:
        _restore(step, state)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            step.step_persistent_full()
        s.synchronize()
        step.check()
        _compare(_outputs(step), ref, "persistent full step, every unit on the re-read path")
    finally:
        ws[off:off + 4] = 0
        torch.cuda.synchronize()
