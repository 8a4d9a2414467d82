"""Shared helpers of the GPU parity tests: seeded inputs of the BitLinear
configurations and bf16 bit-pattern transfers between numpy and torch."""

import numpy as np


def dev():
    import torch

    return torch.device("cuda:0")


def to_dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev()).view(torch.bfloat16)


def bits_of(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_dev(arr: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev())


def activations(orc, m, k, seed, outliers=True, scale=1.0):
    """bf16 bits of x ~ N(0, 1) with 1 % of the channels (fixed by the seed) x20."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32) * scale
    if outliers:
        cols = rng.choice(k, max(1, k // 100), replace=False)
        x[:, cols] *= 20.0
    return orc.f32_to_bf16(x)


def latent(out_f, in_f, seed, std=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((out_f, in_f)) * std).astype(np.float32)


def gamma(orc, n, seed, std=0.1):
    rng = np.random.default_rng(seed)
    return orc.f32_to_bf16((1.0 + std * rng.standard_normal(n)).astype(np.float32))


def ternary(k, n, seed):
    rng = np.random.default_rng(seed)
    return rng.choice([-1, 0, 1], size=(k, n)).astype(np.int8)


def xa_to_rowmajor(xa: np.ndarray, m: int, k: int) -> np.ndarray:
    """Decode the blocked activation layout (32-row blocks, 128-column
    superblocks, 16 bytes per lane) back to [m, k] int8."""
    ks = (k + 127) // 128
    mb = (m + 31) // 32
    a = xa.view(np.int8).reshape(mb, ks, 4, 2, 32, 16)  # mb, ks, q, half, row, byte
    full = a.transpose(0, 4, 1, 2, 3, 5).reshape(mb * 32, ks * 128)
    return full[:m, :k], full


def rowmajor_to_xa(q: np.ndarray) -> np.ndarray:
    """[m, k] int8 -> blocked activation bytes (inverse of xa_to_rowmajor)."""
    m, k = q.shape
    ks = (k + 127) // 128
    mb = (m + 31) // 32
    full = np.zeros((mb * 32, ks * 128), np.int8)
    full[:m, :k] = q
    return np.ascontiguousarray(full.reshape(mb, 32, ks, 4, 2, 16).transpose(0, 2, 3, 4, 1, 5)).reshape(-1).view(np.uint8)


HF_BITLINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                 "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def bitlinear_shapes(cfg):
    """(out, in) of each BitLinear of a layer, by HF module name."""
    H_, F = cfg.hidden_size, cfg.intermediate_size
    qd, kvd = cfg.num_attention_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    return {"self_attn.q_proj": (qd, H_), "self_attn.k_proj": (kvd, H_), "self_attn.v_proj": (kvd, H_),
            "self_attn.o_proj": (H_, qd), "mlp.gate_proj": (F, H_), "mlp.up_proj": (F, H_),
            "mlp.down_proj": (H_, F)}


def write_hf_snapshot(path, cfg, seed, packed=False, embed=True):
    """A small HF-style checkpoint directory (config.json + one safetensors
    file, HF key names).  Latents ~N(0, 0.02) and gains ~N(1, 0.1) stored in
    bf16; with ``packed`` every BitLinear weight is absmean-quantised and
    stored in HF's uint8 layout with a bf16 ``weight_scale`` = 1/scale.
    Returns {hf key: float32 latent or (int8 ternary, float32 scale)}."""
    import json
    import os

    import torch
    from safetensors.torch import save_file

    from bitnet_tt.utils.quantization import weight_quant_ternary
    from bitnet_tt.utils.weights import pack_hf_ternary

    rng = np.random.default_rng(seed)
    tensors, expect = {}, {}

    def bf16(a):
        return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)

    qd = cfg.num_attention_heads * cfg.head_dim
    for i in range(cfg.num_layers):
        pre = f"model.layers.{i}."
        for name, (o, n) in bitlinear_shapes(cfg).items():
            w = bf16(rng.standard_normal((o, n)) * 0.02)
            wf = w.float().numpy()
            key = pre + name + ".weight"
            if packed:
                q, s = weight_quant_ternary(wf)
                tensors[key] = torch.from_numpy(pack_hf_ternary(q))
                ws = bf16([1.0 / float(s)])
                tensors[pre + name + ".weight_scale"] = ws
                expect[key] = (q, np.float32(1.0) / ws.float().numpy()[0])
            else:
                tensors[key] = w
                expect[key] = wf
        for name, n in (("input_layernorm", cfg.hidden_size), ("post_attention_layernorm", cfg.hidden_size),
                        ("self_attn.attn_sub_norm", qd), ("mlp.ffn_sub_norm", cfg.intermediate_size)):
            g = bf16(1.0 + 0.1 * rng.standard_normal(n))
            tensors[pre + name + ".weight"] = g
            expect[pre + name + ".weight"] = g.float().numpy()
    if embed:
        tensors["model.embed_tokens.weight"] = bf16(rng.standard_normal((cfg.vocab_size, cfg.hidden_size)))
    tensors["model.norm.weight"] = bf16(np.ones(cfg.hidden_size))
    os.makedirs(path, exist_ok=True)
    save_file(tensors, os.path.join(path, "model.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({"hidden_size": cfg.hidden_size, "num_hidden_layers": cfg.num_layers,
                   "num_attention_heads": cfg.num_attention_heads, "num_key_value_heads": cfg.num_key_value_heads,
                   "intermediate_size": cfg.intermediate_size, "vocab_size": cfg.vocab_size,
                   "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta}, f)
    return expect


def reference_order_chain(orc, step, hidden_bits, attn_bits, layers=None):
    """The decode step's BitLinear chain in the reference's own CPU order: per
    BitLinear the RMSNorm as HF BitNetRMSNorm computes it in torch (fp32
    mean of squares, rsqrt, bf16 normalised value times the bf16 gain), numpy
    absmax quantisation (src/bitnet_tt/utils/quantization.py:60-91), a torch
    fp32 GEMM of the integer operands (exact), the scale to bf16, relu^2*up
    and the residual adds in bf16.  Weights are read back from the device.
    Returns (hidden bits after the chain, the last layer's qkv bits)."""
    import torch

    from bitnet_tt.utils.quantization import activation_quant_absmax

    bf = torch.bfloat16
    eps = step.eps
    F = step.config.intermediate_size

    def tb(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(bf)

    def wm(pw):
        dev_words = pw.data.cpu().numpy().view(np.uint32)
        w = orc.devlayout_decode(dev_words, pw.in_features, pw.out_features)
        srow = torch.empty(pw.out_features, dtype=torch.float32)
        lo = 0
        for sc, end in zip(pw.segment_scales, pw.segment_ends):
            srow[lo:end] = float(sc)
            lo = end
        return torch.from_numpy(w.astype(np.float32)), srow

    def rmsnorm(x, g):
        x32 = x.float()
        var = x32.pow(2).mean(-1, keepdim=True)
        return g * (x32 * torch.rsqrt(var + eps)).to(bf)

    def bitlinear(x, g, w_s):
        w, srow = w_s
        y = rmsnorm(x, g).float().numpy()
        q, scale = activation_quant_absmax(y)
        acc = torch.from_numpy(q.astype(np.float32)) @ w
        return (acc * (srow * torch.from_numpy((1.0 / scale).astype(np.float32)))).to(bf)

    h, attn, qkv = tb(hidden_bits).clone(), tb(attn_bits), None
    for lw in step.layers[: layers if layers is not None else len(step.layers)]:
        gl = lambda t: tb(bits_of(t))  # noqa: E731
        qkv = bitlinear(h, gl(lw.input_layernorm), wm(lw.qkv))
        h = (h.float() + bitlinear(attn, gl(lw.attn_sub_norm), wm(lw.o_proj)).float()).to(bf)
        gu = bitlinear(h, gl(lw.post_attention_layernorm), wm(lw.gate_up))
        g_, u_ = gu[:, :F].float(), gu[:, F:].float()
        r = (torch.relu(g_).pow(2).to(bf).float() * u_).to(bf)
        h = (h.float() + bitlinear(r, gl(lw.ffn_sub_norm), wm(lw.down)).float()).to(bf)
    return h.view(torch.int16).numpy().view(np.uint16), qkv.view(torch.int16).numpy().view(np.uint16)


def chain_agreement(orc, got_bits, ref_bits):
    """Normwise relative error, max-element error over the largest reference
    magnitude, Pearson correlation and the fraction of equal bf16 values."""
    g = orc.bf16_to_f32(got_bits).astype(np.float64)
    r = orc.bf16_to_f32(ref_bits).astype(np.float64)
    d = g - r
    return {"rel_fro": float(np.linalg.norm(d) / np.linalg.norm(r)),
            "max_rel": float(np.abs(d).max() / np.abs(r).max()),
            "pcc": float(np.corrcoef(g.ravel(), r.ravel())[0, 1]),
            "bits_equal": float((np.asarray(got_bits) == np.asarray(ref_bits)).mean())}
