"""BitLinear portion of a batch-32 BitNet decode step.

Per layer the reference decode loop (src/bitnet_tt/inference/
generator_batch32.py:713-761) issues four ternary-matmul launches:

    qkv    = ternary_matmul(hidden, W_qkv, norm_weight=input_layernorm)   :721-727
    hidden = hidden + o_proj(attn_sub_norm(attention(qkv)))               :739-749
    hidden = hidden + down(ffn_sub_norm(relu(gate)^2 * up))               :752-756
             with gate||up = BitLinear(post_attention_layernorm(hidden))

Here the remaining norms and residual adds ride along with the BitLinears:
attn_sub_norm and post_attention_layernorm become RMSNorm prologues, relu^2*up
the gate||up epilogue, ffn_sub_norm the down prologue, and both residual adds
epilogues.  Two launch structures compute the same bits:

* ``step_persistent``: the whole step's BitLinears as one ``btl_decode_step``
  launch (one workgroup per CU; 32 row workgroups run the elementwise stages
  of the token rows, the others one GEMM unit of each BitLinear, with weights
  loaded one BitLinear ahead).  The fastest on MI355X (0.70 ms for the 2B
  model's 30 layers); it needs the attention width equal to hidden and the
  shape limits of include/btl.h.
* ``step_per_call`` (the default ``step``, which takes any shape the fused
  op takes): one ``btl_bitlinear_fused`` launch per BitLinear (120 per
  30-layer step, 1.0 ms).

``step`` takes the attention output as an input buffer (the BitLinear
portion alone).  After ``alloc_attention`` the step can also run whole:
``step_full`` puts the decode attention (RoPE, KV-cache update, SDPA over the
cached context, one ``btl_decode_attention`` launch per layer) between each
layer's QKV and o_proj (150 launches per 30-layer step).

All buffers are allocated once, so :meth:`BitLinearDecodeStep.step` is
allocation-free and can be captured in a HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native as N
from .config import BitNetConfig
from .ternary_matmul import PackedTernaryWeight, ternary_matmul_into


@dataclass
class LayerWeights:
    qkv: PackedTernaryWeight
    o_proj: PackedTernaryWeight
    gate_up: PackedTernaryWeight
    down: PackedTernaryWeight
    input_layernorm: object  # bf16 [hidden]
    attn_sub_norm: object  # bf16 [q_dim]
    post_attention_layernorm: object  # bf16 [hidden]
    ffn_sub_norm: object  # bf16 [ffn]


def _quant_pack_device(latents_outin, device, segment_ends=None):
    """float32 latent rows (out, in) on the device -> ternary -> device layout.

    ``latents_outin`` is a list of (out_i, in) float32 device tensors that are
    quantised separately (one absmean scale each) and concatenated along out."""
    import torch

    from .layers.bitlinear import pack_for_device
    from .utils.quantization import weight_quant_ternary

    qs, scales, ends = [], [], []
    total = 0
    for w in latents_outin:
        q, s = weight_quant_ternary(w)
        qs.append(q)
        scales.append(s)
        total += w.shape[0]
        ends.append(total)
    q = qs[0] if len(qs) == 1 else torch.cat(qs, dim=0)
    return pack_for_device(q, device, tuple(scales), tuple(ends)), q


def ternary_split(q) -> tuple[float, float, float]:
    """Fractions of +1 / 0 / -1 in an int8 ternary tensor."""
    n = q.numel()
    pos = int((q == 1).sum().item())
    neg = int((q == -1).sum().item())
    return pos / n, (n - pos - neg) / n, neg / n


class BitLinearDecodeStep:
    """All BitLinear weights of a BitNet model plus the decode-step chain."""

    def __init__(self, config: BitNetConfig, device, batch: int = 32):
        self.config = config
        self.device = device
        self.batch = batch
        self.layers: list[LayerWeights] = []
        self.eps = config.rms_norm_eps
        self.ternary_split = None

    # -- weights ---------------------------------------------------------
    @classmethod
    def random_init(cls, config: BitNetConfig, device, seed: int = 0, batch: int = 32, latent_std: float = 0.02,
                    gamma_std: float = 0.1, num_layers: int | None = None):
        """Random-init weights of the architecture (the reference's demo init,
        examples/demo.py:199-268, with latents ~N(0, latent_std) and RMSNorm
        gains ~N(1, gamma_std)), generated and quantised on the device."""
        import torch

        self = cls(config, device, batch)
        c = config
        H, F, qd, kvd = c.hidden_size, c.intermediate_size, c.num_attention_heads * c.head_dim, c.num_kv_heads * c.head_dim
        gen = torch.Generator(device=device)
        counts = torch.zeros(3, dtype=torch.float64)
        n_total = 0

        def latent(rows, cols, tag):
            gen.manual_seed(seed * 1000003 + tag)
            return torch.randn((rows, cols), generator=gen, device=device, dtype=torch.float32) * latent_std

        def gamma(n, tag):
            gen.manual_seed(seed * 1000003 + tag)
            g = 1.0 + gamma_std * torch.randn((n,), generator=gen, device=device, dtype=torch.float32)
            return g.to(torch.bfloat16).contiguous()

        L = c.num_layers if num_layers is None else num_layers
        for i in range(L):
            t = 100 * (i + 1)
            qkv, q1 = _quant_pack_device([latent(qd, H, t + 1), latent(kvd, H, t + 2), latent(kvd, H, t + 3)], device)
            o, q2 = _quant_pack_device([latent(H, qd, t + 4)], device)
            gu, q3 = _quant_pack_device([latent(F, H, t + 5), latent(F, H, t + 6)], device)
            dn, q4 = _quant_pack_device([latent(H, F, t + 7)], device)
            for q in (q1, q2, q3, q4):
                counts[0] += float((q == 1).sum().item())
                counts[2] += float((q == -1).sum().item())
                n_total += q.numel()
            del q1, q2, q3, q4
            self.layers.append(
                LayerWeights(qkv, o, gu, dn, gamma(H, t + 8), gamma(qd, t + 9), gamma(H, t + 10), gamma(F, t + 11))
            )
        pos, neg = counts[0].item() / n_total, counts[2].item() / n_total
        self.ternary_split = (pos, 1.0 - pos - neg, neg)
        return self

    @classmethod
    def from_state_dict(cls, config: BitNetConfig, state_dict: dict, device, batch: int = 32,
                        num_layers: int | None = None):
        """Weights from a state dict under the reference's keys (what
        ``utils.weights.load_bitnet_weights`` returns): float latents are
        quantised on the device by the absmean rule, ``TernaryWeight`` entries
        (HF's pre-packed checkpoint) are taken as they are."""
        from .utils.weights import get_layer_weights

        self = cls(config, device, batch)
        L = config.num_layers if num_layers is None else num_layers
        self.layers = [None] * L
        self._counts = [0, 0, 0]
        for i in range(L):
            lw = get_layer_weights(state_dict, i)
            if not lw:
                raise KeyError(f"layer {i}: the state dict holds no 'layers.{i}.*' entries")
            self.load_layer_weights(i, lw)
        return self

    def load_layer_weights(self, layer_idx: int, weights: dict) -> None:
        """One layer from its state-dict entries (keys without the
        ``layers.<i>.`` prefix, utils/weights.py:158-181): q|k|v fused with
        three scales (attention.py:481-506), o_proj, gate|up fused with two
        scales (ffn.py:22-34), down, and the four RMSNorm gains."""
        import torch

        from .layers.bitlinear import pack_for_device, to_device_bf16
        from .utils.quantization import weight_quant_ternary
        from .utils.weights import TernaryWeight

        c = self.config
        H, F = c.hidden_size, c.intermediate_size
        qd, kvd = c.num_attention_heads * c.head_dim, c.num_kv_heads * c.head_dim

        def entry(name):
            key = name + ".weight"
            if key not in weights:
                raise KeyError(f"layer {layer_idx}: missing {key!r}")
            return weights[key]

        def ternary(name, rows, cols):
            w = entry(name)
            if isinstance(w, TernaryWeight):
                if w.q.shape[1] != cols or w.q.shape[0] < rows:
                    raise ValueError(f"layer {layer_idx} {name}: ternary weight {w.q.shape}, expected ({rows}, {cols})")
                q = torch.from_numpy(np.ascontiguousarray(w.q[:rows])).to(device=self.device)
                return q, float(w.scale)
            a = np.asarray(w, dtype=np.float32)
            if a.shape != (rows, cols):
                raise ValueError(f"layer {layer_idx} {name}: weight {a.shape}, expected ({rows}, {cols})")
            return weight_quant_ternary(torch.from_numpy(a).to(device=self.device))

        def fused(parts):
            qs, scales, ends, total = [], [], [], 0
            for name, rows, cols in parts:
                q, sc = ternary(name, rows, cols)
                qs.append(q)
                scales.append(float(sc))
                total += rows
                ends.append(total)
            q = qs[0] if len(qs) == 1 else torch.cat(qs, dim=0)
            if getattr(self, "_counts", None) is not None:
                self._counts[0] += int((q == 1).sum().item())
                self._counts[1] += int((q == -1).sum().item())
                self._counts[2] += q.numel()
                pos, neg = self._counts[0] / self._counts[2], self._counts[1] / self._counts[2]
                self.ternary_split = (pos, 1.0 - pos - neg, neg)
            return pack_for_device(q, self.device, tuple(scales), tuple(ends))

        def gamma(name, n):
            g = np.asarray(entry(name), dtype=np.float32).reshape(-1)
            if g.size != n:
                raise ValueError(f"layer {layer_idx} {name}: {g.size} gains, expected {n}")
            return to_device_bf16(g, self.device)

        lw = LayerWeights(
            fused([("self_attn.q_proj", qd, H), ("self_attn.k_proj", kvd, H), ("self_attn.v_proj", kvd, H)]),
            fused([("self_attn.o_proj", H, qd)]),
            fused([("mlp.gate_proj", F, H), ("mlp.up_proj", F, H)]),
            fused([("mlp.down_proj", H, F)]),
            gamma("input_layernorm", H),
            gamma("self_attn.attn_sub_norm", qd),
            gamma("post_attention_layernorm", H),
            gamma("mlp.ffn_sub_norm", F),
        )
        while len(self.layers) <= layer_idx:
            self.layers.append(None)
        self.layers[layer_idx] = lw
        self._st = None

    # -- buffers -----------------------------------------------------------
    def alloc_buffers(self, seed: int = 1, outliers: bool = True):
        """hidden [B, H], attention output stand-in [B, q_dim], qkv [B, qkv_dim],
        FFN intermediate [B, F]; hidden and the attention buffer ~N(0, 1), with
        1 % of the channels (drawn from the seed) scaled by 20 for every token
        when ``outliers``."""
        import torch

        c = self.config
        qd = c.num_attention_heads * c.head_dim
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        B = self.batch

        def acts(k):
            x = torch.randn((B, k), generator=gen, device=self.device)
            if outliers:
                cols = torch.randperm(k, generator=gen, device=self.device)[: max(1, k // 100)]
                x[:, cols] *= 20.0
            return x.to(torch.bfloat16)

        self.hidden0 = acts(c.hidden_size)
        self.hidden = self.hidden0.clone()
        self.attn_out = acts(qd)
        self.qkv_out = torch.empty((B, c.qkv_dim), dtype=torch.bfloat16, device=self.device)
        self.ffn_h = torch.empty((B, c.intermediate_size), dtype=torch.bfloat16, device=self.device)
        return self

    def reset_hidden(self):
        self.hidden.copy_(self.hidden0)

    def alloc_attention(self, max_seq_len: int = 512, pos: int | None = None, seed: int = 3,
                        use_fused_rope: bool = False):
        """Decode attention for ``step_full``: one KV cache per layer
        [batch, kv_heads, max_seq_len, head_dim] bf16 holding an earlier
        context ~N(0, 1), every user at position ``pos`` (default: the last,
        so each step attends over the whole context).  The step's Q/K weights
        are unpermuted, so RoPE pairs (i, i + D/2) unless ``use_fused_rope``."""
        import torch

        from .layers.attention import DecodeAttention

        c = self.config
        self.attention = DecodeAttention(c.num_attention_heads, c.num_kv_heads, c.head_dim, max_seq_len, self.device,
                                         rope_theta=c.rope_theta, use_fused_rope=use_fused_rope)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        self.kv = []
        for _ in self.layers:
            kv = self.attention.new_cache(self.batch)
            kv.key_cache.normal_(generator=gen)
            kv.value_cache.normal_(generator=gen)
            self.kv.append(kv)
        self.pos = torch.full((self.batch,), max_seq_len - 1 if pos is None else pos, dtype=torch.int32,
                              device=self.device)
        return self

    def layer_full(self, i: int):
        """Layer i with the decode attention between QKV and o_proj."""
        w = self.layers[i]
        eps = self.eps
        ternary_matmul_into(self.hidden, w.qkv, self.qkv_out, norm_weight=w.input_layernorm, norm_epsilon=eps)
        self.attention(self.qkv_out, self.kv[i], self.pos, out=self.attn_out)
        ternary_matmul_into(self.attn_out, w.o_proj, self.hidden, norm_weight=w.attn_sub_norm, norm_epsilon=eps,
                            residual=self.hidden)
        ternary_matmul_into(self.hidden, w.gate_up, self.ffn_h, norm_weight=w.post_attention_layernorm,
                            norm_epsilon=eps, epilogue="relu2_mul")
        ternary_matmul_into(self.ffn_h, w.down, self.hidden, norm_weight=w.ffn_sub_norm, norm_epsilon=eps,
                            residual=self.hidden)

    def step_full(self):
        for i in range(len(self.layers)):
            self.layer_full(i)
        return self.hidden

    # -- the step ----------------------------------------------------------
    def layer(self, i: int, hidden, attn_out, qkv_out, ffn_h):
        """One layer's four BitLinear launch sequences, in place on ``hidden``."""
        w = self.layers[i]
        eps = self.eps
        ternary_matmul_into(hidden, w.qkv, qkv_out, norm_weight=w.input_layernorm, norm_epsilon=eps)
        ternary_matmul_into(attn_out, w.o_proj, hidden, norm_weight=w.attn_sub_norm, norm_epsilon=eps,
                            residual=hidden)
        ternary_matmul_into(hidden, w.gate_up, ffn_h, norm_weight=w.post_attention_layernorm, norm_epsilon=eps,
                            epilogue="relu2_mul")
        ternary_matmul_into(ffn_h, w.down, hidden, norm_weight=w.ffn_sub_norm, norm_epsilon=eps, residual=hidden)

    def step_per_call(self):
        for i in range(len(self.layers)):
            self.layer(i, self.hidden, self.attn_out, self.qkv_out, self.ffn_h)
        return self.hidden

    def check(self) -> None:
        """Raise RuntimeError if a bounded wait in any launch of this
        device's steps (fused BitLinears, the persistent step, decode attention)
        ran out since the last check; synchronises the device."""
        N.check_errors(self.device)

    # -- one launch for the whole step ----------------------------------------
    def _step_table(self):
        """btl_layer_weight_t[L][4] (qkv, o_proj, gate_up, down with the gain of
        the RMSNorm in front of each), kept alive with the step."""
        if getattr(self, "_st", None) is None:
            n = len(self.layers)
            arr = (N.LayerWeight * (4 * n))()
            for i, w in enumerate(self.layers):
                arr[4 * i + 0] = N.layer_weight(w.qkv, w.input_layernorm)
                arr[4 * i + 1] = N.layer_weight(w.o_proj, w.attn_sub_norm)
                arr[4 * i + 2] = N.layer_weight(w.gate_up, w.post_attention_layernorm)
                arr[4 * i + 3] = N.layer_weight(w.down, w.ffn_sub_norm)
            self._st = arr
        return self._st

    def _step_workspace(self, attention: bool):
        """This stream's workspace of the one-launch step, prepared for the
        weight table (and, with ``attention``, for the KV-cache table) by
        synchronous copies: the first call on a stream must come before a
        graph capture."""
        import ctypes

        import torch

        c = self.config
        B = self.batch
        H, F, qd = c.hidden_size, c.intermediate_size, c.num_attention_heads * c.head_dim
        if qd != H:
            raise ValueError(f"btl_decode_step needs the attention width ({qd}) equal to hidden ({H})")
        nl = len(self.layers)
        L = N.lib()
        table = self._step_table()
        dev = self.hidden.device
        nbytes = int(L.btl_decode_step_workspace_bytes(B, H, F, c.qkv_dim, nl))
        capturing = torch.cuda.is_current_stream_capturing()
        if capturing and not N.has_workspace(dev, nbytes, "step"):
            raise RuntimeError("run one eager decode step on this stream before capturing it in a graph")
        ws = N.workspace(dev, nbytes, kind="step", error_offset=int(L.btl_decode_step_error_offset()))
        caches = None
        if attention:
            if getattr(self, "kv", None) is None:
                raise RuntimeError("step_persistent_full needs alloc_attention() first")
            caches = tuple((kv.key_cache.data_ptr(), kv.value_cache.data_ptr()) for kv in self.kv)
        ready = getattr(self, "_ws_caches", {})
        self._ws_caches = ready
        if N.workspace_prepared_for(ws) is not table or (attention and ready.get(ws.data_ptr()) != caches):
            if capturing:
                raise RuntimeError("run one eager decode step on this stream before capturing it in a graph")
            torch.cuda.current_stream(dev).synchronize()  # earlier launches on this workspace are done

            def prepare():
                N.check(L.btl_decode_step_prepare(B, H, F, c.qkv_dim, nl, table, N.ptr(ws), ws.numel()),
                        "btl_decode_step_prepare")
                N.set_workspace_prepared_for(ws, table)
                cached = ready.get(ws.data_ptr())
                if cached is not None:
                    kp = (ctypes.c_void_p * nl)(*[k for k, _ in cached])
                    vp = (ctypes.c_void_p * nl)(*[v for _, v in cached])
                    N.check(L.btl_decode_step_attention_prepare(B, H, F, c.qkv_dim, nl, kp, vp, N.ptr(ws),
                                                                ws.numel()),
                            "btl_decode_step_attention_prepare")

            if attention:
                ready[ws.data_ptr()] = caches
            prepare()
            N.set_workspace_reset(ws, prepare)
        return ws

    def step_persistent(self):
        """The whole step's BitLinears as one btl_decode_step launch (every
        layer's QKV, o_proj, gate||up and down; o_proj reads the attention
        output buffer).  Bit-identical to step_per_call.  The first call on a
        stream prepares that stream's workspace (a synchronous copy of the
        weight table), so it must happen before a graph capture."""
        c = self.config
        B = self.batch
        H, F = c.hidden_size, c.intermediate_size
        nl = len(self.layers)
        for t, name in ((self.hidden, "hidden"), (self.attn_out, "attn_out"), (self.qkv_out, "qkv_out"),
                        (self.ffn_h, "ffn_h")):
            N.require_cuda(t, name)
        ws = self._step_workspace(attention=False)
        L = N.lib()
        dev = self.hidden.device
        N.check(
            L.btl_decode_step(B, H, F, c.qkv_dim, nl, float(self.eps), N.ptr(self.attn_out), N.ptr(self.hidden),
                              N.ptr(self.qkv_out), N.ptr(self.ffn_h), N.ptr(ws), ws.numel(), N.stream_of(dev)),
            "btl_decode_step",
        )
        return self.hidden

    def step_persistent_full(self):
        """The whole decode step, attention included, as one
        btl_decode_step_full launch: per layer QKV, the decode attention (RoPE,
        KV-cache update at ``pos``, SDPA over the cached context), o_proj,
        gate||up and down (generator_batch32.py:713-761).  Needs
        alloc_attention(); bit-identical to step_full.  The first call on a
        stream (and the first after the caches move) prepares the workspace
        synchronously, so it must happen before a graph capture."""
        c = self.config
        B = self.batch
        H, F = c.hidden_size, c.intermediate_size
        nl = len(self.layers)
        for t, name in ((self.hidden, "hidden"), (self.attn_out, "attn_out"), (self.qkv_out, "qkv_out"),
                        (self.ffn_h, "ffn_h")):
            N.require_cuda(t, name)
        ws = self._step_workspace(attention=True)
        att = self.attention
        L = N.lib()
        dev = self.hidden.device
        N.check(
            L.btl_decode_step_full(B, H, F, c.qkv_dim, nl, float(self.eps), att.num_kv_heads, att.max_seq_len,
                                   N.ptr(self.pos), N.ptr(att.rope_cos), N.ptr(att.rope_sin),
                                   int(att.use_fused_rope), float(att.scale), N.ptr(self.hidden),
                                   N.ptr(self.qkv_out), N.ptr(self.attn_out), N.ptr(self.ffn_h), N.ptr(ws),
                                   ws.numel(), N.stream_of(dev)),
            "btl_decode_step_full",
        )
        return self.hidden

    def step_floor(self):
        """btl_decode_step_floor on this stream's step workspace: the persistent
        step's launch structure (waits and hand-off stores) with no
        arithmetic, whose time is the latency floor of the step's chain of
        dependent hand-offs.  Changes no tensor of the step."""
        c = self.config
        B, H, F = self.batch, c.hidden_size, c.intermediate_size
        nl = len(self.layers)
        L = N.lib()
        dev = self.hidden.device
        nbytes = int(L.btl_decode_step_workspace_bytes(B, H, F, c.qkv_dim, nl))
        import torch

        if torch.cuda.is_current_stream_capturing() and not N.has_workspace(dev, nbytes, "step"):
            raise RuntimeError("run one eager decode step on this stream before capturing it in a graph")
        ws = N.workspace(dev, nbytes, kind="step", error_offset=int(L.btl_decode_step_error_offset()))
        N.check(L.btl_decode_step_floor(B, H, F, c.qkv_dim, nl, N.ptr(ws), ws.numel(), N.stream_of(dev)),
                "btl_decode_step_floor")

    def step(self):
        return self.step_per_call()

    # -- accounting ----------------------------------------------------------
    def algorithmic_bytes(self) -> dict:
        """Compulsory HBM bytes of one step's BitLinear launches: packed
        weights, bf16 inputs and outputs, RMSNorm gains, scales (fp32 per
        token and per weight segment), residual reads."""
        c = self.config
        B, H, F = self.batch, c.hidden_size, c.intermediate_size
        qd = c.num_attention_heads * c.head_dim
        per = {}
        per["qkv"] = H * c.qkv_dim // 4 + 2 * B * H + 2 * B * c.qkv_dim + 2 * H + 4 * 3 + 4 * B
        per["o_proj"] = qd * H // 4 + 2 * B * qd + 2 * B * H * 2 + 2 * qd + 4 + 4 * B
        per["gate_up"] = H * 2 * F // 4 + 2 * B * H + 2 * B * F + 2 * H + 4 * 2 + 4 * B
        per["down"] = F * H // 4 + 2 * B * F + 2 * B * H * 2 + 2 * F + 4 + 4 * B
        per["layer"] = sum(per.values())
        per["step"] = per["layer"] * len(self.layers)
        per["weights_step"] = (H * c.qkv_dim + qd * H + H * 2 * F + F * H) // 4 * len(self.layers)
        return per
