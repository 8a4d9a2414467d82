"""Final RMSNorm + LM head + greedy argmax of a decode step on gfx950.

The reference loads the head as the pre-transposed (hidden, vocab) matrix
(src/bitnet_tt/model/bitnet.py:139-215), runs ``norm`` then the head matmul on
the decode rows (src/bitnet_tt/inference/generator_batch32.py:768-811) and
takes ``ttnn.argmax`` over the vocabulary (:1170-1174).  Here the head stays
bf16 (the checkpoint's dtype; the reference's bfp8 is a Tensix block format)
in an MFMA operand layout made once at load time, and one launch streams it
for up to 32 rows, writing fp32 logits (optional) and the token ids.
"""

from __future__ import annotations

import numpy as np

from . import _native as N


class LMHead:
    """``norm`` + head + argmax; API pieces of bitnet.py:139-215."""

    def __init__(self, hidden_size: int, vocab_size: int, device=None, eps: float = 1e-5) -> None:
        import torch

        self.hidden_size = hidden_size
        self.vocab_size = vocab_size
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.eps = eps
        self.norm_weight = None
        self.weight = None  # device layout (uint8 bytes)

    def load_final_weights(self, norm_weight, lm_head_weight) -> None:
        """Final norm gain [hidden] and head [vocab, hidden] (numpy or tensor,
        any float dtype; stored as bf16)."""
        import torch

        H, V = self.hidden_size, self.vocab_size
        g = torch.as_tensor(np.asarray(norm_weight, dtype=np.float32)) if not isinstance(norm_weight, torch.Tensor) \
            else norm_weight
        g = g.reshape(-1).to(device=self.device, dtype=torch.bfloat16).contiguous()
        if g.numel() != H:
            raise ValueError(f"norm weight has {g.numel()} elements, expected {H}")
        w = lm_head_weight if isinstance(lm_head_weight, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(lm_head_weight, dtype=np.float32)))
        if tuple(w.shape) != (V, H):
            raise ValueError(f"head weight is {tuple(w.shape)}, expected ({V}, {H})")
        w = w.to(device=self.device, dtype=torch.bfloat16).contiguous()
        L = N.lib()
        nbytes = int(L.btl_lm_head_weight_bytes(V, H))
        if nbytes <= 0:
            raise ValueError(f"unsupported head shape vocab={V} hidden={H}")
        dev = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        N.check(L.btl_lm_head_repack(N.ptr(w), V, H, N.ptr(dev), N.stream_of(self.device)), "btl_lm_head_repack")
        self.norm_weight = g
        self.weight = dev

    def __call__(self, hidden, return_logits: bool = True, normed_out=None, logits_out=None, tokens_out=None):
        """bf16 hidden [M, hidden] (M <= 32) -> (fp32 logits [M, vocab] or None,
        int32 token ids [M]).  The ``*_out`` tensors, when given, are written
        in place (no allocation: the call can then be captured in a graph
        after one eager call on the same stream)."""
        import torch

        if self.weight is None:
            raise RuntimeError("Weights not loaded. Call load_final_weights() first.")
        N.require_cuda(hidden, "hidden")
        H, V = self.hidden_size, self.vocab_size
        if hidden.dtype != torch.bfloat16 or hidden.shape[-1] != H:
            raise ValueError("hidden must be bf16 [..., hidden_size]")
        M = hidden.numel() // H
        if M > 32:
            raise ValueError(f"{M} rows: the head launch takes up to 32")
        x = hidden.reshape(M, H)
        xn = normed_out if normed_out is not None else torch.empty((M, H), dtype=torch.bfloat16, device=hidden.device)
        logits = logits_out if logits_out is not None else (
            torch.empty((M, V), dtype=torch.float32, device=hidden.device) if return_logits else None)
        tokens = tokens_out if tokens_out is not None else torch.empty(M, dtype=torch.int32, device=hidden.device)
        L = N.lib()
        stream = N.stream_of(hidden.device)
        nbytes = int(L.btl_lm_head_workspace_bytes())
        if torch.cuda.is_current_stream_capturing() and not N.has_workspace(hidden.device, nbytes, "lm_head"):
            # a workspace made inside a capture would be re-zeroed by every replay
            raise RuntimeError("run one eager head call on this stream before capturing it in a graph")
        ws = N.workspace(hidden.device, nbytes, kind="lm_head")
        N.check(L.btl_rmsnorm(N.ptr(x), M, H, H, N.ptr(self.norm_weight), float(self.eps), N.ptr(xn), stream),
                "btl_rmsnorm")
        N.check(L.btl_lm_head(N.ptr(xn), M, H, V, N.ptr(self.weight), N.ptr(logits) if logits is not None else None,
                              N.ptr(tokens), N.ptr(ws), ws.numel(), stream), "btl_lm_head")
        return logits, tokens

    def weight_bytes(self) -> int:
        """Compulsory HBM bytes of one head call's weights (bf16 vocab x hidden)."""
        return 2 * self.vocab_size * self.hidden_size
