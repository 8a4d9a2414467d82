"""The ternary matmul op: drop-in for ``ttnn.experimental.ternary_matmul``.

bitnet-tt calls ``ttnn.experimental.ternary_matmul(x, W, use_packed_ternary=True,
norm_weight=..., norm_epsilon=...)`` from ``Linear.__call__``
(src/bitnet_tt/layers/bitlinear.py:336-341) and from the decode loop's fused
RMSNorm->QKV (src/bitnet_tt/inference/generator_batch32.py:721-727).  Here the
same call runs one launch sequence of libbtl.so (``btl_bitlinear_fused``):

    [RMSNorm(norm_weight, norm_epsilon) ->] per-token int8 absmax quant ->
    int8 x ternary GEMM (int32, exact) -> epilogue -> bf16

The epilogue applies the activation dequantisation ``a/127`` and the weight
scale(s) in one multiply (Linear's separate ``multiply(out, weight_scale)``,
bitlinear.py:351-352, folds into it), optionally ``relu(g)^2 * u`` for the
gate||up weight (ffn.py:164-170) and a residual add.  There is no other
backend: inputs must live on a ROCm device and libbtl.so must be built.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

from . import _native as N

EPILOGUES = {"none": N.EPI_SCALE, "scale": N.EPI_SCALE, "relu2_mul": N.EPI_RELU2_MUL}

# Check-after-call mode: every call synchronises its device and raises
# RuntimeError at the call when a bounded wait of a fused decode launch ran
# out, as the reference's op raises at its call (bitlinear.py:329-330).  Off by
# default (a synchronisation per call; not allowed inside a graph capture);
# on with set_check_after_call(True) or BTL_CHECK_AFTER_CALL=1, or per call.
_check_after_call = os.environ.get("BTL_CHECK_AFTER_CALL", "0") not in ("", "0")


def set_check_after_call(enabled: bool) -> None:
    """Turn the check-after-call mode on or off for every later call."""
    global _check_after_call
    _check_after_call = bool(enabled)


def check_after_call_enabled() -> bool:
    return _check_after_call


@dataclass
class PackedTernaryWeight:
    """A ternary weight in the GEMM's device layout.

    ``data``: int32 tensor (N/32, ceil(K/128), 256) on the device, made by
    :func:`bitnet_tt.kernels.pack.repack_for_gemm` from the reference tile
    format.  ``segment_scales``/``segment_ends`` are the per-projection weight
    scales of a fused weight (Q|K|V, gate|up) with their exclusive column ends.
    """

    data: "object"
    in_features: int
    out_features: int
    segment_scales: tuple = (1.0,)
    segment_ends: tuple = field(default_factory=tuple)

    def __post_init__(self):
        if not self.segment_ends:
            self.segment_ends = (self.out_features,)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.data.numel() * 4


def ternary_matmul(
    input_tensor_a,
    input_tensor_b,
    *,
    use_packed_ternary: bool = True,
    norm_weight=None,
    norm_epsilon: float | None = None,
    compute_kernel_config=None,
    weight_scale=None,
    epilogue: str = "none",
    residual=None,
    splitk: int = 0,
    acc_out=None,
    xq_out=None,
    check_errors: bool | None = None,
):
    """``y = epilogue(quant(norm(a)) @ W)`` in bf16.

    input_tensor_a: bf16 [..., M, K] on a ROCm device.
    input_tensor_b: :class:`PackedTernaryWeight` (or its ``data`` tensor).
    norm_weight / norm_epsilon: RMSNorm gain [K] (any shape with K elements)
        and epsilon, fused in front of the quantiser when given.
    weight_scale: None -> the weight's own segment scales; a float or a
        sequence of per-segment floats overrides them.
    epilogue: "none" (scale), or "relu2_mul" for a gate||up weight (output has
        N/2 columns).
    residual: optional bf16 [..., M, N] added to the output (may be the output
        buffer's owner tensor; the result is returned as a new tensor unless
        ``residual`` is also the destination, see :func:`ternary_matmul_into`).
    acc_out / xq_out: optional int32 [M, N] / int8 [M, K] tensors receiving the
        exact accumulators and the quantised activations (parity checks).
    compute_kernel_config: accepted for signature compatibility; the gfx950
        path has a single (exact) accumulation mode.
    check_errors: True synchronises after the launch and raises RuntimeError
        if a bounded wait of a fused decode launch ran out (None: the mode set
        by :func:`set_check_after_call`).
    """
    import torch

    if not use_packed_ternary:
        raise ValueError("only the packed ternary path exists on this backend")
    w = input_tensor_b
    if not isinstance(w, PackedTernaryWeight):
        if w.dim() != 3 or w.shape[-1] != 256:
            raise ValueError("input_tensor_b must be a PackedTernaryWeight or an int32 (N/32, KS, 256) tensor")
        w = PackedTernaryWeight(w, input_tensor_a.shape[-1], w.shape[0] * 32)
    x = input_tensor_a
    N.require_cuda(x, "input_tensor_a")
    if x.dtype != torch.bfloat16:
        raise ValueError("input_tensor_a must be bfloat16")
    K = x.shape[-1]
    if K != w.in_features:
        raise ValueError(f"input has K={K}, weight expects {w.in_features}")
    Nf = w.out_features
    epi = EPILOGUES.get(epilogue)
    if epi is None:
        raise ValueError(f"unknown epilogue {epilogue!r}")
    M = x.numel() // K
    n_out = Nf // 2 if epi == N.EPI_RELU2_MUL else Nf
    out = torch.empty(x.shape[:-1] + (n_out,), dtype=torch.bfloat16, device=x.device)
    ternary_matmul_into(
        x, w, out, norm_weight=norm_weight, norm_epsilon=norm_epsilon, weight_scale=weight_scale,
        epilogue=epilogue, residual=residual, splitk=splitk, acc_out=acc_out, xq_out=xq_out,
        check_errors=check_errors,
    )
    return out


def check(device=None) -> None:
    """Raise RuntimeError if a bounded wait of a fused decode launch on
    ``device`` ran out since the last check (the launch then returned invalid
    bf16 values).  Synchronises the device; call it at synchronisation points.
    The reference surfaces op failures as RuntimeError
    (src/bitnet_tt/layers/bitlinear.py:329-330)."""
    N.check_errors(device)


def ternary_matmul_into(
    x,
    w: PackedTernaryWeight,
    out,
    *,
    norm_weight=None,
    norm_epsilon: float | None = None,
    weight_scale=None,
    epilogue: str = "none",
    residual=None,
    splitk: int = 0,
    acc_out=None,
    xq_out=None,
    check_errors: bool | None = None,
):
    """Same as :func:`ternary_matmul` writing into ``out`` (no allocation once
    the per-stream workspace exists, so the call can be captured in a graph).
    ``residual`` may be ``out`` itself for an in-place residual add."""
    import torch

    K = w.in_features
    Nf = w.out_features
    M = x.numel() // K
    epi = EPILOGUES[epilogue]
    for t, name in ((x, "x"), (out, "out"), (residual, "residual"), (acc_out, "acc_out"), (xq_out, "xq_out")):
        N.require_cuda(t, name)
    if out.dtype != torch.bfloat16:
        raise ValueError("out must be bfloat16")
    n_out = Nf // 2 if epi == N.EPI_RELU2_MUL else Nf
    if out.numel() != M * n_out:
        raise ValueError(f"out has {out.numel()} elements, expected {M}x{n_out}")
    if residual is not None and (residual.numel() != M * n_out or residual.dtype != torch.bfloat16):
        raise ValueError("residual must be bf16 with the output's shape")
    if acc_out is not None and (acc_out.dtype != torch.int32 or acc_out.numel() != M * Nf):
        raise ValueError("acc_out must be int32 [M, N]")
    if xq_out is not None and (xq_out.dtype != torch.int8 or xq_out.numel() != M * K):
        raise ValueError("xq_out must be int8 [M, K]")
    gamma = None
    eps = 0.0
    if norm_weight is not None:
        if norm_epsilon is None:
            raise ValueError("norm_weight needs norm_epsilon")
        gamma = norm_weight
        N.require_cuda(gamma, "norm_weight")
        if gamma.dtype != torch.bfloat16 or gamma.numel() != K:
            raise ValueError("norm_weight must be bf16 with K elements")
        eps = float(norm_epsilon)
    if weight_scale is None:
        scales = tuple(w.segment_scales)
        ends = tuple(w.segment_ends)
    elif isinstance(weight_scale, (int, float)):
        scales, ends = (float(weight_scale),), (Nf,)
    else:
        scales = tuple(float(s) for s in weight_scale)
        ends = tuple(w.segment_ends)
        if len(scales) != len(ends):
            raise ValueError("weight_scale needs one value per weight segment")
    sc, en, nseg = N.segments_arrays(scales, ends)
    L = N.lib()
    dev = x.device
    ws_bytes = int(L.btl_fused_workspace_bytes(M, K, Nf, epi, splitk))
    ws = N.workspace(dev, ws_bytes, error_offset=int(L.btl_fused_error_offset()))
    N.check(
        L.btl_bitlinear_fused(
            N.ptr(x), M, K, K, N.ptr(gamma), eps, N.ptr(w.data), Nf, sc, en, nseg, epi, N.ptr(residual),
            N.ptr(out), N.ptr(acc_out), N.ptr(xq_out), N.ptr(ws), ws.numel(), int(splitk), N.stream_of(dev),
        ),
        "btl_bitlinear_fused",
    )
    if _check_after_call if check_errors is None else check_errors:
        N.check_errors(dev)
    return out
