"""BitLinear layer and RMSNorm on gfx950 (API of bitnet-tt's
``src/bitnet_tt/layers/bitlinear.py``).

``Linear`` keeps the reference's constructor, ``load_weights``,
``load_pretransposed_weight`` and ``__call__(x, norm_weight, norm_epsilon)``.
Its weight lives on the GPU in the GEMM's device layout (made from the
reference ``packed_ternary`` tile format), and a forward pass is one fused
launch sequence of libbtl.so: [RMSNorm ->] int8 absmax quant -> ternary GEMM
with int32 accumulation -> scale epilogue (the reference's separate
``multiply(out, weight_scale)``, bitlinear.py:351-352, is part of it).
"""

from __future__ import annotations

import numpy as np

from ..kernels.pack import pack_ternary_tilized_device, repack_for_gemm
from ..ternary_matmul import PackedTernaryWeight, ternary_matmul, ternary_matmul_into
from ..utils.quantization import weight_quant_ternary


def quantize_and_transpose_weight(weight) -> tuple[np.ndarray, float]:
    """Ternary {-1,0,+1} (in, out) float32 matrix and its absmean scale
    (bitlinear.py:104-114)."""
    weight_quant, scale = weight_quant_ternary(np.asarray(weight).astype(np.float32))
    return weight_quant.T.astype(np.float32).copy(), float(scale)


def _device(device):
    import torch

    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


def to_device_bf16(array, device):
    """numpy/torch array -> contiguous bf16 tensor on ``device``."""
    import torch

    t = torch.as_tensor(np.asarray(array, dtype=np.float32)) if not isinstance(array, torch.Tensor) else array
    return t.to(device=device, dtype=torch.bfloat16).contiguous()


def pack_for_device(weight_quant_outin, device, segment_scales=(1.0,), segment_ends=()) -> PackedTernaryWeight:
    """int8 (out, in) ternary matrix (numpy or tensor) -> device-layout weight,
    through the reference tile format (btl_pack_tiles, then btl_repack)."""
    import torch

    q = weight_quant_outin
    if not isinstance(q, torch.Tensor):
        q = torch.from_numpy(np.ascontiguousarray(np.asarray(q, dtype=np.int8)))
    q = q.to(device=device, dtype=torch.int8).contiguous()
    out_f, in_f = q.shape
    packed = pack_ternary_tilized_device(q)
    data = repack_for_gemm(packed, in_f, out_f)
    return PackedTernaryWeight(data, in_f, out_f, tuple(segment_scales), tuple(segment_ends))


class Linear:
    """BitLinear with a pre-quantised ternary weight (bitlinear.py:132-353).

    ``weight_dtype`` keeps the reference's selector; ``"packed_ternary"`` (2-bit
    weights, the only format of this backend) is the default.  The reference's
    bfp4/bfp8/bf16 storage choices are Tensix block-float formats with no
    counterpart here and are rejected.
    """

    _WEIGHT_DTYPE_MAP = {"packed_ternary": "int32 (2-bit codes, GEMM device layout)"}

    def __init__(self, in_features: int, out_features: int, device=None, compute_fidelity: str = "hifi2",
                 weight_dtype: str = "packed_ternary", check_errors: bool | None = None) -> None:
        if weight_dtype not in self._WEIGHT_DTYPE_MAP:
            raise ValueError(
                f"weight_dtype {weight_dtype!r} is a Tensix storage format; this backend stores 'packed_ternary'"
            )
        self.in_features = in_features
        self.out_features = out_features
        self.device = device
        self.weight: PackedTernaryWeight | None = None
        self.weight_scale: float = 1.0
        self._fidelity = compute_fidelity
        self._weight_dtype_name = weight_dtype
        self._use_packed_ternary = True
        self.epilogue = "none"
        # True: every call synchronises and raises RuntimeError at the call if
        # a bounded wait of its launch ran out (None: the library-wide mode,
        # bitnet_tt.ternary_matmul.set_check_after_call)
        self.check_errors = check_errors

    def _check_shape(self, out_f: int, in_f: int) -> None:
        if (out_f, in_f) != (self.out_features, self.in_features):
            raise ValueError(f"weight is ({out_f}, {in_f}), layer is ({self.out_features}, {self.in_features})")
        if in_f % 32 or out_f % 32:
            raise ValueError("K/N must be multiples of 32")  # bitlinear.py:226

    def load_weights(self, weight) -> None:
        """(out_features, in_features) latent weight -> absmean ternary ->
        packed on the device; ``weight_scale`` = the absmean scale
        (bitlinear.py:199-254).  numpy input is quantised on the host exactly
        as the reference does; a float32 device tensor is quantised by the
        gfx950 kernel (same numpy-order scale)."""
        import torch

        dev = _device(self.device)
        if isinstance(weight, torch.Tensor) and weight.is_cuda:
            q, scale = weight_quant_ternary(weight.to(torch.float32).contiguous())
        else:
            q, scale = weight_quant_ternary(np.asarray(weight).astype(np.float32))
        self._check_shape(*q.shape)
        self.weight_scale = float(scale)
        self.weight = pack_for_device(q, dev, (self.weight_scale,))

    def load_pretransposed_weight(self, weight_t, scale: float = 1.0, segment_scales=None,
                                  segment_ends=None) -> None:
        """Already-quantised (in, out) ternary weight (bitlinear.py:256-307).

        ``scale`` is the post-matmul scale.  A fused weight (Q|K|V, gate|up)
        can instead carry one scale per column segment: ``segment_scales``
        with exclusive ``segment_ends``; the epilogue applies them per column.
        """
        wt = np.asarray(weight_t)
        k, n = wt.shape
        if not np.all(np.isin(wt, (-1.0, 0.0, 1.0))):
            raise ValueError("load_pretransposed_weight expects ternary values {-1, 0, +1}")
        self._check_shape(n, k)
        q = np.ascontiguousarray(wt.T).astype(np.int8)
        if segment_scales is None:
            self.weight_scale = float(scale)
            seg_s, seg_e = (self.weight_scale,), (n,)
        else:
            seg_s = tuple(float(s) for s in segment_scales)
            seg_e = tuple(int(e) for e in segment_ends)
            self.weight_scale = 1.0 if len(seg_s) > 1 else seg_s[0]
        self.weight = pack_for_device(q, _device(self.device), seg_s, seg_e)

    def load_packed(self, packed_bytes, scale: float = 1.0) -> None:
        """Weight already in the reference tile format (``pack_ternary_tilized``
        output, (num_tiles, 256) uint8) -> device layout."""
        import torch

        dev = _device(self.device)
        packed = torch.as_tensor(np.ascontiguousarray(packed_bytes)).to(device=dev, dtype=torch.uint8).contiguous()
        data = repack_for_gemm(packed, self.in_features, self.out_features)
        self.weight_scale = float(scale)
        self.weight = PackedTernaryWeight(data, self.in_features, self.out_features, (self.weight_scale,))

    def __call__(self, x, norm_weight=None, norm_epsilon: float | None = None, residual=None, out=None):
        """``x`` bf16 [..., in_features] -> bf16 [..., out_features]
        (bitlinear.py:309-353).  ``norm_weight``/``norm_epsilon`` fuse an
        RMSNorm in front; ``residual`` adds a bf16 tensor to the result;
        ``out`` writes into an existing tensor (may be ``residual``)."""
        if self.weight is None:
            raise RuntimeError("Weights not loaded. Call load_weights() first.")
        if out is None:
            return ternary_matmul(x, self.weight, norm_weight=norm_weight, norm_epsilon=norm_epsilon,
                                  epilogue=self.epilogue, residual=residual, check_errors=self.check_errors)
        return ternary_matmul_into(x, self.weight, out, norm_weight=norm_weight, norm_epsilon=norm_epsilon,
                                   epilogue=self.epilogue, residual=residual, check_errors=self.check_errors)

    def check(self) -> None:
        """Raise RuntimeError if a bounded wait of a launch on this layer's
        device ran out since the last check (its outputs are then invalid);
        synchronises the device."""
        from ..ternary_matmul import check

        check(_device(self.device))


class RMSNorm:
    """RMSNorm ``y = bf16(gamma * bf16(x / sqrt(mean(x^2) + eps)))``
    (bitlinear.py:356-461; HF BitNetRMSNorm order), one gfx950 launch."""

    def __init__(self, hidden_size: int, device=None, eps: float = 1e-6) -> None:
        self.hidden_size = hidden_size
        self.device = device
        self.eps = eps
        self.weight = None

    def load_weights(self, weight) -> None:
        w = np.asarray(weight, dtype=np.float32).reshape(-1)
        if w.size != self.hidden_size:
            raise ValueError(f"gamma has {w.size} elements, expected {self.hidden_size}")
        self.weight = to_device_bf16(w, _device(self.device))

    def enable_sharded_fast_path(self, num_cores: int = 8) -> bool:
        """Tensix width-sharding switch of the reference (bitlinear.py:406-431);
        a workgroup per row is already the gfx950 layout, so nothing changes."""
        return False

    def __call__(self, x, memory_config=None):
        import torch

        from .. import _native as N

        if self.weight is None:
            raise RuntimeError("Weights not loaded. Call load_weights() first.")
        N.require_cuda(x, "x")
        if x.dtype != torch.bfloat16 or x.shape[-1] != self.hidden_size:
            raise ValueError("x must be bf16 [..., hidden_size]")
        k = self.hidden_size
        m = x.numel() // k
        y = torch.empty_like(x)
        N.check(
            N.lib().btl_rmsnorm(N.ptr(x), m, k, k, N.ptr(self.weight), float(self.eps), N.ptr(y),
                                N.stream_of(x.device)),
            "btl_rmsnorm",
        )
        return y
