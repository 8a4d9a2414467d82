"""bitnet_tt -- the BitLinear hot path of BitNet b1.58 on AMD MI355X (gfx950).

Same module layout and names as bitnet-tt's ``src/bitnet_tt`` for the parts
that make up that path:

* ``bitnet_tt.kernels.pack``        2-bit ``packed_ternary`` tile format
* ``bitnet_tt.utils.quantization``  absmean / absmax quantisers
* ``bitnet_tt.layers.bitlinear``    ``Linear`` (BitLinear), ``RMSNorm``
* ``bitnet_tt.layers.ffn``          ``FeedForward`` (gate||up, relu^2, sub-norm, down)
* ``bitnet_tt.layers.attention``    fused RMSNorm->QKV projection builders
* ``bitnet_tt.ternary_matmul``      the ``ternary_matmul`` op
* ``bitnet_tt.decode``              BitLinear chain of a batch-32 decode step

Compute runs in hand-written HIP kernels (libbtl.so, C ABI in include/btl.h).
"""

__version__ = "0.1.0"
