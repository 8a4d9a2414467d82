"""2-bit ternary weight packing (the reference's ``packed_ternary`` tile format).

Same module, names and byte layout as ``src/bitnet_tt/kernels/pack.py`` of
bitnet-tt, so packed weights move between the two unchanged:

* codes ``-1 -> 0b10, 0 -> 0b00, +1 -> 0b01`` (``0b11`` decodes to 0),
  four per byte, first code in bits 7:6 (pack.py:31-76);
* a 32x32 tile is stored as four row-major 16x16 faces
  (f0 rows<16 cols<16, f1 rows<16 cols>=16, f2, f3; pack.py:79-98);
* the (out, in) weight is transposed to (in, out), zero-padded to 32 and cut
  into tiles in row-major tile order ``t = kt*Nt + nt`` (pack.py:101-191).

The numpy functions are the host-side load-time utilities of the reference
API (vectorised rather than looped per tile).  The ``*_device`` functions do
the same work on the GPU through libbtl.so, and :func:`repack_for_gemm`
turns the tile format into the layout the ternary GEMM streams.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

TILE_H = 32
TILE_W = 32
TILE_ELEMENTS = TILE_H * TILE_W
FACE_H = 16
FACE_W = 16
FACE_ELEMENTS = FACE_H * FACE_W
PACKED_TILE_BYTES = TILE_ELEMENTS // 4  # 256 bytes

_ENC_NEG = np.uint8(0b10)
_ENC_ZERO = np.uint8(0b00)
_ENC_POS = np.uint8(0b01)


def _encode_ternary(values: NDArray[np.int8]) -> NDArray[np.uint8]:
    """{-1, 0, +1} -> 2-bit codes {0b10, 0b00, 0b01} (pack.py:37-42)."""
    values = np.asarray(values)
    return np.where(values == 1, _ENC_POS, np.where(values == -1, _ENC_NEG, _ENC_ZERO)).astype(np.uint8)


def _decode_ternary(codes: NDArray[np.uint8]) -> NDArray[np.int8]:
    """2-bit codes -> {-1, 0, +1}; 0b11 decodes to 0 (pack.py:45-50)."""
    codes = np.asarray(codes)
    return np.where(codes == _ENC_POS, 1, np.where(codes == _ENC_NEG, -1, 0)).astype(np.int8)


def _pack_4_to_byte(codes: NDArray[np.uint8]) -> NDArray[np.uint8]:
    """Groups of four codes -> one byte, first code in the top bits (pack.py:53-63)."""
    codes = np.asarray(codes, dtype=np.uint8)
    assert codes.size % 4 == 0
    c = codes.reshape(-1, 4)
    return ((c[:, 0] << 6) | (c[:, 1] << 4) | (c[:, 2] << 2) | c[:, 3]).astype(np.uint8)


def _unpack_byte_to_4(packed: NDArray[np.uint8]) -> NDArray[np.uint8]:
    """One byte -> four codes, top bits first (pack.py:66-76)."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1, 1)
    shifts = np.array([6, 4, 2, 0], dtype=np.uint8)
    return ((packed >> shifts) & 0x03).astype(np.uint8).reshape(-1)


def _tile_to_faces(tile: NDArray) -> NDArray:
    """32x32 tile -> four concatenated row-major 16x16 faces (pack.py:79-86)."""
    tile = np.asarray(tile)
    assert tile.shape == (TILE_H, TILE_W)
    return tile.reshape(2, FACE_H, 2, FACE_W).transpose(0, 2, 1, 3).reshape(-1)


def _faces_to_tile(faces_flat: NDArray) -> NDArray:
    """Inverse of :func:`_tile_to_faces` (pack.py:89-98)."""
    faces_flat = np.asarray(faces_flat)
    assert faces_flat.size == TILE_ELEMENTS
    return faces_flat.reshape(2, 2, FACE_H, FACE_W).transpose(0, 2, 1, 3).reshape(TILE_H, TILE_W)


def _tiles_of(wt: NDArray) -> NDArray:
    """(Kp, Np) -> (Kt*Nt, 1024) in tile order t = kt*Nt + nt, face order inside."""
    kp, np_ = wt.shape
    kt, nt = kp // TILE_H, np_ // TILE_W
    return (
        wt.reshape(kt, 2, FACE_H, nt, 2, FACE_W)
        .transpose(0, 3, 1, 4, 2, 5)  # kt, nt, face-row, face-col, r, c
        .reshape(kt * nt, TILE_ELEMENTS)
    )


def pack_ternary_tilized(
    weight_quant: NDArray[np.int8], scale: float
) -> tuple[NDArray[np.uint8], NDArray[np.float32]]:
    """Quantised (out_features, in_features) int8 -> (num_tiles, 256) packed bytes
    of the transposed (in, out) matrix plus per-tile scales (pack.py:101-155)."""
    weight_quant = np.asarray(weight_quant)
    wt = weight_quant.T
    pad_h = (TILE_H - wt.shape[0] % TILE_H) % TILE_H
    pad_w = (TILE_W - wt.shape[1] % TILE_W) % TILE_W
    if pad_h or pad_w:
        wt = np.pad(wt, ((0, pad_h), (0, pad_w)), constant_values=0)
    tiles = _tiles_of(np.ascontiguousarray(wt))
    packed = _pack_4_to_byte(_encode_ternary(tiles)).reshape(-1, PACKED_TILE_BYTES)
    return packed, np.full(packed.shape[0], scale, dtype=np.float32)


def unpack_ternary_tilized(
    packed_bytes: NDArray[np.uint8],
    tile_scales: NDArray[np.float32],
    in_features: int,
    out_features: int,
) -> NDArray[np.float32]:
    """Inverse of :func:`pack_ternary_tilized`: float32 (in, out) = value * tile scale
    (pack.py:158-191)."""
    kt = (in_features + TILE_H - 1) // TILE_H
    nt = (out_features + TILE_W - 1) // TILE_W
    vals = _decode_ternary(_unpack_byte_to_4(packed_bytes)).reshape(kt, nt, 2, 2, FACE_H, FACE_W)
    wt = vals.transpose(0, 2, 4, 1, 3, 5).reshape(kt * TILE_H, nt * TILE_W).astype(np.float32)
    sc = np.asarray(tile_scales, dtype=np.float32).reshape(kt, nt)
    wt *= np.repeat(np.repeat(sc, TILE_H, axis=0), TILE_W, axis=1)
    return wt[:in_features, :out_features]


def packed_tile_count(in_features: int, out_features: int) -> int:
    """Number of 32x32 tiles (pack.py:194-198)."""
    rows_t = ((in_features + TILE_H - 1) // TILE_H) * TILE_H
    cols_t = ((out_features + TILE_W - 1) // TILE_W) * TILE_W
    return (rows_t // TILE_H) * (cols_t // TILE_W)


def packed_dram_bytes(in_features: int, out_features: int) -> int:
    """Bytes of the packed weight without the scale array (pack.py:201-203)."""
    return packed_tile_count(in_features, out_features) * PACKED_TILE_BYTES


# ------------------------------------------------------------- device ----
def pack_ternary_tilized_device(weight_quant):
    """GPU version of :func:`pack_ternary_tilized` (bytes only): a ROCm int8
    (out, in) tensor -> uint8 (num_tiles, 256) tensor, bit-identical."""
    import torch

    from .. import _native as N

    N.require_cuda(weight_quant, "weight_quant")
    if weight_quant.dtype != torch.int8 or weight_quant.dim() != 2:
        raise ValueError("weight_quant must be a 2-D int8 tensor (out_features, in_features)")
    out_f, in_f = weight_quant.shape
    packed = torch.empty((packed_tile_count(in_f, out_f), PACKED_TILE_BYTES), dtype=torch.uint8,
                         device=weight_quant.device)
    N.check(
        N.lib().btl_pack_tiles(N.ptr(weight_quant), out_f, in_f, N.ptr(packed), N.stream_of(weight_quant.device)),
        "btl_pack_tiles",
    )
    return packed


def unpack_ternary_tilized_device(packed, in_features: int, out_features: int):
    """GPU unpack of the tile format to the int8 (in, out) matrix."""
    import torch

    from .. import _native as N

    N.require_cuda(packed, "packed")
    if packed.dtype != torch.uint8 or packed.numel() != packed_dram_bytes(in_features, out_features):
        raise ValueError("packed must be uint8 with packed_dram_bytes(in, out) elements")
    w = torch.empty((in_features, out_features), dtype=torch.int8, device=packed.device)
    N.check(
        N.lib().btl_unpack_tiles(N.ptr(packed), in_features, out_features, N.ptr(w), N.stream_of(packed.device)),
        "btl_unpack_tiles",
    )
    return w


def repack_for_gemm(packed, in_features: int, out_features: int):
    """Tile format (ROCm uint8 tensor) -> the GEMM's device layout, an int32 tensor
    of shape (out/32, ceil(in/128), 256)."""
    import torch

    from .. import _native as N

    N.require_cuda(packed, "packed")
    if in_features % 32 or out_features % 32:
        raise ValueError("K/N must be multiples of 32")  # bitlinear.py:226, 276
    if packed.dtype != torch.uint8 or packed.numel() != packed_dram_bytes(in_features, out_features):
        raise ValueError("packed must be uint8 with packed_dram_bytes(in, out) elements")
    ks = (in_features + 127) // 128
    wdev = torch.empty((out_features // 32, ks, 256), dtype=torch.int32, device=packed.device)
    N.check(
        N.lib().btl_repack(N.ptr(packed), in_features, out_features, N.ptr(wdev), N.stream_of(packed.device)),
        "btl_repack",
    )
    return wdev
