"""CPU oracle for the BitLinear hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy wrappers over ``liboracle.so`` (``btl_oracle.c``), the plain-C
restatement of bitnet-tt's quantisation, packing and BitLinear arithmetic, plus
the composite BitLinear / fused-QKV / FFN-block semantics built from those
pieces.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product package never does.

Reference semantics restated here (paths relative to the bitnet-tt root):

* ``src/bitnet_tt/kernels/pack.py:31-203`` -- codes, byte packing, faces, tiles;
* ``src/bitnet_tt/utils/quantization.py:15-91`` -- absmean weight quant,
  per-token absmax int8 activation quant;
* ``src/bitnet_tt/layers/bitlinear.py:309-353`` -- Linear forward (matmul then
  weight-scale multiply); ``bitlinear.py:433-461`` RMSNorm;
* ``src/bitnet_tt/layers/ffn.py:129-183`` -- gate||up, relu(g)^2*u, ffn_sub_norm,
  down; ``ffn.py:22-34`` and ``layers/attention.py:462-506`` -- fused builders;
* ``src/bitnet_tt/inference/generator_batch32.py:713-761`` -- per-layer order of
  the decode step (fused RMSNorm->QKV, o_proj, residual, norm, FFN, residual);
  ``:768-811`` and ``:1170-1174`` -- final norm, LM head and greedy argmax
  (float64 matmul, a library routine, with the fp32 rounding bound; the first
  index wins ties, as numpy's and torch's argmax do).

Which check pins each function is listed in ``btl_oracle.c``'s header.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# BTL_ORACLE_LIBRARY names another build of the oracle (the host-sanitizer
# build of tests/host_asan.sh).
_LIB_PATH = os.environ.get("BTL_ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle.so")
_lib = None

ACT_EPS = 1e-5  # quantization.py:63
WEIGHT_EPS = 1e-5  # quantization.py:15


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        F = ctypes.c_float
        sig = {
            "orc_f32_to_bf16": ([P, I64, P], None),
            "orc_bf16_to_f32": ([P, I64, P], None),
            "orc_encode_ternary": ([P, I64, P], None),
            "orc_decode_ternary": ([P, I64, P], None),
            "orc_pack_4_to_byte": ([P, I64, P], None),
            "orc_unpack_byte_to_4": ([P, I64, P], None),
            "orc_tile_to_faces": ([P, P], None),
            "orc_faces_to_tile": ([P, P], None),
            "orc_packed_tile_count": ([I64, I64], I64),
            "orc_packed_dram_bytes": ([I64, I64], I64),
            "orc_pack_ternary_tilized": ([P, I64, I64, P], None),
            "orc_unpack_ternary_tilized": ([P, I64, I64, P], None),
            "orc_sum_f32_numpy": ([P, I64], F),
            "orc_compute_weight_scale": ([P, I64, F], F),
            "orc_weight_quant_ternary": ([P, I64, F, P], F),
            "orc_act_quant_absmax": ([P, I64, I64, F, P, P, P, P], None),
            "orc_rms_inv": ([P, I64, F, ctypes.c_int], F),
            "orc_rmsnorm_bf16": ([P, P, I64, I64, F, ctypes.c_int, P], None),
            "orc_gemm_i8t": ([P, P, I64, I64, I64, P], None),
            "orc_scale_bf16": ([P, I64, I64, P, P, P, ctypes.c_int, P], None),
            "orc_relu2_mul_bf16": ([P, P, I64, P], None),
            "orc_add_bf16": ([P, P, I64, P], None),
            "orc_devlayout_encode": ([P, I64, I64, P], None),
            "orc_devlayout_decode": ([P, I64, I64, P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


# ----------------------------------------------------------------- bf16 ----
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16(_p(x), x.size, _p(y))
    return y


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.empty(x.shape, dtype=np.float32)
    lib().orc_bf16_to_f32(_p(x), x.size, _p(y))
    return y


# ----------------------------------------------------------------- pack ----
def encode_ternary(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.int8)
    c = np.empty(v.shape, dtype=np.uint8)
    lib().orc_encode_ternary(_p(v), v.size, _p(c))
    return c


def decode_ternary(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    v = np.empty(c.shape, dtype=np.int8)
    lib().orc_decode_ternary(_p(c), c.size, _p(v))
    return v


def pack_4_to_byte(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    assert codes.size % 4 == 0
    out = np.empty(codes.size // 4, dtype=np.uint8)
    lib().orc_pack_4_to_byte(_p(codes), codes.size, _p(out))
    return out


def unpack_byte_to_4(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(packed.size * 4, dtype=np.uint8)
    lib().orc_unpack_byte_to_4(_p(packed), packed.size, _p(out))
    return out


def tile_to_faces(tile: np.ndarray) -> np.ndarray:
    tile = np.ascontiguousarray(tile, dtype=np.int8)
    assert tile.shape == (32, 32)
    out = np.empty(1024, dtype=np.int8)
    lib().orc_tile_to_faces(_p(tile), _p(out))
    return out


def faces_to_tile(faces: np.ndarray) -> np.ndarray:
    faces = np.ascontiguousarray(faces, dtype=np.int8).reshape(-1)
    assert faces.size == 1024
    out = np.empty((32, 32), dtype=np.int8)
    lib().orc_faces_to_tile(_p(faces), _p(out))
    return out


def packed_tile_count(in_f: int, out_f: int) -> int:
    return int(lib().orc_packed_tile_count(in_f, out_f))


def packed_dram_bytes(in_f: int, out_f: int) -> int:
    return int(lib().orc_packed_dram_bytes(in_f, out_f))


def pack_ternary_tilized(wq: np.ndarray, scale: float):
    """pack.py:101-155.  wq is (out_f, in_f) int8; returns (tiles, 256) uint8 and scales."""
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    out_f, in_f = wq.shape
    nt = packed_tile_count(in_f, out_f)
    packed = np.empty((nt, 256), dtype=np.uint8)
    lib().orc_pack_ternary_tilized(_p(wq), out_f, in_f, _p(packed))
    return packed, np.full(nt, scale, dtype=np.float32)


def unpack_ternary_tilized_values(packed: np.ndarray, in_f: int, out_f: int) -> np.ndarray:
    """pack.py:158-191 without the scale: (in_f, out_f) int8."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    wt = np.zeros((in_f, out_f), dtype=np.int8)
    lib().orc_unpack_ternary_tilized(_p(packed), in_f, out_f, _p(wt))
    return wt


def unpack_ternary_tilized(packed, tile_scales, in_f: int, out_f: int) -> np.ndarray:
    """pack.py:158-191: values times the (uniform) per-tile scale, float32."""
    vals = unpack_ternary_tilized_values(packed, in_f, out_f).astype(np.float32)
    kt_n, nt_n = (in_f + 31) // 32, (out_f + 31) // 32
    sc = np.asarray(tile_scales, dtype=np.float32).reshape(kt_n, nt_n)
    rows = np.repeat(np.arange(kt_n), 32)[:in_f]
    cols = np.repeat(np.arange(nt_n), 32)[:out_f]
    return vals * sc[rows[:, None], cols[None, :]]


def pack_tile_python(tile_vals: np.ndarray) -> bytes:
    """Pure-Python loop restatement of one tile's packing (pack.py:79-63 chain),
    independent of the C code; small inputs only."""
    out = bytearray(256)
    for p in range(1024):
        f, rr, cc = p // 256, (p % 256) // 16, p % 16
        r, c = 16 * (f // 2) + rr, 16 * (f % 2) + cc
        v = int(tile_vals[r][c])
        code = 1 if v == 1 else (2 if v == -1 else 0)
        out[p // 4] |= code << (6 - 2 * (p % 4))
    return bytes(out)


# ---------------------------------------------------------------- quant ----
def sum_f32_numpy(a: np.ndarray) -> np.float32:
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    return np.float32(lib().orc_sum_f32_numpy(_p(a), a.size))


def compute_weight_scale(w: np.ndarray, eps: float = WEIGHT_EPS) -> np.float32:
    w = np.ascontiguousarray(w, dtype=np.float32)
    return np.float32(lib().orc_compute_weight_scale(_p(w), w.size, eps))


def weight_quant_ternary(w: np.ndarray, eps: float = WEIGHT_EPS):
    w = np.ascontiguousarray(w, dtype=np.float32)
    q = np.empty(w.shape, dtype=np.int8)
    s = lib().orc_weight_quant_ternary(_p(w), w.size, eps, _p(q))
    return q, np.float32(s)


def act_quant_absmax(x: np.ndarray, eps: float = ACT_EPS):
    """quantization.py:60-91 on float32 input.  Returns (q int8, scale=127/a,
    a_dq=a/127, rowsum int32), the last three with shape (..., 1) / (...,)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.size // k
    q = np.empty(x.shape, dtype=np.int8)
    scale = np.empty(rows, dtype=np.float32)
    a_dq = np.empty(rows, dtype=np.float32)
    rowsum = np.empty(rows, dtype=np.int32)
    lib().orc_act_quant_absmax(_p(x), rows, k, eps, _p(q), _p(scale), _p(a_dq), _p(rowsum))
    lead = x.shape[:-1]
    return q, scale.reshape(lead + (1,)), a_dq.reshape(lead), rowsum.reshape(lead)


def rms_inv(x: np.ndarray, eps: float, order: int) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.float32(lib().orc_rms_inv(_p(x), x.size, eps, order))


def rmsnorm_bf16(x_bf16: np.ndarray, gamma_bf16, eps: float, order: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    k = x.shape[-1]
    rows = x.size // k
    y = np.empty(x.shape, dtype=np.uint16)
    g = None if gamma_bf16 is None else np.ascontiguousarray(gamma_bf16, dtype=np.uint16)
    lib().orc_rmsnorm_bf16(_p(x), None if g is None else _p(g), rows, k, eps, order, _p(y))
    return y


# ----------------------------------------------------------------- gemm ----
def gemm_i8t(xq: np.ndarray, w_kn: np.ndarray) -> np.ndarray:
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    w_kn = np.ascontiguousarray(w_kn, dtype=np.int8)
    m, k = xq.shape
    k2, n = w_kn.shape
    assert k == k2
    acc = np.empty((m, n), dtype=np.int32)
    lib().orc_gemm_i8t(_p(xq), _p(w_kn), m, k, n, _p(acc))
    return acc


def scale_bf16(acc: np.ndarray, a_dq: np.ndarray, seg_scales, seg_ends) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    a_dq = np.ascontiguousarray(a_dq, dtype=np.float32).reshape(-1)
    sc = np.ascontiguousarray(seg_scales, dtype=np.float32)
    ends = np.ascontiguousarray(seg_ends, dtype=np.int64)
    out = np.empty((m, n), dtype=np.uint16)
    lib().orc_scale_bf16(_p(acc), m, n, _p(a_dq), _p(sc), _p(ends), int(sc.size), _p(out))
    return out


def relu2_mul_bf16(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.uint16)
    u = np.ascontiguousarray(u, dtype=np.uint16)
    h = np.empty(g.shape, dtype=np.uint16)
    lib().orc_relu2_mul_bf16(_p(g), _p(u), g.size, _p(h))
    return h


def add_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    y = np.empty(a.shape, dtype=np.uint16)
    lib().orc_add_bf16(_p(a), _p(b), a.size, _p(y))
    return y


def devlayout_encode(w_kn: np.ndarray) -> np.ndarray:
    w_kn = np.ascontiguousarray(w_kn, dtype=np.int8)
    k, n = w_kn.shape
    assert n % 32 == 0
    ks = (k + 127) // 128
    dev = np.empty((n // 32, ks, 256), dtype=np.uint32)
    lib().orc_devlayout_encode(_p(w_kn), k, n, _p(dev))
    return dev


def devlayout_decode(dev: np.ndarray, k: int, n: int) -> np.ndarray:
    dev = np.ascontiguousarray(dev, dtype=np.uint32)
    w = np.zeros((k, n), dtype=np.int8)
    lib().orc_devlayout_decode(_p(dev), k, n, _p(w))
    return w


# ------------------------------------------------------------ composite ----
def bitlinear(x_bf16, w_kn, seg_scales, seg_ends=None, gamma_bf16=None, norm_eps=1e-5,
              order: int = 1, residual_bf16=None):
    """One BitLinear: [RMSNorm ->] absmax int8 quant -> int32 GEMM -> scale ->
    bf16 [-> + residual].  Returns a dict of every intermediate."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, k = x.shape
    n = w_kn.shape[1]
    y = rmsnorm_bf16(x, gamma_bf16, norm_eps, order) if gamma_bf16 is not None else x
    q, scale, a_dq, rowsum = act_quant_absmax(bf16_to_f32(y))
    acc = gemm_i8t(q, w_kn)
    if seg_ends is None:
        seg_ends = [n]
    out = scale_bf16(acc, a_dq, seg_scales, seg_ends)
    if residual_bf16 is not None:
        out = add_bf16(residual_bf16, out)
    return {"y": y, "q": q, "scale": scale, "a_dq": a_dq, "rowsum": rowsum, "acc": acc, "out": out}


def gate_up_relu2(x_bf16, w_kn_gu, gate_scale, up_scale, gamma_bf16=None, norm_eps=1e-5, order=1):
    """Fused gate||up BitLinear with the relu(g)^2*u epilogue (ffn.py:140-170)."""
    n2 = w_kn_gu.shape[1]
    f = n2 // 2
    r = bitlinear(x_bf16, w_kn_gu, [gate_scale, up_scale], [f, n2], gamma_bf16, norm_eps, order)
    r["h"] = relu2_mul_bf16(r["out"][:, :f], r["out"][:, f:])
    return r


def permute_halfsplit_to_adjacent(weight_t: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """attention.py:462-478 -- column permutation of a (K, heads*head_dim) matrix:
    new[2k] = old[k], new[2k+1] = old[k + head_dim/2] inside each head."""
    out = weight_t.copy()
    half = head_dim // 2
    for h in range(num_heads):
        for kk in range(half):
            out[:, h * head_dim + 2 * kk] = weight_t[:, h * head_dim + kk]
            out[:, h * head_dim + 2 * kk + 1] = weight_t[:, h * head_dim + kk + half]
    return out


# --------------------------------------------------------------- LM head ----
def lm_head(xn_bf16: np.ndarray, w_bf16: np.ndarray):
    """src/bitnet_tt/inference/generator_batch32.py:768-811 -- logits of the
    normalised rows against the (vocab, hidden) head (model/bitnet.py:139-215)
    in float64 (bf16 x bf16 products are exact there), with the bound on the
    rounding of an fp32 accumulation of the same K products: 2 K 2^-24 sum|x w|."""
    x = bf16_to_f32(np.asarray(xn_bf16, dtype=np.uint16)).astype(np.float64)
    w = bf16_to_f32(np.asarray(w_bf16, dtype=np.uint16)).astype(np.float64)
    k = x.shape[-1]
    return x @ w.T, (2.0 * k * 2.0 ** -24) * (np.abs(x) @ np.abs(w).T)


def argmax_first(logits: np.ndarray) -> np.ndarray:
    """generator_batch32.py:1170-1174 -- greedy token: the first index of each
    row's largest logit (the tie rule of torch/ttnn argmax)."""
    return np.argmax(np.asarray(logits), axis=-1)


# ------------------------------------------------------- decode attention ----
def rope_tables(dim: int, max_pos: int, theta: float):
    """utils/rope.py:7-23 -- float32 frequencies 1/theta^(2i/dim), angles
    position x frequency in float32, cos/sin in float32; [max_pos, dim/2]."""
    freqs = 1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    ang = np.outer(np.arange(max_pos, dtype=np.float32), freqs)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_rotate(x: np.ndarray, c: np.ndarray, s: np.ndarray, adjacent: bool) -> np.ndarray:
    """attention.py:1325-1350 -- rotation of every pair of the last axis by its
    frequency's angle: pairs (2i, 2i+1) (adjacent-pair RoPE of permuted Q/K
    weights) or (i, i + D/2) (HF rotate_half); x float64, c/s [D/2]."""
    d = x.shape[-1]
    i0 = np.arange(0, d, 2) if adjacent else np.arange(d // 2)
    i1 = i0 + 1 if adjacent else i0 + d // 2
    y = np.empty_like(x)
    y[..., i0] = x[..., i0] * c - x[..., i1] * s
    y[..., i1] = x[..., i1] * c + x[..., i0] * s
    return y


def decode_attention(qkv_bf16, kc_bf16, vc_bf16, pos, H, Hkv, cos, sin, adjacent, scale):
    """attention.py:1040-1262 -- split qkv into heads, RoPE q and k at each
    user's position, write k and v at that position of copies of the caches,
    then softmax(scale q k^T) v over positions [0, pos] per query head (head h
    reads key-value head h // (H / Hkv)).  Rotated q and k are rounded to bf16
    (the operands the caches and the score products hold); everything else is
    float64.  Returns (out [B, H*D] float64, new k cache bits, new v cache bits)."""
    qkv = bf16_to_f32(np.asarray(qkv_bf16, dtype=np.uint16)).astype(np.float64)
    B = qkv.shape[0]
    D = kc_bf16.shape[-1]
    G = H // Hkv
    kc = np.array(kc_bf16, dtype=np.uint16, copy=True)
    vc = np.array(vc_bf16, dtype=np.uint16, copy=True)
    out = np.zeros((B, H * D))
    for b in range(B):
        p = int(pos[b])
        c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
        q = qkv[b, :H * D].reshape(H, D)
        k = qkv[b, H * D:(H + Hkv) * D].reshape(Hkv, D)
        v_bits = np.asarray(qkv_bf16, dtype=np.uint16)[b, (H + Hkv) * D:].reshape(Hkv, D)
        qr = bf16_to_f32(f32_to_bf16(rope_rotate(q, c, s, adjacent).astype(np.float32))).astype(np.float64)
        kr_bits = f32_to_bf16(rope_rotate(k, c, s, adjacent).astype(np.float32))
        kc[b, :, p, :] = kr_bits
        vc[b, :, p, :] = v_bits
        K = bf16_to_f32(kc[b, :, : p + 1, :]).astype(np.float64)
        V = bf16_to_f32(vc[b, :, : p + 1, :]).astype(np.float64)
        for h in range(H):
            sc = scale * (K[h // G] @ qr[h])
            e = np.exp(sc - sc.max())
            out[b, h * D:(h + 1) * D] = (e / e.sum()) @ V[h // G]
    return out, kc, vc
