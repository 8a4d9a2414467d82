"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against the reference tests' known answers
(tests/golden/known_answers.json, copied by value from bitnet-tt's tests), brute
force, or an independent computation (numpy / torch on the CPU) of the same
closed form, chosen so that a dropped term, a swapped index or a wrong
rounding mode fails a test.
"""

import itertools

import numpy as np
import pytest
import torch


def bf16_bits_torch(x_f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# --------------------------------------------------------------- bf16 ----
def test_bf16_conversion_matches_torch(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10.0,
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 1e-40, 3.3895314e38], dtype=np.float32),
        # exact halfway cases between two bf16 values: ties to even
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    assert np.array_equal(orc.f32_to_bf16(x), bf16_bits_torch(x))
    nan = orc.f32_to_bf16(np.array([np.nan], dtype=np.float32))
    assert np.isnan(orc.bf16_to_f32(nan))[0]
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    back = orc.bf16_to_f32(bits)
    fin = np.isfinite(back)
    assert np.array_equal(orc.f32_to_bf16(back[fin]), bits[fin])


# ------------------------------------------------------- codes / bytes ----
def test_encode_decode_known_answers(orc, known):
    ka = known["encode_values"]
    assert orc.encode_ternary(np.array(ka["values"], np.int8)).tolist() == ka["codes"]
    kd = known["decode_values"]
    assert orc.decode_ternary(np.array(kd["codes"], np.uint8)).tolist() == kd["values"]
    # reserved code 0b11 reads as 0 (kernels/device/reader_ternary_in1.cpp:43-56)
    assert orc.decode_ternary(np.array([3], np.uint8)).tolist() == [0]


def test_encode_roundtrip_seeded(orc, known):
    rng = np.random.default_rng(known["seeded_roundtrips"]["encode_seed"])
    v = rng.choice([-1, 0, 1], size=1024).astype(np.int8)
    assert np.array_equal(orc.decode_ternary(orc.encode_ternary(v)), v)


def test_pack_byte_known_answers(orc, known):
    k = known["pack_single_byte"]
    assert orc.pack_4_to_byte(np.array(k["codes"], np.uint8)).tolist() == [k["byte"]]
    k2 = known["pack_roundtrip_two_bytes"]
    codes = np.array(k2["codes"], np.uint8)
    packed = orc.pack_4_to_byte(codes)
    assert packed.size == k2["n_bytes"]
    assert np.array_equal(orc.unpack_byte_to_4(packed), codes)
    # MSB first: the first code sits in bits 7:6
    assert orc.pack_4_to_byte(np.array([1, 0, 0, 0], np.uint8)).tolist() == [0b01000000]
    assert orc.pack_4_to_byte(np.array([0, 0, 0, 2], np.uint8)).tolist() == [0b00000010]


def test_pack_byte_brute_force_all_81_tuples(orc):
    for tup in itertools.product([-1, 0, 1], repeat=4):
        v = np.array(tup, np.int8)
        b = orc.pack_4_to_byte(orc.encode_ternary(v))
        expect = sum(({1: 1, -1: 2, 0: 0}[t]) << (6 - 2 * i) for i, t in enumerate(tup))
        assert b.tolist() == [expect]
        assert np.array_equal(orc.decode_ternary(orc.unpack_byte_to_4(b)), v)


# --------------------------------------------------------- faces/tiles ----
def test_face_ordering_known_answer(orc, known):
    k = known["face_ordering"]
    tile = np.zeros((32, 32), np.int8)
    for r, c, v in k["marks"]:
        tile[r, c] = v
    faces = orc.tile_to_faces(tile)
    for idx, v in k["expect"]:
        assert faces[idx] == v


def test_faces_are_row_major_quadrants(orc):
    tile = (np.arange(1024) % 127).astype(np.int8).reshape(32, 32)
    faces = orc.tile_to_faces(tile)
    quads = [tile[:16, :16], tile[:16, 16:], tile[16:, :16], tile[16:, 16:]]
    for f, q in enumerate(quads):
        assert np.array_equal(faces[256 * f: 256 * (f + 1)], q.ravel())
    assert np.array_equal(orc.faces_to_tile(faces), tile)


def test_tile_counts_known_answers(orc, known):
    k = known["tile_counts"]
    for in_f, out_f, tiles in k["cases"]:
        assert orc.packed_tile_count(in_f, out_f) == tiles
        assert orc.packed_dram_bytes(in_f, out_f) == tiles * 256
    assert (2560 * 2560 * 2) / orc.packed_dram_bytes(2560, 2560) > k["bf16_over_packed_min_ratio"]
    assert orc.packed_tile_count(50, 100) == 2 * 4  # padded to 64 x 128


def test_single_tile_against_independent_python(orc):
    rng = np.random.default_rng(5)
    for _ in range(4):
        w_kn = rng.choice([-1, 0, 1], size=(32, 32)).astype(np.int8)
        packed, _ = orc.pack_ternary_tilized(np.ascontiguousarray(w_kn.T), 1.0)
        assert bytes(packed[0]) == orc.pack_tile_python(w_kn)


def test_tile_order_kt_major(orc):
    # (in=64, out=96): Kt=2, Nt=3; a single +1 in tile (kt=1, nt=2) must land in tile 1*3+2
    w_outin = np.zeros((96, 64), np.int8)
    w_outin[2 * 32 + 5, 1 * 32 + 7] = 1  # n = 69, k = 39
    packed, _ = orc.pack_ternary_tilized(w_outin, 1.0)
    nz = np.nonzero(packed.reshape(6, 256).any(axis=1))[0].tolist()
    assert nz == [5]
    # r=7, c=5 -> face 0, p = 16*7 + 5 = 117 -> byte 29, shift 6-2*(117%4)=4
    assert packed[5, 29] == 1 << 4


@pytest.mark.parametrize("seed_key,shape_key", [("matrix_seed", "matrix_shape"), ("nonaligned_seed", "nonaligned_shape")])
def test_tilized_roundtrip_seeded(orc, known, seed_key, shape_key):
    k = known["seeded_roundtrips"]
    rng = np.random.default_rng(k[seed_key])
    out_f, in_f = k[shape_key]
    w = rng.standard_normal((out_f, in_f)).astype(np.float32)
    q, s = orc.weight_quant_ternary(w)
    packed, scales = orc.pack_ternary_tilized(q, float(s))
    assert packed.shape == (orc.packed_tile_count(in_f, out_f), 256)
    un = orc.unpack_ternary_tilized(packed, scales, in_f, out_f)
    np.testing.assert_allclose(un, q.T.astype(np.float32) * float(s), atol=1e-5)


def test_all_zero_and_all_one_tiles(orc, known):
    k = known["all_zeros_tile"]
    packed, sc = orc.pack_ternary_tilized(np.zeros((k["out_features"], k["in_features"]), np.int8), k["scale"])
    assert np.all(orc.unpack_ternary_tilized(packed, sc, k["in_features"], k["out_features"]) == k["expect"])
    k = known["all_ones_tile"]
    packed, sc = orc.pack_ternary_tilized(np.ones((k["out_features"], k["in_features"]), np.int8), k["scale"])
    np.testing.assert_allclose(orc.unpack_ternary_tilized(packed, sc, k["in_features"], k["out_features"]),
                               k["expect"], atol=1e-6)
    assert np.all(packed == 0b01010101)


# ------------------------------------------------------- weight quant ----
@pytest.mark.parametrize("shape", [(7,), (100,), (129,), (4097,), (64, 128), (50, 100), (300, 301), (640, 2560),
                                   (2560, 2560)])
def test_weight_scale_bit_exact_with_numpy(orc, shape):
    rng = np.random.default_rng(sum(shape))
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    assert orc.sum_f32_numpy(np.abs(w)) == np.sum(np.abs(w))
    assert orc.compute_weight_scale(w) == np.maximum(np.mean(np.abs(w)), 1e-5)


def test_weight_quant_known_answers(orc, known):
    k = known["weight_sign"]
    q, _ = orc.weight_quant_ternary(np.array(k["weight"], np.float32))
    assert q[0, 0] == k["q00"] and q[0, 1] == k["q01"]
    q, s = orc.weight_quant_ternary(np.zeros((64, 128), np.float32))
    assert np.all(q == 0) and s == np.float32(1e-5)
    rng = np.random.default_rng(3)
    w = rng.standard_normal((64, 128)).astype(np.float32) * 100
    q, s = orc.weight_quant_ternary(w)
    assert set(np.unique(q).tolist()) <= {-1, 0, 1} and s > 10


def test_weight_quant_ties_to_even(orc):
    # mean|W| = 1 exactly, so W/s = W: 0.5 -> 0, 1.5 -> 2 -> 1, -0.5 -> 0, -1.5 -> -2 -> -1
    w = np.array([0.5, 1.5, -0.5, -1.5, 0.0, 2.0], np.float32)
    q, s = orc.weight_quant_ternary(w)
    assert s == 1.0
    assert q.tolist() == [0, 1, 0, -1, 0, 1]


def test_weight_quant_matches_numpy_expression(orc):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((384, 320)) * 0.02).astype(np.float32)
    q, s = orc.weight_quant_ternary(w)
    s_np = np.maximum(np.mean(np.abs(w)), 1e-5)
    assert s == s_np
    assert np.array_equal(q, np.clip(np.round(w / s_np), -1, 1).astype(np.int8))
    frac = [(q == 1).mean(), (q == 0).mean(), (q == -1).mean()]
    # absmean of a Gaussian: P(|z| < 0.5*mean|z|/sigma) = P(|z| < 0.399) = 0.31
    assert abs(frac[1] - 0.31) < 0.02 and abs(frac[0] - frac[2]) < 0.02


# --------------------------------------------------- activation quant ----
def test_act_quant_known_answers(orc, known):
    k = known["act_scale_known"]
    x = np.zeros(k["shape"], np.float32)
    x[0, 0, 0] = k["x000"]
    q, scale, a_dq, rowsum = orc.act_quant_absmax(x)
    assert scale.shape == (1, 1, 1)
    assert abs(scale[0, 0, 0] - k["scale"]) < k["atol"]
    assert q[0, 0, 0] == 127 and rowsum.item() == 127
    kr = known["act_range"]
    rng = np.random.default_rng(1)
    q, scale, _, _ = orc.act_quant_absmax(rng.standard_normal(kr["shape"]).astype(np.float32))
    assert q.min() >= kr["qmin"] and q.max() <= kr["qmax"]
    assert scale.shape == (2, 16, 1)


def test_act_quant_special_cases(orc):
    # zero row: absmax clamps to eps -> all zeros; exact +-absmax -> +-127;
    # ties to even with scale 1: 2.5 -> 2, 3.5 -> 4, -2.5 -> -2
    x = np.zeros((3, 8), np.float32)
    x[1] = [-4.0, 4.0, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0]
    x[2] = [127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -127.0]
    q, scale, a_dq, rowsum = orc.act_quant_absmax(x)
    assert np.all(q[0] == 0) and a_dq[0] == np.float32(1e-5) / np.float32(127)
    assert q[1, :3].tolist() == [-127, 127, 32]  # 1*127/4 = 31.75 -> 32
    assert q[2].tolist() == [127, 2, 4, -2, 0, 0, 2, -127]
    assert rowsum.tolist() == [0, 32, 6]
    assert a_dq[2] == np.float32(1.0)


def test_act_quant_matches_numpy_expression(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 2560)).astype(np.float32)
    x[:, rng.choice(2560, 26, replace=False)] *= 20
    q, scale, a_dq, rowsum = orc.act_quant_absmax(x)
    a = np.maximum(np.max(np.abs(x), axis=-1, keepdims=True), 1e-5)
    s = 127 / a
    assert np.array_equal(scale, s)
    assert np.array_equal(q, np.clip(np.round(x * s), -128, 127).astype(np.int8))
    assert np.array_equal(rowsum, q.astype(np.int64).sum(-1))
    assert np.array_equal(a_dq, (a / np.float32(127)).reshape(-1))


# ------------------------------------------------------------ RMSNorm ----
def test_rms_orders_agree(orc):
    rng = np.random.default_rng(4)
    for k in (256, 2560, 6912):
        x = orc.bf16_to_f32(orc.f32_to_bf16(rng.standard_normal(k).astype(np.float32) * 3))
        r1, r0 = orc.rms_inv(x, 1e-5, 1), orc.rms_inv(x, 1e-5, 0)
        assert abs(float(r1) - float(r0)) <= 4 * np.spacing(np.float32(r0))


def test_rmsnorm_closed_forms(orc):
    # constant row c: r = 1/sqrt(c^2 + eps) -> y ~ sign(c)
    x = orc.f32_to_bf16(np.full((2, 512), [[3.0], [-0.25]], np.float32))
    y = orc.bf16_to_f32(orc.rmsnorm_bf16(x, None, 1e-5))
    np.testing.assert_allclose(y[0], 1.0, rtol=2 ** -8)
    np.testing.assert_allclose(y[1], -1.0, rtol=2 ** -7)
    # gamma enters after the bf16 rounding of x*r: gamma = 2 doubles y exactly
    rng = np.random.default_rng(8)
    xb = orc.f32_to_bf16(rng.standard_normal((4, 256)).astype(np.float32))
    g1 = orc.f32_to_bf16(np.ones(256, np.float32))
    g2 = orc.f32_to_bf16(np.full(256, 2.0, np.float32))
    y1 = orc.bf16_to_f32(orc.rmsnorm_bf16(xb, g1, 1e-5))
    y2 = orc.bf16_to_f32(orc.rmsnorm_bf16(xb, g2, 1e-5))
    assert np.array_equal(y2, 2 * y1)
    # eps dominates a tiny row: y = bf16(x / sqrt(eps))
    xt = orc.f32_to_bf16(np.full((1, 64), 1e-6, np.float32))
    yt = orc.bf16_to_f32(orc.rmsnorm_bf16(xt, None, 1e-5))
    np.testing.assert_allclose(yt, orc.bf16_to_f32(xt) / np.sqrt(1e-5 + 1e-12), rtol=1e-2)


def test_rmsnorm_matches_torch_hf_formula(orc):
    # HF BitNetRMSNorm.forward (modeling_bitnet.py:53-58) in torch on the CPU
    rng = np.random.default_rng(9)
    x = orc.f32_to_bf16(rng.standard_normal((8, 2560)).astype(np.float32))
    g = orc.f32_to_bf16((1 + 0.1 * rng.standard_normal(2560)).astype(np.float32))
    xt = torch.from_numpy(orc.bf16_to_f32(x)).to(torch.bfloat16)
    gt = torch.from_numpy(orc.bf16_to_f32(g)).to(torch.bfloat16)
    hs = xt.to(torch.float32)
    var = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(var + 1e-5)
    ref = (gt * hs.to(torch.bfloat16)).to(torch.float32).numpy()
    y = orc.bf16_to_f32(orc.rmsnorm_bf16(x, g, 1e-5, order=0))
    ulp = np.abs(ref) * 2 ** -7
    assert np.all(np.abs(y - ref) <= ulp + 1e-30)
    assert np.mean(y == ref) > 0.99


# --------------------------------------------------------------- GEMM ----
def test_gemm_identity_and_rowsums(orc, known):
    k = known["identity_readback"]
    rng = np.random.default_rng(k["seed"])
    w_outin = rng.choice([-1, 0, 1], size=(k["N"], k["K"])).astype(np.int8)
    eye = np.eye(k["M"], k["K"], dtype=np.int8)
    assert np.array_equal(orc.gemm_i8t(eye, np.ascontiguousarray(w_outin.T)), w_outin.T.astype(np.int32))
    g = known["matmul_ones"]
    acc = orc.gemm_i8t(np.ones((g["M"], g["K"]), np.int8), np.ones((g["K"], g["N"]), np.int8))
    assert np.all(acc == int(g["expect"]))
    # activation 0.5 quantises to 127 with a_dq = 0.5/127, so out = 127*32*0.5/127 = 16
    g = known["generic_op_all_plus_one"]
    xb = orc.f32_to_bf16(np.full((g["M"], g["K"]), g["act"], np.float32))
    r = orc.bitlinear(xb, np.ones((g["K"], g["N"]), np.int8), [1.0])
    np.testing.assert_allclose(orc.bf16_to_f32(r["out"]), g["expect"], rtol=1e-2)


def test_gemm_brute_force(orc):
    rng = np.random.default_rng(6)
    for m, k, n in [(1, 32, 32), (5, 96, 64), (32, 256, 96)]:
        x = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
        w = rng.choice([-1, 0, 1], size=(k, n)).astype(np.int8)
        assert np.array_equal(orc.gemm_i8t(x, w), x.astype(np.int64) @ w.astype(np.int64))


def test_scale_epilogue_segments(orc):
    rng = np.random.default_rng(12)
    acc = rng.integers(-50000, 50000, size=(4, 96)).astype(np.int32)
    a_dq = (rng.random(4) * 0.05).astype(np.float32)
    sc = [0.02, 0.03, 0.05]
    out = orc.bf16_to_f32(orc.scale_bf16(acc, a_dq, sc, [32, 64, 96]))
    seg = np.repeat(np.array(sc, np.float32), 32)
    f = (seg[None, :] * a_dq[:, None]).astype(np.float32)
    ref = (acc.astype(np.float32) * f).astype(np.float32)
    assert np.array_equal(out, orc.bf16_to_f32(orc.f32_to_bf16(ref)))
    # against float64 within one bf16 rounding
    ref64 = acc.astype(np.float64) * seg[None, :].astype(np.float64) * a_dq[:, None].astype(np.float64)
    assert np.all(np.abs(out - ref64) <= np.abs(ref64) * 2 ** -8 + 1e-30)


def test_relu2_mul_and_add_match_torch_bf16(orc):
    rng = np.random.default_rng(13)
    g = orc.f32_to_bf16(rng.standard_normal(4096).astype(np.float32) * 3)
    u = orc.f32_to_bf16(rng.standard_normal(4096).astype(np.float32) * 3)
    gt = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    ut = torch.from_numpy(u.view(np.int16)).view(torch.bfloat16)
    ref = (torch.square(torch.relu(gt)) * ut).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.relu2_mul_bf16(g, u), ref)
    ref_add = (gt + ut).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.add_bf16(g, u), ref_add)


def test_bitlinear_against_float64_reference(orc):
    rng = np.random.default_rng(14)
    x = orc.f32_to_bf16(rng.standard_normal((32, 512)).astype(np.float32))
    w_lat = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    q, s = orc.weight_quant_ternary(w_lat)
    r = orc.bitlinear(x, np.ascontiguousarray(q.T), [float(s)])
    xf = orc.bf16_to_f32(x).astype(np.float64)
    a = np.abs(xf).max(-1, keepdims=True)
    xq = np.clip(np.round(xf * (127 / a)), -128, 127)
    ref = (xq @ q.T.astype(np.float64)) * float(s) * a / 127
    out = orc.bf16_to_f32(r["out"])
    assert np.max(np.abs(out - ref)) <= 1e-2 * np.max(np.abs(ref))


# ------------------------------------------------------- device layout ----
def test_devlayout_bijective_and_padded(orc):
    rng = np.random.default_rng(15)
    for k, n in [(128, 32), (96, 64), (2560, 96), (200 - 200 % 32, 32)]:
        w = rng.choice([-1, 0, 1], size=(k, n)).astype(np.int8)
        dev = orc.devlayout_encode(w)
        assert dev.shape == (n // 32, (k + 127) // 128, 256)
        assert np.array_equal(orc.devlayout_decode(dev, k, n), w)


def test_devlayout_is_the_mfma_operand_order(orc):
    # Unpacking word d of lane l as (d >> 2r) & 0x03030303 gives B-operand dword r,
    # whose bytes are rows 4r..4r+3 of that lane's 16 (rows k0+16*(l>>5)+j, column l&31).
    rng = np.random.default_rng(16)
    k, n = 256, 64
    w = rng.choice([-1, 0, 1], size=(k, n)).astype(np.int8)
    dev = orc.devlayout_encode(w)
    for nt in range(n // 32):
        for ks in range(k // 128):
            for lane in (0, 5, 31, 32, 47, 63):
                for q in range(4):
                    d = int(dev[nt, ks, lane * 4 + q])
                    col = nt * 32 + (lane & 31)
                    for r in range(4):
                        dw = (d >> (2 * r)) & 0x03030303
                        for b in range(4):
                            j = 4 * r + b
                            row = ks * 128 + q * 32 + (lane >> 5) * 16 + j
                            assert ((dw >> (8 * b)) & 0xFF) == w[row, col] + 1
    # rows past K read as weight 0 (offset code 1)
    w2 = rng.choice([-1, 0, 1], size=(96, 32)).astype(np.int8)
    d2 = orc.devlayout_encode(w2)
    lane, q = 0, 3  # rows 96..111: padding
    assert int(d2[0, 0, lane * 4 + q]) == 0x55555555


def test_lm_head_oracle_closed_forms(orc):
    """Head rows that are unit vectors pick single columns of the normalised
    rows (W = I gives the rows themselves); a tie takes the first index; the
    bound scales with sum|x w| and vanishes for exact products."""
    rng = np.random.default_rng(4)
    x = orc.f32_to_bf16(rng.standard_normal((3, 64)).astype(np.float32))
    eye = orc.f32_to_bf16(np.eye(64, dtype=np.float32))
    logits, bound = orc.lm_head(x, eye)
    assert np.array_equal(logits, orc.bf16_to_f32(x).astype(np.float64))
    assert np.allclose(bound, 2 * 64 * 2.0 ** -24 * np.abs(orc.bf16_to_f32(x)))
    w = orc.f32_to_bf16(np.stack([np.zeros(64), np.ones(64), np.ones(64), -np.ones(64)]).astype(np.float32))
    ones = orc.f32_to_bf16(np.ones((1, 64), dtype=np.float32))
    lg, _ = orc.lm_head(ones, w)
    assert lg.tolist() == [[0.0, 64.0, 64.0, -64.0]]
    assert orc.argmax_first(lg).tolist() == [1]  # tie between 1 and 2: the first
