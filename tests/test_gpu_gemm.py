"""GPU parity of the ternary GEMM (btl_gemm_i8t2) and the fused entry point.

int32 accumulators are compared bit for bit with the oracle; bf16 outputs too
(the epilogue's rounding is specified exactly).  Decode shapes run every
split-K factor; prefill shapes at full size are compared in every row, with
the reference accumulators from a host fp32 matmul of the integer operands
(exact: every partial sum is an integer below 2^24) that is itself checked
against the oracle's integer GEMM on sampled rows, plus row and column
checksums in int64."""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N

pytestmark = pytest.mark.gpu


def device_weight(orc, w_kn):
    k, n = w_kn.shape
    dev = orc.devlayout_encode(w_kn)
    return H.to_dev(dev.view(np.int32))


def run_gemm(orc, q, w_kn, scales, ends=None, epi=0, splitk=0, residual_bits=None, wdev=None, rowsum=False):
    """int8 q [m,k] x ternary w [k,n] through btl_gemm_i8t2 with a random
    per-row dequantisation factor a_dq.  rowsum=True hands the kernel the row
    sums sum_k q (as btl_quant_absmax writes them); else it sums the operand."""
    L = N.lib()
    d = H.dev()
    m, k = q.shape
    n = w_kn.shape[1]
    rows = 32 * ((m + 31) // 32)
    rng = np.random.default_rng(m + k + n)
    a_dq = np.zeros(rows, np.float32)
    a_dq[:m] = (0.005 + 0.03 * rng.random(m)).astype(np.float32)
    xa = H.to_dev(H.rowmajor_to_xa(q))
    wdev = device_weight(orc, w_kn) if wdev is None else wdev
    ends = ends or [n]
    sc, en, nseg = N.segments_arrays(scales, ends)
    n_out = n // 2 if epi == 1 else n
    out = torch.empty((m, n_out), dtype=torch.bfloat16, device=d)
    acc = torch.empty((m, n), dtype=torch.int32, device=d)
    res = H.to_dev_bf16(residual_bits) if residual_bits is not None else None
    if res is not None:
        out.copy_(res)
        res = out  # in place: out = residual + result
    ws_bytes = int(L.btl_gemm_workspace_bytes(m, k, n, epi, splitk))
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=d)
    a_dq_d = H.to_dev(a_dq)  # keep the tensor alive across the launch
    rs_d = H.to_dev(q.astype(np.int32).sum(1, dtype=np.int64).astype(np.int32)) if rowsum else None
    N.check(L.btl_gemm_i8t2(N.ptr(xa), N.ptr(a_dq_d), N.ptr(rs_d), m, k, n, N.ptr(wdev), sc, en,
                            nseg, epi, N.ptr(res), N.ptr(out), N.ptr(acc), N.ptr(ws), ws.numel(), splitk,
                            N.stream_of(d)), "btl_gemm_i8t2")
    torch.cuda.synchronize()
    counters_clean = ws_bytes == 0 or not ws[: 4 * 2048].cpu().numpy()[: 4 * ((n // 32) or 1)].any()
    return acc.cpu().numpy(), H.bits_of(out), a_dq[:m], counters_clean


def full_acc_ref(orc, q, w, check_rows=8, seed=0):
    """Reference int32 accumulators of q [m,k] int8 x w [k,n] ternary for
    every row: a host torch fp32 matmul of the integer-valued operands.  The
    sums are exact (|acc| <= 128 k < 2^24 for k <= 131072, so every partial
    sum is an integer that fp32 holds), and sampled rows are checked against
    the oracle's integer GEMM."""
    m, k = q.shape
    assert 128 * k < (1 << 24)
    ref = (torch.from_numpy(q.astype(np.float32)) @ torch.from_numpy(w.astype(np.float32))).numpy()
    ref = ref.astype(np.int32)
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(seed).choice(m, check_rows)]))
    assert np.array_equal(ref[rows], orc.gemm_i8t(np.ascontiguousarray(q[rows]), w)), "host fp32 reference"
    return ref


def expected_out(orc, acc, a_dq, scales, ends, epi, residual_bits=None):
    out = orc.scale_bf16(acc, a_dq, scales, ends)
    if epi == 1:
        f = acc.shape[1] // 2
        return orc.relu2_mul_bf16(out[:, :f], out[:, f:])
    if residual_bits is not None:
        out = orc.add_bf16(residual_bits, out)
    return out


def test_identity_readback(orc, known):
    k = known["identity_readback"]
    w_outin = np.random.default_rng(k["seed"]).choice([-1, 0, 1], size=(k["N"], k["K"])).astype(np.int8)
    acc, _, _, _ = run_gemm(orc, np.eye(32, 32, dtype=np.int8), np.ascontiguousarray(w_outin.T), [1.0])
    assert np.array_equal(acc, w_outin.T.astype(np.int32))


def test_all_ones_row_sums(orc):
    rng = np.random.default_rng(2)
    q = rng.integers(-128, 128, size=(32, 256)).astype(np.int8)
    acc, _, _, _ = run_gemm(orc, q, np.ones((256, 64), np.int8), [1.0])
    assert np.all(acc == q.astype(np.int64).sum(1, keepdims=True))
    acc, _, _, _ = run_gemm(orc, q, -np.ones((256, 64), np.int8), [1.0])
    assert np.all(acc == -q.astype(np.int64).sum(1, keepdims=True))


@pytest.mark.parametrize("m,k,n", [(32, 128, 32), (32, 2560, 256), (7, 640, 96), (1, 2560, 64), (32, 6912, 128),
                                   (32, 224, 64)])
@pytest.mark.parametrize("splitk", [1, 2, 3, 0])
def test_decode_gemm_bit_exact(orc, m, k, n, splitk):
    print(f"decode gemm m={m} k={k} n={n} splitk={splitk}", flush=True)
    rng = np.random.default_rng(m * 7 + k + n + splitk)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=k + n)
    acc, out, a_dq, clean = run_gemm(orc, q, w, [0.0173], splitk=splitk)
    ref = orc.gemm_i8t(q, w)
    assert np.array_equal(acc, ref)
    assert np.array_equal(out, expected_out(orc, ref, a_dq, [0.0173], [n], 0))
    assert clean, "split-K counters must be left at zero"


@pytest.mark.parametrize("m,k,n", [(32, 2560, 2560), (7, 640, 96), (32, 6912, 256), (1, 128, 32)])
def test_dot4_variant_bit_exact(orc, m, k, n):
    """The VALU (v_dot4) formulation of the decode GEMM gives the oracle's
    int32 accumulators."""
    print(f"dot4 gemm m={m} k={k} n={n}", flush=True)
    L = N.lib()
    d = H.dev()
    rng = np.random.default_rng(m + 3 * k + n)
    q = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=2 * k + n)
    xa = H.to_dev(H.rowmajor_to_xa(q))
    wdev = device_weight(orc, w)
    rs = H.to_dev(q.astype(np.int64).sum(1).astype(np.int32))
    acc = torch.zeros((m, n), dtype=torch.int32, device=d)
    N.check(L.btl_gemm_i8t2_dot4(N.ptr(xa), N.ptr(rs), m, k, n, N.ptr(wdev), N.ptr(acc), N.stream_of(d)),
            "btl_gemm_i8t2_dot4")
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), orc.gemm_i8t(q, w))


def test_extreme_accumulators(orc):
    # |acc| = 128 * K at its largest: all -128 against all -1 / +1
    k = 16384
    q = np.full((32, k), -128, np.int8)
    w = np.concatenate([np.ones((k, 32), np.int8), -np.ones((k, 32), np.int8)], axis=1)
    acc, _, _, _ = run_gemm(orc, q, w, [1.0], splitk=4)
    assert np.all(acc[:, :32] == -128 * k) and np.all(acc[:, 32:] == 128 * k)


def test_segments_and_residual(orc):
    rng = np.random.default_rng(4)
    m, k, n = 32, 512, 192
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=9)
    scales, ends = [0.011, 0.023, 0.037], [128, 160, 192]
    res = orc.f32_to_bf16(rng.standard_normal((m, n)).astype(np.float32))
    for splitk in (1, 2):
        acc, out, a_dq, _ = run_gemm(orc, q, w, scales, ends, splitk=splitk, residual_bits=res)
        assert np.array_equal(out, expected_out(orc, acc, a_dq, scales, ends, 0, res))
        assert np.array_equal(acc, orc.gemm_i8t(q, w))


@pytest.mark.parametrize("m,k,n", [(100, 512, 192), (64, 160, 96), (2048, 256, 4096), (32, 96, 64), (7, 160, 96)])
def test_residual_segments_all_paths(orc, m, k, n):
    """Residual and per-segment scales through the decode (M <= 32) and both
    prefill tilings (64- and 128-row tiles: 2048 x 4096 fills the CUs with
    128-row tiles); K not a multiple of 128 is zero-padded."""
    print(f"residual m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m + 3 * k + n)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=n + 5)
    ends = [n // 2 - n // 2 % 32, n] if n >= 64 else [n]
    scales = [0.013, 0.029][: len(ends)]
    res = orc.f32_to_bf16(rng.standard_normal((m, n)).astype(np.float32))
    acc, out, a_dq, _ = run_gemm(orc, q, w, scales, ends, residual_bits=res)
    rows = np.arange(m) if m <= 128 else np.sort(rng.choice(m, 24, replace=False))
    ref = orc.gemm_i8t(np.ascontiguousarray(q[rows]), w)
    assert np.array_equal(acc[rows], ref)
    assert np.array_equal(out[rows], expected_out(orc, ref, a_dq[rows], scales, ends, 0, res[rows]))


@pytest.mark.parametrize("m,k,f", [(32, 256, 64), (32, 2560, 512), (5, 640, 96), (100, 256, 128)])
def test_relu2_epilogue(orc, m, k, f):
    rng = np.random.default_rng(m + k + f)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, 2 * f, seed=f)
    scales, ends = [0.021, 0.017], [f, 2 * f]
    acc, out, a_dq, _ = run_gemm(orc, q, w, scales, ends, epi=1)
    assert np.array_equal(acc, orc.gemm_i8t(q, w))
    assert np.array_equal(out, expected_out(orc, acc, a_dq, scales, ends, 1))


@pytest.mark.parametrize("m,k,n", [(33, 256, 128), (64, 512, 96), (100, 640, 160), (512, 256, 64)])
@pytest.mark.parametrize("rowsum", [False, True])
def test_prefill_gemm_bit_exact(orc, m, k, n, rowsum):
    print(f"prefill gemm m={m} k={k} n={n} rowsum={rowsum}", flush=True)
    rng = np.random.default_rng(m + k + n)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=n)
    acc, out, a_dq, _ = run_gemm(orc, q, w, [0.02], rowsum=rowsum)
    ref = orc.gemm_i8t(q, w)
    assert np.array_equal(acc, ref)
    assert np.array_equal(out, expected_out(orc, ref, a_dq, [0.02], [n], 0))


@pytest.mark.parametrize("m,k,f", [(70, 384, 96), (512, 256, 160), (129, 640, 32)])
@pytest.mark.parametrize("rowsum", [False, True])
def test_prefill_relu2_bit_exact(orc, m, k, f, rowsum):
    """relu2 prefill with F not a multiple of the 4 gate tiles of a workgroup."""
    print(f"prefill relu2 m={m} k={k} f={f} rowsum={rowsum}", flush=True)
    rng = np.random.default_rng(m * 7 + f)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, 2 * f, seed=f + 1)
    scales, ends = [0.021, 0.017], [f, 2 * f]
    acc, out, a_dq, _ = run_gemm(orc, q, w, scales, ends, epi=1, rowsum=rowsum)
    assert np.array_equal(acc, orc.gemm_i8t(q, w))
    assert np.array_equal(out, expected_out(orc, acc, a_dq, scales, ends, 1))


@pytest.mark.parametrize("m,k,n,epi", [(64, 2048, 256, 0), (100, 1536, 160, 0), (70, 2048, 192, 1), (130, 992, 96, 0),
                                       (33, 6912, 64, 0)])
def test_prefill_splitk_bit_exact(orc, m, k, n, epi):
    """Prefill grids smaller than the CU count split K between workgroups
    (given row sums); the last workgroup of a tile adds the others' exact
    partials.  Two calls in a row on one workspace, counters left at zero."""
    L = N.lib()
    assert int(L.btl_choose_splitk(m, k, n, epi)) > 1, "shape should take the split-K path"
    print(f"prefill split-K m={m} k={k} n={n} epi={epi}", flush=True)
    rng = np.random.default_rng(m * 3 + k)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=k + 7)
    scales = [0.02] if epi == 0 else [0.021, 0.017]
    ends = [n] if epi == 0 else [n // 2, n]
    d = H.dev()
    rows = 32 * ((m + 31) // 32)
    a_dq = np.zeros(rows, np.float32)
    a_dq[:m] = (0.005 + 0.03 * rng.random(m)).astype(np.float32)
    xa, a_dq_d, wdev = H.to_dev(H.rowmajor_to_xa(q)), H.to_dev(a_dq), device_weight(orc, w)
    rs_d = H.to_dev(q.astype(np.int64).sum(1).astype(np.int32))
    sc, en, nseg = N.segments_arrays(scales, ends)
    ws_bytes = int(L.btl_gemm_workspace_bytes(m, k, n, epi, 0))
    assert ws_bytes > 0
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=d)
    ref = orc.gemm_i8t(q, w)
    for call in range(2):
        n_out = n // 2 if epi == 1 else n
        out = torch.empty((m, n_out), dtype=torch.bfloat16, device=d)
        acc = torch.empty((m, n), dtype=torch.int32, device=d)
        N.check(L.btl_gemm_i8t2(N.ptr(xa), N.ptr(a_dq_d), N.ptr(rs_d), m, k, n, N.ptr(wdev), sc, en, nseg, epi, None,
                                N.ptr(out), N.ptr(acc), N.ptr(ws), ws.numel(), 0, N.stream_of(d)), "btl_gemm_i8t2")
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), ref), f"call {call}: accumulators"
        assert np.array_equal(H.bits_of(out), expected_out(orc, ref, a_dq[:m], scales, ends, epi)), f"call {call}: out"
        # the per-tile arrival counters lead the workspace (256 bytes here); the partials follow them
        assert not ws[:256].cpu().numpy().any(), f"call {call}: arrival counters not back at zero"


# Every prefill shape of the configured sweep (M in {512, 2048}; K = 2560 -> N in
# {3840, 6912, 2560}; 6912 -> 2560), with and without the activation kernel's
# row sums (split-K at M = 512 runs only with them), plus the gate||up pair.
PREFILL_SHAPES = [
    (512, 2560, 3840, 0, False), (512, 2560, 3840, 0, True),
    (512, 2560, 6912, 0, False), (512, 2560, 6912, 0, True),
    (512, 2560, 2560, 0, False), (512, 2560, 2560, 0, True),
    (512, 6912, 2560, 0, False), (512, 6912, 2560, 0, True),
    (2048, 2560, 3840, 0, False), (2048, 2560, 3840, 0, True),
    (2048, 2560, 6912, 0, True), (2048, 2560, 2560, 0, False), (2048, 2560, 2560, 0, True),
    (2048, 6912, 2560, 0, False), (2048, 6912, 2560, 0, True),
    (512, 2560, 13824, 1, True),
]


@pytest.mark.parametrize("m,k,n,epi,rowsum", PREFILL_SHAPES)
def test_prefill_full_size_properties(orc, m, k, n, epi, rowsum):
    """Full prefill shapes: every accumulator and every bf16 output exact,
    and every row and column checksum in int64."""
    print(f"prefill full m={m} k={k} n={n} epi={epi} rowsum={rowsum} splitk={N.lib().btl_choose_splitk(m, k, n, epi)}",
          flush=True)
    rng = np.random.default_rng(m + n + k)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=k + n)
    scales = [0.02] if epi == 0 else [0.02, 0.03]
    ends = [n] if epi == 0 else [n // 2, n]
    acc, out, a_dq, clean = run_gemm(orc, q, w, scales, ends, epi=epi, rowsum=rowsum)
    assert clean, "split-K arrival counters not back at zero"
    ref = full_acc_ref(orc, q, w, seed=m + n)
    bad = np.argwhere(acc != ref)
    assert bad.size == 0, f"{len(bad)} accumulators differ, first at {bad[0].tolist()}"
    q64, w64 = q.astype(np.int64), w.astype(np.int64)
    assert np.array_equal(acc.astype(np.int64).sum(1), q64 @ w64.sum(1))
    assert np.array_equal(acc.astype(np.int64).sum(0), q64.sum(0) @ w64)
    exp = expected_out(orc, ref, a_dq, scales, ends, epi)
    bad = np.argwhere(out != exp)
    assert bad.size == 0, f"{len(bad)} bf16 outputs differ, first at {bad[0].tolist()}"


# Wide-tile prefill (64-row x CT-column tiles, about two per CU; with the row
# sums given, scale epilogue, M >= 256).  The planner's choice on 256 CUs is
# listed per shape as (CT, tiles per wave CTW, k-step groups WQ); together
# they run every instantiated (CTW, WQ) pair, a ragged last row tile
# (M % 64 != 0), a ragged last column group (NT % CT != 0), K not a multiple
# of 128 and fewer superblocks than pipeline stages.
WIDE_SHAPES = [  # m, k, n, (CT, CTW, WQ)
    (300, 640, 2560, (1, 2, 4)),    # 5 superblocks, last row tile 44 rows
    (512, 384, 3840, (2, 2, 2)),    # 3 superblocks
    (1024, 2560, 2560, (3, 3, 4)),  # last column group 2 tiles
    (512, 992, 6912, (4, 2, 1)),    # last superblock 96 deep
    (2048, 2560, 2560, (5, 5, 4)),
    (2048, 512, 3072, (6, 3, 2)),
    (1000, 512, 6912, (7, 2, 1)),   # last row tile 40 rows, last column group 6 tiles
    (2048, 256, 5120, (10, 5, 2)),
    (2048, 256, 6144, (12, 3, 1)),
    (2000, 1056, 6880, (14, 4, 1)),  # last column group 5 tiles, last row tile 16 rows
]


@pytest.mark.parametrize("m,k,n,plan", WIDE_SHAPES)
def test_prefill_wide_tiles(orc, m, k, n, plan):
    """Every accumulator and every bf16 output exact (a residual and three
    weight-scale segments), every row and column checksum exact."""
    t = N.gemm_tiling(m, k, n)
    assert (t["kind"], t["col_tiles"], t["tiles_per_wave"], t["k_groups"]) == ("wide", *plan), t
    print(f"prefill wide m={m} k={k} n={n} tiling={t}", flush=True)
    rng = np.random.default_rng(m * 5 + k + n)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=k * 3 + n)
    ends = [n // 4 - n // 4 % 32, n // 2 - n // 2 % 32, n]
    scales = [0.013, 0.029, 0.021]
    res = orc.f32_to_bf16(rng.standard_normal((m, n)).astype(np.float32))
    acc, out, a_dq, _ = run_gemm(orc, q, w, scales, ends, residual_bits=res, rowsum=True)
    ref = full_acc_ref(orc, q, w, seed=m + k)
    assert np.array_equal(acc, ref)
    q64, w64 = q.astype(np.int64), w.astype(np.int64)
    assert np.array_equal(acc.astype(np.int64).sum(1), q64 @ w64.sum(1))
    assert np.array_equal(acc.astype(np.int64).sum(0), q64.sum(0) @ w64)
    assert np.array_equal(out, expected_out(orc, ref, a_dq, scales, ends, 0, res))


@pytest.mark.parametrize("m,k,n", [(2048, 2560, 3072), (1000, 512, 6912), (512, 1024, 2560)])
def test_prefill_tilings_agree(orc, m, k, n, monkeypatch):
    """The wide tiles and the 128x256 / 64x256 tiles (BTL_PREFILL_WIDE=0,
    read at every call) give the same accumulators and the same bf16 outputs,
    residual and three weight-scale segments included."""
    rng = np.random.default_rng(m + 11 * n)
    q = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    w = H.ternary(k, n, seed=n + 3)
    ends = [n // 4 - n // 4 % 32, n // 2 - n // 2 % 32, n]
    scales = [0.013, 0.029, 0.021]
    res = orc.f32_to_bf16(rng.standard_normal((m, n)).astype(np.float32))
    assert N.gemm_tiling(m, k, n)["kind"] == "wide"
    acc_w, out_w, _, _ = run_gemm(orc, q, w, scales, ends, residual_bits=res, rowsum=True)
    monkeypatch.setenv("BTL_PREFILL_WIDE", "0")
    assert N.gemm_tiling(m, k, n)["kind"] == "tiles"
    acc_t, out_t, _, _ = run_gemm(orc, q, w, scales, ends, residual_bits=res, rowsum=True)
    assert np.array_equal(acc_w, acc_t)
    assert np.array_equal(out_w, out_t)


@pytest.mark.parametrize("m", [512, 2048])
def test_prefill_gate_up_relu2_through_ternary_matmul(orc, m):
    """Prefill gate||up as the layer runs it: ternary_matmul (RMSNorm +
    absmax activation kernel, then the prefill GEMM with its row sums) on
    x ~ N(0, 1) with 1 % outlier channels and gate/up weights absmean-quantised
    from seeded N(0, 0.02) latents.  The quantised activations, every
    accumulator and every relu^2*up output are compared with the oracle bit
    for bit (64 rows through the oracle's whole BitLinear chain as well)."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    k, f = 2560, 6912
    print(f"prefill gate||up relu2 m={m} through ternary_matmul", flush=True)
    xb = H.activations(orc, m, k, seed=m + 3)
    gb = H.gamma(orc, k, seed=m + 4)
    gq, gs = orc.weight_quant_ternary(H.latent(f, k, seed=m + 5))
    uq, us = orc.weight_quant_ternary(H.latent(f, k, seed=m + 6))
    w = np.ascontiguousarray(np.concatenate([gq, uq]).T)  # (K, 2F)
    pw = PackedTernaryWeight(device_weight(orc, w), k, 2 * f, (float(gs), float(us)), (f, 2 * f))
    acc = torch.empty((m, 2 * f), dtype=torch.int32, device=H.dev())
    xq = torch.empty((m, k), dtype=torch.int8, device=H.dev())
    out = ternary_matmul(H.to_dev_bf16(xb), pw, norm_weight=H.to_dev_bf16(gb), norm_epsilon=1e-5,
                         epilogue="relu2_mul", acc_out=acc, xq_out=xq)
    torch.cuda.synchronize()
    y = orc.rmsnorm_bf16(xb, gb, 1e-5)
    q_ref, _, a_dq_ref, _ = orc.act_quant_absmax(orc.bf16_to_f32(y))
    q_got = xq.cpu().numpy()
    assert np.array_equal(q_got, q_ref), "quantised activations differ"
    a = acc.cpu().numpy().astype(np.int64)
    q64, w64 = q_ref.astype(np.int64), w.astype(np.int64)
    assert np.array_equal(a.sum(1), q64 @ w64.sum(1)), "row checksums"
    assert np.array_equal(a.sum(0), q64.sum(0) @ w64), "column checksums"
    rows = np.sort(np.random.default_rng(m).choice(m, 64, replace=False))
    ref = orc.gate_up_relu2(np.ascontiguousarray(xb[rows]), w, float(gs), float(us), gamma_bf16=gb, norm_eps=1e-5)
    assert np.array_equal(a[rows], ref["acc"]), "sampled accumulators"
    assert np.array_equal(H.bits_of(out)[rows], ref["h"]), "sampled relu^2*up outputs"
    full = full_acc_ref(orc, q_ref, w, seed=m)
    assert np.array_equal(a, full), "accumulators"
    exp = expected_out(orc, full, a_dq_ref, [float(gs), float(us)], [f, 2 * f], 1)
    assert np.array_equal(H.bits_of(out), exp), "relu^2*up outputs"


@pytest.mark.parametrize("m", [32, 100])
def test_fused_entry_matches_split_path(orc, m):
    """btl_bitlinear_fused == oracle: one launch at M = 32; at M = 100 the
    activation kernel and the prefill GEMM, which takes its row sums."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    print(f"fused entry m={m}", flush=True)
    k, n = 2560, 3840
    xb = H.activations(orc, m, k, seed=21)
    gb = H.gamma(orc, k, seed=22)
    w = H.ternary(k, n, seed=23)
    pw = PackedTernaryWeight(device_weight(orc, w), k, n, (0.017, 0.019, 0.023), (2560, 3200, 3840))
    acc = torch.empty((m, n), dtype=torch.int32, device=H.dev())
    xq = torch.empty((m, k), dtype=torch.int8, device=H.dev())
    ref = orc.bitlinear(xb, w, [0.017, 0.019, 0.023], [2560, 3200, 3840], gamma_bf16=gb, norm_eps=1e-5)
    for splitk in (0, 1, 2, 4):
        out = ternary_matmul(H.to_dev_bf16(xb), pw, norm_weight=H.to_dev_bf16(gb), norm_epsilon=1e-5,
                             splitk=splitk, acc_out=acc, xq_out=xq)
        torch.cuda.synchronize()
        assert np.array_equal(xq.cpu().numpy(), ref["q"])
        assert np.array_equal(acc.cpu().numpy(), ref["acc"])
        assert np.array_equal(H.bits_of(out), ref["out"])


def test_fused_decode_handshake_clean(orc):
    """The single-launch decode path (activation blocks + GEMM blocks) leaves its
    launch counters all equal (ready words of the 32 activation blocks and the
    512 GEMM slots, across calls with different GEMM grids) and never reports
    a timed-out wait."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    for m, k, n, epi in [(32, 2560, 3840, "none"), (5, 6912, 2560, "none"), (32, 2560, 1024, "relu2_mul")]:
        xb = H.activations(orc, m, k, seed=m + k)
        w = H.ternary(k, n, seed=n)
        ends = (n // 2, n) if epi == "relu2_mul" else (n,)
        pw = PackedTernaryWeight(device_weight(orc, w), k, n, (0.02,) * len(ends), ends)
        ref = orc.bitlinear(xb, w, [0.02] * len(ends), list(ends))
        exp = ref["out"] if epi == "none" else orc.relu2_mul_bf16(ref["out"][:, : n // 2], ref["out"][:, n // 2:])
        for rep in range(6):  # every call checked: a row published before its stores landed shows up as one bad call
            out = ternary_matmul(H.to_dev_bf16(xb), pw, epilogue=epi)
            torch.cuda.synchronize()
            bad = [i for i in range(m) if not np.array_equal(H.bits_of(out)[i], exp[i])]
            assert not bad, f"m={m} k={k} n={n} call {rep}: rows {bad} differ"
    err = int(N.lib().btl_fused_error_offset())
    for key, ws in N._workspaces.items():
        if key[0] != "bitlinear":
            continue  # decode-layer workspaces keep launch counters
        words = ws[:8192].view(torch.int32).cpu().numpy()
        assert words[err // 4] == 0, "a bounded wait ran out"
        ready_idx = np.arange(32) * 32  # one per 128-byte line
        ready = words[ready_idx]
        seen = words[33 * 32:33 * 32 + 512]
        assert ready.min() == ready.max() == seen.min() == seen.max() > 0, "launch counters out of step"
        rest = words.copy()
        rest[ready_idx] = 0
        rest[33 * 32:33 * 32 + 512] = 0
        assert not rest.any(), "stray handshake words"


@pytest.mark.parametrize("m,k,n,epi", [(32, 2560, 2560, "none"), (17, 6912, 2560, "none"), (24, 2560, 640, "none"),
                                        (32, 6912, 96, "none"), (32, 2560, 3840, "qkv"), (17, 2560, 3840, "qkv"),
                                        (32, 2560, 13824, "relu2_mul"), (19, 2560, 13824, "relu2_mul"),
                                        (32, 2560, 1024, "relu2_mul"), (24, 2560, 1024, "relu2_mul"),
                                        (16, 2560, 3840, "qkv"), (1, 6912, 2560, "none"), (8, 2560, 13824, "relu2_mul"),
                                        (13, 2560, 2560, "none"), (16, 6912, 96, "none")])
def test_fused_row_halves_bit_exact(orc, m, k, n, epi):
    """Single-launch BitLinear on the 16-row body.  At M <= 16 one GEMM
    workgroup per column group takes rows 0..15 (every shape).  With more
    than 16 rows two take each column group, one per 16-row half, in these
    cases:
    - the o_proj and down shapes of the 2B model (one column tile a group,
      scale and residual epilogue);
    - fused QKV (two tiles a group, three scale segments);
    - gate||up at 1024 (one gate/up pair a group, relu2 epilogue).
    The 2B gate||up shape keeps whole-tile workgroups.  In every case the int8
    rows, int32 accumulators and bf16 outputs equal the oracle's, also for the
    rows of a half that stops at M.  The two calls take different inputs (a
    half that read the first call's rows after a timed-out wait would fail),
    and no bounded wait runs out."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    print(f"row halves m={m} k={k} n={n} {epi}", flush=True)
    gb = H.gamma(orc, k, seed=n + 3)
    w = H.ternary(k, n, seed=k + 5)
    if epi == "relu2_mul":
        scales, ends = [0.0173, 0.0191], [n // 2, n]
    elif epi == "qkv":
        scales, ends = [0.0173, 0.0191, 0.0229], [2560, 3200, 3840]
    else:
        scales, ends = [0.0173], [n]
    res = H.activations(orc, m, n, seed=n + 11) if epi == "none" else None
    pw = PackedTernaryWeight(device_weight(orc, w), k, n, tuple(scales), tuple(ends))
    acc = torch.empty((m, n), dtype=torch.int32, device=H.dev())
    xq = torch.empty((m, k), dtype=torch.int8, device=H.dev())
    kw = dict(residual=H.to_dev_bf16(res)) if res is not None else {}
    for rep in range(2):
        xb = H.activations(orc, m, k, seed=m + k + 7 + 1000 * rep)
        ref = orc.bitlinear(xb, w, scales, ends, gamma_bf16=gb, norm_eps=1e-5, residual_bf16=res)
        exp = ref["out"] if epi != "relu2_mul" else orc.relu2_mul_bf16(ref["out"][:, : n // 2], ref["out"][:, n // 2:])
        out = ternary_matmul(H.to_dev_bf16(xb), pw, norm_weight=H.to_dev_bf16(gb), norm_epsilon=1e-5,
                             epilogue="relu2_mul" if epi == "relu2_mul" else "none", acc_out=acc, xq_out=xq, **kw)
        torch.cuda.synchronize()
        assert np.array_equal(xq.cpu().numpy(), ref["q"]), f"call {rep}: int8 rows differ"
        assert np.array_equal(acc.cpu().numpy(), ref["acc"]), f"call {rep}: accumulators differ"
        assert np.array_equal(H.bits_of(out), exp), f"call {rep}: outputs differ"
    N.check_errors(H.dev())  # raises if a bounded wait of these calls ran out


def test_fused_workspace_shared_across_shapes(orc):
    """One stream's workspace carries calls of different K, M and N, with a
    prefill call (M > 32, the split path) in between: a shorter row before a
    longer one, or the split path's own buffers, never leave bytes or counters
    that a later launch takes for its own."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    seq = [(32, 2560, 512, None), (32, 6912, 256, "g"), (5, 2560, 384, "g"), (64, 2560, 256, "g"),
           (32, 8192, 256, "g"), (1, 6912, 512, None), (32, 2560, 512, "g"), (31, 4096, 256, None)]
    for i, (m, k, n, norm) in enumerate(seq):
        xb = H.activations(orc, m, k, seed=100 + i)
        gb = H.gamma(orc, k, seed=200 + i) if norm else None
        w = H.ternary(k, n, seed=300 + i)
        pw = PackedTernaryWeight(device_weight(orc, w), k, n, (0.021,), (n,))
        acc = torch.empty((m, n), dtype=torch.int32, device=H.dev())
        kw = dict(norm_weight=H.to_dev_bf16(gb), norm_epsilon=1e-5) if norm else {}
        print(f"call {i}: M={m} K={k} N={n} norm={bool(norm)}", flush=True)
        out = ternary_matmul(H.to_dev_bf16(xb), pw, acc_out=acc, **kw)
        torch.cuda.synchronize()
        ref = orc.bitlinear(xb, w, [0.021], [n], gamma_bf16=gb, norm_eps=1e-5)
        assert np.array_equal(acc.cpu().numpy(), ref["acc"]), f"call {i}: accumulators differ"
        assert np.array_equal(H.bits_of(out), ref["out"]), f"call {i}: outputs differ"
    err = int(N.lib().btl_fused_error_offset())
    for key, ws in N._workspaces.items():
        if key[0] == "bitlinear":
            assert int(ws[:8192].view(torch.int32)[err // 4]) == 0, "a bounded wait ran out"


def test_check_raises_on_sticky_error_word(orc):
    """check() reads the fused workspace's sticky error word: set from the host
    (as a timed-out wait would set it), it raises RuntimeError and leaves the
    workspace zero-filled, so the next call computes correct results."""
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, check, ternary_matmul

    m, k, n = 32, 512, 256
    xb = H.activations(orc, m, k, seed=5)
    w = H.ternary(k, n, seed=6)
    pw = PackedTernaryWeight(device_weight(orc, w), k, n, (0.02,), (n,))
    ref = orc.bitlinear(xb, w, [0.02])
    out = ternary_matmul(H.to_dev_bf16(xb), pw)
    check()  # clean
    key = next(key for key in N._workspaces if key[0] == "bitlinear" and key[1] == str(H.dev()))
    ws = N._workspaces[key]
    off = int(N.lib().btl_fused_error_offset())
    ws[off:off + 4].view(torch.int32).fill_(1)
    with pytest.raises(RuntimeError, match="bounded wait ran out"):
        check()
    assert not ws.cpu().numpy().any(), "workspace not reset"
    out = ternary_matmul(H.to_dev_bf16(xb), pw)
    check()
    assert np.array_equal(H.bits_of(out), ref["out"])


def test_check_after_call_raises_at_the_call(orc):
    """Check-after-call mode: a call whose launch finds the error word set (as
    a bounded wait that ran out sets it; here set from the host) raises
    RuntimeError at that call, as the reference's op raises at its call; the
    workspace is reset and the next call returns the oracle's bits."""
    from bitnet_tt.layers.bitlinear import Linear
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    m, k, n = 32, 512, 256
    xb = H.activations(orc, m, k, seed=15)
    w = H.ternary(k, n, seed=16)
    pw = PackedTernaryWeight(device_weight(orc, w), k, n, (0.02,), (n,))
    ref = orc.bitlinear(xb, w, [0.02])
    out = ternary_matmul(H.to_dev_bf16(xb), pw, check_errors=True)
    assert np.array_equal(H.bits_of(out), ref["out"])
    key = next(key for key in N._workspaces if key[0] == "bitlinear" and key[1] == str(H.dev()))
    ws = N._workspaces[key]
    off = int(N.lib().btl_fused_error_offset())
    ws[off:off + 4].view(torch.int32).fill_(1)
    with pytest.raises(RuntimeError, match="bounded wait ran out"):
        ternary_matmul(H.to_dev_bf16(xb), pw, check_errors=True)
    out = ternary_matmul(H.to_dev_bf16(xb), pw, check_errors=True)
    assert np.array_equal(H.bits_of(out), ref["out"])
    lin = Linear(k, n, H.dev(), check_errors=True)
    lin.load_pretransposed_weight(w.astype(np.float32), scale=0.02)
    ws[off:off + 4].view(torch.int32).fill_(1)
    with pytest.raises(RuntimeError, match="bounded wait ran out"):
        lin(H.to_dev_bf16(xb))
    assert np.array_equal(H.bits_of(lin(H.to_dev_bf16(xb))), ref["out"])


def _hip():
    import ctypes

    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    pytest.skip("libamdhip64 not found")


def test_cu_masked_stream_coresidency(orc):
    """A stream limited to 32 CUs (hipExtStreamCreateWithCUMask): the
    persistent step (one workgroup per CU of the device, all waiting on each
    other) is refused with RuntimeError before anything is launched, and the
    fused decode BitLinear, whose one-launch grid does not fit there, takes
    its two-launch path and returns the oracle's bits."""
    import ctypes

    from bitnet_tt.config import BitNetMiniConfig
    from bitnet_tt.decode import BitLinearDecodeStep
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    hip = _hip()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    words = (cus + 31) // 32
    mask = (ctypes.c_uint32 * words)(*([0xFFFFFFFF] + [0] * (words - 1)))
    raw = ctypes.c_void_p()
    assert hip.hipExtStreamCreateWithCUMask(ctypes.byref(raw), ctypes.c_uint32(words), mask) == 0
    try:
        back = (ctypes.c_uint32 * words)()
        assert hip.hipExtStreamGetCUMask(raw, ctypes.c_uint32(words), back) == 0
        if sum(bin(v).count("1") for v in back) != 32:
            pytest.skip("the runtime does not report the stream's CU mask")
        s = torch.cuda.ExternalStream(raw.value)
        m, k, f = 32, 2560, 6912
        xb = H.activations(orc, m, k, seed=21)
        gq, uq = H.ternary(f, k, seed=22), H.ternary(f, k, seed=23)
        w = np.ascontiguousarray(np.concatenate([gq, uq]).T)
        pw = PackedTernaryWeight(device_weight(orc, w), k, 2 * f, (0.02, 0.03), (f, 2 * f))
        ref = orc.gate_up_relu2(xb, w, 0.02, 0.03)
        step = BitLinearDecodeStep.random_init(BitNetMiniConfig(num_layers=1), H.dev(), seed=24).alloc_buffers(seed=25)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            out = ternary_matmul(H.to_dev_bf16(xb), pw, epilogue="relu2_mul", check_errors=True)
            s.synchronize()
            assert np.array_equal(H.bits_of(out), ref["h"])
            with pytest.raises(RuntimeError, match="fit at once"):
                step.step_persistent()
        s.synchronize()
    finally:
        torch.cuda.synchronize()
        hip.hipStreamDestroy(raw)
