"""The C ABI of libbtl.so (CPU only: loading, exports, sizes, argument checks).

No call here reaches a kernel launch: the size helpers are host arithmetic and
every argument-check case is rejected before the library touches HIP.
"""

import ctypes
import os
import re
import subprocess
import sys

import pytest

from bitnet_tt import _native as N

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "btl.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int64_t|int)\s+(btl_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def L():
    return N.lib()


def test_library_loads_and_exports_every_declaration(L):
    names = declared_functions()
    assert len(names) >= 17
    for name in names:
        assert hasattr(L, name), f"{name} declared in include/btl.h but not exported"
        assert name in N.EXPORTS, f"{name} has no ctypes signature"
    assert set(N.EXPORTS) == set(names)
    assert L.btl_version() == 200
    assert L.btl_fused_error_offset() % 4 == 0 and 0 < L.btl_fused_error_offset() < 8192


def test_size_helpers(L):
    assert L.btl_packed_tile_count(2560, 6912) == 80 * 216
    assert L.btl_packed_dram_bytes(2560, 2560) == 6400 * 256
    assert L.btl_packed_tile_count(50, 100) == 8
    assert L.btl_devlayout_words(2560, 3840) == 120 * 20 * 256
    assert L.btl_devlayout_words(6912, 2560) == 80 * 54 * 256
    assert L.btl_devlayout_words(96, 64) == 2 * 1 * 256
    assert L.btl_devlayout_words(64, 33) == 0
    assert L.btl_act_bytes(32, 2560) == 20 * 4096
    assert L.btl_act_bytes(33, 2560) == 2 * 20 * 4096
    assert L.btl_weight_quant_scratch_bytes(8193) == 8
    # device layout is exactly 2 bits per weight when K % 128 == 0
    assert L.btl_devlayout_words(2560, 2560) * 4 == L.btl_packed_dram_bytes(2560, 2560)


def test_split_k_plans(L):
    # decode shapes of the 2B model: about one workgroup per CU
    assert L.btl_choose_splitk(32, 2560, 3840, 0) == 2
    assert L.btl_choose_splitk(32, 2560, 2560, 0) == 3
    assert L.btl_choose_splitk(32, 2560, 13824, 1) == 1
    assert L.btl_choose_splitk(32, 6912, 2560, 0) == 3
    assert L.btl_choose_splitk(2048, 2560, 6912, 0) == 1  # prefill: no split
    assert L.btl_gemm_workspace_bytes(32, 2560, 13824, 1, 0) == 0
    assert L.btl_gemm_workspace_bytes(32, 2560, 3840, 0, 0) > 2 * 120 * 4096
    assert L.btl_fused_workspace_bytes(32, 2560, 3840, 0, 0) > L.btl_act_bytes(32, 2560)
    # a split request larger than K allows is capped (one superblock per wave)
    assert L.btl_choose_splitk(32, 256, 64, 0) == 1


def test_gemm_tiling_query(L):
    t = N.gemm_tiling
    # 2048 x 2560 -> N on 256 CUs: 64-row tiles, 16 column groups (two tiles a CU)
    assert t(2048, 2560, 6912) == {"kind": "wide", "rows": 64, "col_tiles": 14, "splitk": 1, "k_groups": 1,
                                   "tiles_per_wave": 4}
    assert t(2048, 2560, 2560) == {"kind": "wide", "rows": 64, "col_tiles": 5, "splitk": 1, "k_groups": 4,
                                   "tiles_per_wave": 5}
    assert t(512, 2560, 3840)["col_tiles"] == 2
    # without row sums, for relu2 and below 256 rows: the 128x256 / 64x256 tiles
    assert t(2048, 2560, 6912, rowsum_given=False)["kind"] == "tiles"
    assert t(2048, 2560, 13824, N.EPI_RELU2_MUL)["kind"] == "tiles"
    assert t(100, 1536, 160)["kind"] == "tiles" and t(100, 1536, 160)["splitk"] > 1
    assert t(32, 2560, 3840) == {"kind": "decode", "rows": 32, "col_tiles": 1, "splitk": 2, "k_groups": 0,
                                 "tiles_per_wave": 0}
    with pytest.raises(RuntimeError):
        t(64, 100, 64)


def test_gemm_tiling_invariants():
    """Over a sweep of prefill shapes: a wide plan's wave ranges cover its
    column tiles (spans of CT / (4 / WQ) tiles, at most CTW each), CTW is an
    instantiated size, and shapes the wide tiles do not take fall back to
    the 128x256 / 64x256 tiles."""
    for m in (256, 300, 512, 777, 1024, 2048, 4096, 8192):
        for n in (32, 96, 640, 2560, 3072, 3840, 5120, 6912, 8192, 13824):
            for k in (256, 2560, 6912):
                t = N.gemm_tiling(m, k, n)
                if t["kind"] == "tiles":
                    assert t["rows"] in (64, 128)
                    continue
                assert t["kind"] == "wide" and t["rows"] == 64 and t["splitk"] == 1
                ct, wq, ctw = t["col_tiles"], t["k_groups"], t["tiles_per_wave"]
                assert wq in (1, 2, 4) and ctw in ((2, 3, 4) if wq == 1 else (2, 3, 5)), t
                parts = 4 // wq
                assert 1 <= ct and -(-ct // parts) <= ctw, t
                # about two tiles per CU on 256 CUs, at least one
                tiles = -(-m // 64) * -(-(n // 32) // ct)
                assert tiles <= 2 * 256, t


FAKE = 0x100000  # never dereferenced: every call below is rejected first


def _p(x):
    return ctypes.c_void_p(x)


def call_gemm(L, **kw):
    a = dict(xa=_p(FAKE), a_dq=_p(FAKE), rowsum=None, M=32, K=256, N=64, wdev=_p(FAKE), nseg=1, epi=0,
             residual=None, out=_p(FAKE), acc=None, ws=None, ws_bytes=0, splitk=1)
    a.update(kw)
    sc = (ctypes.c_float * 4)(1.0, 1.0, 1.0, 1.0)
    en = (ctypes.c_int64 * 4)(*(kw.get("ends") or (a["N"], a["N"], a["N"], a["N"])))
    return L.btl_gemm_i8t2(a["xa"], a["a_dq"], a["rowsum"], a["M"], a["K"], a["N"], a["wdev"], sc, en, a["nseg"],
                           a["epi"], a["residual"], a["out"], a["acc"], a["ws"], a["ws_bytes"], a["splitk"], None)


def test_gemm_argument_checks(L):
    assert call_gemm(L, xa=None) == 1
    assert call_gemm(L, wdev=None) == 1
    assert call_gemm(L, K=250) == 2
    assert call_gemm(L, N=48) == 2
    assert call_gemm(L, K=32768) == 2
    assert call_gemm(L, M=0) == 2
    assert call_gemm(L, epi=7) == 5
    assert call_gemm(L, epi=1, N=96) == 2  # relu2 needs N = 2F with F % 32 == 0
    assert call_gemm(L, nseg=0) == 5
    assert call_gemm(L, nseg=2, N=64, ends=(16, 64, 0, 0)) == 5  # not a multiple of 32
    assert call_gemm(L, nseg=2, N=64, ends=(32, 96, 0, 0)) == 5  # last end != N
    assert call_gemm(L, wdev=_p(FAKE + 4)) == 3
    assert "16-byte" in N.last_error()
    assert call_gemm(L, xa=_p(FAKE + 8)) == 3
    assert "misaligned" in N.last_error()
    assert call_gemm(L, M=64, rowsum=_p(FAKE + 2)) == 3
    assert "rowsum" in N.last_error()
    # split-K needs a workspace of the advertised size
    assert call_gemm(L, M=32, K=2560, N=3840, splitk=2, ws=None) == 1
    assert call_gemm(L, M=32, K=2560, N=3840, splitk=2, ws=_p(FAKE), ws_bytes=16) == 4
    assert call_gemm(L, splitk=-1) == 5
    assert "splitk" in N.last_error()


def test_fused_and_prep_argument_checks(L):
    sc = (ctypes.c_float * 1)(1.0)
    en = (ctypes.c_int64 * 1)(64)
    f = L.btl_bitlinear_fused
    args = [_p(FAKE), 32, 256, 256, None, 1e-5, _p(FAKE), 64, sc, en, 1, 0, None, _p(FAKE), None, None, _p(FAKE),
            1 << 20, 0, None]
    bad = list(args)
    bad[0] = None
    assert f(*bad) == 1
    bad = list(args)
    bad[3] = 250  # ldx < K
    assert f(*bad) == 3
    bad = list(args)
    bad[16] = None  # workspace
    assert f(*bad) == 1
    bad = list(args)
    bad[17] = 64  # workspace too small
    assert f(*bad) == 4
    bad = list(args)
    bad[4] = _p(FAKE + 2)  # misaligned gamma
    assert f(*bad) == 3
    assert L.btl_quant_absmax(_p(FAKE), 32, 100, 104, None, 0.0, _p(FAKE), _p(FAKE), _p(FAKE), None, None, None,
                              None) == 2
    assert L.btl_quant_absmax(_p(FAKE), 32, 256, 256, None, 0.0, None, _p(FAKE), _p(FAKE), None, None, None,
                              None) == 1
    assert L.btl_rmsnorm(_p(FAKE), 4, 256, 256, None, 1e-5, None, None) == 1
    assert L.btl_repack(_p(FAKE), 100, 64, _p(FAKE), None) == 2
    assert L.btl_repack(_p(FAKE), 128, 64, _p(FAKE + 4), None) == 3
    assert L.btl_pack_tiles(None, 32, 32, _p(FAKE), None) == 1
    assert L.btl_unpack_tiles(_p(FAKE), 0, 32, _p(FAKE), None) == 2
    assert L.btl_weight_quant_ternary(_p(FAKE), 100, 1e-5, _p(FAKE), _p(FAKE), _p(FAKE), 0, None) == 4


def test_python_errors_are_loud(L):
    torch = pytest.importorskip("torch")
    from bitnet_tt.ternary_matmul import PackedTernaryWeight, ternary_matmul

    w = PackedTernaryWeight(torch.zeros((2, 2, 256), dtype=torch.int32), 256, 64)
    with pytest.raises(ValueError, match="ROCm GPU"):
        ternary_matmul(torch.zeros((32, 256), dtype=torch.bfloat16), w)
    with pytest.raises(RuntimeError, match="BTL_ERR_SHAPE"):
        N.check(2, "probe")


def test_decode_step_sizes_and_argument_checks(L):
    # one hand-off region reused by every layer: the workspace does not grow with L
    ws1 = L.btl_decode_step_workspace_bytes(32, 2560, 6912, 3840, 1)
    ws30 = L.btl_decode_step_workspace_bytes(32, 2560, 6912, 3840, 30)
    tiles = 32 * (3 * 2560 + 6912)
    words = 32 * (3840 + 2560 + 6912 + 2560) // 2 * 8
    assert ws1 == ws30 and ws30 >= tiles + words + 4 * 32 * 128
    assert L.btl_decode_step_workspace_bytes(33, 2560, 6912, 3840, 30) == 0
    assert L.btl_decode_step_workspace_bytes(32, 2560, 6912, 3840, 65) == 0
    assert L.btl_decode_step_error_offset() % 4 == 0 and 0 < L.btl_decode_step_error_offset() < ws30

    def step(M=32, H=2560, F=6912, NQ=3840, nl=30, attn=FAKE, ws_bytes=1 << 28):
        return L.btl_decode_step(M, H, F, NQ, nl, 1e-5, _p(attn) if attn else None, _p(FAKE), _p(FAKE), _p(FAKE),
                                 _p(FAKE), ws_bytes, None)

    # every case below fails a shape check that runs before the library touches HIP
    assert step(M=0) == 2 and step(M=33) == 2
    assert step(nl=0) == 2 and step(nl=65) == 2
    assert step(H=2500) == 2 and step(NQ=3850) == 2
    assert step(F=8192) == 2  # 64 superblocks of K = F exceed the down projection's weight registers
    assert "weight registers" in N.last_error()
    assert step(H=3200) == 2  # 25 superblocks of K = H exceed three register slots
    table = (N.LayerWeight * 4)()
    assert L.btl_decode_step_prepare(0, 2560, 6912, 3840, 1, table, _p(FAKE), 1 << 28) == 2


def test_coresidency_rule(L):
    """The rule the fused one-launch decode path and the persistent step apply
    before launching (their workgroups wait on each other): the grid must fit
    on the stream's CUs at once, occupancy x CUs.  A refusal is an error with a
    message, never a launch that would wait for workgroups that cannot run."""
    assert L.btl_check_coresident(256, 1, 256) == 0
    assert L.btl_check_coresident(280, 2, 256) == 0
    assert L.btl_check_coresident(257, 1, 256) == 6
    msg = N.last_error()
    assert "257 workgroups" in msg and "only 256 fit" in msg
    assert L.btl_check_coresident(256, 1, 64) == 6  # a stream masked to 64 CUs
    assert L.btl_check_coresident(10, 0, 256) == 6  # the kernel fits no workgroup at all
    assert "no workgroup" in N.last_error()


def test_check_after_call_mode():
    """The opt-in check-after-call mode: off by default, switched by
    set_check_after_call or BTL_CHECK_AFTER_CALL, and carried per layer."""
    from bitnet_tt import ternary_matmul as T
    from bitnet_tt.layers.bitlinear import Linear

    assert T.check_after_call_enabled() is False
    T.set_check_after_call(True)
    try:
        assert T.check_after_call_enabled() is True
    finally:
        T.set_check_after_call(False)
    code = "from bitnet_tt import ternary_matmul as T; print(T.check_after_call_enabled())"
    env = dict(os.environ, BTL_CHECK_AFTER_CALL="1",
               PYTHONPATH=os.pathsep.join([os.path.join(REPO, "bitnet-tt_amd"), REPO]))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.stdout.strip() == "True", r.stderr
    assert Linear(64, 64, check_errors=True).check_errors is True
    assert Linear(64, 64).check_errors is None


def test_noalloc_scratch_holds_every_decode_shape(L):
    """The header's promise for btl_bitlinear_fused_noalloc: every decode shape
    (M <= 32, K and N multiples of 32 up to 16384, either epilogue, no split-K
    request) has a workspace within BTL_NOALLOC_SCRATCH_BYTES."""
    text = open(HEADER).read()
    limit = eval(re.search(r"#define BTL_NOALLOC_SCRATCH_BYTES \((\d+ << \d+)\)", text).group(1))
    worst = 0
    for epi, step in ((0, 32), (1, 64)):
        for k in range(32, 16385, 32):
            for n in range(step, 16385, step):
                worst = max(worst, L.btl_fused_workspace_bytes(32, k, n, epi, 0))
    assert 0 < worst <= limit, (worst, limit)
    # M below 32 uses the same 32-row blocks
    assert L.btl_fused_workspace_bytes(1, 16288, 8192, 0, 0) <= limit
    # a prefill shape does not fit, and is refused by the entry point (GPU test)
    assert L.btl_fused_workspace_bytes(2048, 6912, 2560, 0, 0) > limit


def _line_rows(ln):
    """Rows whose operand bytes line ln of a step tile holds (row r at bytes
    32 r .. 32 r + 31 of each 1 KiB block)."""
    return {(ln * 128 % 1024 + b) // 32 for b in range(0, 128, 32)}


def _clear_share(L, m, KS):
    out = (ctypes.c_int64 * (16 * KS))()
    assert L.btl_decode_step_clear_share(m, KS, out, 16 * KS) == 0
    return list(out)


@pytest.mark.parametrize("KS", [1, 3, 20, 54])
def test_decode_step_tile_clear_shares(L, KS):
    """The persistent step's between-use clears of an operand tile (the
    function the kernel calls).  Operand layout of a tile: in each 1 KiB
    k-step block, row r's 32 bytes (both k-groups) start at offset 32 r, so a
    128-byte line holds rows of one 4-row group.  Each row's share must lie in
    whole lines of its own 16-row half (a row of the other half may already be
    writing the tile's next use), be 8-byte aligned, and the 32 shares must
    cover the tile's 32*KS*128 bytes exactly once."""
    tile_bytes = 32 * KS * 128
    seen = {}
    for m in range(32):
        offs = _clear_share(L, m, KS)
        lines = {o // 128 for o in offs}
        assert len(lines) == KS  # whole lines: 16 pieces of 8 bytes each
        for o in offs:
            assert o % 8 == 0 and 0 <= o < tile_bytes
            assert o not in seen, f"piece {o} cleared by rows {seen[o]} and {m}"
            seen[o] = m
        for ln in lines:
            rows = _line_rows(ln)
            assert {r >> 4 for r in rows} == {m >> 4}, f"row {m} clears line {ln} holding rows {sorted(rows)}"
    assert len(seen) == tile_bytes // 8
    # argument checks
    out = (ctypes.c_int64 * 4)()
    assert L.btl_decode_step_clear_share(32, KS, out, 4) == 5
    assert L.btl_decode_step_clear_share(0, 0, out, 4) == 5
    assert L.btl_decode_step_clear_share(0, KS, None, 4) == 1


def test_decode_step_tile_clear_planted_mistake_is_caught(L):
    """The coverage check above fails for a share map that splits the tile
    into 32 contiguous ranges (lines shared by both halves)."""
    KS = 20
    bad = {m: [m * KS * 128 + 8 * pc for pc in range(16 * KS)] for m in range(32)}
    crossing = 0
    for m, offs in bad.items():
        for ln in {o // 128 for o in offs}:
            rows = _line_rows(ln)
            crossing += {r >> 4 for r in rows} != {m >> 4}
    assert crossing > 0


def test_lm_head_sizes_and_argument_checks(L):
    # 16 vocab rows x 32 k per KiB, K padded to the supported multiple of 256
    assert L.btl_lm_head_weight_bytes(128256, 2560) == 128256 * 2560 * 2
    assert L.btl_lm_head_weight_bytes(37, 272) == 3 * 16 * 512 * 2  # 3 tiles, K 272 -> 512
    assert L.btl_lm_head_weight_bytes(1000, 100) == 0  # K % 16
    assert L.btl_lm_head_weight_bytes(1000, 4096) == 0  # K > 3072
    assert L.btl_lm_head_workspace_bytes() == 512
    SHAPE, NULL, ALIGN, WS = 2, 1, 3, 4

    def call(M=32, K=2560, V=128256, xn=FAKE, w=FAKE, logits=FAKE, tok=FAKE, ws=FAKE, nbytes=512):
        return L.btl_lm_head(xn, M, K, V, w, logits, tok, ws, nbytes, None)

    assert call(M=0) == SHAPE
    assert call(M=33) == SHAPE
    assert call(K=100) == SHAPE
    assert call(V=0) == SHAPE
    assert call(xn=None) == NULL
    assert call(tok=None) == NULL
    assert call(ws=None) == NULL
    assert call(xn=FAKE + 4) == ALIGN
    assert call(nbytes=100) == WS
    assert L.btl_lm_head_repack(None, 100, 256, FAKE, None) == NULL
    assert L.btl_lm_head_repack(FAKE, 100, 250, FAKE, None) == SHAPE
