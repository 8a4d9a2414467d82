"""btl_bitlinear_fused_noalloc (the entry point that allocates nothing) against
btl_bitlinear_fused on the same inputs, through the C ABI.

Two calls in a row share the library's static scratch, the second with a
smaller input; a third call takes the prefill path (M > 32: activation kernel
then the prefill GEMM, both on the scratch).  Outputs, exact accumulators and
quantised activations must equal the workspace entry point's bit for bit, and
the caller's error word must stay zero.  A shape whose workspace exceeds the
scratch is refused with BTL_ERR_WORKSPACE before anything is launched.

The entry point is for callers that cannot allocate, graph capture among
them: the first test captures a call in a HIP graph (in a fresh process that
call is the library's first on the device, so the graph also records the
fill kernel that clears the scratch) and replays it, with eager calls of both
entry points on other inputs in between, against the workspace entry point's
eager result.  It runs first in this file so that, in a fresh process, the
captured call is the first one."""

import ctypes

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N

pytestmark = pytest.mark.gpu


def _weight(orc, k, n, seed):
    w = H.ternary(k, n, seed=seed)
    return w, H.to_dev(orc.devlayout_encode(w).view(np.int32))


def _call(L, noalloc, x, m, k, gamma, wdev, n, scales, ends, epi, residual, err_word):
    d = H.dev()
    sc, en, nseg = N.segments_arrays(scales, ends)
    n_out = n // 2 if epi == N.EPI_RELU2_MUL else n
    out = torch.empty((m, n_out), dtype=torch.bfloat16, device=d)
    if residual is not None:
        out.copy_(residual)
    acc = torch.empty((m, n), dtype=torch.int32, device=d)
    xq = torch.empty((m, k), dtype=torch.int8, device=d)
    res_ptr = N.ptr(out) if residual is not None else None
    stream = N.stream_of(d)
    if noalloc:
        rc = L.btl_bitlinear_fused_noalloc(N.ptr(x), m, k, k, N.ptr(gamma), 1e-5, N.ptr(wdev), n, sc, en, nseg, epi,
                                           res_ptr, N.ptr(out), N.ptr(acc), N.ptr(xq), N.ptr(err_word), 0, stream)
        N.check(rc, "btl_bitlinear_fused_noalloc")
    else:
        nbytes = int(L.btl_fused_workspace_bytes(m, k, n, epi, 0))
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=d)
        rc = L.btl_bitlinear_fused(N.ptr(x), m, k, k, N.ptr(gamma), 1e-5, N.ptr(wdev), n, sc, en, nseg, epi, res_ptr,
                                   N.ptr(out), N.ptr(acc), N.ptr(xq), N.ptr(ws), ws.numel(), 0, stream)
        N.check(rc, "btl_bitlinear_fused")
        torch.cuda.synchronize()
        off = int(L.btl_fused_error_offset())
        assert int(ws[off:off + 4].view(torch.int32).item()) == 0
    torch.cuda.synchronize()
    return H.bits_of(out), acc.cpu().numpy(), xq.cpu().numpy()


def test_noalloc_under_graph_capture(orc):
    L = N.lib()
    d = H.dev()
    m, k, n = 32, 2560, 3840
    scales, ends = [0.017, 0.019, 0.023], [2560, 3200, 3840]
    err_word = torch.zeros(1, dtype=torch.int32, device=d)
    xb, gb = H.activations(orc, m, k, seed=910), H.gamma(orc, k, seed=911)
    w, wdev = _weight(orc, k, n, seed=912)
    x, g = H.to_dev_bf16(xb), H.to_dev_bf16(gb)
    ref = _call(L, False, x, m, k, g, wdev, n, scales, ends, N.EPI_SCALE, None, err_word)
    # other inputs for the eager calls between replays (they share the static scratch)
    xb2 = H.activations(orc, m, k, seed=913)
    x2 = H.to_dev_bf16(xb2)
    ref2 = _call(L, False, x2, m, k, g, wdev, n, scales, ends, N.EPI_SCALE, None, err_word)

    out = torch.empty((m, n), dtype=torch.bfloat16, device=d)
    acc = torch.empty((m, n), dtype=torch.int32, device=d)
    xq = torch.empty((m, k), dtype=torch.int8, device=d)
    sc, en, nseg = N.segments_arrays(scales, ends)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("noalloc: capturing one call", flush=True)
    with torch.cuda.graph(graph):
        rc = L.btl_bitlinear_fused_noalloc(N.ptr(x), m, k, k, N.ptr(g), 1e-5, N.ptr(wdev), n, sc, en, nseg,
                                           N.EPI_SCALE, None, N.ptr(out), N.ptr(acc), N.ptr(xq), N.ptr(err_word), 0,
                                           N.stream_of(d))
    N.check(rc, "btl_bitlinear_fused_noalloc (captured)")
    for r in range(4):
        print(f"noalloc: replay {r}", flush=True)
        out.zero_()
        acc.zero_()
        xq.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert int(err_word.item()) == 0, f"replay {r}: a bounded wait ran out"
        assert np.array_equal(xq.cpu().numpy(), ref[2]), f"replay {r}: quantised activations differ"
        assert np.array_equal(acc.cpu().numpy(), ref[1]), f"replay {r}: accumulators differ"
        assert np.array_equal(H.bits_of(out), ref[0]), f"replay {r}: bf16 outputs differ"
        # eager work between replays: both entry points on other inputs
        got2 = _call(L, True, x2, m, k, g, wdev, n, scales, ends, N.EPI_SCALE, None, err_word)
        assert np.array_equal(got2[0], ref2[0]) and np.array_equal(got2[1], ref2[1]), f"eager call after replay {r}"
        _call(L, False, x2, m, k, g, wdev, n, scales, ends, N.EPI_SCALE, None, err_word)
    o = orc.bitlinear(xb, w, scales, ends, gamma_bf16=gb, norm_eps=1e-5)
    assert np.array_equal(ref[0], o["out"]), "the eager reference differs from the oracle"


def test_noalloc_matches_workspace_entry_point(orc):
    L = N.lib()
    err_word = torch.zeros(1, dtype=torch.int32, device=H.dev())
    cases = [
        # (m, k, n, scales, ends, epilogue, residual): QKV with three segments; then a smaller
        # o_proj-like call with a residual; then gate||up relu2; then a prefill-path call
        (32, 2560, 3840, [0.017, 0.019, 0.023], [2560, 3200, 3840], N.EPI_SCALE, False),
        (16, 2560, 2560, [0.02], [2560], N.EPI_SCALE, True),
        (32, 2560, 13824, [0.021, 0.018], [6912, 13824], N.EPI_RELU2_MUL, False),
        (64, 1024, 512, [0.02], [512], N.EPI_SCALE, True),
    ]
    for i, (m, k, n, scales, ends, epi, with_res) in enumerate(cases):
        print(f"noalloc case {i}: m={m} k={k} n={n} epi={epi} residual={with_res}", flush=True)
        xb = H.activations(orc, m, k, seed=100 + i)
        gb = H.gamma(orc, k, seed=200 + i)
        w, wdev = _weight(orc, k, n, seed=300 + i)
        x, g = H.to_dev_bf16(xb), H.to_dev_bf16(gb)
        res = H.to_dev_bf16(H.activations(orc, m, n // 2 if epi else n, seed=400 + i, outliers=False)) \
            if with_res else None
        ref = _call(L, False, x, m, k, g, wdev, n, scales, ends, epi, res, err_word)
        got = _call(L, True, x, m, k, g, wdev, n, scales, ends, epi, res, err_word)
        assert np.array_equal(got[2], ref[2]), f"case {i}: quantised activations differ"
        assert np.array_equal(got[1], ref[1]), f"case {i}: accumulators differ"
        assert np.array_equal(got[0], ref[0]), f"case {i}: bf16 outputs differ"
        assert int(err_word.item()) == 0, f"case {i}: a bounded wait ran out"
        # and against the oracle, for the decode cases
        if epi == N.EPI_SCALE and m <= 32:
            o = orc.bitlinear(xb, w, scales, ends, gamma_bf16=gb, norm_eps=1e-5,
                              residual_bf16=H.bits_of(res) if res is not None else None)
            assert np.array_equal(got[0], o["out"]), f"case {i}: differs from the oracle"


def test_noalloc_refuses_oversized_shapes():
    L = N.lib()
    d = H.dev()
    m, k, n = 2048, 6912, 2560
    need = int(L.btl_fused_workspace_bytes(m, k, n, 0, 0))
    assert need > (3 << 20)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device=d)
    wdev = torch.zeros((n // 32, (k + 127) // 128, 256), dtype=torch.int32, device=d)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=d)
    sc, en, nseg = N.segments_arrays([0.02], [n])
    rc = L.btl_bitlinear_fused_noalloc(N.ptr(x), m, k, k, None, 1e-5, N.ptr(wdev), n, sc, en, nseg, 0, None,
                                       N.ptr(out), None, None, None, 0, N.stream_of(d))
    assert rc == 4  # BTL_ERR_WORKSPACE
    assert "scratch" in N.last_error()
