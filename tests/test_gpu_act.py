"""GPU parity of the activation prologue: RMSNorm, absmax int8 quantisation,
the blocked operand layout, per-token scales and row sums.  Bit-exact
against the oracle (RMS statistic in this build's fixed fp32 order)."""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N
from bitnet_tt.layers.bitlinear import RMSNorm
from bitnet_tt.utils import quantization as Q

pytestmark = pytest.mark.gpu


def run_quant(m, k, xb, gb=None, eps=1e-5):
    L = N.lib()
    d = H.dev()
    rows = 32 * ((m + 31) // 32)
    x = H.to_dev_bf16(xb)
    g = H.to_dev_bf16(gb) if gb is not None else None
    xa = torch.full((int(L.btl_act_bytes(m, k)),), 0x5A, dtype=torch.uint8, device=d)
    a_dq = torch.empty(rows, dtype=torch.float32, device=d)
    rowsum = torch.empty(rows, dtype=torch.int32, device=d)
    scale = torch.empty(m, dtype=torch.float32, device=d)
    xq = torch.empty((m, k), dtype=torch.int8, device=d)
    y = torch.empty((m, k), dtype=torch.bfloat16, device=d)
    N.check(L.btl_quant_absmax(N.ptr(x), m, k, k, N.ptr(g), eps, N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum), N.ptr(scale),
                               N.ptr(xq), N.ptr(y), N.stream_of(d)), "btl_quant_absmax")
    torch.cuda.synchronize()
    return dict(xa=xa.cpu().numpy(), a_dq=a_dq.cpu().numpy(), rowsum=rowsum.cpu().numpy(),
                scale=scale.cpu().numpy(), xq=xq.cpu().numpy(), y=H.bits_of(y))


# For K <= 8192 the prologue runs two waves per row from 256 rows and one wave
# per row from 1024: (300, 2560) and (500, 6912) take the first kernel,
# (1000, 2560) and (1100, 6912) the second, with padding rows in the last row
# block.
@pytest.mark.parametrize("m,k", [(1, 32), (5, 256), (32, 2560), (33, 2560), (70, 640), (32, 6912), (3, 16384),
                                 (300, 2560), (500, 6912), (1000, 2560), (1100, 6912)])
@pytest.mark.parametrize("norm", [False, True])
def test_quant_absmax_bit_exact(orc, m, k, norm):
    print(f"quant m={m} k={k} norm={norm}", flush=True)
    xb = H.activations(orc, m, k, seed=m * 131 + k)
    gb = H.gamma(orc, k, seed=k) if norm else None
    r = run_quant(m, k, xb, gb)
    y = orc.rmsnorm_bf16(xb, gb, 1e-5, order=1) if norm else xb
    q, scale, a_dq, rowsum = orc.act_quant_absmax(orc.bf16_to_f32(y))
    if norm:
        assert np.array_equal(r["y"], y)
    assert np.array_equal(r["xq"], q)
    assert np.array_equal(r["scale"], scale.reshape(-1))
    assert np.array_equal(r["a_dq"][:m], a_dq)
    assert np.array_equal(r["rowsum"][:m], rowsum)
    rm, full = H.xa_to_rowmajor(r["xa"], m, k)
    assert np.array_equal(rm, q)
    # padding rows and columns are zero, as are their scales
    assert not full[m:].any() and not full[:, k:].any()
    assert not r["a_dq"][m:].any() and not r["rowsum"][m:].any()


def test_quant_special_rows(orc):
    x = np.zeros((3, 32), np.float32)
    x[1, :4] = [-4.0, 4.0, 1.0, 0.0]
    x[2, :8] = [127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -127.0]
    r = run_quant(3, 32, orc.f32_to_bf16(x))
    assert not r["xq"][0].any() and r["a_dq"][0] == np.float32(1e-5) / np.float32(127)
    assert r["xq"][1, :3].tolist() == [-127, 127, 32]
    assert r["xq"][2, :8].tolist() == [127, 2, 4, -2, 0, 0, 2, -127]
    assert r["rowsum"][:3].tolist() == [0, 32, 6]


@pytest.mark.parametrize("m,k", [(4, 256), (32, 2560), (32, 6912)])
def test_rmsnorm_kernel_bit_exact(orc, m, k):
    xb = H.activations(orc, m, k, seed=k + 1)
    gb = H.gamma(orc, k, seed=k + 2)
    norm = RMSNorm(k, H.dev(), eps=1e-5)
    norm.load_weights(orc.bf16_to_f32(gb))
    y = norm(H.to_dev_bf16(xb))
    assert np.array_equal(H.bits_of(y), orc.rmsnorm_bf16(xb, gb, 1e-5, order=1))


def test_activation_quant_api_device(orc):
    xb = H.activations(orc, 2 * 16, 256, seed=3).reshape(2, 16, 256)
    q, s = Q.activation_quant_absmax(H.to_dev_bf16(xb))
    oq, os_, _, _ = orc.act_quant_absmax(orc.bf16_to_f32(xb))
    assert q.shape == (2, 16, 256) and s.shape == (2, 16, 1)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy(), os_)
