"""GPU parity of the load-time kernels: absmean weight quantisation, the
reference tile format (pack / unpack) and the repack into the GEMM layout.
All integer/byte work: bit-exact against the oracle."""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt.kernels import pack as P
from bitnet_tt.utils import quantization as Q

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(7,), (64, 128), (300, 301), (640, 2560), (6912, 2560)])
def test_weight_quant_device_matches_numpy(orc, shape):
    w = H.latent(int(np.prod(shape[:-1])) if len(shape) > 1 else 1, shape[-1], seed=sum(shape))
    w = w.reshape(shape)
    print(f"weight quant shape={shape}", flush=True)
    q_d, s_d = Q.weight_quant_ternary(H.to_dev(w))
    q_h, s_h = orc.weight_quant_ternary(w)
    assert np.float32(s_d) == s_h
    assert np.array_equal(q_d.cpu().numpy(), q_h)


def test_weight_quant_device_unaligned_and_partial(orc):
    """Full 8192-blocks plus a partial last block, from a buffer that is not
    16-byte aligned (the one-thread block sums) and from an aligned one (one
    wave per full block): the scale and codes equal numpy's either way."""
    w = H.latent(1, 3 * 8192 + 12, seed=41).reshape(-1)
    d = H.to_dev(w)
    print("weight quant unaligned / aligned, n=%d" % (w.size - 1), flush=True)
    for view, host in ((d[1:], w[1:]), (d[:-1], w[:-1])):
        q_d, s_d = Q.weight_quant_ternary(view)
        q_h, s_h = orc.weight_quant_ternary(np.ascontiguousarray(host))
        assert np.float32(s_d) == s_h
        assert np.array_equal(q_d.cpu().numpy(), q_h)


def test_weight_quant_device_special_cases(orc):
    z = torch.zeros((4, 64), dtype=torch.float32, device=H.dev())
    q, s = Q.weight_quant_ternary(z)
    assert np.float32(s) == np.float32(1e-5) and int(q.abs().sum()) == 0
    w = np.array([0.5, 1.5, -0.5, -1.5, 0.0, 2.0], np.float32)
    q, s = Q.weight_quant_ternary(H.to_dev(w))
    assert s == 1.0 and q.cpu().tolist() == [0, 1, 0, -1, 0, 1]


@pytest.mark.parametrize("out_f,in_f", [(32, 32), (64, 128), (50, 100), (33, 65), (3840, 2560)])
def test_pack_unpack_device(orc, out_f, in_f):
    print(f"pack out={out_f} in={in_f}", flush=True)
    q = H.ternary(out_f, in_f, seed=out_f + in_f)
    packed = P.pack_ternary_tilized_device(H.to_dev(q))
    ref, _ = orc.pack_ternary_tilized(q, 1.0)
    assert np.array_equal(packed.cpu().numpy(), ref)
    un = P.unpack_ternary_tilized_device(packed, in_f, out_f)
    assert np.array_equal(un.cpu().numpy(), q.T)


def test_unpack_device_reads_reserved_code_as_zero(orc):
    packed = torch.full((1, 256), 0xFF, dtype=torch.uint8, device=H.dev())
    un = P.unpack_ternary_tilized_device(packed, 32, 32)
    assert int(un.abs().sum()) == 0


@pytest.mark.parametrize("k,n", [(32, 32), (96, 64), (128, 96), (224, 32), (2560, 3840), (6912, 2560)])
def test_repack_matches_oracle_layout(orc, k, n):
    print(f"repack K={k} N={n}", flush=True)
    w_kn = H.ternary(k, n, seed=k * 7 + n)
    packed, _ = orc.pack_ternary_tilized(np.ascontiguousarray(w_kn.T), 1.0)
    wdev = P.repack_for_gemm(H.to_dev(packed), k, n)
    got = wdev.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, orc.devlayout_encode(w_kn))
    assert np.array_equal(orc.devlayout_decode(got, k, n), w_kn)
