"""GPU parity of the final norm + LM head + argmax (generator_batch32.py:
768-811 and 1170-1174; head weights of model/bitnet.py:139-215).

Logits are fp32 accumulations of bf16 products, so they are compared with the
float64 oracle within the fp32 rounding bound 2 K 2^-24 sum|x w| (an error in
a dropped term, a wrong row or a transposed operand is orders of magnitude
larger).  Tokens must equal the first index of the maximum of the returned
logits exactly, and be the oracle's argmax up to logits closer than the bound.
"""

import numpy as np
import pytest
import torch

import helpers as H
from bitnet_tt import _native as N
from bitnet_tt.lm_head import LMHead

pytestmark = pytest.mark.gpu


def run_head(orc, m, k, v, seed, w_bits=None, x_bits=None):
    rng = np.random.default_rng(seed)
    if x_bits is None:
        x_bits = orc.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    g_bits = H.gamma(orc, k, seed + 1)
    if w_bits is None:
        w_bits = orc.f32_to_bf16((rng.standard_normal((v, k)) * 0.05).astype(np.float32))
    head = LMHead(k, v, H.dev(), eps=1e-5)
    head.load_final_weights(orc.bf16_to_f32(g_bits), H.to_dev_bf16(w_bits))
    logits, tokens = head(H.to_dev_bf16(x_bits))
    torch.cuda.synchronize()
    xn = orc.rmsnorm_bf16(x_bits, g_bits, 1e-5)
    return head, x_bits, xn, w_bits, logits.cpu().numpy(), tokens.cpu().numpy()


def check(orc, xn, w_bits, logits, tokens):
    ref, bound = orc.lm_head(xn, w_bits)
    assert np.all(np.abs(logits - ref) <= bound + 1e-30), np.max(np.abs(logits - ref) / (bound + 1e-30))
    assert np.array_equal(tokens, orc.argmax_first(logits))
    r = np.arange(ref.shape[0])
    assert np.all(ref[r, tokens] >= ref.max(1) - 2 * bound.max(1))


@pytest.mark.parametrize("m,k,v", [(1, 2560, 4096), (5, 128, 1000), (32, 288, 37), (32, 2560, 3000), (17, 1024, 8224)])
def test_lm_head_small_shapes(orc, m, k, v):
    print(f"lm head m={m} k={k} v={v}", flush=True)
    head, x, xn, w, logits, tokens = run_head(orc, m, k, v, seed=m * 7 + v)
    normed = torch.empty((m, k), dtype=torch.bfloat16, device=H.dev())
    head(H.to_dev_bf16(x), normed_out=normed)
    torch.cuda.synchronize()
    assert np.array_equal(H.bits_of(normed), xn)  # the final norm is the fixed-order RMSNorm
    check(orc, xn, w, logits, tokens)


def test_lm_head_ties_take_the_first_index(orc):
    """Rows 700 and 5 of the head equal and larger than all others: token 5;
    and a row whose every logit is equal picks index 0."""
    k, v = 256, 1024
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((v, k)) * 0.01).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    w[5] = w[700] = np.sign(x[0]) * 0.5
    x[1] = 0.0
    print("lm head ties", flush=True)
    _, _, xn, wb, logits, tokens = run_head(orc, 2, k, v, seed=3, w_bits=orc.f32_to_bf16(w),
                                             x_bits=orc.f32_to_bf16(x))
    assert logits[0, 5] == logits[0, 700]
    assert tokens[0] == 5 and tokens[1] == 0


def test_lm_head_2b_full_vocab(orc):
    """32 rows against the 128256 x 2560 head: every logit of two rows and the
    tokens of all rows against the oracle; logits of all rows at sampled
    columns."""
    m, k, v = 32, 2560, 128256
    print("lm head 2B shape", flush=True)
    head, x, xn, w, logits, tokens = run_head(orc, m, k, v, seed=11)
    assert np.array_equal(tokens, orc.argmax_first(logits))
    rows = [0, 31]
    ref, bound = orc.lm_head(xn[rows], w)
    assert np.all(np.abs(logits[rows] - ref) <= bound)
    cols = np.random.default_rng(12).choice(v, 2048, replace=False)
    ref_s, bound_s = orc.lm_head(xn, w[cols])
    assert np.all(np.abs(logits[:, cols] - ref_s) <= bound_s)
    assert np.all(ref[np.arange(2), tokens[rows]] >= ref.max(1) - 2 * bound.max(1))


def test_lm_head_repeats_graph_and_clean_workspace(orc):
    """Repeated calls and graph replays give the same tokens; the workspace's
    argmax keys and done counter are zero after every call."""
    m, k, v = 32, 512, 5000
    print("lm head repeats + graph", flush=True)
    head, x, xn, w, logits, tokens = run_head(orc, m, k, v, seed=21)
    xd = H.to_dev_bf16(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    xn_buf = torch.empty((m, k), dtype=torch.bfloat16, device=H.dev())
    lg = torch.empty((m, v), dtype=torch.float32, device=H.dev())
    tk = torch.empty(m, dtype=torch.int32, device=H.dev())
    with torch.cuda.stream(s):
        for _ in range(5):
            head(xd, normed_out=xn_buf, logits_out=lg, tokens_out=tk)
    torch.cuda.synchronize()
    assert np.array_equal(tk.cpu().numpy(), tokens)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        head(xd, normed_out=xn_buf, logits_out=lg, tokens_out=tk)
    for _ in range(3):
        tk.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(tk.cpu().numpy(), tokens)
    for key, ws in N._workspaces.items():
        if key[0] == "lm_head":
            assert not ws[:384].cpu().numpy().any()
