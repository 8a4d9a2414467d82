"""Benchmark: BitLinear portion of a batch-32 BitNet b1.58 2B decode step on one MI355X.

A step is the 30-layer chain of the model's BitLinear launches at M = 32
tokens: per layer the fused RMSNorm->QKV (2560->3840), o_proj (2560->2560,
attn_sub_norm prologue, residual epilogue), gate||up (2560->2x6912,
post-attention RMSNorm prologue, relu^2*up epilogue) and down (6912->2560,
ffn_sub_norm prologue, residual epilogue).  Weights are random-init ternary
(latents ~N(0, 0.02), absmean-quantised on the device), RMSNorm gains ~N(1,
0.1), activations ~N(0, 1): synthetic, seeded.  The attention core between
QKV and o_proj is not part of the BitLinear path; o_proj reads a seeded
stand-in buffer.  The step is captured once in a HIP graph and replayed.

Printed JSON (one line): value = algorithmic HBM bytes of a step / step time
(GB/s), ms_per_step = BitLinear ms per decode step, plus the roofline of the
dominant kernel (the BitLinear kind with the longest launch) measured with HIP
events on the launch stream, the prefill MFMA-i8 utilisation, and the CPU
oracle timed on the host as a reported baseline.  ``--pmc-pass`` runs only
the workload of the rocprofv3 --pmc traffic measurement.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "bitnet-tt_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=10, help="repetitions of the per-kernel event pass")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-lm-head", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="approximate CPU-baseline sample length")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="run only the workload of the rocprofv3 --pmc traffic runs and exit")
    return ap.parse_args()


# --------------------------------------------------------------- kernels ----
KINDS = ("qkv", "o_proj", "gate_up", "down")


def kind_launcher(step, kind):
    """(launch(layer_index), description) of one BitLinear kind of the step,
    with exactly the arguments the step's own chain passes."""
    from bitnet_tt.ternary_matmul import ternary_matmul_into

    eps = step.eps
    if kind == "qkv":
        def launch(i):
            w = step.layers[i]
            ternary_matmul_into(step.hidden, w.qkv, step.qkv_out, norm_weight=w.input_layernorm, norm_epsilon=eps)
    elif kind == "o_proj":
        def launch(i):
            w = step.layers[i]
            ternary_matmul_into(step.attn_out, w.o_proj, step.hidden, norm_weight=w.attn_sub_norm,
                                norm_epsilon=eps, residual=step.hidden)
    elif kind == "gate_up":
        def launch(i):
            w = step.layers[i]
            ternary_matmul_into(step.hidden, w.gate_up, step.ffn_h, norm_weight=w.post_attention_layernorm,
                                norm_epsilon=eps, epilogue="relu2_mul")
    else:
        def launch(i):
            w = step.layers[i]
            ternary_matmul_into(step.ffn_h, w.down, step.hidden, norm_weight=w.ffn_sub_norm, norm_epsilon=eps,
                                residual=step.hidden)
    return launch


def kernel_event_timing(step, torch, reps):
    """Average duration of each BitLinear kind's single-launch decode kernel,
    measured with HIP events on the launch stream.  For every kind the 30
    layers' launches (distinct weights: 265 MB for gate||up, more than the
    256 MB last-level cache) are recorded into a graph; a replay is bracketed
    by two events on that stream and divided by the number of launches."""
    dev = step.device
    res = {}
    s = torch.cuda.Stream(device=dev)
    n = len(step.layers)
    for kind in KINDS:
        launch = kind_launcher(step, kind)
        step.reset_hidden()
        torch.cuda.synchronize()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(n):  # eager pass: workspace allocation happens outside capture
                launch(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                launch(i)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        times = []
        with torch.cuda.stream(s):
            g.replay()
            for _ in range(reps):
                step.reset_hidden()
                e0.record(s)
                g.replay()
                e1.record(s)
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1e3 / n)  # us per launch
        torch.cuda.synchronize()
        times.sort()
        res[kind] = {"us_per_launch_median": times[len(times) // 2], "us_per_launch_min": times[0]}
        del g
    step.reset_hidden()
    torch.cuda.synchronize()
    return res


def pmc_pass(step, torch):
    """Workload for the rocprofv3 --pmc traffic runs: a plain 256 MiB device
    copy (the counter calibration: it reads and writes exactly 256 MiB), then
    two eager passes of each BitLinear kind over all layers."""
    dev = step.device
    a = torch.empty(128 << 20, dtype=torch.int16, device=dev).fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    for kind in KINDS:
        launch = kind_launcher(step, kind)
        for _ in range(2):
            step.reset_hidden()
            for i in range(len(step.layers)):
                launch(i)
        torch.cuda.synchronize()
        log(f"[bench] pmc pass: {kind} done")


TRAFFIC_FILE = os.path.join(REPO, "profiles", "bitlinear_decode_b32_traffic.md")


def committed_traffic(kind):
    """HBM bytes per launch of a kind from the committed rocprofv3 --pmc
    summary (lines 'traffic_bytes_per_launch <kind> <bytes>'), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kind:
                    return int(parts[2])
    except OSError:
        return None
    return None


def gemm_algorithmic_bytes(M, K, N, epi, nseg, residual):
    n_out = N // 2 if epi == 1 else N
    b = K * N // 4 + 32 * K + 8 * 32 + 4 * nseg + 2 * M * n_out
    if residual:
        b += 2 * M * n_out
    return b


def prefill_mfma(torch, N, dev):
    """MFMA-i8 utilisation of the prefill GEMM at the configured shapes."""
    L = N.lib()
    shapes = [(512, 2560, 3840), (512, 2560, 6912), (512, 2560, 2560), (512, 6912, 2560),
              (2048, 2560, 3840), (2048, 2560, 6912), (2048, 2560, 2560), (2048, 6912, 2560)]
    out = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    for M, K, Nf in shapes:
        KS = (K + 127) // 128
        # activations as the layer makes them: absmax int8 operand, scales and
        # row sums from the activation kernel
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        xa = torch.empty((int(L.btl_act_bytes(M, K)),), dtype=torch.int8, device=dev)
        a_dq = torch.empty((32 * ((M + 31) // 32),), dtype=torch.float32, device=dev)
        rowsum = torch.empty((32 * ((M + 31) // 32),), dtype=torch.int32, device=dev)
        N.check(L.btl_quant_absmax(N.ptr(x), M, K, K, None, 0.0, N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum), None, None,
                                   None, N.stream_of(dev)), "prefill activations")
        copies = 4
        wd = [torch.randint(0, 1 << 30, (Nf // 32, KS, 256), generator=gen, device=dev, dtype=torch.int32) & 0x55555555
              for _ in range(copies)]  # codes 0/1 only: valid ternary offsets
        o = torch.empty((M, Nf), dtype=torch.bfloat16, device=dev)
        sc, en, nseg = N.segments_arrays([0.02], [Nf])
        stream = N.stream_of(dev)
        # split-K partials and counters (zero-filled once; every call leaves them clean)
        ws = torch.zeros(max(int(L.btl_gemm_workspace_bytes(M, K, Nf, 0, 0)), 256), dtype=torch.uint8, device=dev)

        def launch(i):
            N.check(L.btl_gemm_i8t2(N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum), M, K, Nf, N.ptr(wd[i % copies]), sc, en,
                                    nseg, 0, None, N.ptr(o), None, N.ptr(ws), ws.numel(), 0, stream), "prefill gemm")

        reps = 20
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            stream = N.stream_of(dev)
            for i in range(3):
                launch(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            stream = N.stream_of(dev)
            for i in range(reps):
                launch(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            g.replay()
            e0.record(s)
            g.replay()
            e1.record(s)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        del g
        tops = 2.0 * M * K * Nf / (us * 1e-6) / 1e12
        out.append({"M": M, "K": K, "N": Nf, "us": round(us, 2), "tops": round(tops, 1),
                    "mfma_i8_util": round(tops / MFMA_I8_PEAK_TOPS, 4)})
    return out


# ------------------------------------------------------------ full step ----
def full_step_timing(step, torch, s, args, ctx=512):
    """The 30-layer step with the decode attention in place (150 launches,
    one graph), and the attention launches alone (a graph of one per layer,
    bracketed by HIP events on the launch stream)."""
    step.alloc_attention(max_seq_len=ctx)
    with torch.cuda.stream(s):
        step.reset_hidden()
        step.step_full()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step.step_full()
    with torch.cuda.stream(s):
        for _ in range(max(args.warmup, 1)):
            g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(s):
        for _ in range(args.steps):
            g.replay()
    torch.cuda.synchronize()
    us_full = (time.perf_counter() - t0) * 1e6 / args.steps
    del g
    n = len(step.layers)
    ga = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ga, stream=s):
        for i in range(n):
            step.attention(step.qkv_out, step.kv[i], step.pos, out=step.attn_out)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    with torch.cuda.stream(s):
        ga.replay()
        for _ in range(3):
            e0.record(s)
            ga.replay()
            e1.record(s)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / n)
    del ga
    torch.cuda.synchronize()
    c = step.config
    B, Hkv, D, H_ = step.batch, c.num_kv_heads, c.head_dim, c.num_attention_heads
    # compulsory bytes: cached K and V rows [0, pos], the qkv rows, the new cache rows, the output
    nbytes = 2 * B * Hkv * ctx * D * 2 + B * c.qkv_dim * 2 + 2 * B * Hkv * D * 2 + B * H_ * D * 2
    us_att = sorted(times)[1]
    for kv in step.kv:  # release the caches (1.3 GB)
        del kv.key_cache, kv.value_cache
    step.kv = None
    return {
        "workload": f"30 layers x (QKV, decode attention over context {ctx}, o_proj, gate||up, down), batch 32",
        "us_per_step": round(us_full, 1),
        "attention_us_per_layer": round(us_att, 2),
        "attention_bytes_per_launch": nbytes,
        "attention_GBps": round(nbytes / (us_att * 1e-6) / 1e9, 1),
        "attention_roofline_frac": round(nbytes / (us_att * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
    }


# ------------------------------------------------------------------ LM head ----
def lm_head_timing(torch, N, dev, reps=20):
    """Final norm + LM head + argmax at the 2B shape (32 rows, hidden 2560,
    vocab 128256; a random bf16 head of 656 MB in the kernel's layout).  The
    head kernel alone and norm + head are each timed as a graph of `reps`
    calls bracketed by HIP events on the launch stream."""
    from bitnet_tt.lm_head import LMHead

    M, H_, V = 32, 2560, 128256
    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    head = LMHead(H_, V, dev, eps=1e-5)
    w = (torch.randn((V, H_), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    g = (1.0 + 0.1 * torch.randn(H_, generator=gen, device=dev))
    head.load_final_weights(g, w)
    del w
    x = torch.randn((M, H_), generator=gen, device=dev).to(torch.bfloat16)
    xn = torch.empty((M, H_), dtype=torch.bfloat16, device=dev)
    logits = torch.empty((M, V), dtype=torch.float32, device=dev)
    tokens = torch.empty(M, dtype=torch.int32, device=dev)
    L = N.lib()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        head(x, normed_out=xn, logits_out=logits, tokens_out=tokens)  # eager: workspace exists before capture
    torch.cuda.synchronize()
    ws = N.workspace(dev, int(L.btl_lm_head_workspace_bytes()), kind="lm_head")

    def kernel_only(rows=M):
        N.check(L.btl_lm_head(N.ptr(xn), rows, H_, V, N.ptr(head.weight), N.ptr(logits), N.ptr(tokens), N.ptr(ws),
                              ws.numel(), N.stream_of(dev)), "btl_lm_head")

    res = {}
    for name, fn in (("kernel", kernel_only), ("kernel_row0", lambda: kernel_only(1)),
                     ("norm_and_head", lambda: head(x, normed_out=xn, logits_out=logits, tokens_out=tokens))):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            for _ in range(reps):
                fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        times = []
        with torch.cuda.stream(s):
            gr.replay()
            for _ in range(3):
                e0.record(s)
                gr.replay()
                e1.record(s)
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1e3 / reps)
        res[name] = sorted(times)[1]
        del gr
    torch.cuda.synchronize()
    wbytes = 2 * V * H_
    nbytes = wbytes + 2 * M * H_ + 4 * M * V + 4 * M  # head + normed rows + fp32 logits + tokens
    us = res["kernel"]
    return {
        "workload": "final RMSNorm + LM head 2560 -> 128256 (bf16 weights) + argmax, 32 rows",
        "us_kernel": round(us, 2),
        "us_norm_and_head": round(res["norm_and_head"], 2),
        "us_kernel_one_row": round(res["kernel_row0"], 2),
        "bytes_per_launch": nbytes,
        "achieved_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
        "roofline_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
    }


# ------------------------------------------------------------ CPU baseline ----
def cpu_baseline(step, torch, seconds):
    """Scalar C oracle (one thread) on a bounded sample of the same workload:
    whole decode layers (4 BitLinears at M = 32), run until `seconds` pass."""
    import numpy as np

    from oracle import oracle as orc

    orc.lib()
    c = step.config

    def wkn(pw):
        return orc.devlayout_decode(pw.data.cpu().numpy().view(np.uint32), pw.in_features, pw.out_features)

    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    eps = step.eps
    hidden = bits(step.hidden0)
    attn = bits(step.attn_out)
    per_layer = step.algorithmic_bytes()["layer"]
    done, t_total = 0, 0.0
    for i, w in enumerate(step.layers):
        mats = (wkn(w.qkv), wkn(w.o_proj), wkn(w.gate_up), wkn(w.down))
        g = [bits(t) for t in (w.input_layernorm, w.attn_sub_norm, w.post_attention_layernorm, w.ffn_sub_norm)]
        t0 = time.perf_counter()
        orc.bitlinear(hidden, mats[0], list(w.qkv.segment_scales), list(w.qkv.segment_ends), gamma_bf16=g[0],
                      norm_eps=eps)
        hidden = orc.bitlinear(attn, mats[1], list(w.o_proj.segment_scales), gamma_bf16=g[1], norm_eps=eps,
                               residual_bf16=hidden)["out"]
        r = orc.gate_up_relu2(hidden, mats[2], w.gate_up.segment_scales[0], w.gate_up.segment_scales[1],
                              gamma_bf16=g[2], norm_eps=eps)
        hidden = orc.bitlinear(r["h"], mats[3], list(w.down.segment_scales), gamma_bf16=g[3], norm_eps=eps,
                               residual_bf16=hidden)["out"]
        t_total += time.perf_counter() - t0
        done += 1
        if t_total >= seconds:
            break
    gbs = per_layer * done / t_total / 1e9
    ms_step = t_total / done * len(step.layers) * 1e3
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{done} of {len(step.layers)} decode layers (4 BitLinears each, M=32) through the scalar C "
                  f"oracle; {t_total:.1f} s; extrapolated {ms_step:.0f} ms per 30-layer step",
        "ms_per_step_extrapolated": round(ms_step, 1),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the BitLinear path is measured on a single MI355X "
              f"(--gpus {args.gpus} is not supported).", file=sys.stderr)
        sys.exit(2)

    import torch

    from bitnet_tt import _native as N
    from bitnet_tt.config import BitNet2B4TConfig
    from bitnet_tt.decode import BitLinearDecodeStep

    N.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = BitNet2B4TConfig()
    t0 = time.time()
    step = BitLinearDecodeStep.random_init(cfg, dev, seed=args.seed, num_layers=args.layers).alloc_buffers(seed=1)
    torch.cuda.synchronize()
    log(f"[bench] model ready: {args.layers} layers in {time.time() - t0:.1f} s; "
        f"ternary split +1/0/-1 = {'/'.join(f'{v:.4f}' for v in step.ternary_split)}")

    if args.pmc_pass:
        pmc_pass(step, torch)
        return

    # warm-up (eager), then capture the step on a side stream
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(args.warmup, 1)):
            step.reset_hidden()
            step.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step.step()
    with torch.cuda.stream(s):
        for _ in range(args.warmup):
            graph.replay()
    torch.cuda.synchronize()
    log("[bench] graph captured; timing")

    torch.cuda.synchronize()
    t_start = time.perf_counter()
    with torch.cuda.stream(s):
        for _ in range(args.steps):
            graph.replay()
    torch.cuda.synchronize()
    t_el = time.perf_counter() - t_start
    ms_per_step = t_el * 1e3 / args.steps
    nbytes = step.algorithmic_bytes()
    value = nbytes["step"] / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] {ms_per_step * 1e3:.1f} us per step, {value:.0f} GB/s")

    # the same step as persistent per-layer launches (btl_decode_layer)
    with torch.cuda.stream(s):
        step.reset_hidden()
        step.step_layers()
    torch.cuda.synchronize()
    graph_l = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph_l, stream=s):
        step.step_layers()
    with torch.cuda.stream(s):
        for _ in range(args.warmup):
            graph_l.replay()
    torch.cuda.synchronize()
    t_l = time.perf_counter()
    with torch.cuda.stream(s):
        for _ in range(args.steps):
            graph_l.replay()
    torch.cuda.synchronize()
    us_layers = (time.perf_counter() - t_l) * 1e6 / args.steps
    del graph_l
    log(f"[bench] persistent per-layer launches: {us_layers:.1f} us per step")

    # the whole step: decode attention (context 512, every user at the last
    # position) between each layer's QKV and o_proj
    full = None
    if not args.no_attention:
        full = full_step_timing(step, torch, s, args)
        log(f"[bench] full step with decode attention (context 512): {full['us_per_step']:.1f} us; attention "
            f"{full['attention_us_per_layer']:.2f} us per layer, {full['attention_GBps']:.0f} GB/s, "
            f"{100 * full['attention_roofline_frac']:.1f} % of HBM")

    kt = kernel_event_timing(step, torch, args.kernel_reps)
    for name, r in kt.items():
        log(f"[bench] {name}: {r['us_per_launch_median']:.2f} us per launch (median of {args.kernel_reps})")
    # dominant kernel: the kind with the largest share of the step
    dom = max(KINDS, key=lambda k: kt[k]["us_per_launch_median"])
    dom_bytes = nbytes[dom]
    dom_us = kt[dom]["us_per_launch_median"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic = committed_traffic(dom)
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": f"k_bitlinear_decode ({dom}: " + {
            "qkv": "RMSNorm->QKV 2560->3840", "o_proj": "attn_sub_norm->o_proj 2560->2560 +residual",
            "gate_up": "RMSNorm->gate||up 2560->2x6912, relu2*up", "down": "ffn_sub_norm->down 6912->2560 +residual",
        }[dom] + ", M=32)",
        "bytes_per_launch": dom_bytes,
        "us_per_launch": round(dom_us, 3),
    }
    kernel_us = {k: round(v["us_per_launch_median"], 3) for k, v in kt.items()}
    kernel_frac = {k: round(nbytes[k] / (kt[k]["us_per_launch_median"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                   for k in KINDS}

    prefill = None
    if not args.no_prefill:
        prefill = prefill_mfma(torch, N, dev)
        for p in prefill:
            log(f"[bench] prefill M={p['M']} K={p['K']} N={p['N']}: {p['us']} us, {p['tops']} TOPS, "
                f"MFMA-i8 {100 * p['mfma_i8_util']:.1f}%")

    head = None
    if not args.no_lm_head:
        head = lm_head_timing(torch, N, dev)
        log(f"[bench] LM head (32 x 2560 -> 128256 + argmax): {head['us_kernel']} us kernel, "
            f"{head['us_norm_and_head']} us with the final norm, {head['us_kernel_one_row']} us for one row; "
            f"{head['achieved_GBps']} GB/s, "
            f"{100 * head['roofline_frac']:.1f} % of HBM")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) ...")
        cpu = cpu_baseline(step, torch, args.cpu_seconds)
        log(f"[bench] CPU: {cpu['sample']}")

    line = {
        "metric": "ternary GEMM HBM GB/s (% roofline) at M=32; BitLinear ms per batch-32 decode step",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xternary->int32 (bf16 in/out)",
        "data": "synthetic (seeded random-init ternary weights, N(0,1) activations)",
        "config": {
            "workload": f"BitLinear portion of a batch-32 BitNet b1.58 2B decode step ({args.layers} layers x "
                        "4 fused BitLinear launches: RMSNorm->QKV 2560->3840, o_proj 2560->2560, "
                        "gate||up 2560->2x6912 relu2, down 6912->2560), HIP-graph replay",
            "batch": 32,
            "layers": args.layers,
            "bytes_per_step": nbytes["step"],
            "step_roofline_frac": round(value / HBM_PEAK_GBS, 4),
            "us_per_step_layer_launches": round(us_layers, 1),
            "us_per_launch": kernel_us,
            "roofline_frac_per_launch": kernel_frac,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill_mfma": prefill,
        "lm_head": head,
        "full_step": full,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
