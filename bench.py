"""Benchmark: BitLinear portion of a batch-32 BitNet b1.58 2B decode step on one MI355X.

A step is the 30-layer chain of the model's BitLinear launches at M = 32
tokens: per layer the fused RMSNorm->QKV (2560->3840), o_proj (2560->2560,
attn_sub_norm prologue, residual epilogue), gate||up (2560->2x6912,
post-attention RMSNorm prologue, relu^2*up epilogue) and down (6912->2560,
ffn_sub_norm prologue, residual epilogue), all 120 of them in one persistent
kernel launch (btl_decode_step).  Weights are random-init ternary
(latents ~N(0, 0.02), absmean-quantised on the device), RMSNorm gains ~N(1,
0.1), activations ~N(0, 1): synthetic, seeded.  The attention core between
QKV and o_proj is not part of the BitLinear path; o_proj reads a seeded
stand-in buffer.  The step is captured once in a HIP graph and replayed.  The
same step as 120 per-BitLinear launches and as 31 per-layer launches is timed
beside it, and the three structures are checked to give the same bits.

Printed JSON (one line): value = algorithmic HBM bytes of a step / step time
(GB/s), ms_per_step = BitLinear ms per decode step, plus the roofline of the
step kernel measured with HIP events on the launch stream, each BitLinear
kind's single-launch kernel time, the prefill MFMA-i8 utilisation, and the CPU
reference CPU path (numpy absmax quantisation + torch fp32 GEMM of the same
step) timed on the host as a reported baseline.  ``--pmc-pass`` runs only
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
    ap.add_argument("--cpu-reps", type=int, default=20, help="timed CPU-baseline steps (after 3 warm-ups)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="run only the workload of the rocprofv3 --pmc traffic runs and exit")
    ap.add_argument("--step-trace", action="store_true",
                    help="load the -DBTL_TRACE build (bitnet_tt/_lib/libbtl_trace.so, from "
                         "python bitnet-tt_amd/bitnet_tt/_build.py --trace), run persistent steps and print the "
                         "phase table of layer 10 (then that of the one-launch step with the decode attention, "
                         "unless --no-attention), then exit")
    ap.add_argument("--prefill-pmc-pass", action="store_true",
                    help="run only the prefill GEMMs (5 launches per configured shape) for rocprofv3 --pmc and exit")
    return ap.parse_args()


# --------------------------------------------------------------- kernels ----
KINDS = ("qkv", "o_proj", "gate_up", "down")


KIND_ATTR = {"qkv": "qkv", "o_proj": "o_proj", "gate_up": "gate_up", "down": "down"}
ROTATION_BYTES = 512 << 20  # distinct weight bytes a per-kind pass cycles through (> 256 MB last-level cache)


def kind_launcher(step, kind):
    """launch(layer_index, weight=None) of one BitLinear kind of the step, with
    exactly the arguments the step's own chain passes (``weight`` replaces the
    layer's weight by a copy with the same values)."""
    from bitnet_tt.ternary_matmul import ternary_matmul_into

    eps = step.eps
    attr = KIND_ATTR[kind]

    def wt(i, w):
        return getattr(step.layers[i], attr) if w is None else w

    if kind == "qkv":
        def launch(i, w=None):
            L_ = step.layers[i]
            ternary_matmul_into(step.hidden, wt(i, w), step.qkv_out, norm_weight=L_.input_layernorm, norm_epsilon=eps)
    elif kind == "o_proj":
        def launch(i, w=None):
            L_ = step.layers[i]
            ternary_matmul_into(step.attn_out, wt(i, w), step.hidden, norm_weight=L_.attn_sub_norm,
                                norm_epsilon=eps, residual=step.hidden)
    elif kind == "gate_up":
        def launch(i, w=None):
            L_ = step.layers[i]
            ternary_matmul_into(step.hidden, wt(i, w), step.ffn_h, norm_weight=L_.post_attention_layernorm,
                                norm_epsilon=eps, epilogue="relu2_mul")
    else:
        def launch(i, w=None):
            L_ = step.layers[i]
            ternary_matmul_into(step.ffn_h, wt(i, w), step.hidden, norm_weight=L_.ffn_sub_norm, norm_epsilon=eps,
                                residual=step.hidden)
    return launch


def rotation_plan(step, kind):
    """[(layer, weight)] covering every layer's weight of a kind, repeated with
    device copies until the distinct weight bytes reach ROTATION_BYTES, so a
    pass cannot run out of the 256 MB last-level cache."""
    import dataclasses

    attr = KIND_ATTR[kind]
    n = len(step.layers)
    per_pass = sum(getattr(L_, attr).nbytes for L_ in step.layers)
    copies = max(1, -(-ROTATION_BYTES // per_pass))
    plan = [(i, None) for i in range(n)]
    for _ in range(copies - 1):
        for i in range(n):
            w = getattr(step.layers[i], attr)
            plan.append((i, dataclasses.replace(w, data=w.data.clone())))
    return plan, per_pass * copies


def kernel_event_timing(step, torch, reps):
    """Average duration of each BitLinear kind's single-launch decode kernel,
    measured with HIP events on the launch stream.  For every kind the 30
    layers' launches, over copies of their weights until at least 512 MB of
    distinct weights are cycled (more than the 256 MB last-level cache), are
    recorded into a graph; a replay is bracketed by two events on that stream
    and divided by the number of launches."""
    dev = step.device
    res = {}
    s = torch.cuda.Stream(device=dev)
    for kind in KINDS:
        launch = kind_launcher(step, kind)
        plan, wbytes = rotation_plan(step, kind)
        step.reset_hidden()
        torch.cuda.synchronize()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i, w in plan:  # eager pass: workspace allocation happens outside capture
                launch(i, w)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i, w in plan:
                launch(i, w)
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
                times.append(e0.elapsed_time(e1) * 1e3 / len(plan))  # us per launch
        torch.cuda.synchronize()
        times.sort()
        res[kind] = {"us_per_launch_median": times[len(times) // 2], "us_per_launch_min": times[0],
                     "launches_per_replay": len(plan), "distinct_weight_bytes": wbytes}
        del g, plan
    step.reset_hidden()
    torch.cuda.synchronize()
    return res


def pmc_pass(step, torch):
    """Workload for the rocprofv3 --pmc traffic runs: a plain 256 MiB device
    copy (the counter calibration: it reads and writes exactly 256 MiB), then
    two eager passes of each BitLinear kind over all layers, then three
    persistent steps (one k_decode_step launch each)."""
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
    for _ in range(3):
        step.reset_hidden()
        step.step_persistent()
    step.check()
    log("[bench] pmc pass: persistent step done")


TRAFFIC_FILES = [os.path.join(REPO, "profiles", f) for f in
                 ("decode_step_b32_traffic.md", "bitlinear_decode_b32_traffic.md")]


def committed_traffic(kind):
    """HBM bytes per launch of a kind ("step" for the persistent step kernel)
    from the committed rocprofv3 --pmc summaries (lines
    'traffic_bytes_per_launch <kind> <bytes>'), or None."""
    for path in TRAFFIC_FILES:
        try:
            with open(path) as f:
                for line in f:
                    parts = line.strip().strip("`").split()
                    if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kind:
                        return int(parts[2])
        except OSError:
            continue
    return None


def gemm_algorithmic_bytes(M, K, N, epi, nseg, residual):
    n_out = N // 2 if epi == 1 else N
    b = K * N // 4 + 32 * K + 8 * 32 + 4 * nseg + 2 * M * n_out
    if residual:
        b += 2 * M * n_out
    return b


PREFILL_SHAPES = [(512, 2560, 3840), (512, 2560, 6912), (512, 2560, 2560), (512, 6912, 2560),
                  (2048, 2560, 3840), (2048, 2560, 6912), (2048, 2560, 2560), (2048, 6912, 2560)]
PREFILL_SEED = 77


def graph_time_us(torch, dev, launch, reps=20, warm=3):
    """Average us per call of `reps` calls of launch(i) recorded into one
    graph, bracketed by HIP events on the capture stream (eager warm-up calls
    first, so workspaces exist before the capture)."""
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(warm):
            launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
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
    torch.cuda.synchronize()
    return us


def prefill_mfma(torch, N, dev, shapes=PREFILL_SHAPES, pmc_reps=0):
    """MFMA-i8 utilisation of the prefill BitLinear at the configured shapes.

    Inputs as the prefill configuration states them: x bf16 ~N(0, 1) with 1 %
    of the channels x20, gain ~N(1, 0.1), weights absmean-quantised from
    seeded N(0, 0.02) latents (4 copies with distinct latents, cycled).  Two
    figures per shape: the GEMM alone (btl_gemm_i8t2 on the activation
    kernel's int8 operand, scales and row sums) and the whole BitLinear
    (btl_bitlinear_fused: RMSNorm + absmax activation kernel, then the GEMM).
    With pmc_reps > 0 nothing is timed: each shape's GEMM runs pmc_reps times
    eagerly, in the order of `shapes` (the workload of the rocprofv3 --pmc
    MFMA counter runs)."""
    from bitnet_tt.layers.bitlinear import pack_for_device
    from bitnet_tt.ternary_matmul import ternary_matmul_into
    from bitnet_tt.utils.quantization import weight_quant_ternary

    L = N.lib()
    out = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(PREFILL_SEED)
    for M, K, Nf in shapes:
        x = torch.randn((M, K), generator=gen, device=dev)
        cols = torch.randperm(K, generator=gen, device=dev)[: K // 100]
        x[:, cols] *= 20.0
        x = x.to(torch.bfloat16)
        gamma = (1.0 + 0.1 * torch.randn((K,), generator=gen, device=dev)).to(torch.bfloat16)
        xa = torch.empty((int(L.btl_act_bytes(M, K)),), dtype=torch.int8, device=dev)
        a_dq = torch.empty((32 * ((M + 31) // 32),), dtype=torch.float32, device=dev)
        rowsum = torch.empty((32 * ((M + 31) // 32),), dtype=torch.int32, device=dev)
        N.check(L.btl_quant_absmax(N.ptr(x), M, K, K, N.ptr(gamma), 1e-5, N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum),
                                   None, None, None, N.stream_of(dev)), "prefill activations")
        copies = 4
        pws = []
        for _ in range(copies):
            lat = torch.randn((Nf, K), generator=gen, device=dev) * 0.02
            q, sc_w = weight_quant_ternary(lat)
            pws.append(pack_for_device(q, dev, (sc_w,), (Nf,)))
            del lat, q
        o = torch.empty((M, Nf), dtype=torch.bfloat16, device=dev)
        # split-K partials and counters (zero-filled once; every call leaves them clean)
        ws = torch.zeros(max(int(L.btl_gemm_workspace_bytes(M, K, Nf, 0, 0)), 256), dtype=torch.uint8, device=dev)

        def gemm(i):
            pw = pws[i % copies]
            sc, en, nseg = N.segments_arrays(pw.segment_scales, pw.segment_ends)
            N.check(L.btl_gemm_i8t2(N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum), M, K, Nf, N.ptr(pw.data), sc, en,
                                    nseg, 0, None, N.ptr(o), None, N.ptr(ws), ws.numel(), 0, N.stream_of(dev)),
                    "prefill gemm")

        def bitlinear(i):
            ternary_matmul_into(x, pws[i % copies], o, norm_weight=gamma, norm_epsilon=1e-5)

        if pmc_reps:
            for i in range(pmc_reps):
                gemm(i)
            torch.cuda.synchronize()
            log(f"[bench] prefill pmc pass: M={M} K={K} N={Nf}: {pmc_reps} GEMM launches")
            out.append({"M": M, "K": K, "N": Nf})
            del pws
            continue
        us = graph_time_us(torch, dev, gemm)
        us_bl = graph_time_us(torch, dev, bitlinear)
        ops = 2.0 * M * K * Nf
        tops = ops / (us * 1e-6) / 1e12
        # The vendor library's int8 GEMM on the same shape (torch._int_mm, hipBLASLt on ROCm): int8 operands
        # already unpacked, int32 output, no scale epilogue -- a reference point, not this path.
        us_lib = None
        try:
            glib = torch.Generator(device=dev)
            glib.manual_seed(PREFILL_SEED + 1)
            a8 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=glib)
            b8 = torch.randint(-1, 2, (Nf, K), dtype=torch.int8, device=dev, generator=glib)
            c32 = torch.empty((M, Nf), dtype=torch.int32, device=dev)
            us_lib = graph_time_us(torch, dev, lambda i: torch._int_mm(a8, b8.t(), out=c32))
            del a8, b8, c32
        except (RuntimeError, TypeError) as e:
            log(f"[bench] torch._int_mm unavailable for {M}x{K}x{Nf}: {e}")
        tl = N.gemm_tiling(M, K, Nf)
        tiling = (f"{tl['rows']}x{32 * tl['col_tiles']}" + (f" wq{tl['k_groups']}" if tl["kind"] == "wide" else "")
                  + (f" sk{tl['splitk']}" if tl["splitk"] > 1 else ""))
        out.append({"M": M, "K": K, "N": Nf, "tiling": tiling,
                    "us": round(us, 2), "tops": round(tops, 1), "mfma_i8_util": round(tops / MFMA_I8_PEAK_TOPS, 4),
                    "us_bitlinear": round(us_bl, 2),
                    "mfma_i8_util_bitlinear": round(ops / (us_bl * 1e-6) / 1e12 / MFMA_I8_PEAK_TOPS, 4),
                    "us_hipblaslt_int8": None if us_lib is None else round(us_lib, 2),
                    "mfma_i8_util_hipblaslt_int8": None if us_lib is None else
                    round(ops / (us_lib * 1e-6) / 1e12 / MFMA_I8_PEAK_TOPS, 4)})
        del pws
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
    # the same step as one launch (btl_decode_step_full): attention on the
    # GEMM workgroups between QKV and o_proj; its bits equal step_full's
    state = (step.hidden.clone(), [(kv.key_cache.clone(), kv.value_cache.clone()) for kv in step.kv])

    def restore():
        step.hidden.copy_(state[0])
        for kv, (k, v) in zip(step.kv, state[1]):
            kv.key_cache.copy_(k)
            kv.value_cache.copy_(v)

    with torch.cuda.stream(s):
        restore()
        step.step_full()
    torch.cuda.synchronize()
    ref = step.hidden.clone()
    with torch.cuda.stream(s):
        restore()
        step.step_persistent_full()
    torch.cuda.synchronize()
    step.check()
    full_bits_equal = bool(torch.equal(step.hidden.view(torch.int16), ref.view(torch.int16)))
    gp = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gp, stream=s):
        step.step_persistent_full()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        for _ in range(max(args.warmup, 1)):
            gp.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(s):
        e0.record(s)
        for _ in range(args.steps):
            gp.replay()
        e1.record(s)
    torch.cuda.synchronize()
    us_one = (time.perf_counter() - t0) * 1e6 / args.steps
    us_one_event = e0.elapsed_time(e1) * 1e3 / args.steps
    step.check()
    del gp, state
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
        "us_per_step_one_launch": round(us_one, 1),
        "us_per_step_one_launch_event": round(us_one_event, 1),
        "one_launch_bits_equal": full_bits_equal,
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
def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the process's CPU affinity, capped
    by OMP_NUM_THREADS when the environment sets it (the GPU box gives one GPU
    a share of its cores and says so there)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(n, 1)


def cpu_baseline(step, torch, gpu_hidden, reps=20, warmup=3):
    """The reference's CPU path of the same 30-layer BitLinear step, timed on
    the host: per BitLinear the RMSNorm in HF BitNetRMSNorm order (torch fp32),
    numpy per-token absmax quantisation (activation_quant_absmax,
    src/bitnet_tt/utils/quantization.py:60-91), a torch fp32 GEMM of the
    int-valued operands (exact: |acc| < 2^24), and the scale to bf16; relu^2*up
    and the residual adds in bf16 as the model does.  Same weights, gains and
    inputs as the GPU step.  Median of `reps` full steps after `warmup`."""
    import numpy as np

    from bitnet_tt.utils.quantization import activation_quant_absmax
    from oracle import oracle as orc

    orc.lib()
    n_thr = cpu_threads()
    torch.set_num_threads(n_thr)
    c = step.config
    eps = step.eps
    bf = torch.bfloat16

    def w_f32(pw):  # ternary (K, N) as float32, from the device weight
        w = orc.devlayout_decode(pw.data.cpu().numpy().view(np.uint32), pw.in_features, pw.out_features)
        return torch.from_numpy(w.astype(np.float32))

    def seg_scale_row(pw):
        v = torch.empty(pw.out_features, dtype=torch.float32)
        lo = 0
        for sc, end in zip(pw.segment_scales, pw.segment_ends):
            v[lo:end] = float(sc)
            lo = end
        return v

    layers = []
    for w in step.layers:
        layers.append({
            "qkv": (w_f32(w.qkv), seg_scale_row(w.qkv)), "o": (w_f32(w.o_proj), seg_scale_row(w.o_proj)),
            "gu": (w_f32(w.gate_up), seg_scale_row(w.gate_up)), "dn": (w_f32(w.down), seg_scale_row(w.down)),
            "g_in": w.input_layernorm.cpu(), "g_sub": w.attn_sub_norm.cpu(),
            "g_post": w.post_attention_layernorm.cpu(), "g_ffn": w.ffn_sub_norm.cpu(),
        })
    hidden0 = step.hidden0.cpu()
    attn = step.attn_out.cpu()
    F = c.intermediate_size

    def rmsnorm(x, g):  # HF BitNetRMSNorm: fp32 statistic, bf16 normalised value times the bf16 gain
        x32 = x.float()
        var = x32.pow(2).mean(-1, keepdim=True)
        return g * (x32 * torch.rsqrt(var + eps)).to(bf)

    def bitlinear(x, g, wm):
        w, srow = wm
        y = rmsnorm(x, g).float().numpy()
        q, scale = activation_quant_absmax(y)
        acc = torch.from_numpy(q.astype(np.float32)) @ w
        a_dq = torch.from_numpy((1.0 / scale).astype(np.float32))  # a/127 per token
        return (acc * (srow * a_dq)).to(bf)

    def run_step():
        h = hidden0.clone()
        qkv = None
        for L_ in layers:
            qkv = bitlinear(h, L_["g_in"], L_["qkv"])
            h = (h.float() + bitlinear(attn, L_["g_sub"], L_["o"]).float()).to(bf)
            gu = bitlinear(h, L_["g_post"], L_["gu"])
            g_, u_ = gu[:, :F].float(), gu[:, F:].float()
            r = (torch.relu(g_).pow(2).to(bf).float() * u_).to(bf)
            h = (h.float() + bitlinear(r, L_["g_ffn"], L_["dn"]).float()).to(bf)
        return h, qkv

    for _ in range(warmup):
        run_step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        h, _qkv = run_step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    nbytes = step.algorithmic_bytes()["step"]
    equal = float((h.view(torch.int16) == gpu_hidden.view(torch.int16)).float().mean().item())
    # the GPU's hidden state against this reference-order chain: normwise
    # relative error, largest element error over the largest magnitude, PCC
    g64, r64 = gpu_hidden.float().cpu().double(), h.float().double()
    d = g64 - r64
    agree = {"rel_fro": float(d.norm() / r64.norm()), "max_rel": float(d.abs().max() / r64.abs().max()),
             "pcc": float(np.corrcoef(g64.numpy().ravel(), r64.numpy().ravel())[0, 1])}
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": n_thr,
        "kind": "port",
        "sample": f"the full {len(layers)}-layer BitLinear step (4 BitLinears per layer, M=32) on the host: numpy "
                  f"absmax quantisation + torch fp32 GEMM on {n_thr} threads; median of {reps} steps after {warmup} "
                  "warm-ups",
        "ms_per_step": round(med * 1e3, 2),
        "ms_per_step_min": round(times[0] * 1e3, 2),
        "us_per_bitlinear": round(med * 1e6 / (4 * len(layers)), 1),
        "cpu_model": cpu_model_name(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "torch": torch.__version__,
        "numpy": np.__version__,
        "hidden_bits_equal_to_gpu": round(equal, 6),
        "hidden_vs_gpu": {k: round(v, 7) for k, v in agree.items()},
    }


def dot4_variant_timing(step, torch, N, reps=10):
    """The decode GEMM of each BitLinear kind at M = 32 as the library runs it
    (btl_gemm_i8t2: MFMA) and formulated on the VALU (btl_gemm_i8t2_dot4:
    v_dot4_i32_i8), on the same int8 operand tile and the 30 layers' weights:
    a graph of 30 launches per kernel, timed with events on its stream, in us
    per launch (median of reps).  The GEMM alone: the operand tile comes from
    one btl_quant_absmax call made beforehand."""
    L = N.lib()
    dev = step.device
    c = step.config
    H_, F_ = c.hidden_size, c.intermediate_size
    shapes = {"qkv": (H_, c.qkv_dim), "o_proj": (H_, H_), "gate_up": (H_, 2 * F_), "down": (F_, H_)}
    s = torch.cuda.Stream(device=dev)
    gen = torch.Generator(device="cpu")
    gen.manual_seed(53)
    res = {}
    for kind, (K, Nn) in shapes.items():
        x = torch.randn(32, K, generator=gen).to(torch.bfloat16).to(dev)
        xa = torch.empty(int(L.btl_act_bytes(32, K)), dtype=torch.uint8, device=dev)
        a_dq = torch.empty(32, dtype=torch.float32, device=dev)
        rs = torch.empty(32, dtype=torch.int32, device=dev)
        N.check(L.btl_quant_absmax(N.ptr(x), 32, K, K, None, 0.0, N.ptr(xa), N.ptr(a_dq), N.ptr(rs), None, None,
                                   None, N.stream_of(dev)), "btl_quant_absmax")
        out = torch.empty(32, Nn, dtype=torch.bfloat16, device=dev)
        acc = torch.zeros(32, Nn, dtype=torch.int32, device=dev)
        wsb = int(L.btl_gemm_workspace_bytes(32, K, Nn, 0, 0))
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
        sc, en, nseg = N.segments_arrays([1.0], [Nn])
        ws_ = [getattr(Lr, KIND_ATTR[kind]).data for Lr in step.layers]

        def mfma(w):
            N.check(L.btl_gemm_i8t2(N.ptr(xa), N.ptr(a_dq), N.ptr(rs), 32, K, Nn, N.ptr(w), sc, en, nseg, 0, None,
                                    N.ptr(out), None, N.ptr(ws), ws.numel(), 0, N.stream_of(dev)), "btl_gemm_i8t2")

        def dot4(w):  # accumulates into acc (no clearing inside the timed graph)
            N.check(L.btl_gemm_i8t2_dot4(N.ptr(xa), N.ptr(rs), 32, K, Nn, N.ptr(w), N.ptr(acc), N.stream_of(dev)),
                    "btl_gemm_i8t2_dot4")

        res[kind] = {"K": K, "N": Nn}
        for name, fn in (("us_mfma", mfma), ("us_dot4", dot4)):
            torch.cuda.synchronize()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for w in ws_:
                    fn(w)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for w in ws_:
                    fn(w)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            times = []
            with torch.cuda.stream(s):
                g.replay()
                for _ in range(reps):
                    e0.record(s)
                    g.replay()
                    e1.record(s)
                    e1.synchronize()
                    times.append(e0.elapsed_time(e1) * 1e3 / len(ws_))
            torch.cuda.synchronize()
            times.sort()
            res[kind][name] = round(times[len(times) // 2], 2)
            del g
    return res


STEP_TRACE_EVENTS = {
    # row workgroups (wave 0): event -> name
    0: "row: QKV row stage starts", 1: "row: QKV flag set", 2: "row: QKV words in", 3: "row: o_proj flag set",
    4: "row: o_proj words in", 5: "row: gate||up flag set", 6: "row: gate||up words in", 7: "row: down flag set",
    # GEMM workgroups (wave 0)
    8: "GEMM: QKV rows seen", 9: "GEMM: QKV outputs stored", 10: "GEMM: o_proj rows seen",
    11: "GEMM: o_proj outputs stored", 12: "GEMM: gate||up rows seen", 13: "GEMM: gate||up outputs stored",
    14: "GEMM: down rows seen", 15: "GEMM: down outputs stored",
}
STEP_TRACE_ORDER = (0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15)
# The full step (btl_decode_step_full): the attention units' events 0-7 (GEMM
# workgroups) come between QKV and o_proj; row event 2 is then "the user's
# attention output words in".
STEP_TRACE_ATT_EVENTS = {
    100: "attention: cache loads issued", 101: "attention: QKV rows in", 103: "attention: RoPE done",
    104: "attention: softmax done", 105: "attention: values done", 106: "attention: merge barriers passed",
    107: "attention: outputs stored",
}
STEP_TRACE_FULL_ORDER = (0, 1, 8, 9, 100, 101, 103, 104, 105, 106, 107, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15)


def step_trace(step, torch, N, runs=5, full=False):
    """Phase timestamps (s_memrealtime, 100 MHz) of layer 10 of the persistent
    step from the -DBTL_TRACE build: per event, min / median / max over the
    workgroups that record it, in us from the first row workgroup's start;
    the median over `runs` launches of each statistic.  full: the one-launch
    step with the decode attention (context 512) instead of the BitLinears."""
    import ctypes

    import numpy as np

    L = N.lib()
    rd = L.btl_trace_read_step
    rd.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    rd.restype = ctypes.c_int
    buf = np.zeros((2048, 16, 16), dtype=np.uint64)
    fn = step.step_persistent_full if full else step.step_persistent
    order = STEP_TRACE_FULL_ORDER if full else STEP_TRACE_ORDER
    names = {**STEP_TRACE_EVENTS, **STEP_TRACE_ATT_EVENTS}
    if full:
        names[2] = "row: attention words in"
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    rd(buf.ctypes.data, buf.nbytes)  # clears the table
    stats = {ev: [] for ev in order}
    for _ in range(runs):
        fn()
        torch.cuda.synchronize()
        rd(buf.ctypes.data, buf.nbytes)
        t0 = int(buf[:32, 0, 0][buf[:32, 0, 0] > 0].min())
        for ev in order:
            v = buf[:32, 0, ev] if ev < 8 else buf[32:, 0, ev % 100]
            v = v[v > 0].astype(np.int64)
            if len(v):
                d = (v - t0) / 100.0
                stats[ev].append((d.min(), np.median(d), d.max(), len(v)))
    step.check()
    rows = []
    for ev in order:
        if stats[ev]:
            a = np.array(stats[ev])
            rows.append({"event": names[ev], "workgroups": int(a[0, 3]),
                         "min_us": round(float(np.median(a[:, 0])), 2), "median_us": round(float(np.median(a[:, 1])), 2),
                         "max_us": round(float(np.median(a[:, 2])), 2)})
    return rows


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

    if args.step_trace:
        from bitnet_tt import _build

        if not os.path.exists(_build.OUT_TRACE):
            raise SystemExit(f"{_build.OUT_TRACE} is not built: python bitnet-tt_amd/bitnet_tt/_build.py --trace")
        N.LIB_PATH = _build.OUT_TRACE
    N.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.prefill_pmc_pass:
        prefill_mfma(torch, N, dev, pmc_reps=5)
        return
    cfg = BitNet2B4TConfig()
    t0 = time.time()
    step = BitLinearDecodeStep.random_init(cfg, dev, seed=args.seed, num_layers=args.layers).alloc_buffers(seed=1)
    torch.cuda.synchronize()
    log(f"[bench] model ready: {args.layers} layers in {time.time() - t0:.1f} s; "
        f"ternary split +1/0/-1 = {'/'.join(f'{v:.4f}' for v in step.ternary_split)}")

    if args.pmc_pass:
        pmc_pass(step, torch)
        return
    if args.step_trace:
        rows = step_trace(step, torch, N)
        print(f"{'event (layer 10)':36s} {'WGs':>4s} {'min':>7s} {'median':>7s} {'max':>7s}  (us)")
        for r in rows:
            print(f"{r['event']:36s} {r['workgroups']:4d} {r['min_us']:7.2f} {r['median_us']:7.2f} {r['max_us']:7.2f}")
        if not args.no_attention:
            step.alloc_attention(max_seq_len=512)
            rows = step_trace(step, torch, N, full=True)
            print(f"\nfull step with decode attention (context 512), {'event (layer 10)':36s}")
            for r in rows:
                print(f"{r['event']:36s} {r['workgroups']:4d} {r['min_us']:7.2f} {r['median_us']:7.2f} "
                      f"{r['max_us']:7.2f}")
        return

    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())

    def capture(fn):
        """Eager warm-up calls of fn on stream s (workspaces are prepared
        outside the capture), then fn captured into a graph on s."""
        with torch.cuda.stream(s):
            for _ in range(max(args.warmup, 1)):
                step.reset_hidden()
                fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
        with torch.cuda.stream(s):
            for _ in range(args.warmup):
                g.replay()
        torch.cuda.synchronize()
        return g

    def timed(g, n):
        """Wall-clock us per replay of n replays, and the same span from two
        HIP events recorded on the launch stream around them."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t = time.perf_counter()
        with torch.cuda.stream(s):
            e0.record(s)
            for _ in range(n):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t) * 1e6 / n
        return wall, e0.elapsed_time(e1) * 1e3 / n

    # the headline step: the whole step's BitLinears as one persistent launch
    graph = capture(step.step_persistent)
    log("[bench] persistent step captured; timing")
    us_wall, us_event = timed(graph, args.steps)
    step.check()  # a bounded wait that ran out inside the timed replays raises here
    ms_per_step = us_wall * 1e-3
    nbytes = step.algorithmic_bytes()
    value = nbytes["step"] / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] {us_wall:.1f} us per step ({us_event:.1f} us between events on the launch stream), "
        f"{value:.0f} GB/s")
    del graph

    # the same step as 120 per-BitLinear launches
    graph_c = capture(step.step_per_call)
    us_per_call, _ = timed(graph_c, args.steps)
    step.check()
    del graph_c
    log(f"[bench] per-BitLinear launches: {us_per_call:.1f} us per step")
    # the latency floor of the persistent step's launch structure: the same
    # waits and hand-off stores with no arithmetic and no weight traffic
    graph_f = capture(step.step_floor)
    us_floor, _ = timed(graph_f, args.steps)
    step.check()
    del graph_f
    log(f"[bench] hand-off floor of the persistent step (waits and hand-off stores only): {us_floor:.1f} us per step")

    # the two launch structures compute the same bits from the same input
    outs = {}
    for name, fn in (("persistent", step.step_persistent), ("per_call", step.step_per_call)):
        step.reset_hidden()
        fn()
        step.check()
        outs[name] = step.hidden.clone()
    same_bits = all(torch.equal(outs["persistent"].view(torch.int16), o.view(torch.int16)) for o in outs.values())
    log(f"[bench] persistent / per-call hidden bits equal: {same_bits}")
    if not same_bits:
        raise SystemExit("launch structures disagree")

    # the whole step: decode attention (context 512, every user at the last
    # position) between each layer's QKV and o_proj
    full = None
    if not args.no_attention:
        full = full_step_timing(step, torch, s, args)
        log(f"[bench] full step with decode attention (context 512): {full['us_per_step']:.1f} us as 150 launches, "
            f"{full['us_per_step_one_launch']:.1f} us as one launch (bits equal: {full['one_launch_bits_equal']}); attention "
            f"{full['attention_us_per_layer']:.2f} us per layer, {full['attention_GBps']:.0f} GB/s, "
            f"{100 * full['attention_roofline_frac']:.1f} % of HBM")

    dot4 = dot4_variant_timing(step, torch, N, args.kernel_reps)
    for kind, r in dot4.items():
        log(f"[bench] decode GEMM {kind} ({r['K']}->{r['N']}): MFMA {r['us_mfma']} us, v_dot4 on the VALU "
            f"{r['us_dot4']} us per launch")
    kt = kernel_event_timing(step, torch, args.kernel_reps)
    for name, r in kt.items():
        log(f"[bench] {name}: {r['us_per_launch_median']:.2f} us per launch (median of {args.kernel_reps})")
    # dominant kernel: the persistent step kernel, the only launch of a step
    achieved = nbytes["step"] / (us_event * 1e-6) / 1e9
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": committed_traffic("step"),
        "kernel": f"k_decode_step (all {args.layers} layers' QKV, o_proj, gate||up, down at M=32 in one launch)",
        "bytes_per_launch": nbytes["step"],
        "us_per_launch": round(us_event, 3),
    }
    kernel_us = {k: round(v["us_per_launch_median"], 3) for k, v in kt.items()}
    kernel_frac = {k: round(nbytes[k] / (kt[k]["us_per_launch_median"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                   for k in KINDS}

    prefill = None
    if not args.no_prefill:
        prefill = prefill_mfma(torch, N, dev)
        for p in prefill:
            lib = ("" if p["us_hipblaslt_int8"] is None else
                   f"; hipBLASLt int8 GEMM {p['us_hipblaslt_int8']} us ({100 * p['mfma_i8_util_hipblaslt_int8']:.1f}%)")
            log(f"[bench] prefill M={p['M']} K={p['K']} N={p['N']}: {p['us']} us, {p['tops']} TOPS, "
                f"MFMA-i8 {100 * p['mfma_i8_util']:.1f}% (BitLinear {100 * p['mfma_i8_util_bitlinear']:.1f}%){lib}")

    head = None
    if not args.no_lm_head:
        head = lm_head_timing(torch, N, dev)
        log(f"[bench] LM head (32 x 2560 -> 128256 + argmax): {head['us_kernel']} us kernel, "
            f"{head['us_norm_and_head']} us with the final norm, {head['us_kernel_one_row']} us for one row; "
            f"{head['achieved_GBps']} GB/s, "
            f"{100 * head['roofline_frac']:.1f} % of HBM")

    cpu = None
    if not args.no_cpu_baseline:
        # the GPU's result of one step from the seeded input, for the CPU path's agreement figure
        # (the attention timing above rewrote attn_out, so the GPU step runs again here)
        step.reset_hidden()
        step.step_persistent()
        step.check()
        gpu_hidden = step.hidden.cpu()
        log("[bench] CPU baseline (reference CPU path: numpy absmax + torch fp32 GEMM) ...")
        cpu = cpu_baseline(step, torch, gpu_hidden, reps=args.cpu_reps)
        log(f"[bench] CPU: {cpu['ms_per_step']} ms per step on {cpu['cores']} threads ({cpu['cpu_model']}); "
            f"{cpu['value']} GB/s; hidden bits equal to the GPU's: {cpu['hidden_bits_equal_to_gpu']}; "
            f"against the GPU's: {cpu['hidden_vs_gpu']}")

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
        "data": "synthetic (seeded random-init ternary weights from N(0,0.02) latents, RMSNorm gains N(1,0.1), "
                "activations N(0,1) with 1% outlier channels x20)",
        "config": {
            "workload": f"BitLinear portion of a batch-32 BitNet b1.58 2B decode step ({args.layers} layers x "
                        "4 fused BitLinears: RMSNorm->QKV 2560->3840, o_proj 2560->2560, "
                        "gate||up 2560->2x6912 relu2, down 6912->2560) as one persistent launch, HIP-graph replay",
            "batch": 32,
            "layers": args.layers,
            "bytes_per_step": nbytes["step"],
            "step_roofline_frac": round(value / HBM_PEAK_GBS, 4),
            "us_per_step_event": round(us_event, 1),
            "us_per_step_per_bitlinear_launches": round(us_per_call, 1),
            "us_per_step_handoff_floor": round(us_floor, 1),
            "launch_structures_bits_equal": same_bits,
            "us_per_bitlinear_launch": kernel_us,
            "roofline_frac_per_launch": kernel_frac,
            "per_kind_rotation_bytes": {k: v["distinct_weight_bytes"] for k, v in kt.items()},
            "seeds": {"weights": args.seed, "activations": 1, "kv_cache": 3, "prefill": PREFILL_SEED,
                      "lm_head": 31, "dot4_variant": 53},
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill_mfma": prefill,
        "lm_head": head,
        "full_step": full,
        "decode_gemm_dot4_vs_mfma": dot4,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
