"""DASH attention benchmark on one MI355X.

Headline: one DASH prefill pass (k_bar -> block scores -> entmax routing -> fused
block-sparse attention) over B=1, 27,300 tokens (100 pages x 273), 10 heads,
head_dim 128, 64-token blocks, 1,024-token window, 16 routed blocks, in bf16 with
fp32 accumulation; reported as TFLOP/s of algorithmic attention work
(4*D*H*sum_t |window(t) U routed(t)|, counted from the routing the pass emits).

Every other workload is timed in the same run, each with the roofline of its
product kernels and the CPU oracle timed on a bounded sample on this host:
  * 2,730-token prefill (block 64, window 512, cap 8)
  * decode step, B = 8 x 27,300 cached tokens (window 1,024, cap 16)
  * 16-document packed prefill (cu_seqlens, window 512, cap 8)
  * 12-layer paged decode step, B = 32 sequences of 2,730..27,300 tokens
  * training step at 27,300 tokens (training routing, attention forward and backward,
    routing backward; k = 16)
  * page-aware candidate masks of a 100-page OCR prompt (prefill rows, decode row)
  * the fused router front end at 27,300 tokens, hidden 1,280, block 32 (index
    projections, norms, RoPE, block summaries in one launch)

HBM traffic and executed MFMA work per launch come from hardware-counter runs
(rocprofv3 --pmc over ``bench.py --counter-probe WORKLOAD``), summarised by
``bench.py --summarize-counters`` into profiles/counters_per_launch.txt together
with a hash of the kernel sources; a summary whose hash differs from the current
sources is reported as stale (null).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--only NAME,...]
  python bench.py --counter-probe WORKLOAD
  python bench.py --summarize-counters COUNTER_DIR [COUNTER_DIR ...]
"""

import argparse
import csv
import glob
import hashlib
import json
import math
import os
import re
import statistics
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from ananta_ocr_amd import ops, pipeline  # noqa: E402
from ananta_ocr_amd import workloads as W  # noqa: E402

METRIC = "DASH attn prefill TFLOP/s @27.3k tok + decode µs/step; % of MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2516.6          # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBS = 8000.0
COUNTERS_FILE = os.path.join(ROOT, "profiles", "counters_per_launch.txt")
CSRC = os.path.join(ROOT, "ananta_ocr_amd", "csrc")
CALIB_BYTES = 256 * 2 ** 20        # the counter runs' device-copy calibration


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_source_hash():
    """sha256 over the HIP sources (name and contents, sorted), first 16 hex digits."""
    h = hashlib.sha256()
    for p in sorted(glob.glob(os.path.join(CSRC, "*"))):
        h.update(os.path.basename(p).encode())
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def host_cpu():
    """(model name, physical cores, logical CPUs) of this host."""
    model, phys, logical = "unknown", None, os.cpu_count()
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL,
                             text=True, timeout=10).stdout
        f = dict(l.split(":", 1) for l in out.splitlines() if ":" in l)
        f = {k.strip(): v.strip() for k, v in f.items()}
        model = f.get("Model name", model)
        cps = int(f.get("Core(s) per socket", "0") or 0)
        sockets = int(f.get("Socket(s)", "0") or 0)
        if cps and sockets:
            phys = cps * sockets
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if phys is None:
        try:
            pairs = set()
            pid = None
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                if line.startswith("physical id"):
                    pid = line.split(":", 1)[1].strip()
                if line.startswith("core id"):
                    pairs.add((pid, line.split(":", 1)[1].strip()))
            phys = len(pairs) or None
        except OSError:
            pass
    return model, phys, logical


# ------------------------------------------------------------------ work counting

def prefill_pairs(idx, valid, S, bs, lw):
    """sum_t |window(t) U routed(t)| for routing idx/valid [S,K] of one sequence
    (routed ids are distinct, as routing emits them)."""
    t = torch.arange(S, device=idx.device)
    ls = t - lw + 1
    win = torch.minimum(t + 1, torch.full_like(t, lw))
    c = idx.long()
    hi = torch.minimum(torch.minimum((c + 1) * bs, ls[:, None]), torch.full_like(c, S))
    rk = (hi - c * bs).clamp(min=0) * (valid & (c >= 0)).long()
    return int(win.sum().item() + rk.sum().item())


def decode_keys(idx, valid, lens, bs, lw):
    """|window U routed| per sequence for the query at lens-1."""
    qp = lens.long() - 1
    ls = qp - lw + 1
    win = torch.minimum(qp + 1, torch.full_like(qp, lw))
    c = idx.long()
    hi = torch.minimum(torch.minimum((c + 1) * bs, ls[:, None]), lens.long()[:, None])
    rk = (hi - c * bs).clamp(min=0) * (valid & (c >= 0)).long()
    return win + rk.sum(-1)


def decode_step_bytes(nkeys, lens, bs, d=W.D):
    """HBM bytes one decode step must move per layer: K and V of window U routed keys
    for every head, the query and the fp32 output, the k_bar rows the scores read and
    the tail block's index keys the refresh reads."""
    B = lens.numel()
    nblk = (lens.long() + bs - 1) // bs
    kv = float(nkeys.sum().item()) * W.H * W.D * 2 * 2
    qo = B * W.H * W.D * (2 + 4)
    kbar = float(nblk.sum().item()) * d * 4
    tail = float((lens.long() - (nblk - 1) * bs).sum().item()) * d * 4
    return kv, qo + kbar + tail


# ------------------------------------------------------------------ timing helpers

def time_steps(fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def time_kernel(fn, reps):
    """Average duration of fn's launches with HIP events on the current stream
    (the stream the kernels are enqueued on)."""
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # A spin kernel first keeps the GPU busy while the host enqueues every launch, so
    # that the event pair around the back-to-back launches brackets GPU work only (an
    # event pair per launch would add its own gaps).  The spin covers three times the
    # host time of one untimed call per launch (at least 100 us each): a spin shorter
    # than the enqueueing lets the GPU idle inside the bracket.
    t0 = time.perf_counter()
    fn(0)
    host = time.perf_counter() - t0
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.4e9 * (2e-3 + reps * max(100e-6, 3.0 * host))))
    a.record(st)
    for i in range(reps):
        fn(i)
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / reps


# ------------------------------------------------------------------ counter summaries

def read_counters():
    """{(workload, quantity): value} from the committed counter summary, or {} when it
    is missing or was measured on other kernel sources."""
    try:
        text = open(COUNTERS_FILE).read()
    except OSError:
        return {}, "no counter summary"
    m = re.findall(r"^kernel_source_sha\s+([0-9a-f]{16})\s*$", text, flags=re.M)
    if not m or m[-1] != kernel_source_hash():
        return {}, "counter summary measured on other kernel sources (stale)"
    vals = {}
    for wl, qty, v in re.findall(r"^per_launch\s+(\S+)\s+(\S+)\s+([0-9.eE+]+)", text, flags=re.M):
        vals[(wl, qty)] = float(v)
    return vals, None


# ------------------------------------------------------------------ prefill

def _prefill_inputs(cfg, copies):
    d = W.make_prefill(cfg, device="cuda")
    sets = [(d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"])]
    for _ in range(copies - 1):   # distinct buffers so repeated steps do not reuse the MALL
        sets.append(tuple(t.clone() for t in sets[0]))
    return d, sets


def _maxlen(d):
    cl = d.get("cu_list")
    return None if cl is None else max(b - a for a, b in zip(cl[:-1], cl[1:]))


def bench_prefill(cfg, steps, warmup, copies=3):
    log(f"[bench] prefill {cfg.name}: generating inputs")
    d, sets = _prefill_inputs(cfg, copies)
    cu = d.get("cu_seqlens")
    ml = _maxlen(d)
    hc = torch.zeros(W.D, device="cuda")
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)

    def step(i):
        qq, kk, vv, a, b = sets[i % len(sets)]
        return pipeline.prefill(qq, kk, vv, a, b, hc, cfg.bs, lb, W.IDX_SCALE, W.FLOOR,
                                W.SIGMA, cfg.cap, cfg.cap, scale, cu_seqlens=cu, max_seqlen=ml)

    out, (idx, bias, valid) = pipeline.prefill(*sets[0], hc, cfg.bs, lb, W.IDX_SCALE,
                                               W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale,
                                               cu_seqlens=cu, max_seqlen=ml, return_routing=True)
    torch.cuda.synchronize()
    if cu is None:
        pairs = sum(prefill_pairs(idx[b], valid[b], d["S"], cfg.bs, cfg.lw)
                    for b in range(d["B"]))
    else:
        cl = d["cu_list"]
        pairs = sum(prefill_pairs(idx[s0:s1], valid[s0:s1], s1 - s0, cfg.bs, cfg.lw)
                    for s0, s1 in zip(cl[:-1], cl[1:]))
    flops = 4.0 * W.D * W.H * pairs
    log(f"[bench] prefill {cfg.name}: {d['S']} tokens, {pairs} query-key pairs/head, "
        f"{flops / 1e9:.1f} GFLOP; timing {steps} steps")
    t_step = time_steps(step, steps, warmup)

    def attn(i):
        qq, kk, vv, _, _ = sets[i % len(sets)]
        ops.attn_prefill(qq, kk, vv, idx, bias, valid, cfg.bs, cfg.lw, scale, cu_seqlens=cu,
                         max_seqlen=ml)

    t_attn = time_kernel(attn, max(steps, 5))
    return dict(pairs=pairs, flops=flops, t_step=t_step, t_attn=t_attn, data=d,
                routing=(idx, bias, valid))


def prefill_entry(cfg, res, counters):
    fl, ta = res["flops"], res["t_attn"]
    tf = fl / ta / 1e12
    roof = {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "traffic": None, "kernel": "prefill attention (plan, sparse, tile)",
            "flop_per_launch": fl, "avg_launch_ms": round(ta * 1e3, 4)}
    tr = counters.get((cfg.name, "hbm_bytes"))
    if tr is not None:
        roof["traffic"] = int(tr)
    ex = counters.get((cfg.name, "mfma_flop"))
    if ex is not None:
        roof["executed_flop_per_launch"] = ex
        roof["executed_frac"] = round(ex / ta / 1e12 / PEAK_BF16_TFLOPS, 4)
    return {"workload": cfg.name, "value": round(fl / res["t_step"] / 1e12, 2),
            "unit": "TFLOP/s", "ms_per_step": round(res["t_step"] * 1e3, 4),
            "tokens": res["data"]["S"], "roofline": roof}


# ------------------------------------------------------------------ decode

def bench_decode(cfg, steps, warmup, copies=8):
    log(f"[bench] decode {cfg.name}: generating inputs")
    d = W.make_decode(cfg, device="cuda")
    hc = torch.zeros(W.D, device="cuda")
    lb = cfg.lw // cfg.bs
    nblk = (cfg.S + cfg.bs - 1) // cfg.bs
    scale = 1.0 / math.sqrt(W.D)
    # distinct caches: the per-step read set (~84 MB) must not stay in the 256 MB MALL
    sets = [(d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"])]
    for _ in range(copies - 1):
        sets.append(tuple(t.clone() for t in sets[0]))
    states = [pipeline.init_decode_state(s[4], hc, cfg.bs, nblk) for s in sets]
    args = (hc, cfg.bs, lb, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale)

    def step(i):
        return pipeline.decode_step(states[i % len(sets)], *sets[i % len(sets)], *args)

    out, (idx, bias, valid) = pipeline.decode_step(states[0], *sets[0], *args,
                                                   return_routing=True)
    torch.cuda.synchronize()
    lens = torch.full((cfg.B,), cfg.S, device="cuda")
    nkeys = decode_keys(idx[:, 0], valid[:, 0], lens, cfg.bs, cfg.lw)
    kv_bytes, other_bytes = decode_step_bytes(nkeys, lens, cfg.bs)
    log(f"[bench] decode {cfg.name}: {kv_bytes / 1e6:.1f} MB K/V per step; timing")
    t_step_eager = time_steps(step, max(steps, 20), warmup)
    # the same steps as a serving loop runs them: one captured graph per cache set
    graphs = [pipeline.DecodeGraph(states[i], *sets[i], *args) for i in range(len(sets))]
    t_step = time_steps(lambda i: graphs[i % len(graphs)].replay(), max(steps, 20), warmup)
    # the same replays timed on the device (the host enqueues ahead of the GPU)
    t_step_dev = time_kernel(lambda i: graphs[i % len(graphs)].replay(), max(steps, 20))
    # the step's own launches back to back, timed on the device: the kernels' time
    # without the graph launches' overhead between replays
    t_step_kern = time_kernel(step, max(steps, 20))

    def attn(i):
        qq, kk, vv, _, _ = sets[i % len(sets)]
        ops.attn_decode(qq, kk, vv, idx[:, 0], bias[:, 0], valid[:, 0], cfg.bs, cfg.lw, scale)

    t_attn = time_kernel(attn, max(steps, 20))
    return dict(kv_bytes=kv_bytes, other_bytes=other_bytes, t_step=t_step,
                t_step_eager=t_step_eager, t_step_dev=t_step_dev, t_step_kern=t_step_kern,
                t_attn=t_attn, data=d, routing=(idx, bias, valid))


def decode_entry(cfg, res, counters):
    step_bytes = res["kv_bytes"] + res["other_bytes"]
    gbs = step_bytes / res["t_step_kern"] / 1e9
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
            "kernel": "decode step (router + window + routed blocks, merge), its launches "
                      "back to back",
            "bytes_per_launch": step_bytes, "avg_launch_us": round(res["t_step_kern"] * 1e6, 2)}
    tr = counters.get((cfg.name, "hbm_bytes"))
    if tr is not None:
        roof["traffic"] = int(tr)
    qo = cfg.B * W.H * W.D * (2 + 4)
    sk = (res["kv_bytes"] + qo) / res["t_attn"] / 1e9
    return {"workload": cfg.name, "value": round(res["t_step"] * 1e6, 2), "unit": "us/step",
            "us_per_step_eager": round(res["t_step_eager"] * 1e6, 2),
            "us_per_step_device": round(res["t_step_dev"] * 1e6, 2),
            "us_per_step_device_note": "graph replays timed on the device (each replay adds "
                                       "the graph launch's overhead)",
            "step": "routing + attention, replayed as one HIP graph per cache set",
            "roofline": roof,
            "split_k_attention_only": {"achieved_GBps": round(sk, 1),
                                       "frac": round(sk / PEAK_HBM_GBS, 4),
                                       "avg_launch_us": round(res["t_attn"] * 1e6, 2),
                                       "kernel": "decode_attn + decode_merge on the step's "
                                                 "routing (not the product step)"}}


def bench_paged_decode(cfg, steps, warmup):
    """12 stacked layers of paged decode over B=32 sequences: one step = every layer's
    fused decode step, captured as one HIP graph."""
    lengths, table = W.paged_layout(cfg)
    layers = []
    hc = torch.zeros(W.D, device="cuda")
    lb = cfg.lw // cfg.bs
    nblk = int(table.shape[1])
    scale = 1.0 / math.sqrt(W.D)
    log(f"[bench] paged decode {cfg.name}: generating {cfg.layers} layers "
        f"({int(lengths.sum())} cached tokens each)")
    for layer in range(cfg.layers):
        d = W.make_paged_decode(cfg, "cuda", layer, lengths, table)
        st = pipeline.init_decode_state(d["idx_k"], hc, cfg.bs, nblk, seq_lens=d["seq_lens"],
                                        block_table=d["block_table"], page_size=cfg.bs)
        layers.append((d, st))
    kv_bytes = other = 0.0
    for d, st in layers:
        _, (idx, bias, valid) = pipeline.decode_step(
            st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs, lb, W.IDX_SCALE,
            W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale, seq_lens=d["seq_lens"],
            block_table=d["block_table"], page_size=cfg.bs, return_routing=True)
        nk = decode_keys(idx[:, 0], valid[:, 0], d["seq_lens"], cfg.bs, cfg.lw)
        a, b = decode_step_bytes(nk, d["seq_lens"], cfg.bs)
        kv_bytes += a
        other += b

    def step(i=0):
        for d, st in layers:
            pipeline.decode_step(st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs,
                                 lb, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale,
                                 seq_lens=d["seq_lens"], block_table=d["block_table"],
                                 page_size=cfg.bs)

    t_step_eager = time_steps(step, steps, warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    t_step = time_steps(lambda i: graph.replay(), steps, warmup)
    t_dev = time_kernel(lambda i: graph.replay(), steps)
    return dict(t_step=t_step, t_step_eager=t_step_eager, t_step_dev=t_dev, kv_bytes=kv_bytes,
                other_bytes=other, lengths=lengths, table=table, layers=layers)


def paged_entry(cfg, res, counters):
    step_bytes = res["kv_bytes"] + res["other_bytes"]
    gbs = step_bytes / res["t_step_dev"] / 1e9
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
            "kernel": f"{cfg.layers} x decode step (route + window, routed blocks, merge)",
            "bytes_per_launch": step_bytes, "avg_launch_us": round(res["t_step_dev"] * 1e6, 1)}
    tr = counters.get((cfg.name, "hbm_bytes"))
    if tr is not None:
        roof["traffic"] = int(tr)
    return {"workload": cfg.name, "value": round(res["t_step"] * 1e6, 1),
            "unit": "us per 12-layer step", "us_per_step_eager": round(res["t_step_eager"] * 1e6, 1),
            "us_per_step_device": round(res["t_step_dev"] * 1e6, 1),
            "cached_tokens_per_layer": int(res["lengths"].sum()), "roofline": roof}


# ------------------------------------------------------------------ training step

TRAIN_NAME = "train_s27300_lw1024_k16"


def bench_train(steps, warmup):
    """One training step of the routed attention at 27,300 tokens (block 64, window
    1,024, k = 16): training routing of the block scores, fused attention forward,
    its backward (dq, dk, dv, bias gradient) and the routing backward to the scores.
    Stage-0 scores come from the inference kernels (their autograd runs in PyTorch in
    DashAttention and is not timed)."""
    cfg = W.PREFILL_27300
    log(f"[bench] training step {TRAIN_NAME}: generating inputs")
    d = W.make_prefill(cfg, device="cuda")
    hc = torch.zeros(W.D, device="cuda")
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)
    kb = ops.kbar(d["idx_k"], hc, cfg.bs)
    z = ops.block_scores(d["idx_q"], kb, cfg.bs, lb)
    q, k, v = d["q"], d["k"], d["v"]
    gen = torch.Generator(device="cuda").manual_seed(11)
    dout = torch.randn(q.shape, device="cuda", generator=gen).bfloat16()
    K = cfg.cap

    def fwd_bwd(i=0):
        idx, bias, valid, topv, stat = ops.train_route_raw(z, None, W.IDX_SCALE, W.FLOOR,
                                                           W.SIGMA, K)
        out, lse = ops.attn_prefill(q, k, v, idx, bias, valid, cfg.bs, cfg.lw, scale,
                                    return_lse=True)
        dq, dk, dv, db = ops.attn_prefill_backward(q, k, v, out, lse, dout, idx, bias, valid,
                                                   cfg.bs, cfg.lw, scale)
        ops.train_route_backward(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, idx, valid, topv, stat,
                                 db)

    idx, bias, valid, topv, stat = ops.train_route_raw(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, K)
    torch.cuda.synchronize()
    pairs = prefill_pairs(idx[0], valid[0], d["S"], cfg.bs, cfg.lw)
    fwd_flops = 4.0 * W.D * W.H * pairs
    bwd_flops = 2.5 * fwd_flops            # S recomputed, dP, dV, dK, dQ: five products
    t_step = time_steps(fwd_bwd, steps, warmup)
    out, lse = ops.attn_prefill(q, k, v, idx, bias, valid, cfg.bs, cfg.lw, scale, return_lse=True)

    def bwd(i):
        ops.attn_prefill_backward(q, k, v, out, lse, dout, idx, bias, valid, cfg.bs, cfg.lw,
                                  scale)

    t_bwd = time_kernel(bwd, max(steps, 5))
    t_route = time_kernel(lambda i: ops.train_route_raw(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA,
                                                        K), max(steps, 5))
    tf = bwd_flops / t_bwd / 1e12
    log(f"[bench] training step: {t_step * 1e3:.3f} ms, attention backward {t_bwd * 1e3:.3f} ms")
    return dict(cfg=cfg, data=d, z=z, K=K, pairs=pairs, t_step=t_step, t_bwd=t_bwd,
                t_route=t_route,
                entry={"workload": TRAIN_NAME,
                       "value": round((fwd_flops + bwd_flops) / t_step / 1e12, 2),
                       "unit": "TFLOP/s", "ms_per_step": round(t_step * 1e3, 4),
                       "step": "training routing + attention forward + attention backward + "
                               "routing backward, one sequence of 27,300 tokens, k = 16",
                       "train_route_forward_us": round(t_route * 1e6, 2),
                       "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                                    "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None,
                                    "kernel": "attention backward (delta, plan, dK/dV, dQ, "
                                              "bias gradient)",
                                    "flop_per_launch": bwd_flops,
                                    "avg_launch_ms": round(t_bwd * 1e3, 4)}})


def train_entry(res, counters):
    e = res["entry"]
    roof = e["roofline"]
    tr = counters.get((TRAIN_NAME, "hbm_bytes"))
    if tr is not None:
        roof["traffic"] = int(tr)
    ex = counters.get((TRAIN_NAME, "mfma_flop"))
    if ex is not None:
        roof["executed_flop_per_launch"] = ex
        roof["executed_frac"] = round(ex / res["t_bwd"] / 1e12 / PEAK_BF16_TFLOPS, 4)
    return e


def cpu_train_baseline(res, rows=512, reps=3):
    """The oracle's training path on this host, differentiated by torch autograd: the
    training routing and dense attention for the last `rows` query rows, forward and
    backward."""
    from oracle import dash_oracle as O
    cfg, d = res["cfg"], res["data"]
    S = d["S"]
    r0 = S - rows
    scale = 1.0 / math.sqrt(W.D)
    q, k, v = d["q"].float().cpu(), d["k"].float().cpu(), d["v"].float().cpu()
    z = res["z"][:, r0:].cpu()

    def run():
        zz = z.clone().requires_grad_()
        qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
        ti, bi, va = O.train_route_select(zz, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, res["K"])
        full = torch.zeros(1, S, ti.shape[-1], dtype=torch.long)
        fv = torch.zeros(1, S, ti.shape[-1], dtype=torch.bool)
        full[:, r0:], fv[:, r0:] = ti, va
        fb = torch.cat([torch.zeros(1, r0, ti.shape[-1]), bi], dim=1)
        out = O.dense_attend(qq, kk, vv, full, fb, fv, cfg.bs, cfg.lw, scale, rows=(r0, S))
        out.sum().backward()
        return ti, va

    t = _median_time(run, reps)
    ti, va = run()
    pairs = prefill_pairs(torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.long), ti[0]]),
                          torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.bool), va[0]]),
                          S, cfg.bs, cfg.lw)
    pairs -= sum(min(t_ + 1, cfg.lw) for t_ in range(r0))
    sample = (f"oracle fp32 training routing + dense attention, forward and autograd backward, "
              f"on the last {rows} of {S} query rows; median of {reps} after 1 warm-up; "
              f"{t:.2f} s per sample")
    return _cpu_fields(14.0 * W.D * W.H * pairs / t / 1e12, "TFLOP/s", sample)


# ------------------------------------------------------------------ page-aware candidates

PAGES_NAME = "page_candidates_s27300_100pages"


def ocr_prompt_ids(pages_n=100, per_page=W.PAGE_TOKENS, seed=6):
    """Token ids [1, L] of a 100-page OCR prompt: BOS, per page a <PAGE> marker and 273
    image tokens, an instruction, then the response: per page a marker and text.  Ids:
    1 BOS, 5 image, 9 marker, 7 text."""
    g = torch.Generator().manual_seed(seed)
    ids = [1]
    for _ in range(pages_n):
        ids += [9] + [5] * per_page
    ids += [7] * 8
    for _ in range(pages_n):
        ids += [9] + [7] * int(torch.randint(20, 60, (1,), generator=g))
    return torch.tensor([ids], dtype=torch.int64)


def bench_pages(steps):
    """Prefill candidates of a 100-page prompt (page ids, block pages, [S, nblk] rows) and
    the decode allow row of its batch of 8 copies."""
    from ananta_ocr_amd import pages
    ids = ocr_prompt_ids().to("cuda")
    S = ids.shape[1]
    bs = 64
    nblk = (S + bs - 1) // bs
    pos = torch.arange(S, device="cuda", dtype=torch.int32)[None]
    out = torch.empty(1, S, nblk, dtype=torch.bool, device="cuda")

    def prefill(i=0):
        img, ipi, qpi, _ = pages.page_ids(ids, 5, 9, S, W.PAGE_TOKENS, True)
        pages.block_cand(pos, nblk, bs, img, ipi, qpi, out=out)

    prefill()
    t_pre = time_kernel(prefill, max(steps, 10))
    ids8 = ids.expand(8, -1).contiguous()
    st = pages.DecodePageState(ids8, 5, 9, bs)
    new = torch.full((8,), 7, dtype=torch.int64, device="cuda")
    arow = torch.empty(8, nblk + 1, dtype=torch.bool, device="cuda")
    t_dec = time_kernel(lambda i: st.allow(new, S + 1, out=arow), max(steps, 20))
    nbytes = S * 8 * 3 + S * (1 + 4 + 4) * 2 + S * nblk     # ids reads, page ids, rows
    gbs = nbytes / t_pre / 1e9
    return {"workload": PAGES_NAME, "value": round(t_pre * 1e6, 2), "unit": "us per prefill",
            "tokens": S, "blocks": nblk,
            "decode_allow_us": round(t_dec * 1e6, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                         "kernel": "page_ids + block_pages + block_cand",
                         "bytes_per_launch": nbytes, "avg_launch_us": round(t_pre * 1e6, 2)}}


FRONT_NAME = W.FRONT_NAME


def front_bytes(S, hidden, bs):
    """Algorithmic HBM bytes of one fused front-end call: hidden states and weights read,
    bf16 cos/sin read, idx_q / idx_k and the block summaries written."""
    nblk = (S + bs - 1) // bs
    return S * hidden * 2 + 2 * W.D * hidden * 2 + 2 * S * W.D * 2 + 2 * S * W.D * 4 + \
        nblk * W.D * 4


def bench_front(steps):
    """The fused router front end (projections, norms, RoPE, guards, block summaries in
    one launch) against the unfused sequence it replaces (nan_to_num, one library GEMM
    for both projections, the norm / RoPE kernel, the block-summary kernel)."""
    d = W.make_front(device="cuda")
    S, hid, bs = W.FRONT_S, W.FRONT_HIDDEN, W.FRONT_BS
    wpack = ops.router_front_pack(d["wq"], d["wk"])
    wcat = torch.cat([d["wq"], d["wk"]], 0)

    def fused(i=0):
        ops.router_front(d["hs"], d["wq"], d["wk"], d["nq"], d["nk"], 1e-6, d["cos"], d["sin"],
                         head_cls=d["hc"], block_size=bs, w_pack=wpack)

    def unfused(i=0):
        h = torch.nan_to_num(d["hs"], nan=0.0, posinf=0.0, neginf=0.0)
        proj = torch.nn.functional.linear(h, wcat)
        iq, ik = ops.router_qk_norm(proj, d["nq"], d["nk"], 1e-6, d["cos"], d["sin"])
        ops.kbar(ik, d["hc"], bs)

    for _ in range(3):                    # first calls (library GEMM set-up) off the clock
        fused()
        unfused()
    torch.cuda.synchronize()
    t = time_kernel(fused, max(steps, 10))
    t_un = time_kernel(unfused, max(steps, 10))
    nbytes = front_bytes(S, hid, bs)
    gbs = nbytes / t / 1e9
    flop = 2.0 * S * hid * 2 * W.D
    return {"workload": FRONT_NAME, "value": round(t * 1e6, 2), "unit": "us per call",
            "tokens": S, "hidden": hid, "block": bs,
            "unfused_us": round(t_un * 1e6, 2),
            "mfma_tflops": round(flop / t / 1e12, 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                         "kernel": "router_front_kernel", "bytes_per_launch": nbytes,
                         "avg_launch_us": round(t * 1e6, 2)}}


def front_entry(res, counters):
    tr = counters.get((FRONT_NAME, "hbm_bytes"))
    if tr is not None:
        res["roofline"]["traffic"] = int(tr)
    return res


def cpu_front_baseline(rows=2048, reps=3):
    """The oracle's router_qk (float64 projections rounded to bf16, then the norm and RoPE
    of the reference in fp32/bf16) and k_bar pooling for the last `rows` tokens, scaled to
    the whole sequence (the work is linear in the tokens)."""
    from oracle import dash_oracle as O
    d = W.make_front()
    S, bs = W.FRONT_S, W.FRONT_BS
    sl = slice(S - rows, S)

    def run():
        iq, ik = O.router_qk(d["hs"][:, sl], d["wq"], d["wk"], d["nq"], d["nk"], 1e-6,
                             d["cos"][:, sl], d["sin"][:, sl])
        O.kbar_headcls(ik, d["hc"], bs)

    t = _median_time(run, reps) * S / rows
    return _cpu_fields(round(t * 1e6, 1), "us per call",
                       f"oracle router_qk + kbar_headcls on the last {rows} of {S} tokens, "
                       f"scaled by {S / rows:.2f}; median of {reps} after 1 warm-up")


# ------------------------------------------------------------------ CPU baselines

def _median_time(run, reps):
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _cpu_fields(value, unit, sample):
    model, phys, logical = host_cpu()
    return dict(value=value, unit=unit, cores=torch.get_num_threads(), kind="port",
                sample=sample, cpu_model=model, physical_cores=phys, logical_cpus=logical)


def cpu_prefill_baseline(res, cfg, rows=None, reps=3, docs=None):
    """The oracle (the reference's torch path restated in fp32) on this host: k_bar and
    scores for the whole sequence, routing and dense attention for the last `rows` query
    rows (None: every row, the whole workload); for packed inputs, whole documents
    (`docs` of them) on their own block grids."""
    from oracle import dash_oracle as O
    d = res["data"]
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)
    q, k, v = d["q"].float().cpu(), d["k"].float().cpu(), d["v"].float().cpu()
    iq, ik = d["idx_q"].cpu(), d["idx_k"].cpu()
    if d.get("cu_list") is not None:
        cl = d["cu_list"][:docs + 1]

        def run():
            out = []
            for s0, s1 in zip(cl[:-1], cl[1:]):
                out.append(O.prefill_pipeline(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1],
                                              iq[:, s0:s1], ik[:, s0:s1], torch.zeros(W.D),
                                              cfg.bs, lb, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap,
                                              cfg.cap, scale)[1:])
            return out

        t = _median_time(run, reps)
        pairs = 0
        for (s0, s1), (ti, bi, va) in zip(zip(cl[:-1], cl[1:]), run()):
            pairs += prefill_pairs(ti[0], va[0], s1 - s0, cfg.bs, cfg.lw)
        sample = (f"oracle fp32 on the first {len(cl) - 1} of {len(d['cu_list']) - 1} documents "
                  f"({cl[-1]} of {d['S']} tokens), each on its own block grid; median of {reps} "
                  f"after 1 warm-up; {t:.2f} s per sample")
        return _cpu_fields(4.0 * W.D * W.H * pairs / t / 1e12, "TFLOP/s", sample)
    S = d["S"]
    r0 = 0 if rows is None else max(0, S - rows)

    def run():
        kb, cv = O.kbar_headcls(ik, torch.zeros(W.D), cfg.bs)
        z = O.block_scores_headcls(iq[:, r0:], kb, cv, torch.arange(r0, S)[None], cfg.bs, lb)
        ti, bi, va = O.infer_route_select(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap,
                                          cfg.cap)
        full = torch.zeros(1, S, ti.shape[-1], dtype=torch.long)
        fb = torch.zeros(1, S, ti.shape[-1])
        fv = torch.zeros(1, S, ti.shape[-1], dtype=torch.bool)
        full[:, r0:], fb[:, r0:], fv[:, r0:] = ti, bi, va
        O.dense_attend(q, k, v, full, fb, fv, cfg.bs, cfg.lw, scale, rows=(r0, S))
        return ti, va

    t = _median_time(run, reps)
    ti, va = run()
    pairs = prefill_pairs(torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.long), ti[0]]),
                          torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.bool), va[0]]),
                          S, cfg.bs, cfg.lw)
    pairs -= sum(min(t_ + 1, cfg.lw) for t_ in range(r0))
    rows_txt = (f"all {S} query rows" if r0 == 0 else
                f"the last {S - r0} of {S} query rows (full k_bar/scores over the sequence)")
    sample = (f"oracle fp32 on {rows_txt}; dense masked SDPA as the reference's CPU path; "
              f"median of {reps} after 1 warm-up; {t:.2f} s per sample")
    return _cpu_fields(4.0 * W.D * W.H * pairs / t / 1e12, "TFLOP/s", sample)


def cpu_decode_baseline(res, cfg, reps=3):
    """The oracle decode step (k_bar over the whole cache, as the reference rebuilds it
    every step, scores, routing, dense fp32 attention over the cache)."""
    from oracle import dash_oracle as O
    d = res["data"]
    q = d["q"].float().cpu()[:, :, None]
    k, v = d["k"].cpu(), d["v"].cpu()
    iq, ik = d["idx_q"].cpu(), d["idx_k"].cpu()
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)

    def run():
        O.decode_pipeline(q, k, v, iq, ik, torch.zeros(W.D), cfg.bs, lb, W.IDX_SCALE, W.FLOOR,
                          W.SIGMA, cfg.cap, cfg.cap, scale)

    t = _median_time(run, reps)
    return _cpu_fields(t * 1e6, "us/step",
                       f"oracle fp32 decode step on all {cfg.B} sequences ({cfg.S} cached tokens "
                       f"each); median of {reps} after 1 warm-up")


def cpu_paged_baseline(res, cfg, nseq=8, reps=3):
    """The oracle decode step of layer 0 for `nseq` of the 32 sequences, on their caches
    gathered out of the pages (the reference's decode reads a contiguous cache), scaled
    to 32 sequences x 12 layers."""
    from oracle import dash_oracle as O
    d, _ = res["layers"][0]
    lengths, table = res["lengths"], res["table"]
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)
    seqs = []
    for b in range(nseq):
        L = int(lengths[b])
        npg = (L + cfg.bs - 1) // cfg.bs
        pg = table[b, :npg].long().to(d["k"].device)
        kk = d["k"][pg].reshape(-1, W.H, W.D)[:L].permute(1, 0, 2)[None].cpu()
        vv = d["v"][pg].reshape(-1, W.H, W.D)[:L].permute(1, 0, 2)[None].cpu()
        ik = d["idx_k"][pg].reshape(-1, W.D)[:L][None].cpu()
        seqs.append((d["q"][b:b + 1].float().cpu()[:, :, None], kk, vv,
                     d["idx_q"][b:b + 1].cpu(), ik))

    def run():
        for q, kk, vv, iq, ik in seqs:
            O.decode_pipeline(q, kk, vv, iq, ik, torch.zeros(W.D), cfg.bs, lb, W.IDX_SCALE,
                              W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale)

    t = _median_time(run, reps)
    per_step = t / nseq * cfg.B * cfg.layers
    return _cpu_fields(per_step * 1e6, "us per 12-layer step",
                       f"oracle fp32 decode step of layer 0 for {nseq} of {cfg.B} sequences "
                       f"(caches gathered from the pages), scaled x{cfg.B / nseq:.0f} sequences "
                       f"x{cfg.layers} layers; median of {reps} after 1 warm-up; "
                       f"{t:.2f} s per sample")


# ------------------------------------------------------------------ counter probes

def counter_probe(name):
    """One launch of one workload's measured kernels, for hardware-counter runs: after
    warm-up, a 256 MiB device-to-device copy (the counters' calibration), then one
    launch of the workload's product kernels, separated by synchronisations.  The last
    dispatches in the counter output belong to that launch."""
    dev = "cuda"
    hc = torch.zeros(W.D, device=dev)
    scale = 1.0 / math.sqrt(W.D)
    cfgs = {c.name: c for c in (W.PREFILL_2730, W.PREFILL_27300, W.PACKED_16DOC, W.DECODE_B8,
                                W.PAGED_12L)}
    cfgs[TRAIN_NAME] = TRAIN_NAME
    cfgs[FRONT_NAME] = FRONT_NAME
    cfg = cfgs[name]
    if cfg == FRONT_NAME:
        d = W.make_front(device=dev)
        wpack = ops.router_front_pack(d["wq"], d["wk"])

        def launch():
            ops.router_front(d["hs"], d["wq"], d["wk"], d["nq"], d["nk"], 1e-6, d["cos"],
                             d["sin"], head_cls=d["hc"], block_size=W.FRONT_BS, w_pack=wpack)
    elif cfg == TRAIN_NAME:
        c27 = W.PREFILL_27300
        d = W.make_prefill(c27, device=dev)
        kb = ops.kbar(d["idx_k"], hc, c27.bs)
        z = ops.block_scores(d["idx_q"], kb, c27.bs, c27.lw // c27.bs)
        idx, bias, valid, _, _ = ops.train_route_raw(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA,
                                                     c27.cap)
        out, lse = ops.attn_prefill(d["q"], d["k"], d["v"], idx, bias, valid, c27.bs, c27.lw,
                                    scale, return_lse=True)
        gen = torch.Generator(device=dev).manual_seed(11)
        dout = torch.randn(d["q"].shape, device=dev, generator=gen).bfloat16()

        def launch():
            ops.attn_prefill_backward(d["q"], d["k"], d["v"], out, lse, dout, idx, bias, valid,
                                      c27.bs, c27.lw, scale)
    elif isinstance(cfg, W.Prefill):
        d = W.make_prefill(cfg, device=dev)
        cu, ml = d.get("cu_seqlens"), _maxlen(d)
        _, (idx, bias, valid) = pipeline.prefill(d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"],
                                                 hc, cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE,
                                                 W.FLOOR, W.SIGMA, cfg.cap, cfg.cap,
                                                 cu_seqlens=cu, max_seqlen=ml,
                                                 return_routing=True)

        def launch():
            ops.attn_prefill(d["q"], d["k"], d["v"], idx, bias, valid, cfg.bs, cfg.lw, scale,
                             cu_seqlens=cu, max_seqlen=ml)
    elif not cfg.paged:
        d = W.make_decode(cfg, device=dev)
        nblk = (cfg.S + cfg.bs - 1) // cfg.bs
        st = pipeline.init_decode_state(d["idx_k"], hc, cfg.bs, nblk)

        def launch():
            pipeline.decode_step(st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs,
                                 cfg.lw // cfg.bs, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap,
                                 cfg.cap, scale)
    else:
        lengths, table = W.paged_layout(cfg)
        layers = []
        for layer in range(cfg.layers):
            dd = W.make_paged_decode(cfg, dev, layer, lengths, table)
            st = pipeline.init_decode_state(dd["idx_k"], hc, cfg.bs, int(table.shape[1]),
                                            seq_lens=dd["seq_lens"],
                                            block_table=dd["block_table"], page_size=cfg.bs)
            layers.append((dd, st))

        def launch():
            for dd, st in layers:
                pipeline.decode_step(st, dd["q"], dd["k"], dd["v"], dd["idx_q"], dd["idx_k"], hc,
                                     cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE, W.FLOOR, W.SIGMA,
                                     cfg.cap, cfg.cap, scale, seq_lens=dd["seq_lens"],
                                     block_table=dd["block_table"], page_size=cfg.bs)
    for _ in range(2):
        launch()
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    launch()
    torch.cuda.synchronize()
    log(f"[bench] counter probe {name}: copy {CALIB_BYTES} B, then one launch")


# Kernels of one launch of each workload, and how many of each one launch dispatches.
PROBE_KERNELS = {
    "prefill": ["prefill_clear_kernel", "prefill_plan_kernel", "prefill_scan_kernel",
                "prefill_scatter_kernel", "prefill_sparse_kernel", "prefill_tile_kernel"],
    "decode": ["decode_route_window_kernel", "decode_routed_kernel", "decode_step_merge_kernel"],
    "front": ["router_front_kernel"],
    "train": ["bwd_delta_kernel", "prefill_clear_kernel", "prefill_plan_kernel",
              "prefill_scan_kernel", "prefill_scatter_kernel", "bwd_kv_kernel", "bwd_q_kernel",
              "bwd_dbias_kernel"],
}


def summarize_counters(dirs):
    """Per-launch HBM bytes and executed MFMA FLOP from rocprofv3 counter CSVs (one
    directory per probe run; the run's workload is named in its directory).  Prints the
    summary lines that profiles/counters_per_launch.txt keeps."""
    lines = []
    for dr in dirs:
        files = glob.glob(os.path.join(dr, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            log(f"no counter_collection.csv under {dr}")
            continue
        rows = []
        for f in files:
            with open(f) as fh:
                rows.extend(csv.DictReader(fh))
        rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0)))
        # one value per dispatch and counter
        per = {}
        for r in rows:
            key = (int(r["Dispatch_Id"]), r["Kernel_Name"], r["Counter_Name"])
            per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
        counters = sorted({k[2] for k in per})
        names = [c.name for c in (W.PREFILL_2730, W.PREFILL_27300, W.PACKED_16DOC, W.DECODE_B8,
                                  W.PAGED_12L)] + [TRAIN_NAME, FRONT_NAME]
        wl = next((nm for nm in names if nm in dr), None)
        if wl is None:
            log(f"{dr}: directory names no workload")
            continue
        kind = "train" if wl == TRAIN_NAME else "front" if wl == FRONT_NAME else \
            "decode" if "decode" in wl else "prefill"
        disp = sorted({(k[0], k[1]) for k in per})
        copy = [x for x in disp if "copyBuffer" in x[1]
                and per.get((x[0], x[1], counters[0]), 0.0) > 1024]
        if not copy:
            log(f"{dr}: no calibration copy found")
            continue
        cid = copy[-1][0]
        after = [x for x in disp if x[0] > cid]
        for cn in counters:
            calib = per.get((cid, copy[-1][1], cn))
            tot = 0.0
            agg = {}                      # kernel -> (dispatches, sum)
            for did, kn in after:
                if any(k in kn for k in PROBE_KERNELS[kind]):
                    v = per.get((did, kn, cn), 0.0)
                    tot += v
                    name = kn.split('(')[0].replace('void ', '').replace('dash::', '')
                    n0, v0 = agg.get(name, (0, 0.0))
                    agg[name] = (n0 + 1, v0 + v)
            parts = [f"{k}{'' if n == 1 else f' x{n}'} {v:.0f}" for k, (n, v) in agg.items()]
            if cn in ("FETCH_SIZE", "WRITE_SIZE"):
                factor = calib * 1024 / CALIB_BYTES if calib else float("nan")
                nbytes = tot * 1024 / factor
                lines.append(f"# {wl} {cn}: copy {calib:.0f} KiB (factor {factor:.5f}); "
                             f"{'; '.join(parts)} | {tot:.0f} KiB -> {nbytes / 1e6:.1f} MB")
                lines.append(f"per_launch {wl} {cn.lower()}_bytes {nbytes:.0f}")
            elif cn == "SQ_INSTS_VALU_MFMA_MOPS_BF16":
                lines.append(f"# {wl} {cn}: {'; '.join(parts)} | {tot:.0f} MOPS x 512 FLOP")
                lines.append(f"per_launch {wl} mfma_flop {tot * 512:.0f}")
            else:
                lines.append(f"# {wl} {cn}: {'; '.join(parts)} | {tot:.0f}")
    # HBM bytes = reads + writes where both were measured
    vals = {}
    for l in lines:
        m = re.match(r"per_launch (\S+) (\S+) (\S+)", l)
        if m:
            vals[(m.group(1), m.group(2))] = float(m.group(3))
    for wl in sorted({k[0] for k in vals}):
        f, w = vals.get((wl, "fetch_size_bytes")), vals.get((wl, "write_size_bytes"))
        if f is not None and w is not None:
            lines.append(f"per_launch {wl} hbm_bytes {f + w:.0f}")
    lines.append(f"kernel_source_sha {kernel_source_hash()}")
    print("\n".join(lines))


# ------------------------------------------------------------------ main

ALL = [W.PREFILL_27300, W.DECODE_B8, W.PREFILL_2730, W.PACKED_16DOC, W.PAGED_12L]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma-separated workload names to time (default: all five)")
    ap.add_argument("--counter-probe", default=None, metavar="WORKLOAD",
                    help="run one launch of WORKLOAD's kernels for a counter run and exit")
    ap.add_argument("--summarize-counters", nargs="+", default=None, metavar="DIR",
                    help="print per-launch figures from rocprofv3 counter directories")
    args = ap.parse_args()
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.counter_probe:
        torch.cuda.set_device(0)
        counter_probe(args.counter_probe)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this benchmark measures one GPU only (no figure at several GPUs is "
              "produced; the path's sharding is design only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    torch.backends.cuda.matmul.allow_tf32 = False
    only = set(filter(None, args.only.split(",")))
    todo = [c for c in ALL if not only or c.name in only]
    if only and not todo and not ({PAGES_NAME, TRAIN_NAME, FRONT_NAME} & only):
        sys.exit(f"bench.py: unknown workload(s) {sorted(only)}")
    counters, cnote = read_counters()
    res, entries = {}, {}
    for cfg in todo:
        if isinstance(cfg, W.Prefill):
            res[cfg.name] = bench_prefill(cfg, args.steps, args.warmup,
                                          copies=1 if cfg.doc_pages or cfg is W.PACKED_16DOC
                                          else 3)
            entries[cfg.name] = prefill_entry(cfg, res[cfg.name], counters)
        elif cfg.paged:
            res[cfg.name] = bench_paged_decode(cfg, max(3, args.steps // 2), 1)
            entries[cfg.name] = paged_entry(cfg, res[cfg.name], counters)
        else:
            res[cfg.name] = bench_decode(cfg, args.steps, args.warmup)
            entries[cfg.name] = decode_entry(cfg, res[cfg.name], counters)
    if not args.no_cpu:
        log("[bench] CPU baselines (oracle on host cores)")
        for cfg in todo:
            r = res[cfg.name]
            if cfg is W.PACKED_16DOC:
                cb = cpu_prefill_baseline(r, cfg, docs=3)
            elif isinstance(cfg, W.Prefill):
                cb = cpu_prefill_baseline(r, cfg)
            elif cfg.paged:
                cb = cpu_paged_baseline(r, cfg)
            else:
                cb = cpu_decode_baseline(r, cfg)
            entries[cfg.name]["cpu_baseline"] = cb
    if not only or TRAIN_NAME in only:
        tr = bench_train(max(3, args.steps // 2), 1)
        entries[TRAIN_NAME] = train_entry(tr, counters)
        if not args.no_cpu:
            entries[TRAIN_NAME]["cpu_baseline"] = cpu_train_baseline(tr)
    if not only or PAGES_NAME in only:
        entries[PAGES_NAME] = bench_pages(args.steps)
        if not args.no_cpu:
            from oracle import dash_oracle as O
            ids = ocr_prompt_ids()
            S = ids.shape[1]
            nblk = (S + 63) // 64

            def cpu_pages():
                itm, ipi, qpi = O.page_aware_ids(ids, 5, 9, S, W.PAGE_TOKENS, True)
                for c0 in range(0, S, 2048):             # the reference's query chunks
                    c1 = min(c0 + 2048, S)
                    O.kl_candidate_mask(torch.arange(c0, c1)[None], nblk, itm, 1, c1 - c0, 64,
                                        ipi, qpi)

            t = _median_time(cpu_pages, 3)
            entries[PAGES_NAME]["cpu_baseline"] = _cpu_fields(
                t * 1e6, "us per prefill", "oracle page ids and candidate rows of the same "
                "100-page prompt in 2,048-query chunks; median of 3 after 1 warm-up")
    if not only or FRONT_NAME in only:
        entries[FRONT_NAME] = front_entry(bench_front(args.steps), counters)
        if not args.no_cpu:
            entries[FRONT_NAME]["cpu_baseline"] = cpu_front_baseline()
    head = entries.get(W.PREFILL_27300.name)
    if head is None:                      # a partial run: the first workload timed
        head = next(iter(entries.values()))
    hcfg = next((c for c in ALL if c.name == head["workload"]), None)
    if hcfg is not None:
        hconf = {"workload": hcfg.name, "B": hcfg.B, "seq_len": hcfg.S, "heads": W.H,
                 "head_dim": W.D, "block": hcfg.bs, "window": hcfg.lw,
                 "routed_cap": hcfg.cap, "parallelism": "single-gpu"}
    else:
        hconf = {"workload": head["workload"], "parallelism": "single-gpu"}
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head.get("ms_per_step", round(head["value"] / 1e3, 4)),
        "higher_is_better": head["unit"] == "TFLOP/s",
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": hconf,
        "roofline": head["roofline"],
    }
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
    line["workloads"] = {k: v for k, v in entries.items() if k != head["workload"]}
    if cnote:
        line["counters_note"] = cnote
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
