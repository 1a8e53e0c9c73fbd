"""DASH attention benchmark on one MI355X.

Headline: one DASH prefill pass (k_bar -> block scores -> entmax routing -> fused
block-sparse attention) over B=1, 27,300 tokens (100 pages x 273), 10 heads,
head_dim 128, 64-token blocks, 1,024-token window, 16 routed blocks, in bf16 with
fp32 accumulation; reported as TFLOP/s of algorithmic attention work
(4*D*H*sum_t |window(t) U routed(t)|, counted from the routing the pass emits).
Beside it: the decode step (B=8 sequences of 27,300 cached tokens, 1,024 window,
16 routed blocks) in microseconds, each with the roofline of its dominant
kernel, and the CPU oracle timed on a bounded sample on this host.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--extras]
"""

import argparse
import json
import math
import os
import statistics
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


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ work counting

def prefill_pairs(idx, valid, S, bs, lw, lens=None):
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
    # event pair per launch would add its own gaps).
    torch.cuda._sleep(int(2.4e9 * 2e-3 + reps * 2.4e9 * 100e-6))
    a.record(st)
    for i in range(reps):
        fn(i)
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / reps


# ------------------------------------------------------------------ prefill

def bench_prefill(cfg, steps, warmup, copies=3):
    dev = "cuda"
    log(f"[bench] prefill {cfg.name}: generating inputs")
    d = W.make_prefill(cfg, device=dev)
    q, k, v, iq, ik = d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"]
    cu = d.get("cu_seqlens")
    sets = [(q, k, v, iq, ik)]
    for _ in range(copies - 1):   # distinct buffers so repeated steps do not reuse the MALL
        sets.append(tuple(t.clone() for t in sets[0]))
    hc = torch.zeros(W.D, device=dev)
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)

    def step(i):
        qq, kk, vv, a, b = sets[i % len(sets)]
        return pipeline.prefill(qq, kk, vv, a, b, hc, cfg.bs, lb, W.IDX_SCALE, W.FLOOR,
                                W.SIGMA, cfg.cap, cfg.cap, scale, cu_seqlens=cu)

    out, (idx, bias, valid) = pipeline.prefill(q, k, v, iq, ik, hc, cfg.bs, lb, W.IDX_SCALE,
                                               W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale,
                                               cu_seqlens=cu, return_routing=True)
    torch.cuda.synchronize()
    if cu is None:
        pairs = sum(prefill_pairs(idx[b], valid[b], d["S"], cfg.bs, cfg.lw)
                    for b in range(d["B"]))
    else:
        cl = d["cu_list"]
        pairs = sum(prefill_pairs(idx[s0:s1], valid[s0:s1], s1 - s0, cfg.bs, cfg.lw)
                    for s0, s1 in zip(cl[:-1], cl[1:]))
    flops = 4.0 * W.D * W.H * pairs
    log(f"[bench] prefill {cfg.name}: {pairs} query-key pairs/head, "
        f"{flops / 1e9:.1f} GFLOP; timing {steps} steps")
    t_step = time_steps(step, steps, warmup)

    def attn(i):
        qq, kk, vv, _, _ = sets[i % len(sets)]
        ops.attn_prefill(qq, kk, vv, idx, bias, valid, cfg.bs, cfg.lw, scale, cu_seqlens=cu)

    t_attn = time_kernel(attn, max(steps, 5))
    return dict(pairs=pairs, flops=flops, t_step=t_step, t_attn=t_attn, data=d,
                routing=(idx, bias, valid))


# ------------------------------------------------------------------ decode

def bench_decode(cfg, steps, warmup, copies=8):
    dev = "cuda"
    log(f"[bench] decode {cfg.name}: generating inputs")
    d = W.make_decode(cfg, device=dev)
    hc = torch.zeros(W.D, device=dev)
    lb = cfg.lw // cfg.bs
    nblk = (cfg.S + cfg.bs - 1) // cfg.bs
    scale = 1.0 / math.sqrt(W.D)
    # distinct caches: the per-step read set (~84 MB) must not stay in the 256 MB MALL
    sets = [(d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"])]
    for _ in range(copies - 1):
        sets.append(tuple(t.clone() for t in sets[0]))
    states = [pipeline.init_decode_state(s[4], hc, cfg.bs, nblk) for s in sets]

    def step(i):
        qq, kk, vv, a, b = sets[i % len(sets)]
        return pipeline.decode_step(states[i % len(sets)], qq, kk, vv, a, b, hc, cfg.bs, lb,
                                    W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale)

    out, (idx, bias, valid) = pipeline.decode_step(states[0], *sets[0], hc, cfg.bs, lb,
                                                   W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap,
                                                   cfg.cap, scale, return_routing=True)
    torch.cuda.synchronize()
    lens = torch.full((cfg.B,), cfg.S, device=dev)
    nkeys = decode_keys(idx[:, 0], valid[:, 0], lens, cfg.bs, cfg.lw)
    kv_bytes = float(nkeys.sum().item()) * W.H * W.D * 2 * 2
    qo_bytes = cfg.B * W.H * W.D * (2 + 4)
    kbar_bytes = cfg.B * nblk * W.D * 4
    log(f"[bench] decode {cfg.name}: {kv_bytes / 1e6:.1f} MB K/V per step; timing")
    t_step_eager = time_steps(step, max(steps, 20), warmup)
    # the same steps as a serving loop runs them: one captured graph per cache set
    graphs = [pipeline.DecodeGraph(states[i], *sets[i], hc, cfg.bs, lb, W.IDX_SCALE, W.FLOOR,
                                   W.SIGMA, cfg.cap, cfg.cap, scale) for i in range(len(sets))]
    t_step = time_steps(lambda i: graphs[i % len(graphs)].replay(), max(steps, 20), warmup)
    # the same replays timed on the device (the host enqueues ahead of the GPU)
    t_step_dev = time_kernel(lambda i: graphs[i % len(graphs)].replay(), max(steps, 20))

    def attn(i):
        qq, kk, vv, _, _ = sets[i % len(sets)]
        ops.attn_decode(qq, kk, vv, idx[:, 0], bias[:, 0], valid[:, 0], cfg.bs, cfg.lw, scale)

    t_attn = time_kernel(attn, max(steps, 20))
    return dict(kv_bytes=kv_bytes, qo_bytes=qo_bytes, kbar_bytes=kbar_bytes, t_step=t_step,
                t_step_eager=t_step_eager, t_step_dev=t_step_dev,
                t_attn=t_attn, data=d, routing=(idx, bias, valid))


def bench_paged_decode(cfg, steps, warmup):
    """12 stacked layers of paged decode over B=32 sequences: us per 12-layer step."""
    dev = "cuda"
    lengths, table = W.paged_layout(cfg)
    layers = []
    hc = torch.zeros(W.D, device=dev)
    lb = cfg.lw // cfg.bs
    nblk = int(table.shape[1])
    scale = 1.0 / math.sqrt(W.D)
    for l in range(cfg.layers):
        d = W.make_paged_decode(cfg, dev, l, lengths, table)
        st = pipeline.init_decode_state(d["idx_k"], hc, cfg.bs, nblk, seq_lens=d["seq_lens"],
                                        block_table=d["block_table"], page_size=cfg.bs)
        layers.append((d, st))
    kv_bytes = 0.0
    for d, st in layers[:1]:
        _, (idx, bias, valid) = pipeline.decode_step(
            st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs, lb, W.IDX_SCALE,
            W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale, seq_lens=d["seq_lens"],
            block_table=d["block_table"], page_size=cfg.bs, return_routing=True)
        nk = decode_keys(idx[:, 0], valid[:, 0], d["seq_lens"], cfg.bs, cfg.lw)
        kv_bytes = float(nk.sum().item()) * W.H * W.D * 4 * cfg.layers

    def step(i):
        for d, st in layers:
            pipeline.decode_step(st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs,
                                 lb, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, scale,
                                 seq_lens=d["seq_lens"], block_table=d["block_table"],
                                 page_size=cfg.bs)

    t_step = time_steps(step, steps, warmup)
    return dict(t_step=t_step, kv_bytes=kv_bytes)


# ------------------------------------------------------------------ CPU baselines

def cpu_prefill_baseline(res, cfg, rows=8192, reps=3):
    """The oracle (the reference's torch path restated in fp32) on this host:
    k_bar and scores for the whole sequence, routing and dense attention for the
    last `rows` query rows."""
    from oracle import dash_oracle as O
    d = res["data"]
    S = d["S"]
    q, k, v = d["q"].float().cpu(), d["k"].float().cpu(), d["v"].float().cpu()
    iq, ik = d["idx_q"].cpu(), d["idx_k"].cpu()
    r0 = max(0, S - rows)
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)

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

    ti, va = run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    pairs = prefill_pairs(torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.long), ti[0]]),
                          torch.cat([torch.zeros(r0, ti.shape[-1], dtype=torch.bool), va[0]]),
                          S, cfg.bs, cfg.lw)
    pairs -= sum(min(t + 1, cfg.lw) for t in range(r0))
    fl = 4.0 * W.D * W.H * pairs
    return dict(value=fl / t / 1e12, unit="TFLOP/s", cores=torch.get_num_threads(),
                kind="port",
                sample=f"oracle fp32 on the last {S - r0} of {S} query rows (full k_bar/scores "
                       f"over the sequence; dense masked SDPA as the reference's CPU path); "
                       f"median of {reps} after 1 warm-up; {t:.2f} s per sample")


def cpu_decode_baseline(res, cfg, reps=3):
    """The oracle decode step (k_bar over the whole cache, as the reference rebuilds
    it every step, scores, routing, dense fp32 attention over the cache)."""
    from oracle import dash_oracle as O
    d = res["data"]
    nb = cfg.B
    q = d["q"][:nb].float().cpu()[:, :, None]
    k, v = d["k"][:nb].cpu(), d["v"][:nb].cpu()
    iq, ik = d["idx_q"][:nb].cpu(), d["idx_k"][:nb].cpu()
    lb = cfg.lw // cfg.bs
    scale = 1.0 / math.sqrt(W.D)

    def run():
        O.decode_pipeline(q, k, v, iq, ik, torch.zeros(W.D), cfg.bs, lb, W.IDX_SCALE, W.FLOOR,
                          W.SIGMA, cfg.cap, cfg.cap, scale)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times) * cfg.B / nb
    return dict(value=t * 1e6, unit="us/step", cores=torch.get_num_threads(), kind="port",
                sample=f"oracle fp32 decode step on {nb} of {cfg.B} sequences "
                       f"(27,300 cached tokens each); median of {reps} after 1 warm-up")


# ------------------------------------------------------------------ main

# HBM bytes per launch of the measured kernel groups, from two hardware-counter
# runs of ``bench.py --traffic-probe`` under rocprofv3 --pmc (FETCH_SIZE, then
# WRITE_SIZE), each divided by the counter's reading for a 256 MiB device copy
# (FETCH_SIZE reads 0.500 of the copied bytes, WRITE_SIZE 1.000).  Re-measure when
# the kernels change.
PREFILL_ATTN_TRAFFIC_BYTES = int((1659.8 + 703.1) * 1e6)
# Executed bf16 MFMA FLOP of one prefill attention launch (tile + sparse kernels), from
# SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 in a counter run of ``bench.py --traffic-probe``
# (re-measure when the kernels change).
PREFILL_ATTN_EXECUTED_FLOP = (293.7 + 79.4) * 1e9
DECODE_ATTN_TRAFFIC_BYTES = int((87.2 + 1.5) * 1e6)


def traffic_probe():
    """One launch of each measured kernel group, for hardware-counter runs: after
    warm-up, a 256 MiB device-to-device copy (the counters' calibration), then one
    27,300-token prefill attention launch and one B=8 decode attention launch,
    separated by synchronisations.  The last dispatch of each kernel name is the
    measured one."""
    dev = "cuda"
    cfg = W.PREFILL_27300
    d = W.make_prefill(cfg, device=dev)
    hc = torch.zeros(W.D, device=dev)
    scale = 1.0 / math.sqrt(W.D)
    _, (idx, bias, valid) = pipeline.prefill(d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc,
                                             cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE, W.FLOOR,
                                             W.SIGMA, cfg.cap, cfg.cap, return_routing=True)
    dc = W.DECODE_B8
    dd = W.make_decode(dc, device=dev)
    nblk = (dc.S + dc.bs - 1) // dc.bs
    st = pipeline.init_decode_state(dd["idx_k"], hc, dc.bs, nblk)
    _, (didx, dbias, dvalid) = pipeline.decode_step(st, dd["q"], dd["k"], dd["v"], dd["idx_q"],
                                                    dd["idx_k"], hc, dc.bs, dc.lw // dc.bs,
                                                    W.IDX_SCALE, W.FLOOR, W.SIGMA, dc.cap,
                                                    dc.cap, scale, return_routing=True)

    def prefill_attn():
        ops.attn_prefill(d["q"], d["k"], d["v"], idx, bias, valid, cfg.bs, cfg.lw, scale)

    def decode_attn():
        ops.attn_decode(dd["q"], dd["k"], dd["v"], didx[:, 0], dbias[:, 0], dvalid[:, 0], dc.bs,
                        dc.lw, scale)

    for _ in range(2):
        prefill_attn()
        decode_attn()
    src = torch.ones(64 * 2 ** 20, dtype=torch.float32, device=dev)      # 256 MiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    prefill_attn()
    torch.cuda.synchronize()
    decode_attn()
    torch.cuda.synchronize()
    log("[bench] traffic probe: copy 268435456 B, then prefill attention, then decode attention")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--extras", action="store_true",
                    help="also time the 2,730-token, packed and 12-layer paged workloads")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run one launch of each measured kernel for counter runs and exit")
    args = ap.parse_args()
    if args.traffic_probe:
        torch.cuda.set_device(0)
        traffic_probe()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this benchmark measures one GPU only (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    torch.backends.cuda.matmul.allow_tf32 = False

    pre = bench_prefill(W.PREFILL_27300, args.steps, args.warmup)
    tflops_step = pre["flops"] / pre["t_step"] / 1e12
    tflops_attn = pre["flops"] / pre["t_attn"] / 1e12
    dec = bench_decode(W.DECODE_B8, args.steps, args.warmup)
    dec_gbs = (dec["kv_bytes"] + dec["qo_bytes"]) / dec["t_attn"] / 1e9

    line = {
        "metric": METRIC,
        "value": round(tflops_step, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["t_step"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": W.PREFILL_27300.name, "B": 1, "seq_len": 27300, "heads": W.H,
                   "head_dim": W.D, "block": 64, "window": 1024, "routed_cap": 16,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(tflops_attn, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops_attn / PEAK_BF16_TFLOPS, 4),
                     "traffic": PREFILL_ATTN_TRAFFIC_BYTES,
                     "kernel": "prefill attention", "flop_per_launch": pre["flops"],
                     "avg_launch_ms": round(pre["t_attn"] * 1e3, 4),
                     "executed_flop_per_launch": PREFILL_ATTN_EXECUTED_FLOP,
                     "executed_frac": round(PREFILL_ATTN_EXECUTED_FLOP / pre["t_attn"] / 1e12 /
                                            PEAK_BF16_TFLOPS, 4)},
        "decode": {"workload": W.DECODE_B8.name, "us_per_step": round(dec["t_step"] * 1e6, 2),
                   "us_per_step_eager": round(dec["t_step_eager"] * 1e6, 2),
                   "us_per_step_device": round(dec["t_step_dev"] * 1e6, 2),
                   "step": "routing + attention, replayed as one HIP graph per cache set",
                   "step_hbm_gbs_device": round((dec["kv_bytes"] + dec["qo_bytes"] +
                                                 dec["kbar_bytes"]) / dec["t_step_dev"] / 1e9, 1),
                   "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1),
                                "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                "frac": round(dec_gbs / PEAK_HBM_GBS, 4),
                                "traffic": DECODE_ATTN_TRAFFIC_BYTES,
                                "kernel": "decode attention (split + merge)",
                                "bytes_per_launch": dec["kv_bytes"] + dec["qo_bytes"],
                                "avg_launch_us": round(dec["t_attn"] * 1e6, 2)}},
    }
    if args.extras:
        ex = {}
        p1 = bench_prefill(W.PREFILL_2730, args.steps, args.warmup)
        ex[W.PREFILL_2730.name] = {"tflops": round(p1["flops"] / p1["t_step"] / 1e12, 2),
                                   "ms_per_step": round(p1["t_step"] * 1e3, 4)}
        p4 = bench_prefill(W.PACKED_16DOC, args.steps, args.warmup, copies=1)
        ex[W.PACKED_16DOC.name] = {"tflops": round(p4["flops"] / p4["t_step"] / 1e12, 2),
                                   "ms_per_step": round(p4["t_step"] * 1e3, 4),
                                   "tokens": p4["data"]["S"]}
        p5 = bench_paged_decode(W.PAGED_12L, max(3, args.steps // 2), 1)
        ex[W.PAGED_12L.name] = {"us_per_step": round(p5["t_step"] * 1e6, 1),
                                "kv_GBps": round(p5["kv_bytes"] / p5["t_step"] / 1e9, 1)}
        line["extras"] = ex
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle on host cores)")
        line["cpu_baseline"] = cpu_prefill_baseline(pre, W.PREFILL_27300)
        line["decode"]["cpu_baseline"] = cpu_decode_baseline(dec, W.DECODE_B8)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
