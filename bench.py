#!/usr/bin/env python3
"""Benchmark of the fused attention hot path on one MI355X.

One step = one call of the Laya drop-in op (tfd_laya_attention_block_f32:
keep packing + fused split/RoPE/attention kernel) on the ModernBERT-base
global configuration ("C2": batch 8, seq 512,
hidden 768, 12 heads x 64, right-padded rows), inputs resident in HBM.

Prints ONE JSON line: the metric (algorithmic fused-attention TFLOP/s), its
fraction of the f32 MFMA peak, prefill tokens/s, the dominant kernel's
roofline (its launches timed with HIP events on the stream it runs on) and
the CPU baseline (the oracle's restatement of the reference rayon path, timed
on this host). The other configurations run once each under "also".
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "tenferro-decision-rs_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

F32_MFMA_PEAK = 157.3   # TFLOP/s, MI355X dense f32 matrix
BF16_MFMA_PEAK = 2500.0  # TFLOP/s, MI355X dense bf16 matrix
HBM_PEAK = 8000.0        # GB/s


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_threads():
    """(threads the CPU baseline uses, CPUs this process may run on): every
    CPU in the process's affinity mask, capped by OMP_NUM_THREADS where the
    host sets it (the GPU boxes give each GPU a 16-CPU share that way)."""
    allowed = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return (min(allowed, int(cap)) if cap.isdigit() and int(cap) > 0 else allowed), allowed


SETTLE_S = 0.08
_settled = {"steps": 0}


def settle(fn, seconds=SETTLE_S):
    """Untimed steps until the GPU has run `fn` back to back for `seconds` of
    wall time. Its clocks ramp up over the first ~30 ms of continuous work
    (kernel times fall 8-10% and then stay flat), so the timed steps measure
    the steady state. The count is reported as "settle_steps"."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        n += 20
    _settled["steps"] += n


def time_gpu(fn, steps, warmup, ctx):
    """(ms per step by torch events on the shared stream, avg attention-kernel ms).

    Before the `warmup` steps, settle() runs untimed steps until the clocks
    are steady.
    Two passes of `steps` steps: the whole-op time, then the attention
    kernel's own mean duration from the library's HIP event pairs, which the
    kernel dispatches themselves record on the op's stream (start of the
    first attention kernel, end of the last; hipExtLaunchKernel)."""
    import torch
    import tenferro_ext as te

    with te.asynchronous():
        settle(fn)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        ctx.take_kernel_time()
        ctx.set_timing(True)
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        ctx.set_timing(False)
    total, launches = ctx.take_kernel_time()
    return start.elapsed_time(end) / steps, total / max(1, launches)


def host_call_line(w, ctx, flops, calls=10, warmup=3):
    """The C2 drop-in called the way the reference's op is: host buffers in,
    host buffer out (TFD_HOST_PTRS: upload, kernels, download, then the call
    returns), timed on the host clock. Pageable numpy arrays, as the
    reference's Vec<f32> tensors are, and pinned host tensors. PCIe-inclusive,
    so never the headline `value`."""
    import time

    import numpy as np
    import torch
    import tenferro_ext as te

    shape = (3 * w.hidden, w.length, w.batch)
    n_out = w.hidden * w.length * w.batch
    h2d = 4 * w.qkv.size + w.keep.size
    d2h = 4 * n_out
    res = {"h2d_bytes": int(h2d), "d2h_bytes": int(d2h),
           "note": "wall time of synchronous host-pointer calls (upload, attention, download)"}
    pinned = (torch.from_numpy(w.qkv).pin_memory(), torch.from_numpy(w.keep).pin_memory(),
              torch.empty(n_out, dtype=torch.float32).pin_memory())
    variants = {"pageable": (w.qkv, w.keep, np.empty(n_out, np.float32)), "pinned": pinned}
    for name, (q, k, o) in variants.items():
        for _ in range(warmup):
            te.laya_attention_block(q, k, w.hidden, w.heads, w.rope_base, qkv_shape=shape,
                                    ctx=ctx, out=o)
        t0 = time.perf_counter()
        for _ in range(calls):
            te.laya_attention_block(q, k, w.hidden, w.heads, w.rope_base, qkv_shape=shape,
                                    ctx=ctx, out=o)
        ms = (time.perf_counter() - t0) * 1e3 / calls
        res[name] = {"ms_per_call": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
                     "prefill_tokens_per_s": round(w.valid_tokens() / (ms * 1e-3), 1),
                     "host_device_gb_per_s": round((h2d + d2h) / (ms * 1e-3) / 1e9, 2)}
    return res


def laya_bytes(w):
    """Algorithmic bytes of one attention-kernel launch: the (3d, L, B) qkv
    read once and the (d, L, B) output written once (f32), plus the packed
    keep words (4 bytes per query per 32-key tile)."""
    words = 4 * w.length * w.batch * ((w.length + 31) // 32)
    return 4 * (3 * w.hidden * w.length * w.batch) + 4 * w.hidden * w.length * w.batch + words


def cpu_laya(w, threads, reps=15, warmup=5):
    import oracle

    oracle.set_threads(threads)
    times = []
    for i in range(warmup + reps):
        t = time.perf_counter()
        oracle.laya_attention_block(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
        if i >= warmup:
            times.append(time.perf_counter() - t)
    return statistics.median(times)


def cpu_jeff_rows(w, rows, threads, reps=3):
    import oracle

    oracle.set_threads(threads)
    L, W, KW = w.length, w.heads * w.head_dim, w.kv_heads * w.head_dim
    sl = lambda x, n: x[: rows * L * n]
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        oracle.jeff_rows(sl(w.q, W), sl(w.k, KW), sl(w.v, KW), sl(w.gate, W), w.q_norm, w.k_norm,
                         w.mask[: rows * L], rows, L, w.heads, w.kv_heads, w.head_dim, w.rotary_dim,
                         w.theta, w.eps)
        times.append(time.perf_counter() - t)
    return statistics.median(times)


# The reference's own CPU micro-benchmark of this op (8 rayon threads,
# median of 15 after 5; fixtures/bench-laya-attention-gemm-2026-10-09/
# micro.json, produced by that directory's microbenchmark.rs:142-210): d 1024,
# 16 heads x 64, RoPE 160000, qkv[i] = ((17 i mod 101) - 50) * 0.002,
# keep = (k mod 13 != 7) and, sliding, |q - k| <= window. Published
# `gemm_ms` (the tile path the op takes) per (L, B, window).
MICRO_PUBLISHED_MS = {
    (64, 1, None): 0.116962, (64, 1, 64): 0.113356,
    (128, 1, None): 0.322324, (128, 1, 64): 0.283323,
    (256, 1, None): 0.997085, (256, 1, 64): 0.636693,
    (512, 1, None): 3.742275, (512, 1, 64): 1.444846,
    (8, 8, None): 0.066831, (8, 8, 64): 0.067832,
}
# The reference's GPU figure for the same op at L 512 (its NVRTC flash
# kernel on an RTX 3060, f32, per call; docs/agents/specs/docs/
# 23_TENFERRO_NATIVE.md:457).
RTX3060_L512_US = 311.5


def micro_inputs(L, B, window):
    import numpy as np

    d = 1024
    i = np.arange(3 * d * L * B, dtype=np.int64)
    qkv = (((i * 17) % 101).astype(np.float32) - np.float32(50.0)) * np.float32(0.002)
    j = np.arange(L * L * B, dtype=np.int64)
    q, k = j % L, (j // L) % L
    keep = (k % 13) != 7
    if window is not None:
        keep &= np.abs(q - k) <= window
    return qkv, keep.astype(np.uint8)


def micro_lines(args, ctx, dev):
    """The reference micro-benchmark's shapes (MICRO_PUBLISHED_MS): the GPU op
    (Laya drop-in, device pointers, ms per call) and the CPU port at the
    reference's 8 threads with its protocol (median of 15 after 5), beside
    the published reference medians."""
    import numpy as np
    import torch

    import oracle
    import tenferro_ext as te

    rows = []
    for (L, B, window), pub in MICRO_PUBLISHED_MS.items():
        qkv, keep = micro_inputs(L, B, window)
        d, H = 1024, 16
        flops = 4 * (d // H) * int(keep.astype(np.int64).sum()) * H
        tq, tk = torch.from_numpy(qkv).to(dev), torch.from_numpy(keep).to(dev)
        to = torch.empty(d * L * B, dtype=torch.float32, device=dev)
        shape = (3 * d, L, B)
        ms, kern = time_gpu(lambda: te.laya_attention_block(tq, tk, d, H, 160000.0, qkv_shape=shape,
                                                            ctx=ctx, out=to),
                            args.steps, args.warmup, ctx)
        row = {"length": L, "batch": B, "window": window, "gpu_ms": round(ms, 5),
               "gpu_kernel_ms": round(kern, 5), "gpu_tflops": round(flops / (ms * 1e-3) / 1e12, 3),
               "reference_published_ms_8_threads": pub}
        if not args.no_cpu:
            oracle.set_threads(8)
            times = []
            for it in range(20):
                t0 = time.perf_counter()
                oracle.laya_attention_block(qkv, keep, d, H, L, B, 160000.0)
                if it >= 5:
                    times.append(time.perf_counter() - t0)
            cpu_ms = statistics.median(times) * 1e3
            row["cpu_port_ms_8_threads"] = round(cpu_ms, 4)
            row["cpu_port_over_published"] = round(cpu_ms / pub, 2)
        row["published_over_gpu"] = round(pub / ms, 1)
        if (L, B, window) == (512, 1, None):
            row["rtx3060_published_us"] = RTX3060_L512_US
        rows.append(row)
        del tq, tk, to
    return {"rows": rows, "cpu": _cpu_model(),
            "note": "cpu_port_over_published compares this host's CPU with the reference's "
                    "benchmark machine (x86_64, 16 logical CPUs) as well as the two codes"}


def run(args):
    import numpy as np
    import torch

    import tenferro_ext as te
    from tenferro_ext.workloads import jeff_config, laya_config

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # One dedicated stream for the library and torch's timing events.
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    ctx = te.Context(0, stream=stream.cuda_stream)
    gpu_name = torch.cuda.get_device_name(0)

    # ------------------------------------------------------------ C2 headline
    w = laya_config(2)
    pairs = w.kept_pairs()
    flops = 4 * w.head_dim * pairs * w.heads
    qkv = torch.from_numpy(w.qkv).to(dev)
    keep = torch.from_numpy(w.keep).to(dev)
    out = torch.empty(w.hidden * w.length * w.batch, dtype=torch.float32, device=dev)
    shape = (3 * w.hidden, w.length, w.batch)

    def step():
        te.laya_attention_block(qkv, keep, w.hidden, w.heads, w.rope_base, qkv_shape=shape,
                                ctx=ctx, out=out)

    log(f"[bench] C2 drop-in: {args.warmup} warmup + {args.steps} timed steps")
    ms, kern_ms = time_gpu(step, args.steps, args.warmup, ctx)
    settle_steps = _settled["steps"]
    value = flops / (ms * 1e-3) / 1e12
    achieved = flops / (kern_ms * 1e-3) / 1e12
    tokens = w.valid_tokens()
    result = {
        "metric": "fused-attention TFLOP/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": SETTLE_S, "untimed_steps": settle_steps,
                   "note": "untimed steps before the warmup until the clocks are steady"},
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded LCG + Box-Muller, BASELINE configs[1])",
        "config": {"workload": "C2 ModernBERT-base global attention layer, Laya drop-in op",
                   "batch": w.batch, "seq_len": w.length, "hidden": w.hidden, "heads": w.heads,
                   "head_dim": w.head_dim, "rope_base": w.rope_base,
                   "mask": "right padding, valid lengths U{64..512}, keep (L,L,B) tensor",
                   "parallelism": "single GPU"},
        "pct_of_f32_mfma_peak": round(100.0 * value / F32_MFMA_PEAK, 2),
        "prefill_tokens_per_s": round(tokens / (ms * 1e-3), 1),
        "algorithmic_flops_per_step": flops,
        "roofline": {"bound": "mfma", "kernel": "laya_attention_kernel<64, keep bits>",
                     "achieved": round(achieved, 3), "peak": F32_MFMA_PEAK, "unit": "TFLOP/s",
                     "frac": round(achieved / F32_MFMA_PEAK, 4), "kernel_ms": round(kern_ms, 5),
                     "traffic": _traffic("laya_attention_kernel"),
                     "algorithmic_bytes": laya_bytes(w)},
        "gpu": gpu_name,
        "provenance": provenance(),
        "timing_note": ("ms_per_step: torch events around `steps` back-to-back calls with the "
                        "library's timing off; kernel_ms (and roofline.achieved): a second pass "
                        "of `steps` calls with timing on, the mean span from the start of the "
                        "op's first kernel to the end of its last, recorded by the dispatches "
                        "themselves (hipExtLaunchKernel events). For the Jeff rows that span "
                        "covers the K prep and the attention kernel and the gap between them; "
                        "the per-kernel durations are in profiles/ (rocprofv3)."),
    }

    # ------------------------------------------------------------ other configs
    also = {}
    if not args.no_extra:
        # C2 through the structured entry (no keep tensor: one kernel per step)
        valid = torch.from_numpy(w.valid).to(dev)

        def step_s():
            te.laya_attention_structured(qkv, valid, w.hidden, w.heads, w.length, w.batch,
                                         w.window, w.rope_base, ctx=ctx, out=out)

        ms_s, k_s = time_gpu(step_s, args.steps, args.warmup, ctx)
        also["C2_structured"] = {"ms_per_step": round(ms_s, 5), "kernel_ms": round(k_s, 5),
                                 "tflops": round(flops / (ms_s * 1e-3) / 1e12, 3),
                                 "kernel_tflops": round(flops / (k_s * 1e-3) / 1e12, 3)}
        del valid
        also["C2_host_pointers"] = host_call_line(w, ctx, flops)

        w3 = laya_config(3)
        f3 = 4 * w3.head_dim * w3.kept_pairs() * w3.heads
        q3 = torch.from_numpy(w3.qkv).to(dev)
        k3 = torch.from_numpy(w3.keep).to(dev)
        v3 = torch.from_numpy(w3.valid).to(dev)
        o3 = torch.empty(w3.hidden * w3.length * w3.batch, dtype=torch.float32, device=dev)
        sh3 = (3 * w3.hidden, w3.length, w3.batch)
        ms3, k3ms = time_gpu(lambda: te.laya_attention_block(q3, k3, w3.hidden, w3.heads, w3.rope_base,
                                                             qkv_shape=sh3, ctx=ctx, out=o3),
                             args.steps, args.warmup, ctx)
        ms3s, k3s = time_gpu(lambda: te.laya_attention_structured(q3, v3, w3.hidden, w3.heads, w3.length,
                                                                  w3.batch, w3.window, w3.rope_base,
                                                                  ctx=ctx, out=o3),
                             args.steps, args.warmup, ctx)
        if not args.no_cpu:
            t3 = cpu_laya(w3, host_threads()[0], reps=3, warmup=1)
        also["C3"] = {"ms_per_step": round(ms3, 5), "kernel_ms": round(k3ms, 5),
                      "tflops": round(f3 / (ms3 * 1e-3) / 1e12, 3),
                      "kernel_tflops": round(f3 / (k3ms * 1e-3) / 1e12, 3),
                      "structured_ms_per_step": round(ms3s, 5),
                      "structured_kernel_tflops": round(f3 / (k3s * 1e-3) / 1e12, 3),
                      "tokens_per_s": round(w3.valid_tokens() / (ms3 * 1e-3), 1),
                      "algorithmic_flops": f3}
        if not args.no_cpu:
            also["C3"]["cpu_port_tflops"] = round(f3 / t3 / 1e12, 5)
            also["C3"]["cpu_port_sample"] = (f"full C3 workload, median of 3 after 1, "
                                             f"{host_threads()[0]} threads, {t3 * 1e3:.1f} ms")
        del q3, k3, v3, o3

        for cfg in (4, 5):
            wj = jeff_config(cfg)
            fj = 4 * wj.head_dim * wj.kept_pairs() * wj.heads
            bf = wj.bf16
            conv = (lambda x: torch.from_numpy(te.to_bf16_bits(x).view(np.int16)).to(dev)) if bf else \
                (lambda x: torch.from_numpy(x).to(dev))
            tq, tk, tv, tg = (conv(getattr(wj, n)) for n in ("q", "k", "v", "gate"))
            tqn, tkn, tm = (torch.from_numpy(getattr(wj, n)).to(dev) for n in ("q_norm", "k_norm", "mask"))
            oj = torch.empty(wj.rows * wj.length * wj.heads * wj.head_dim, dtype=torch.float32, device=dev)

            def step_j():
                te.jeff_full_attention_rows(tq, tk, tv, tg, tqn, tkn, tm, wj.rows, wj.length, wj.heads,
                                            wj.kv_heads, wj.head_dim, wj.rotary_dim, wj.theta, wj.eps,
                                            bf16=bf, ctx=ctx, out=oj)

            try:
                msj, kj = time_gpu(step_j, args.steps, args.warmup, ctx)
            except te.Unsupported as e:
                also[f"C{cfg}"] = {"skipped": str(e)}
                continue
            peak = BF16_MFMA_PEAK if bf else F32_MFMA_PEAK
            also[f"C{cfg}"] = {"ms_per_step": round(msj, 5), "kernel_ms": round(kj, 5),
                               "tflops": round(fj / (msj * 1e-3) / 1e12, 3),
                               "kernel_tflops": round(fj / (kj * 1e-3) / 1e12, 3),
                               "pct_of_peak": round(100.0 * fj / (kj * 1e-3) / 1e12 / peak, 2),
                               "peak": peak, "dtype": "bf16" if bf else "f32",
                               "tokens_per_s": round(wj.valid_tokens() / (msj * 1e-3), 1),
                               "algorithmic_flops": fj}
            if cfg == 4:
                also["C4_dropin_per_row"] = dropin_rows_line(args, ctx, wj, tq, tk, tv, tg, tqn,
                                                             tkn, tm, kj)
            if cfg == 4 and not args.no_cpu:
                cores = host_threads()[0]
                t = cpu_jeff_rows(wj, wj.rows, cores)
                also["C4"]["cpu_port_tokens_per_s"] = round(wj.valid_tokens() / t, 1)
                also["C4"]["cpu_port_tflops"] = round(fj / t / 1e12, 5)
                also["C4"]["cpu_port_sample"] = (f"full C4 workload (16 rows), median of 3, "
                                                 f"{cores} threads (one task per head, as the "
                                                 f"reference), {t * 1e3:.1f} ms")
            if cfg == 5 and not args.no_cpu:
                cores = host_threads()[0]
                log("[bench] C5 CPU leg: the full workload once (about 20-40 s)")
                t = cpu_jeff_rows(wj, wj.rows, cores, reps=1)
                also["C5"]["cpu_port_tflops"] = round(fj / t / 1e12, 5)
                also["C5"]["cpu_port_tokens_per_s"] = round(wj.valid_tokens() / t, 1)
                also["C5"]["cpu_port_sample"] = (f"full C5 workload (2 x 8192, the bf16 inputs' "
                                                 f"f32 values), once, {cores} threads, {t:.2f} s")
            del tq, tk, tv, tg, tqn, tkn, tm, oj
        log("[bench] reference micro-benchmark shapes")
        also["micro_reference_shapes"] = micro_lines(args, ctx, dev)
        also.update(layer_lines(args, ctx, dev))
        also["laya_model_forward"] = model_line(args, ctx, dev)
    result["also"] = also

    # ------------------------------------------------------------ CPU baseline
    if not args.no_cpu:
        cores, allowed = host_threads()
        log(f"[bench] CPU baseline: oracle port of the rayon path, {cores} threads")
        t_all = cpu_laya(w, cores)
        t_8 = cpu_laya(w, 8) if cores != 8 else t_all
        result["cpu_baseline"] = {
            "value": round(flops / t_all / 1e12, 5), "unit": "TFLOP/s", "cores": cores,
            "cpus_allowed": allowed,
            "kind": "port",
            "sample": "full C2 workload per call, median of 15 after 5 warmups",
            "ms": round(t_all * 1e3, 3),
            "tokens_per_s": round(tokens / t_all, 1),
            "ms_8_threads": round(t_8 * 1e3, 3),
            "cpu": _cpu_model(),
        }
        result["gpu_over_cpu"] = round(value / (flops / t_all / 1e12), 1)
    ctx.close()
    return result


def dropin_rows_line(args, ctx, w, tq, tk, tv, tg, tqn, tkn, tm, rows_kernel_ms):
    """C4 through the drop-in op the way jeff-infer calls it (model.rs:755-768):
    one call per question row, q/gate (L, 2048) and K/V expanded to all 8
    heads (checkpoint.rs:307-319), with TFD_KV_HEADS(2) (one head per GQA
    group read) and without (every copy read). Kernel time per row (the
    calls' own dispatch events) beside the rows entry's per-row share."""
    import torch

    import tenferro_ext as te

    R, L, H, KV, hd = w.rows, w.length, w.heads, w.kv_heads, w.head_dim
    W, G = H * hd, H // KV
    # (row, kv head, hd, L) -> every kv head repeated G times: the expansion
    expand = lambda t: t.view(R, KV, hd * L).repeat_interleave(G, dim=1).reshape(-1).contiguous()
    ke, ve = expand(tk), expand(tv)
    oj = torch.empty(R * L * W, dtype=torch.float32, device=tq.device)
    out = {}
    for name, kvh in (("kv_heads_flag", KV), ("every_copy", None)):
        def step():
            for r in range(R):
                sl = slice(r * L * W, (r + 1) * L * W)
                te.jeff_full_attention(tq[sl], ke[sl], ve[sl], tg[sl], tqn, tkn,
                                       tm[r * L:(r + 1) * L], H, hd, w.rotary_dim, w.theta, w.eps,
                                       q_shape=(L, W), ctx=ctx, out=oj[sl], kv_heads=kvh)
        ms, kern = time_gpu(step, max(5, args.steps // 5), max(2, args.warmup // 5), ctx)
        out[name] = {"kernel_us_per_row": round(kern * 1e3, 3),
                     "wall_us_per_row": round(ms * 1e3 / R, 3)}
    out["rows_entry_kernel_us_per_row"] = round(rows_kernel_ms * 1e3 / R, 3)
    out["flag_over_rows_entry"] = round(out["kv_heads_flag"]["kernel_us_per_row"]
                                        / out["rows_entry_kernel_us_per_row"], 2)
    out["note"] = ("one launch of the fused kernel per 256-token row: a row is 128 work items "
                   "for 256 CUs, and its longest query tile walks 16 key tiles on one CU, so "
                   "per-call latency, not the GQA reads, bounds it")
    return out


def _layer_steps(ctx, dev):
    """Step functions of the two layer entries at the C2 and C4 shapes:
    (name, step, attention flops, projection flops, valid tokens)."""
    import numpy as np
    import torch

    import tenferro_ext as te
    from tenferro_ext.workloads import jeff_layer_config, laya_layer_config

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    lw = laya_layer_config(2)
    la = [t(a) for a in (lw.x, lw.keep, lw.w_in, lw.w_out)]
    lo = torch.empty(lw.hidden * lw.length * lw.batch, dtype=torch.float32, device=dev)
    lf = 4 * (lw.hidden // lw.heads) * int(lw.keep.astype(np.int64).sum()) * lw.heads

    def laya_step():
        te.laya_attention_layer(la[0], la[1], la[2], None, la[3], None, lw.hidden, lw.heads,
                                lw.length, lw.batch, lw.rope_base, ctx=ctx, out=lo)

    jw = jeff_layer_config(4)
    ja = [t(getattr(jw, n)) for n in ("x", "w_q", "w_gate", "w_k", "w_v", "w_o", "q_norm",
                                      "k_norm", "mask")]
    jo = torch.empty(jw.rows * jw.length * jw.hidden, dtype=torch.float32, device=dev)
    m = jw.mask.reshape(jw.rows, jw.length) != 0
    # pairs counted as the C4 line counts them: each position t with the
    # active keys at or before it
    jf = 4 * jw.head_dim * int(np.cumsum(m, axis=1).sum()) * jw.heads

    def jeff_step():
        te.jeff_full_attention_layer_rows(*ja, jw.rows, jw.length, jw.hidden, jw.heads,
                                          jw.kv_heads, jw.head_dim, jw.rotary_dim, jw.theta,
                                          jw.eps, ctx=ctx, out=jo)

    def laya_cpu():
        import oracle

        oracle.laya_attention_layer(lw.x, lw.keep, lw.w_in, None, lw.w_out, None, lw.hidden,
                                    lw.heads, lw.length, lw.batch, lw.rope_base)

    def jeff_cpu():
        import oracle

        oracle.jeff_layer_rows(jw.x, jw.w_q, jw.w_gate, jw.w_k, jw.w_v, jw.w_o, jw.q_norm,
                               jw.k_norm, jw.mask, jw.rows, jw.length, jw.hidden, jw.heads,
                               jw.kv_heads, jw.head_dim, jw.rotary_dim, jw.theta, jw.eps)

    return [("C2_layer", laya_step, lf, lw.gemm_flops(), lw.valid.astype(np.int64).sum(),
             laya_cpu),
            ("C4_layer", jeff_step, jf, jw.gemm_flops(), int(m.sum()), jeff_cpu)]


def layer_lines(args, ctx, dev):
    """Whole attention layers (projections by rocBLAS sgemm + the fused op):
    step time, the attention kernels' share, and the layer's f32 TFLOP/s."""
    out = {}
    for name, step, att_flops, gemm_flops, tokens, cpu_fn in _layer_steps(ctx, dev):
        log(f"[bench] {name}")
        ms, kern = time_gpu(step, args.steps, args.warmup, ctx)
        total = att_flops + gemm_flops
        out[name] = {"ms_per_step": round(ms, 5), "attention_kernel_ms": round(kern, 5),
                     "tflops": round(total / (ms * 1e-3) / 1e12, 3),
                     "pct_of_f32_mfma_peak": round(100.0 * total / (ms * 1e-3) / 1e12
                                                   / F32_MFMA_PEAK, 2),
                     "tokens_per_s": round(float(tokens) / (ms * 1e-3), 1),
                     "projection_flops": gemm_flops, "attention_flops": att_flops}
        if not args.no_cpu:
            import oracle

            cores = host_threads()[0]
            oracle.set_threads(cores)
            times = []
            for _ in range(3):
                t0 = time.perf_counter()
                cpu_fn()
                times.append(time.perf_counter() - t0)
            t = statistics.median(times[1:])
            out[name]["cpu_port_tflops"] = round(total / t / 1e12, 5)
            out[name]["cpu_port_sample"] = (f"full workload, oracle (numpy sgemm + C op), median "
                                            f"of 2 after 1, {cores} threads, {t * 1e3:.1f} ms")
    return out


def _model_step(ctx, dev):
    """The Laya decision-model forward at ModernBERT-base shape (22 layers,
    d 768, 12 heads, intermediate 1152, local_attention 128, vocab 50368,
    one head layer) on a C2-shaped batch (L 512, B 8, right padding with
    valid lengths U{64..512}, 8 marker slots): (step, flops, valid tokens)."""
    import numpy as np

    from tenferro_ext.laya_model import LayaModel
    from tenferro_ext.workloads import laya_config, laya_model_batch, laya_model_checkpoint

    d, inter, layers, L, B, K = 768, 1152, 22, 512, 8, 8
    ckpt = laya_model_checkpoint(vocab=50368, hidden=d, intermediate=inter, layers=layers,
                                 heads=12, local_attention=128, seed=2, fast=True)
    ids, _mask, pos, mm, qtype = laya_model_batch(L, B, K, 50368, min_len=64)
    valid = laya_config(2, with_keep=False).valid.astype(bool)  # C2's row lengths
    pos = np.minimum(pos, 63)                                   # markers inside every row
    model = LayaModel(ckpt, ctx=ctx)
    # Flops of the valid tokens only (projections per valid token, attention
    # per kept (query, key) pair of valid queries): the forward computes the
    # padded tokens that no output reads as little as it can.
    T = int(valid.sum())
    proj = 2 * T * (d * 3 * d + d * d + d * 2 * inter + inter * d) * layers
    head = 2 * T * (d * 3 * d + d * d + 2 * d * 4 * d)
    lens = [int(valid[b * L:(b + 1) * L].sum()) for b in range(B)]
    pairs_global = sum(n * n for n in lens)
    q = np.arange(L)
    pairs_local = sum(int((np.abs(q[:n, None] - q[None, :n]) <= 64).sum()) for n in lens)
    att = 0
    for kind in ckpt.encoder.layer_types:
        att += 4 * d * (pairs_global if kind == "full_attention" else pairs_local)
    att += 4 * d * pairs_global  # the head layer
    import torch

    dl = torch.empty(K * B, dtype=torch.float32, device=dev)
    da = torch.empty(ckpt.agent.action_count() * B, dtype=torch.float32, device=dev)

    def step():
        model.forward(ids, valid, pos, mm, qtype, logits=dl, action=da)

    return step, proj + head + att, int(valid.sum()), layers + 1


def model_line(args, ctx, dev):
    """Whole Laya forward: ms, tokens/s, f32 TFLOP/s (projections + attention
    algorithmic flops) and the attention kernels' share of the step."""
    step, flops, tokens, att_launches = _model_step(ctx, dev)
    log("[bench] Laya model forward")
    steps = max(3, args.steps // 5)
    ms, kern = time_gpu(step, steps, max(1, args.warmup // 5), ctx)
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
            "attention_ms_per_step": round(kern * att_launches, 4), "steps": steps,
            "workload": "ModernBERT-base shape (22 layers) + decision head, L 512, B 8, "
                        "synthetic weights; flops of the valid tokens"}


def run_only(args):
    """One configuration's op alone (for rocprofv3 runs of a single kernel)."""
    import numpy as np
    import torch

    import tenferro_ext as te
    from tenferro_ext.workloads import jeff_config, laya_config

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    if args.only == "copy":
        # Calibration for PMC byte counters: a plain device copy of known size.
        n = 1 << 27  # 128 Mi floats = 512 MiB each way
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        return {"only": "copy", "bytes_read_per_copy": 4 * n, "bytes_written_per_copy": 4 * n}
    ctx = te.Context(0, stream=stream.cuda_stream)
    if args.only == "model":
        res = model_line(args, ctx, dev)
        ctx.close()
        return {"only": "model", **res}
    if args.only.endswith("l"):
        name, fn, att, gemm, _, _ = [s for s in _layer_steps(ctx, dev)
                                  if s[0] == f"C{args.only[1]}_layer"][0]
        ms, kern = time_gpu(fn, args.steps, args.warmup, ctx)
        ctx.close()
        return {"only": name, "ms_per_step": round(ms, 5), "attention_kernel_ms": round(kern, 5),
                "tflops": round((att + gemm) / (ms * 1e-3) / 1e12, 3)}
    if args.only == "c2host":
        w = laya_config(2)
        res = host_call_line(w, ctx, 4 * w.head_dim * w.kept_pairs() * w.heads)
        ctx.close()
        return {"only": "C2_host_pointers", **res}
    if args.only == "micro":
        # The reference micro-benchmark's largest shape (L 512, B 1, d 1024,
        # 16 heads, global keep k % 13 != 7): the small-grid Laya path.
        L, d, H = 512, 1024, 16
        qkv, keep = micro_inputs(L, 1, None)
        flops = 4 * (d // H) * int(keep.astype(np.int64).sum()) * H
        tq, tk = torch.from_numpy(qkv).to(dev), torch.from_numpy(keep).to(dev)
        to = torch.empty(d * L, dtype=torch.float32, device=dev)
        fn = lambda: te.laya_attention_block(tq, tk, d, H, 160000.0, qkv_shape=(3 * d, L, 1),
                                             ctx=ctx, out=to)
        ms, kern = time_gpu(fn, args.steps, args.warmup, ctx)
        ctx.close()
        return {"only": "micro L512 B1", "ms_per_step": round(ms, 5), "kernel_ms": round(kern, 5),
                "tflops": round(flops / (ms * 1e-3) / 1e12, 3)}
    if args.only == "c4row":
        # The drop-in op once per C4 row with TFD_KV_HEADS (dropin_rows_line's
        # flag case), for a kernel trace of the per-row path.
        w = jeff_config(4)
        R, L, H, KV, hd = w.rows, w.length, w.heads, w.kv_heads, w.head_dim
        W, G = H * hd, H // KV
        t = {n: torch.from_numpy(getattr(w, n)).to(dev)
             for n in ("q", "k", "v", "gate", "q_norm", "k_norm", "mask")}
        expand = lambda x: x.view(R, KV, hd * L).repeat_interleave(G, dim=1).reshape(-1).contiguous()
        ke, ve = expand(t["k"]), expand(t["v"])
        oj = torch.empty(R * L * W, dtype=torch.float32, device=dev)

        def fn():
            for r in range(R):
                sl = slice(r * L * W, (r + 1) * L * W)
                te.jeff_full_attention(t["q"][sl], ke[sl], ve[sl], t["gate"][sl], t["q_norm"],
                                       t["k_norm"], t["mask"][r * L:(r + 1) * L], H, hd,
                                       w.rotary_dim, w.theta, w.eps, q_shape=(L, W), ctx=ctx,
                                       out=oj[sl], kv_heads=KV)
        ms, kern = time_gpu(fn, args.steps, args.warmup, ctx)
        ctx.close()
        return {"only": "C4_dropin_per_row", "ms_per_16_rows": round(ms, 5),
                "kernel_us_per_row": round(kern * 1e3, 3)}
    cfg = int(args.only[1])
    structured = args.only.endswith("s")
    if cfg in (2, 3):
        w = laya_config(cfg, with_keep=not structured)
        flops = 4 * w.head_dim * w.kept_pairs() * w.heads
        qkv = torch.from_numpy(w.qkv).to(dev)
        out = torch.empty(w.hidden * w.length * w.batch, dtype=torch.float32, device=dev)
        if structured:
            valid = torch.from_numpy(w.valid).to(dev)
            fn = lambda: te.laya_attention_structured(qkv, valid, w.hidden, w.heads, w.length,
                                                      w.batch, w.window, w.rope_base, ctx=ctx,
                                                      out=out)
        else:
            keep = torch.from_numpy(w.keep).to(dev)
            shape = (3 * w.hidden, w.length, w.batch)
            fn = lambda: te.laya_attention_block(qkv, keep, w.hidden, w.heads, w.rope_base,
                                                 qkv_shape=shape, ctx=ctx, out=out)
    else:
        w = jeff_config(cfg)
        flops = 4 * w.head_dim * w.kept_pairs() * w.heads
        conv = (lambda x: torch.from_numpy(te.to_bf16_bits(x).view(np.int16)).to(dev)) if w.bf16 \
            else (lambda x: torch.from_numpy(x).to(dev))
        t = [conv(getattr(w, n)) for n in ("q", "k", "v", "gate")]
        t += [torch.from_numpy(getattr(w, n)).to(dev) for n in ("q_norm", "k_norm", "mask")]
        out = torch.empty(w.rows * w.length * w.heads * w.head_dim, dtype=torch.float32, device=dev)
        fn = lambda: te.jeff_full_attention_rows(*t, w.rows, w.length, w.heads, w.kv_heads,
                                                 w.head_dim, w.rotary_dim, w.theta, w.eps,
                                                 bf16=w.bf16, ctx=ctx, out=out)
    ms, kern = time_gpu(fn, args.steps, args.warmup, ctx)
    ctx.close()
    return {"only": f"C{cfg}" + ("_structured" if structured else ""),
            "ms_per_step": round(ms, 5), "kernel_ms": round(kern, 5),
            "kernel_tflops": round(flops / (kern * 1e-3) / 1e12, 3), "algorithmic_flops": flops}


def _traffic(kernel):
    """HBM bytes per launch of `kernel` on C2, from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE measurement (profiles/traffic_c2.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_c2.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def provenance():
    """Where and from what the line was measured (the reference's bench-suite
    BenchMetadata, crates/bench-suite/src/lib.rs:14-73: git revision,
    timestamp, OS and architecture): the git revision when the tree is a git
    checkout (GPU boxes receive a snapshot without .git), a hash of the
    sources the measured library and this script are built from, UTC time,
    OS/arch, Python, torch and HIP versions."""
    import hashlib
    import platform
    import subprocess
    import datetime

    rev = None
    try:
        rev = subprocess.run(["git", "-C", ROOT, "rev-parse", "HEAD"], capture_output=True,
                             text=True, timeout=10).stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        rev = None
    h = hashlib.sha256()
    for sub in ("tenferro-decision-rs_amd/csrc", "include"):
        d = os.path.join(ROOT, sub)
        for name in sorted(os.listdir(d)):
            fp = os.path.join(d, name)
            if os.path.isfile(fp):
                h.update(name.encode())
                h.update(open(fp, "rb").read())
    h.update(open(os.path.abspath(__file__), "rb").read())
    out = {"git_rev": rev, "sources_sha16": h.hexdigest()[:16],
           "timestamp_utc": datetime.datetime.now(datetime.timezone.utc).isoformat(timespec="seconds"),
           "os": platform.platform(), "arch": platform.machine(),
           "python": platform.python_version()}
    try:
        import torch

        out["torch"] = torch.__version__
        out["hip"] = getattr(torch.version, "hip", None)
    except ImportError:
        pass
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the C2 headline")
    ap.add_argument("--only", choices=["c2", "c3", "c4", "c5", "c2s", "c3s", "c2l", "c4l", "c4row", "c2host", "micro", "model",
                             "copy"], default=None,
                    help="profiling aid: run one configuration's op (steps + warmup calls), "
                         "print its timing line and skip everything else")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    print(json.dumps(run_only(args) if args.only else run(args)), flush=True)


if __name__ == "__main__":
    main()
