"""Benchmark of the quantized KV-cache path on one MI355X.

Default workload (the headline metric): a Gemma-4 global-attention layer at
long context -- batch 1, 16 query heads, 2 KV heads, head_dim 512, 8-bit
group-64 cache prefilled to 32768 tokens, then decode steps. One step = one
decode step of the layer: append the new token (rotate, quantize, slot
write) and run decode attention over the whole cache. K ~ Student-t(3),
V and q ~ N(0,1), seeded (synthetic data; no checkpoint).

Prints ONE JSON line:
  value      decode-step throughput in GB/s over the algorithmic bytes of the
             step (cache read + q/out + the append's rows), inputs resident in HBM;
  roofline   the split-K attention kernel's own GB/s (algorithmic bytes per
             launch / its average duration from HIP events) vs 8 TB/s;
  cpu_baseline  the reference's decode step (TurboQuant round trip of the new
             rows, O(T) concat, SDPA over its bf16 cache in MLX CPU op order)
             timed with the oracle on this host's cores, all and one.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "gemma4-moe-flash-mlx-turbo_amd"
sys.path.insert(0, str(PKG))

HBM_PEAK_GBS = 8000.0
# HBM bytes per decode_attn_kernel launch at this workload, from rocprofv3
# FETCH_SIZE / WRITE_SIZE passes scaled by a plain copy's readings
# (profiles/decode_attn_c3_hbm_traffic.md holds the runs and the commands);
# counters cannot be read inside the timed run itself.
TRAFFIC_BYTES_PER_LAUNCH = 76_025_037
TRAFFIC_SOURCE = "profiles/decode_attn_c3_hbm_traffic.md"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def bytes_per_token_head(D: int, bits: int, codebook: bool = False, plain: bool = False) -> int:
    """K+V codes plus f16 scale and bias per 64-dim group (affine), one f16
    norm per row (codebook) or the bf16 rows alone (plain), one token, one KV
    head."""
    if plain:
        return 2 * D * 2
    if codebook:
        return 2 * (D * bits // 8 + 2)
    return 2 * (D * bits // 8 + 4 * (D // 64))


def run_c3(args) -> dict:
    import torch

    import fmkv
    import synth

    cb = args.mode == "codebook"
    plain = args.mode == "plain"
    quant = not (cb or plain)  # affine
    Hq, Hkv, D, T0 = 16, 2, 512, args.context
    bits = 16 if plain else (args.bits or (3 if cb else 8))
    mode = fmkv.MODE_CODEBOOK if cb else fmkv.MODE_PLAIN if plain else fmkv.MODE_AFFINE
    per_tok = bytes_per_token_head(D, bits, cb, plain)
    # steps: warmup, timed, two event-timed passes, then warmup + timed
    # projected steps and warmup + timed sparse-V steps
    n_dec = 3 * args.warmup + 5 * args.steps + 1
    cache = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=T0 + n_dec + args.graph_steps + 16,
                                       mode=mode)

    # ---- prefill: chunked appends of 2048 tokens (timed separately) ----
    chunk = 2048
    host_k, host_v = [], []
    dk, dv = [], []
    for c0 in range(0, T0, chunk):
        n = min(chunk, T0 - c0)
        k = synth.kv_rows(31, n, Hkv, D, None, dist="t3", offset=c0)
        v = synth.kv_rows(32, n, Hkv, D, None, offset=c0)
        host_k.append(k)
        host_v.append(v)
        dk.append(dev_bf16(k))
        dv.append(dev_bf16(v))
    # the global layer's prologue (k_norm + RoPE over 128 of 512 dims at
    # theta 1e6; K==V: V = v_norm(k)) for the projected-append rate below
    rng = np.random.default_rng(33)
    w = dev_bf16(synth.f32_to_bf16_bits((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)))
    pro = fmkv.make_prologue(w, 1e-6, 128, 1e6, v_from_k=True)
    # one untimed chunk through each path first (first-launch costs)
    warm = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=2 * chunk, mode=mode)
    warm.append(dk[0], dv[0])
    if quant:
        warm.append_projected(dk[0], None, pro)
    torch.cuda.synchronize()
    del warm
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for k, v in zip(dk, dv):
        cache.append(k, v)
    ev1.record()
    torch.cuda.synchronize()
    prefill_ms = ev0.elapsed_time(ev1)
    append_prefill_tps = T0 / (prefill_ms / 1e3)
    log(f"prefill {T0} tokens in {prefill_ms:.2f} ms ({append_prefill_tps/1e6:.2f} M tokens/s)")

    # the same chunks as raw projections through the prologue (affine caches)
    prologue_tps = None
    if quant:
        pcache = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=T0)
        torch.cuda.synchronize()
        ev0.record()
        for k in dk:
            pcache.append_projected(k, None, pro)
        ev1.record()
        torch.cuda.synchronize()
        prologue_tps = T0 / (ev0.elapsed_time(ev1) / 1e3)
        log(f"prefill with prologue (K==V): {prologue_tps/1e6:.2f} M tokens/s")
        del pcache
    del dk, dv

    # ---- decode inputs resident on the device; raw pointers per step ----
    kd = dev_bf16(synth.kv_rows(41, n_dec, Hkv, D, None, dist="t3"))
    vd = dev_bf16(synth.kv_rows(42, n_dec, Hkv, D, None))
    qd = dev_bf16(synth.q_rows(43, Hq, Hkv, D, None, batch=n_dec))
    out = torch.empty((Hq, D), dtype=torch.bfloat16, device="cuda")
    lib, h = fmkv.load_library(), cache._h
    stream = torch.cuda.current_stream().cuda_stream
    row = Hkv * D * 2
    kp = [kd.data_ptr() + t * row for t in range(n_dec)]
    vp = [vd.data_ptr() + t * row for t in range(n_dec)]
    qp = [qd.data_ptr() + t * Hq * D * 2 for t in range(n_dec)]
    outp = out.data_ptr()
    i = 0

    tau = float(args.sparse_v_tau)

    def step():
        nonlocal i
        if args.unfused:
            rc = lib.fmkv_cache_append(h, kp[i], vp[i], 1, stream)
            rc |= lib.fmkv_decode_attention(h, qp[i], Hq, 1.0, tau, outp, fmkv.DTYPE_BF16, stream)
        else:
            rc = lib.fmkv_decode_step(h, kp[i], vp[i], 1, qp[i], Hq, 1.0, tau, outp,
                                      fmkv.DTYPE_BF16, stream)
        if rc:
            raise RuntimeError(lib.fmkv_last_error().decode())
        i += 1

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_begin = cache.offset()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    t_end = cache.offset()
    ms_per_step = elapsed / args.steps * 1e3
    # algorithmic bytes: cache read (every visible token, both KV heads) + q + out
    # + the append (bf16 K/V rows in, codes + scale/bias out)
    # after the append of a step, T = offset tokens are visible (current included)
    read = sum(T * Hkv * per_tok for T in range(t_begin + 1, t_end + 1))
    qo = args.steps * 2 * Hq * D * 2
    app = args.steps * (2 * Hkv * D * 2 + Hkv * per_tok)
    value = (read + qo + app) / elapsed / 1e9

    # ---- split-K kernel duration from HIP events around each launch ----
    # (a first pass over freshly created event pairs, discarded: the pairs
    # are reused for the timed pass)
    fmkv.profile_enable(args.steps)
    for _ in range(args.steps):
        step()
    fmkv.profile_collect_each(args.steps)
    tb = cache.offset()
    for _ in range(args.steps):
        step()
    each_ms = fmkv.profile_collect_each(args.steps)
    fmkv.profile_enable(0)
    n_rec = len(each_ms)
    te = cache.offset()
    avg_T = (tb + te + 1) / 2.0
    kern_s = sum(each_ms) / n_rec / 1e3
    each_us = sorted(m * 1e3 for m in each_ms)
    kern_pct = {q: round(each_us[min(n_rec - 1, int(q / 100 * n_rec))], 3) for q in (10, 50, 90)}
    # (sparse-V: the statistics pass reads the keys, half of each token's
    # bytes; the gated pass reads only the blocks that hold kept tokens, and
    # its figure counts every block)
    gather = tau > 0.0 and args.sparse_v_path == "gather"
    launch_bytes = avg_T * Hkv * (per_tok // 2 if gather else per_tok) + 2 * Hq * D * 2
    achieved = launch_bytes / kern_s / 1e9
    log(f"step {ms_per_step*1e3:.1f} us, split kernel {kern_s*1e6:.2f} us over {n_rec} launches, "
        f"{achieved:.0f} GB/s, splits={cache.decode_splits()}; per launch p10/p50/p90 "
        f"{kern_pct[10]:.2f}/{kern_pct[50]:.2f}/{kern_pct[90]:.2f} us")

    # The next graph_steps steps captured into a HIP graph and replayed: a
    # replay repeats the same appends (the same codes into the same slots)
    # and the same attention reads, so it redoes exactly the steps' work,
    # without the per-launch cost of eager submission. Informational; the
    # headline value above is eager.
    graph_us = None
    if args.graph_steps > 0:
        gs = torch.cuda.Stream()
        gs.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        j0 = i
        try:
            with torch.cuda.graph(g, stream=gs):
                for j in range(args.graph_steps):
                    t = (j0 + j) % n_dec
                    rc = lib.fmkv_decode_step(h, kp[t], vp[t], 1, qp[t], Hq, 1.0, tau, outp,
                                              fmkv.DTYPE_BF16, gs.cuda_stream)
                    if rc:
                        raise RuntimeError(lib.fmkv_last_error().decode())
        except RuntimeError as e:  # e.g. a workspace that would have to grow
            log(f"graph capture skipped: {e}")
            g = None
        if g is not None:
            with torch.cuda.stream(gs):  # replay() launches on the current stream
                g.replay()
                gs.synchronize()
                reps = 4
                gev0, gev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                gev0.record(gs)
                for _ in range(reps):
                    g.replay()
                gev1.record(gs)
                gs.synchronize()
            graph_us = gev0.elapsed_time(gev1) * 1e3 / (reps * args.graph_steps)
            log(f"graph: {graph_us:.2f} us/step over {reps} replays of {args.graph_steps} steps")

    # The integrated step from raw projections (K==V global layer: k_norm +
    # RoPE on K, v_norm of the raw K as V, quantize, store, attend) in the
    # same single attention launch plus combine. Informational, eager.
    proj_us = None
    if quant and tau == 0.0:
        pro_ref = ctypes.byref(pro)

        def proj_step():
            nonlocal i
            rc = lib.fmkv_decode_step_projected(h, kp[i], None, 1, pro_ref, qp[i], Hq, 1.0, 0.0,
                                                outp, fmkv.DTYPE_BF16, stream)
            if rc:
                raise RuntimeError(lib.fmkv_last_error().decode())
            i += 1

        for _ in range(args.warmup):
            proj_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            proj_step()
        torch.cuda.synchronize()
        proj_us = (time.perf_counter() - t0) / args.steps * 1e6
        log(f"projected step (prologue in the new-token column): {proj_us:.1f} us")

    # The same decode step with sparse-V at tau 1e-3 (the reference's gate,
    # src/model/gemma4_attention.rs:196-234: the statistics pass over the
    # keys, then the gather of the kept tokens' V rows) on the same cache.
    # Informational, eager; the headline value above is the dense step.
    sv_us = None
    if tau == 0.0:
        def sv_step():
            nonlocal i
            rc = lib.fmkv_decode_step(h, kp[i], vp[i], 1, qp[i], Hq, 1.0, 1e-3, outp,
                                      fmkv.DTYPE_BF16, stream)
            if rc:
                raise RuntimeError(lib.fmkv_last_error().decode())
            i += 1

        for _ in range(args.warmup):
            sv_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            sv_step()
        torch.cuda.synchronize()
        sv_us = (time.perf_counter() - t0) / args.steps * 1e6
        log(f"sparse-V step (tau 1e-3, gather): {sv_us:.1f} us against {ms_per_step * 1e3:.1f} us dense")

    copy_gbs = device_copy_gbs()
    log(f"device copy (256 MiB, read + write): {copy_gbs:.0f} GB/s")
    res = {
        "metric": "decode-attn GB/s & % HBM peak over quantized KV at 32K ctx; append tokens/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded SplitMix64: K Student-t(3), V and q N(0,1))",
        "config": {
            "workload": (f"gemma4-global-layer decode at {T0 // 1024}K: Hq 16, Hkv 2, head_dim 512, "
                         + (f"{bits}-bit TurboQuant codebook, f16 norm per row" if cb else
                            "plain bf16 rows (no quantization)" if plain else
                            f"{bits}-bit group-64 affine, f16 scale/bias")
                         + ", 1 token append + attention per step"),
            "context": T0, "batch": 1, "n_q_heads": Hq, "n_kv_heads": Hkv, "head_dim": D,
            "bits": bits, "mode": args.mode, "group": 64, "sparse_v_tau": tau,
            **({"sparse_v_path": args.sparse_v_path} if tau > 0.0 else {}),
        },
        "hbm_frac_of_value": round(value / HBM_PEAK_GBS, 4),
        "append_tokens_per_s": {"chunked_prefill_2048": round(append_prefill_tps, 1),
                                "chunked_prefill_2048_prologue_k_eq_v":
                                    None if prologue_tps is None else round(prologue_tps, 1),
                                **single_token_append_rates()},
        "graph_step_us": None if graph_us is None else round(graph_us, 3),
        "sparse_v_step_us": None if sv_us is None else {
            "tau": 1e-3, "path": "gather", "us": round(sv_us, 2),
            "dense_us": round(ms_per_step * 1e3, 2)},
        "projected_step_us": None if proj_us is None else round(proj_us, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if (not quant or bits != 8) else TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_source": None if (not quant or bits != 8) else TRAFFIC_SOURCE,
            "kernel": ((f"cb_decode_kernel<512, {bits}>" if cb else "plain_decode_kernel<512>" if plain
                        else f"decode_attn_kernel<512, {bits}, {0 if tau == 0.0 else 1 if gather else 2}>")
                       + ("" if tau == 0.0 else " (statistics pass)" if gather else " (gated pass)")),
            "avg_kernel_us": round(kern_s * 1e6, 3),
            # the same kernel against a plain device copy measured in this run
            "device_copy_gbs": round(copy_gbs, 1),
            "frac_of_device_copy": round(achieved / copy_gbs, 4),
            "kernel_us_p10_p50_p90": [kern_pct[10], kern_pct[50], kern_pct[90]],
            "bytes_per_launch": int(launch_bytes),
        },
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_c3(args, np.concatenate(host_k), np.concatenate(host_v),
                                              Hq, Hkv, D, per_tok)
    return res


def single_token_append_rates() -> dict:
    """Single-token appends at the sliding-layer shape (Hkv 8, head_dim 256,
    4-bit group 64): 4096 one-token appends into a linear cache (the C1
    store, the reference's decode-loop store, src/cache.rs:266-310) and 8192
    into a ring of 1024 slots (the C2 store, 7 wraps), timed as stream time
    between two events around the whole run (launch costs included)."""
    import torch

    import fmkv
    import synth

    Hkv, D, bits = 8, 256, 4
    lib = fmkv.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for name, n, window in (("single_token_linear_4096", 4096, 0),
                            ("single_token_ring_1024_8192", 8192, 1024)):
        k = dev_bf16(synth.kv_rows(51, n, Hkv, D, None))
        v = dev_bf16(synth.kv_rows(52, n, Hkv, D, None))
        row = Hkv * D * 2
        for rep in range(2):  # the first pass warms the kernel up, untimed
            cache = fmkv.KVCache.new_quantized_with_window(D, bits, window or None, Hkv,
                                                           0 if window else n)
            h = cache._h
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
            kp, vp = k.data_ptr(), v.data_ptr()
            for t in range(n):
                if lib.fmkv_cache_append(h, kp + t * row, vp + t * row, 1, stream):
                    raise RuntimeError(lib.fmkv_last_error().decode())
            ev1.record()
            torch.cuda.synchronize()
            del cache
        us = ev0.elapsed_time(ev1) * 1e3 / n
        out[name] = round(1e6 / us, 1)
        log(f"append {name}: {us:.2f} us per token ({1e6 / us:.0f} tokens/s)")
    return out


def _step_fn(lib, fmkv, h, kd, vd, qd, Hq, Hkv, D, out, stream, pool, tau=0.0):
    """fmkv_decode_step of one token; inputs cycle through `pool` resident rows."""
    row, qrow = Hkv * D * 2, Hq * D * 2
    kp, vp, qp, op = kd.data_ptr(), vd.data_ptr(), qd.data_ptr(), out.data_ptr()

    def step(i):
        t = i % pool
        rc = lib.fmkv_decode_step(h, kp + t * row, vp + t * row, 1, qp + t * qrow, Hq, 1.0, tau, op,
                                  fmkv.DTYPE_BF16, stream)
        if rc:
            raise RuntimeError(lib.fmkv_last_error().decode())
    return step


def run_c2(args) -> dict:
    """Sliding-window layer: batch 1, Hq 16, Hkv 8, head_dim 256, a ring of
    1024 slots, 4-bit group 64; 8192 single-token decode steps (8 wraps),
    attention after every append. Eager: one fmkv_decode_step call per step
    from Python. Graph: one wrap (1024 steps) captured into a HIP graph and
    replayed -- in steady state a ring step depends on the position only
    through (T - 1) mod W, so the same graph replays exactly."""
    import torch

    import fmkv
    import synth

    Hq, Hkv, D, bits, W = 16, 8, 256, 4, 1024
    per_tok = bytes_per_token_head(D, bits)
    pool = 1024
    ch = synth.outlier_channels(7, Hkv, D)
    kd = dev_bf16(synth.kv_rows(51, pool, Hkv, D, ch))
    vd = dev_bf16(synth.kv_rows(52, pool, Hkv, D, ch))
    qd = dev_bf16(synth.q_rows(53, Hq, Hkv, D, ch, batch=pool))
    cache = fmkv.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    out = torch.empty((Hq, D), dtype=torch.bfloat16, device="cuda")
    lib = fmkv.load_library()
    s = torch.cuda.Stream()
    n_steps = 8192
    with torch.cuda.stream(s):
        step = _step_fn(lib, fmkv, cache._h, kd, vd, qd, Hq, Hkv, D, out, s.cuda_stream, pool)
        for i in range(W + 64):  # fill the ring, then steady state
            step(i)
        s.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(s)
        for i in range(n_steps):
            step(i)
        ev1.record(s)
        s.synchronize()
        eager_wall = time.perf_counter() - t0
        eager_gpu_ms = ev0.elapsed_time(ev1)

        # one wrap in a graph (no allocation or memset inside the captured region)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(W):
                step(i)
        s.synchronize()
        g.replay()
        s.synchronize()
        reps = n_steps // W
        ev0.record(s)
        for _ in range(reps):
            g.replay()
        ev1.record(s)
        s.synchronize()
        graph_ms = ev0.elapsed_time(ev1)
    read = W * Hkv * per_tok + 2 * Hq * D * 2 + Hkv * (2 * D * 2 + per_tok)
    graph_us = graph_ms * 1e3 / (reps * W)
    log(f"c2: eager {eager_wall / n_steps * 1e6:.1f} us/step wall ({eager_gpu_ms * 1e3 / n_steps:.1f} "
        f"us GPU span), graph {graph_us:.2f} us/step")
    return {
        "metric": "sliding-window decode steps/s (ring W=1024, 8192 steps, attention after every append)",
        "value": round(1e6 / graph_us, 1),
        "unit": "steps/s",
        "n_gpus": 1, "steps": n_steps, "warmup": W + 64,
        "ms_per_step": round(graph_us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (seeded N(0,1), 4 outlier channels x20; 1024 resident input rows cycled)",
        "config": {"workload": "gemma4-sliding-layer ring decode: Hq 16, Hkv 8, head_dim 256, window "
                               "1024, 4-bit group-64, 1 token append + attention per step, HIP graph "
                               "of 1024 steps replayed 8 times",
                   "batch": 1, "window": W, "n_q_heads": Hq, "n_kv_heads": Hkv, "head_dim": D,
                   "bits": bits},
        "tokens_per_s": round(1e6 / graph_us, 1),
        "step_GBps": round(read / (graph_us * 1e-6) / 1e9, 1),
        "eager": {"us_per_step_wall": round(eager_wall / n_steps * 1e6, 2),
                  "us_per_step_gpu_span": round(eager_gpu_ms * 1e3 / n_steps, 2)},
    }


def run_c4(args) -> dict:
    """Batched ragged decode: 32 sequences with lengths uniform in
    [512, 16384] (seeded), Hq 16, Hkv 8, head_dim 256, 4-bit group 64, paged
    pool of 16-token blocks with block ids in a seeded shuffled order. One
    step appends one token per sequence and attends over all of them
    (fmkv_paged_decode_step)."""
    import torch

    import fmkv
    import synth

    Hq, Hkv, D, bits, n_seqs = 16, 8, 256, 4, 32
    if args.c4_heads:
        Hkv, D, bits = {8: (8, 256, 4), 2: (2, 512, 8)}[args.c4_heads]
    per_tok = bytes_per_token_head(D, bits)
    steps, warm = args.steps if args.steps < 256 else 64, 8
    lens = (512 + (synth.splitmix64(404, n_seqs) % np.uint64(16384 - 512 + 1))).astype(np.int64)
    if args.c4_seqs:  # a uniform batch instead: c4_seqs sequences of c4_len tokens
        n_seqs = args.c4_seqs
        lens = np.full(n_seqs, args.c4_len, np.int64)
    cap = lens + warm + steps + 1
    need = (cap + 15) // 16
    max_blocks = int(need.max())
    n_blocks = int(need.sum())
    perm = np.argsort(synth.splitmix64(405, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s_, nb in enumerate(need):
        tables[s_, :nb] = perm[o:o + nb]
        o += int(nb)
    pool = fmkv.PagedPool(fmkv.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    ch = synth.outlier_channels(9, Hkv, D)
    chunk = 2048
    kc = dev_bf16(synth.kv_rows(61, chunk, Hkv, D, ch))[None]
    vc = dev_bf16(synth.kv_rows(62, chunk, Hkv, D, ch))[None]
    for s_ in range(n_seqs):  # prefill each sequence from a resident 2048-row chunk
        for p0 in range(0, int(lens[s_]), chunk):
            n = min(chunk, int(lens[s_]) - p0)
            pool.append(kc[:, :n].contiguous(), vc[:, :n].contiguous(), dtab[s_:s_ + 1].contiguous(),
                        torch.tensor([p0], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    kd = dev_bf16(synth.kv_rows(63, n_seqs * (warm + steps), Hkv, D, ch))
    vd = dev_bf16(synth.kv_rows(64, n_seqs * (warm + steps), Hkv, D, ch))
    qd = dev_bf16(synth.q_rows(65, Hq, Hkv, D, ch, batch=n_seqs * (warm + steps)))
    out = torch.empty((n_seqs, Hq, D), dtype=torch.bfloat16, device="cuda")
    starts = [torch.tensor(lens + i, dtype=torch.int32, device="cuda") for i in range(warm + steps)]
    slens = [t + 1 for t in starts]
    lib = fmkv.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    row, qrow = n_seqs * Hkv * D * 2, n_seqs * Hq * D * 2

    tau = float(args.sparse_v_tau)

    def step(i):
        mx = int(lens.max()) + i + 1
        rc = lib.fmkv_paged_decode_step(pool._h, kd.data_ptr() + i * row, vd.data_ptr() + i * row,
                                        dtab.data_ptr(), max_blocks, starts[i].data_ptr(),
                                        slens[i].data_ptr(), n_seqs, 1, mx, qd.data_ptr() + i * qrow,
                                        Hq, 1.0, tau, out.data_ptr(), fmkv.DTYPE_BF16, stream)
        if rc:
            raise RuntimeError(lib.fmkv_last_error().decode())

    for i in range(warm):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(warm, warm + steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    tok = float((lens + warm + steps / 2 + 1).sum())
    read = tok * Hkv * per_tok + n_seqs * (2 * Hq * D * 2 + Hkv * (2 * D * 2 + per_tok))
    gbs = read / (us * 1e-6) / 1e9
    log(f"c4: {n_seqs} seqs (Hkv {Hkv}): {us:.1f} us/step, {gbs:.0f} GB/s over {read / 1e6:.0f} MB/step")
    return {
        "metric": "batched ragged paged decode GB/s (32 seqs, lengths U[512,16384])",
        "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (seeded N(0,1), 4 outlier channels x20; prefill from a resident 2048-row chunk)",
        "config": {"workload": "batched ragged decode, paged pool of 16-token blocks (shuffled ids): "
                               f"{n_seqs} sequences, Hq 16, Hkv {Hkv}, head_dim {D}, {bits}-bit group-64, "
                               "1 token append + attention per sequence per step",
                   "n_seqs": n_seqs, "total_context": int(lens.sum()), "n_q_heads": Hq,
                   "n_kv_heads": Hkv, "head_dim": D, "bits": bits, "sparse_v_tau": tau,
                   **({"sparse_v_path": args.sparse_v_path} if tau > 0.0 else {})},
        "hbm_frac_of_value": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_step": int(read),
    }


def run_prefill(args) -> dict:
    """Chunked-prefill attention of one layer (fmkv_prefill_step): 2048-token
    chunks after a prefix of --context tokens. Global layer: Hq 16, Hkv 2,
    head_dim 512, 8-bit, causal; --prefill-sliding: Hq 16, Hkv 8, head_dim
    256, 4-bit, ring W 1024 (band mask). A step appends the chunk and attends
    its 2048 queries. Algorithmic FLOPs: 4 * Hq * D per visible (query, key)
    pair (QK and PV multiply-adds)."""
    import torch

    import fmkv
    import synth

    cb = args.mode == "codebook"
    plain = args.mode == "plain"
    if args.prefill_sliding:
        Hq, Hkv, D, bits, W = 16, 8, 256, 4, 1024
    else:
        Hq, Hkv, D, bits, W = 16, 2, 512, 8, 0
    if cb:
        bits = args.bits or 3
    elif plain:
        bits = 16
    elif args.bits:
        bits = args.bits
    mode = fmkv.MODE_CODEBOOK if cb else fmkv.MODE_PLAIN if plain else fmkv.MODE_AFFINE
    L, T0 = 2048, args.context
    steps = args.steps if args.steps <= 16 else 4
    warm = 1
    cap = 0 if W else T0 + (steps + warm) * L + 16
    cache = fmkv.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap, mode=mode)
    for c0 in range(0, T0, L):
        n = min(L, T0 - c0)
        k = dev_bf16(synth.kv_rows(31, n, Hkv, D, None, dist="t3", offset=c0))
        v = dev_bf16(synth.kv_rows(32, n, Hkv, D, None, offset=c0))
        cache.append(k, v)
    kc = dev_bf16(synth.kv_rows(51, L, Hkv, D, None, dist="t3"))
    vc = dev_bf16(synth.kv_rows(52, L, Hkv, D, None))
    qc = dev_bf16(synth.q_rows(53, Hq, Hkv, D, None, batch=L))
    out = torch.empty((L, Hq, D), dtype=torch.bfloat16, device="cuda")

    def visible_pairs(p0):
        p = np.arange(p0, p0 + L, dtype=np.float64)
        lo = np.maximum(0.0, p - W + 1) if W else np.zeros_like(p)
        return float(np.sum(p - lo + 1))

    for _ in range(warm):
        cache.prefill_step(kc, vc, qc, 1.0, out=out)
    torch.cuda.synchronize()
    pairs = 0.0
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_begin = cache.offset()
    ev0.record()
    for i in range(steps):
        pairs += visible_pairs(t_begin + i * L)
        cache.prefill_step(kc, vc, qc, 1.0, out=out)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    flops = 4.0 * Hq * D * pairs / steps
    tflops = flops / (ms * 1e-3) / 1e12
    tps = L / (ms * 1e-3)
    log(f"prefill chunk {L} at {t_begin}..{cache.offset()}: {ms:.3f} ms/chunk, {tps/1e6:.2f} M tokens/s, "
        f"{tflops:.1f} TFLOP/s")
    name = "sliding (ring W 1024)" if W else "global"
    kind = (f"{bits}-bit TurboQuant codebook" if cb else "plain bf16" if plain else
            f"{bits}-bit group-64 affine")
    return {
        "metric": "prefill attention tokens/s (2048-token chunks)",
        "value": round(tps, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if plain else "u8" if bits == 8 else f"u{bits}",
        "data": "synthetic (seeded SplitMix64: K Student-t(3), V and q N(0,1))",
        "config": {"workload": f"{name} layer chunked prefill: Hq {Hq}, Hkv {Hkv}, head_dim {D}, "
                               f"{kind}, 2048-token chunks after {T0} tokens",
                   "context": T0, "chunk": L, "mode": args.mode, "bits": bits},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None,
                     "kernel": "prefill_attn_kernel (with the chunk's append)"},
    }


def run_append(args) -> dict:
    """The global layer's chunked prefill store at the C3 shape: 2048-token
    chunks of K and V rows (Hkv 2, head_dim 512, 8-bit) appended into a
    32K cache -- rotate, quantize, write (src/cache.rs:266-310) -- and the
    same chunks as raw K projections through the K==V layer prologue
    (src/model/gemma4_attention.rs:52-81). One step = one chunk; the append
    kernel's duration comes from HIP events recorded by its own dispatches."""
    import torch

    import fmkv
    import synth

    Hkv, D, bits, chunk = 2, 512, 8, 2048
    n_chunks = max(1, args.context // chunk)
    per_tok = bytes_per_token_head(D, bits)
    k = dev_bf16(synth.kv_rows(31, chunk, Hkv, D, None, dist="t3"))
    v = dev_bf16(synth.kv_rows(32, chunk, Hkv, D, None))
    rng = np.random.default_rng(33)
    w = dev_bf16(synth.f32_to_bf16_bits((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)))
    pro = fmkv.make_prologue(w, 1e-6, 128, 1e6, v_from_k=True)
    # algorithmic bytes per chunk: bf16 K and V rows in, codes + scale/bias out
    in_bytes = {"plain": 2 * chunk * Hkv * D * 2, "prologue_k_eq_v": chunk * Hkv * D * 2}
    out_bytes = chunk * Hkv * per_tok
    res_rows = {}
    for kind in ("plain", "prologue_k_eq_v"):
        cache = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=n_chunks * chunk)

        def step():
            if kind == "plain":
                cache.append(k, v)
            else:
                cache.append_projected(k, None, pro)

        for _ in range(min(args.warmup, n_chunks)):  # untimed, into a cache dropped after
            step()
        cache = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=n_chunks * chunk)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(n_chunks):
            step()
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / n_chunks
        res_rows[kind] = {"us_per_chunk": round(us, 3), "tokens_per_s": round(chunk / (us * 1e-6), 1),
                          "algorithmic_GBps": round((in_bytes[kind] + out_bytes) / (us * 1e-6) / 1e9, 1)}
        log(f"append {kind}: {us:.2f} us per {chunk}-token chunk (stream time), "
            f"{chunk / us:.1f} M tokens/s")
    main = res_rows["plain"]
    achieved = main["algorithmic_GBps"]
    return {
        "metric": "append tokens/s (2048-token chunked prefill into the quantized cache)",
        "value": main["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": n_chunks,
        "warmup": args.warmup, "ms_per_step": round(main["us_per_chunk"] / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (seeded SplitMix64: K Student-t(3), V N(0,1))",
        "config": {"workload": "gemma4-global-layer chunked prefill store: 2048-token chunks, Hkv 2, "
                               "head_dim 512, 8-bit group-64 affine, into a 32K cache",
                   "chunk": chunk, "n_kv_heads": Hkv, "head_dim": D, "bits": bits},
        "append": res_rows,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "append_kernel<512, 8, 0, false>",
                     "bytes_per_launch": in_bytes["plain"] + out_bytes,
                     "note": "stream time per chunk (launch gaps included)"},
    }


def run_c5(args) -> dict:
    """Decode-step cache traffic of a 30-layer Gemma-4-26B-A4B-shaped stack:
    25 sliding layers (ring of 1024, Hkv 8, head_dim 256, 4-bit) and 5 global
    layers (Hkv 2, head_dim 512, 8-bit) at i % 6 == 5; chunked-prefill appends
    of 2048 tokens to 131072 positions, then decode steps of every layer
    (with --sparse-v-tau, every layer's decode step gated, as the reference
    gates every layer at decode: src/model/gemma4_attention.rs:91-93)."""
    import torch

    import fmkv
    import synth

    Hq, T0, chunk = 16, args.c5_context, 2048
    steps, warm = 16, 4
    glob = [i % 6 == 5 for i in range(30)]
    caches, shapes = [], []
    for g in glob:
        if g:
            caches.append(fmkv.KVCache.new_quantized(512, 8, 2, capacity=T0 + warm + steps + 16))
            shapes.append((2, 512, 8))
        else:
            caches.append(fmkv.KVCache.new_quantized_with_window(256, 4, 1024, 8))
            shapes.append((8, 256, 4))
    inputs = {}
    for (Hkv, D, bits) in set(shapes):
        ch = synth.outlier_channels(11 + D, Hkv, D)
        inputs[D] = (dev_bf16(synth.kv_rows(71 + D, chunk, Hkv, D, ch)),
                     dev_bf16(synth.kv_rows(72 + D, chunk, Hkv, D, ch)),
                     dev_bf16(synth.q_rows(73 + D, Hq, Hkv, D, ch, batch=64)))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for p0 in range(0, T0, chunk):
        for c_, (Hkv, D, bits) in zip(caches, shapes):
            c_.append(inputs[D][0], inputs[D][1])
    ev1.record()
    torch.cuda.synchronize()
    prefill_ms = ev0.elapsed_time(ev1)
    lib = fmkv.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    outs = {D: torch.empty((Hq, D), dtype=torch.bfloat16, device="cuda") for D in inputs}
    tau = float(args.sparse_v_tau)
    fns = [_step_fn(lib, fmkv, c_._h, inputs[D][0], inputs[D][1], inputs[D][2], Hq, Hkv, D, outs[D],
                    stream, 64, tau) for c_, (Hkv, D, bits) in zip(caches, shapes)]
    for i in range(warm):
        for f in fns:
            f(i)
    torch.cuda.synchronize()
    ev0.record()
    for i in range(warm, warm + steps):
        for f in fns:
            f(i)
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    Tg = T0 + warm + steps / 2 + 1
    read = 5 * Tg * 2 * bytes_per_token_head(512, 8) + 25 * 1024 * 8 * bytes_per_token_head(256, 4)
    gbs = read / (us * 1e-6) / 1e9
    log(f"c5: prefill {prefill_ms:.1f} ms, decode {us:.1f} us/step (30 layers), {gbs:.0f} GB/s")
    return {
        "metric": "30-layer stack decode-step cache GB/s at 131072 context",
        "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (seeded N(0,1), 4 outlier channels x20; resident 2048-row chunks reused)",
        "config": {"workload": "gemma4-26B-A4B-shaped 30-layer stack: 25 sliding (W 1024, Hkv 8, "
                               "head_dim 256, 4-bit) + 5 global (Hkv 2, head_dim 512, 8-bit) layers, "
                               "chunked prefill of 2048, then 1-token decode steps",
                   "context": T0, "layers": 30, "batch": 1, "sparse_v_tau": tau,
                   **({"sparse_v_path": args.sparse_v_path} if tau > 0.0 else {})},
        "hbm_frac_of_value": round(gbs / HBM_PEAK_GBS, 4),
        "prefill_ms": round(prefill_ms, 2),
        "prefill_tokens_per_s_per_layer": round(T0 / (prefill_ms / 1e3) * 30, 1),
        "bytes_per_step": int(read),
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Host threads for the all-cores run: the cores this process may use,
    capped by OMP_NUM_THREADS when it is set."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(avail, env) if env > 0 else avail)


class ReferenceLayer:
    """The reference's per-layer decode work on the CPU, restated with the
    oracle (src/cache.rs:266-310 and src/model/gemma4_attention.rs:94-103):
    update_and_fetch runs turbo_round_trip_kv on the new K and V rows (dense
    x.R and .Rt matmuls, Lloyd-Max binning; R built once), concatenates them
    onto the stored bf16 arrays (a fresh array each call, O(T)), and SDPA
    reads the whole bf16 cache in MLX's unfused op order."""

    def __init__(self, oracle, k0, v0, capacity, Hq, bits, n_threads):
        self.ora, self.Hq, self.bits, self.threads = oracle, Hq, bits, n_threads
        T, Hkv, D = k0.shape
        self.r, self.rt = oracle.build_rht(D)
        # two buffers per array: each append writes a fresh array (MLX's
        # allocator recycles the freed one, so no page is touched twice)
        self.kb = [np.empty((capacity, Hkv, D), np.uint16) for _ in range(2)]
        self.vb = [np.empty((capacity, Hkv, D), np.uint16) for _ in range(2)]
        self.kb[0][:T], self.vb[0][:T] = k0, v0
        self.cur, self.T = 0, T
        self.out = np.empty((Hq, D), np.uint16)

    def append(self, k_new, v_new):
        o = self.ora
        kq = o.turbo_round_trip_rt(k_new, self.bits, self.r, self.rt)
        vq = o.turbo_round_trip_rt(v_new, self.bits, self.r, self.rt)
        nxt = 1 - self.cur
        o.concat_rows(self.kb[self.cur], self.T, kq, self.kb[nxt], self.threads)
        o.concat_rows(self.vb[self.cur], self.T, vq, self.vb[nxt], self.threads)
        self.cur, self.T = nxt, self.T + k_new.shape[0]

    def attend(self, q):
        k, v = self.kb[self.cur][:self.T], self.vb[self.cur][:self.T]
        return self.ora.sdpa_bf16_decode(q, k, v, 1.0, self.threads)


def cpu_baseline_c3(args, k_bf16, v_bf16, Hq, Hkv, D, per_tok) -> dict:
    """The reference's decode step at 32K, timed with the oracle on this
    host: append (TurboQuant round trip of the token's K/V rows + the O(T)
    concat) and SDPA over the bf16 cache, on all cores for about
    args.cpu_seconds and on one core for two steps; then C1 in full (4096
    single-token appends into a Hq 16, Hkv 8, head_dim 256 layer, then one
    decode step) on all cores."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    import synth

    T = k_bf16.shape[0]
    # TurboQuant takes 2-4 bits (src/cache.rs:87 panics otherwise); its cost
    # is the two dense D x D matmuls per row whatever the bit width
    rt_bits = 4
    q = synth.q_rows(43, Hq, Hkv, D, None)
    kn = synth.kv_rows(44, 64, Hkv, D, None, dist="t3")
    vn = synth.kv_rows(45, 64, Hkv, D, None)
    threads = cpu_threads()

    def run(n_threads, seconds, max_reps):
        lay = ReferenceLayer(oracle, k_bf16, v_bf16, T + max_reps + 1, Hq, rt_bits, n_threads)
        lay.append(kn[:1], vn[:1])  # warm (first touch of the second buffers)
        lay.attend(q)
        reps, t0 = 0, time.perf_counter()
        while reps < max_reps:
            lay.append(kn[reps + 1:reps + 2], vn[reps + 1:reps + 2])
            lay.attend(q)
            reps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        return (time.perf_counter() - t0) / reps, reps, lay.T

    dt, reps, t_end = run(threads, args.cpu_seconds, 60)
    dt1, reps1, _ = run(1, float("inf"), 2)
    step_bytes = (T + 1) * Hkv * per_tok + 2 * Hq * D * 2 + Hkv * (2 * D * 2 + per_tok)
    gbs, gbs1 = step_bytes / dt / 1e9, step_bytes / dt1 / 1e9
    log(f"cpu baseline: {dt*1e3:.1f} ms per 32K decode step on {threads} threads, "
        f"{dt1*1e3:.1f} ms on 1")
    c1 = cpu_baseline_c1(oracle, synth, threads)
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} reference decode step(s) at T={T}..{t_end} on {threads} threads: "
                  f"TurboQuant round trip of the token's K/V rows ({rt_bits}-bit, dense R), O(T) "
                  f"concat onto the bf16 cache, SDPA over it (MLX CPU op order) -- {dt*1e3:.1f} "
                  f"ms/step; GB/s over the same algorithmic bytes as the GPU step",
        "ms_per_step": round(dt * 1e3, 3),
        "one_core": {"value": round(gbs1, 3), "unit": "GB/s", "ms_per_step": round(dt1 * 1e3, 3),
                     "steps": reps1},
        "nproc": os.cpu_count(),
        "cpu_model": cpu_model(),
        "c1_full": c1,
    }


def cpu_baseline_c1(oracle, synth, threads) -> dict:
    """C1 on the reference path, in full: 4096 single-token appends (round
    trip at 4 bits + O(T) concat each) into a Hq 16, Hkv 8, head_dim 256
    layer, then one decode step (append + SDPA)."""
    Hq, Hkv, D, T = 16, 8, 256, 4096
    ch = synth.outlier_channels(1, Hkv, D)
    k = synth.kv_rows(81, T + 1, Hkv, D, ch)
    v = synth.kv_rows(82, T + 1, Hkv, D, ch)
    q = synth.q_rows(83, Hq, Hkv, D, ch)
    lay = ReferenceLayer(oracle, k[:0], v[:0], T + 1, Hq, 4, threads)
    t0 = time.perf_counter()
    for i in range(T):
        lay.append(k[i:i + 1], v[i:i + 1])
    t1 = time.perf_counter()
    lay.append(k[T:], v[T:])
    lay.attend(q)
    t2 = time.perf_counter()
    log(f"cpu baseline C1: {T} appends in {t1 - t0:.2f} s, decode step {(t2 - t1)*1e3:.1f} ms "
        f"({threads} threads)")
    return {"append_tokens_per_s": round(T / (t1 - t0), 1), "appends": T,
            "decode_step_ms": round((t2 - t1) * 1e3, 3), "threads": threads,
            "workload": "Hq 16, Hkv 8, head_dim 256, 4-bit TurboQuant round trip, bf16 cache"}


def device_copy_gbs(mib: int = 256, reps: int = 8) -> float:
    """A plain device-to-device copy of `mib` MiB, timed with events: bytes
    read plus bytes written per second, in GB/s (the reference point for
    what this GPU's HBM delivers to a simple streaming kernel)."""
    import torch

    n = mib * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(reps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    del src, dst
    return 2 * n / ms / 1e6


def copy_calibration(mib: int) -> int:
    """A plain copy of known size: its FETCH_SIZE / WRITE_SIZE readings per
    dispatch against the bytes it moves give the factor that turns the same
    counters on the decode kernel into HBM bytes."""
    import torch

    n = mib * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(8):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / 8
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "ms_per_copy": round(ms, 4),
                      "GB/s (read+write)": round(2 * n / ms / 1e6, 1)}), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--bps", type=int, default=0, help="blocks per split-K work-group (0: auto)")
    ap.add_argument("--graph-steps", type=int, default=64,
                    help="c3: also time this many steps captured in a HIP graph (0: skip)")
    ap.add_argument("--sparse-v-tau", type=float, default=0.0,
                    help="c3, c4, c5: sparse-V threshold (0: dense softmax attention; > 0: the "
                         "statistics pass, then the second half --sparse-v-path names)")
    ap.add_argument("--sparse-v-path", choices=["gather", "gated"], default="gather",
                    help="sparse-V after the statistics pass: the gather of the kept V rows "
                         "(default; the statistics pass is the timed kernel) or the gated pass "
                         "and the split merge (the gated pass is the timed kernel)")
    ap.add_argument("--unfused", action="store_true",
                    help="time fmkv_cache_append + fmkv_decode_attention instead of fmkv_decode_step")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 8 device-to-device copies of MIB MiB (the reference kernel "
                         "for scaling HBM byte counters) and exit")
    ap.add_argument("--workload", choices=["c3", "c2", "c4", "c5", "prefill", "append"], default="c3",
                    help="c3 (default): global layer at 32K; c2: sliding ring, 8192 steps; "
                         "c4: 32 ragged paged sequences; c5: 30-layer stack; prefill: "
                         "2048-token chunked-prefill attention after --context tokens; append: "
                         "the C3 chunked-prefill store alone")
    ap.add_argument("--prefill-sliding", action="store_true",
                    help="prefill workload on the sliding-layer shape (ring W 1024)")
    ap.add_argument("--c5-context", type=int, default=131072)
    ap.add_argument("--mode", choices=["affine", "codebook", "plain"], default="affine",
                    help="c3 and prefill: cache mode (codebook = the reference's TurboQuant "
                         "indices + norm; plain = unquantized bf16 rows)")
    ap.add_argument("--bits", type=int, default=0,
                    help="c3 and prefill: code bits (0: the shape's affine bits, 3 for codebook, "
                         "the reference's default)")
    ap.add_argument("--c4-seqs", type=int, default=0,
                    help="c4: a uniform batch of this many sequences of --c4-len tokens instead")
    ap.add_argument("--c4-len", type=int, default=32768)
    ap.add_argument("--c4-heads", type=int, default=0, choices=[0, 2, 8],
                    help="c4: 8 (Hkv 8, head_dim 256, 4-bit; default) or 2 (Hkv 2, head_dim 512, 8-bit)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the KV path is "
              "built and measured on a single MI355X).", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    import fmkv

    if args.bps:
        fmkv.set_blocks_per_split(args.bps)
    fmkv.set_sparse_v_gather(args.sparse_v_path == "gather")
    res = {"c3": run_c3, "c2": run_c2, "c4": run_c4, "c5": run_c5,
           "prefill": run_prefill, "append": run_append}[args.workload](args)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
