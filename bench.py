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
  cpu_baseline  the reference's decode read (SDPA over its bf16 cache, MLX
             CPU op order) timed with the oracle on this host's cores.
"""
from __future__ import annotations

import argparse
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
TRAFFIC_BYTES_PER_LAUNCH = 75_860_000
TRAFFIC_SOURCE = "profiles/decode_attn_c3_hbm_traffic.md"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def bytes_per_token_head(D: int, bits: int) -> int:
    """K+V codes plus f16 scale and bias per 64-dim group, one token, one KV head."""
    return 2 * (D * bits // 8 + 4 * (D // 64))


def run_c3(args) -> dict:
    import torch

    import fmkv
    import synth

    Hq, Hkv, D, bits, T0 = 16, 2, 512, 8, args.context
    per_tok = bytes_per_token_head(D, bits)
    n_dec = args.warmup + 2 * args.steps + 1
    cache = fmkv.KVCache.new_quantized(D, bits, Hkv, capacity=T0 + n_dec + 16)

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
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for k, v in zip(dk, dv):
        cache.append(k, v)
    ev1.record()
    torch.cuda.synchronize()
    prefill_ms = ev0.elapsed_time(ev1)
    append_prefill_tps = T0 / (prefill_ms / 1e3)
    log(f"prefill {T0} tokens in {prefill_ms:.2f} ms ({append_prefill_tps/1e6:.2f} M tokens/s)")
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

    def step():
        nonlocal i
        if args.unfused:
            rc = lib.fmkv_cache_append(h, kp[i], vp[i], 1, stream)
            rc |= lib.fmkv_decode_attention(h, qp[i], Hq, 1.0, 0.0, outp, fmkv.DTYPE_BF16, stream)
        else:
            rc = lib.fmkv_decode_step(h, kp[i], vp[i], 1, qp[i], Hq, 1.0, 0.0, outp,
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
    fmkv.profile_enable(args.steps)
    tb = cache.offset()
    for _ in range(args.steps):
        step()
    kernel_ms, n_rec = fmkv.profile_collect()
    fmkv.profile_enable(0)
    te = cache.offset()
    avg_T = (tb + te + 1) / 2.0
    kern_s = kernel_ms / n_rec / 1e3
    launch_bytes = avg_T * Hkv * per_tok + 2 * Hq * D * 2
    achieved = launch_bytes / kern_s / 1e9
    log(f"step {ms_per_step*1e3:.1f} us, split kernel {kern_s*1e6:.2f} us over {n_rec} launches, "
        f"{achieved:.0f} GB/s, splits={cache.decode_splits()}")

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
            "workload": "gemma4-global-layer decode at 32K: Hq 16, Hkv 2, head_dim 512, "
                        "8-bit group-64 affine, f16 scale/bias, 1 token append + attention per step",
            "context": T0, "batch": 1, "n_q_heads": Hq, "n_kv_heads": Hkv, "head_dim": D,
            "bits": bits, "group": 64,
        },
        "hbm_frac_of_value": round(value / HBM_PEAK_GBS, 4),
        "append_tokens_per_s": {"chunked_prefill_2048": round(append_prefill_tps, 1)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_source": TRAFFIC_SOURCE,
            "kernel": "decode_attn_kernel<512, 8>",
            "avg_kernel_us": round(kern_s * 1e6, 3),
            "bytes_per_launch": int(launch_bytes),
        },
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_c3(args, np.concatenate(host_k), np.concatenate(host_v),
                                              Hq, Hkv, D, per_tok)
    return res


def cpu_baseline_c3(args, k_bf16, v_bf16, Hq, Hkv, D, per_tok) -> dict:
    """The reference's decode read on its bf16 cache (SDPA, MLX CPU op order),
    timed with the oracle on this host: one full 32K-context step per rep,
    repeated for about args.cpu_seconds."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    import synth

    T = k_bf16.shape[0]
    q = synth.q_rows(43, Hq, Hkv, D, None)
    threads = min(os.cpu_count() or 1, 16, Hq)
    oracle.sdpa_bf16_decode(q, k_bf16[:64], v_bf16[:64], 1.0, threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.sdpa_bf16_decode(q, k_bf16, v_bf16, 1.0, threads)
        reps += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    gbs = (T * Hkv * per_tok + 2 * Hq * D * 2) / dt / 1e9
    log(f"cpu baseline: {dt*1e3:.1f} ms per 32K decode step on {threads} threads")
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} decode step(s) at T={T}: SDPA over the bf16 cache (reference read, MLX CPU "
                  f"op order), {dt*1e3:.1f} ms/step; GB/s over the same algorithmic bytes as the GPU",
        "ms_per_step": round(dt * 1e3, 3),
    }


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
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--bps", type=int, default=0, help="blocks per split-K work-group (0: auto)")
    ap.add_argument("--unfused", action="store_true",
                    help="time fmkv_cache_append + fmkv_decode_attention instead of fmkv_decode_step")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 8 device-to-device copies of MIB MiB (the reference kernel "
                         "for scaling HBM byte counters) and exit")
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
    if args.bps:
        import fmkv

        fmkv.set_blocks_per_split(args.bps)
    res = run_c3(args)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
