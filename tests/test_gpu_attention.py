"""Decode attention on the GPU against the oracle (exact f64 softmax attention
over the oracle's dequantized, un-rotated cache). Tolerance: max-abs 2e-2,
mean-abs 2e-3 (bf16 outputs: 2e-2 plus half a bf16 ulp of the exact value)."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, kv_batch

pytestmark = pytest.mark.gpu


def q_batch(seed, Hq, Hkv, D, outliers=True):
    ch = synth.outlier_channels(seed, Hkv, D) if outliers else None
    return synth.q_rows(seed + 100, Hq, Hkv, D, ch)


def filled_cache(gpu, ora, D, bits, Hkv, T, window=0, chunks=None, seed=0):
    cap = 0 if window else T + 16
    cache = gpu.KVCache.new_quantized_with_window(D, bits, window, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, window, cap)
    chunks = chunks or [T]
    for i, n in enumerate(chunks):
        k = kv_batch(seed + 2 * i, n, Hkv, D)
        v = kv_batch(seed + 2 * i + 1, n, Hkv, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    return cache, oc


CONFIGS = [  # D, bits, Hkv, Hq
    (256, 4, 8, 16),
    (256, 8, 8, 16),
    (512, 8, 2, 16),
    (512, 4, 2, 16),
    (128, 4, 4, 4),
    (256, 4, 2, 12),
]


@pytest.mark.parametrize("D,bits,Hkv,Hq", CONFIGS)
@pytest.mark.parametrize("T", [1, 7, 16, 33, 300, 1500])
def test_attention_linear(gpu, ora, D, bits, Hkv, Hq, T):
    import torch

    cache, oc = filled_cache(gpu, ora, D, bits, Hkv, T, chunks=[T // 2, T - T // 2] if T > 1 else [1])
    q = q_batch(T, Hq, Hkv, D)
    for scale in (1.0, 0.03):  # peaked (Gemma-4 scale 1.0) and soft softmax
        ref = oc.attention(q, scale)
        out32 = cache.attention(dev_bf16(q), scale, dtype=torch.float32)
        out16 = cache.attention(dev_bf16(q), scale, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        check_attention(out32, ref, f"f32 T={T} scale={scale}")
        check_attention(out16, ref, f"bf16 T={T} scale={scale}")


@pytest.mark.parametrize("bps", [1, 2, 3, 5])
def test_attention_split_counts_agree(gpu, ora, bps):
    import torch

    D, bits, Hkv, Hq, T = 512, 8, 2, 16, 700
    cache, oc = filled_cache(gpu, ora, D, bits, Hkv, T, seed=4)
    q = q_batch(9, Hq, Hkv, D)
    ref = oc.attention(q, 0.05)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), 0.05, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, ref, f"bps={bps}")


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(256, 4, 8, 16), (128, 4, 4, 4), (128, 8, 2, 12),
                                           (256, 4, 2, 12)])
@pytest.mark.parametrize("bps", [7, 8, 13, 40])
def test_attention_stream_kinds_agree(gpu, ora, D, bits, Hkv, Hq, bps):
    """Head-blocks of at most 1024 code bits per token are streamed by wave
    pairs in work-groups of fewer than 8 blocks and by single waves from 8
    blocks on: both kinds, dense and sparse-V, against the oracle over a
    context that ends inside a block."""
    import torch

    T, tau = 1500, 1.0 / 3000
    cache, oc = filled_cache(gpu, ora, D, bits, Hkv, T, chunks=[700, 800], seed=11)
    q = q_batch(12, Hq, Hkv, D)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), 1.0, dtype=torch.float32)
        gated = cache.attention(dev_bf16(q), 1.0, sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, oc.attention(q, 1.0), f"dense bps={bps}")
    check_attention(gated, oc.attention(q, 1.0, tau), f"sparse-V bps={bps}")


@pytest.mark.parametrize("D,bits", [(256, 4), (256, 8)])
def test_attention_ring_through_wraps(gpu, ora, D, bits):
    """Sliding layer: W = 64, one append per decode step, attention after every
    append (the reference attends to the last W positions incl. the current)."""
    import torch

    Hkv, Hq, W = 8, 16, 64
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    oc = ora.OracleCache(Hkv, D, bits, W)
    for step in range(150):
        k = kv_batch(1000 + 2 * step, 1, Hkv, D, special=False)
        v = kv_batch(1001 + 2 * step, 1, Hkv, D, special=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
        if step in (0, 1, 15, 16, 63, 64, 65, 100, 127, 128, 149):
            q = q_batch(step, Hq, Hkv, D)
            out = cache.attention(dev_bf16(q), 0.05, dtype=torch.float32)
            torch.cuda.synchronize()
            assert cache.stored_len() == min(step + 1, W)
            check_attention(out, oc.attention(q, 0.05), f"ring step {step}")


def test_attention_after_trim(gpu, ora):
    import torch

    cache, oc = filled_cache(gpu, ora, 256, 4, 8, 300, seed=21)
    for keep in (290, 50, 17, 1):
        cache.trim(keep)
        oc.trim(keep)
        assert cache.stored_len() == oc.stored_len() == keep
        q = q_batch(keep, 16, 8, 256)
        out = cache.attention(dev_bf16(q), 0.05, dtype=torch.float32)
        torch.cuda.synchronize()
        check_attention(out, oc.attention(q, 0.05), f"trim {keep}")


def test_empty_cache_attention_is_zero(gpu):
    import torch

    cache = gpu.KVCache.new_quantized(256, 4, 2, capacity=32)
    q = torch.ones((4, 256), dtype=torch.bfloat16, device="cuda")
    out = cache.attention(q, dtype=torch.float32)
    torch.cuda.synchronize()
    assert not out.any()


def test_attention_rejects_bad_arguments(gpu):
    import torch

    cache = gpu.KVCache.new_quantized(256, 4, 2, capacity=32)
    q = torch.ones((4, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(gpu.Exception_) as ei:
        cache.attention(q, sparse_v_tau=-1e-4)
    assert ei.value.code == gpu.FMKV_ERR_INVALID_ARG
    with pytest.raises(gpu.Exception_):
        cache.attention(torch.ones((3, 256), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(gpu.Exception_):
        cache.attention(torch.ones((18, 256), dtype=torch.bfloat16, device="cuda"))
