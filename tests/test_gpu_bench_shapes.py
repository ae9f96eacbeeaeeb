"""The shapes the benchmark and the committed profiles time, checked against
the oracle at full size.

  * a 2048-token fmkv_prefill_step chunk after a 32768-token global prefill
    (Hq 16, Hkv 2, head_dim 512, 8-bit; the chunk the prefill profile times):
    every stored code of the chunk bit-exact, and sampled query rows of the
    chunk -- its first and last rows among them -- against
    OracleCache.prefill (src/model/gemma4_attention.rs:84-104, causal mask
    src/model/mod.rs:682-704);
  * the same on a sliding ring of W 1024 (Hq 16, Hkv 8, head_dim 256,
    4-bit): 2048-token chunks longer than the window, banded mask
    (src/model/mod.rs:717-753);
  * 3-bit codebook (TurboQuant, the reference's default cache,
    src/main.rs:84) decode steps at 32K context under the default split plan
    (about 120 splits of 16-17 blocks per KV head), against the oracle's
    attention over the stored indices (src/cache.rs:94-129).

Tolerance of the path: max-abs 2e-2, mean-abs 2e-3 (bf16 outputs: 2e-2 plus
half a bf16 ulp of the exact value)."""
import numpy as np
import pytest

from gpu_util import check_attention, check_codes, dev_bf16, fast_kv, fast_q

pytestmark = pytest.mark.gpu


def _prefill_rows(n):
    return sorted({0, 1, 2, 17, n // 2 - 1, n // 2, n - 2, n - 1})


def test_prefill_2048_chunk_after_32k_global(gpu, ora):
    import torch

    Hq, Hkv, D, bits, T0, L = 16, 2, 512, 8, 32768, 2048
    cap = T0 + L
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap)
    for c0 in range(0, T0, L):
        k = fast_kv(500 + c0, L, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(100500 + c0, L, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    k = fast_kv(591, L, Hkv, D, dist="t3", outliers=False)
    v = fast_kv(592, L, Hkv, D, outliers=False)
    q = fast_q(593, L, Hq, Hkv, D, outliers=False)
    out32 = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 0.05, dtype=torch.float32)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    rows = _prefill_rows(L)
    ref = oc.prefill(k, v, q, 0.05, rows=rows)
    check_codes(codes, meta, oc, slots=np.arange(T0 - 16, T0 + L), what="32K + 2048 chunk codes")
    got = out32[rows]
    check_attention(got, ref, "2048-token chunk after 32K, sampled rows")
    assert cache.offset() == T0 + L


def test_prefill_2048_chunks_on_ring_1024(gpu, ora):
    import torch

    Hq, Hkv, D, bits, W, L = 16, 8, 256, 4, 1024, 2048
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    oc = ora.OracleCache(Hkv, D, bits, W)
    rows = _prefill_rows(L) + [W - 1, W, W + 1]
    for c in range(3):
        k, v = fast_kv(700 + 2 * c, L, Hkv, D), fast_kv(701 + 2 * c, L, Hkv, D)
        q = fast_q(700 + 2 * c, L, Hq, Hkv, D)
        scale = 1.0 if c % 2 == 0 else 0.01
        dt = torch.float32 if c < 2 else torch.bfloat16
        out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), scale, dtype=dt)
        codes, meta = cache.read_codes()
        torch.cuda.synchronize()
        ref = oc.prefill(k, v, q, scale, rows=rows)
        check_codes(codes, meta, oc, what=f"ring chunk {c} codes")
        check_attention(out[rows], ref, f"ring chunk {c} (scale {scale}, {dt}), sampled rows")
    assert cache.offset() == 3 * L and cache.stored_len() == W


def test_codebook3_32k_decode_steps_default_plan(gpu, ora):
    import torch

    Hq, Hkv, D, bits, T0, L, steps = 16, 2, 512, 3, 32768, 2048, 4
    cap = T0 + 16
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap, mode=gpu.MODE_CODEBOOK)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap, mode=1)
    for c0 in range(0, T0, L):
        k = fast_kv(800 + c0, L, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(100800 + c0, L, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    splits = cache.decode_splits()
    assert splits > 64, f"the 32K plan has many splits (got {splits})"
    k1 = fast_kv(891, steps, Hkv, D, dist="t3", outliers=False)
    v1 = fast_kv(892, steps, Hkv, D, outliers=False)
    q = fast_q(893, steps, Hq, Hkv, D, outliers=False)
    outs = []
    for i in range(steps):
        scale = 1.0 if i % 2 == 0 else 0.01
        dt = torch.float32 if i < 2 else torch.bfloat16
        outs.append((scale, cache.decode_step(dev_bf16(k1[i:i + 1]), dev_bf16(v1[i:i + 1]),
                                              dev_bf16(q[i]), scale, dtype=dt)))
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    for i in range(steps):
        oc.append(k1[i:i + 1], v1[i:i + 1])
        scale, out = outs[i]
        check_attention(out, oc.attention(q[i], scale), f"codebook 3-bit step {i} scale {scale}")
    check_codes(codes, meta, oc, slots=np.arange(T0 - 64, T0 + steps), what="codebook 32K steps")
