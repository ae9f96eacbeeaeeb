"""Sliding windows that are not a multiple of the 16-token head-block, on the
GPU against the oracle.

The reference takes any sliding_window from the model config
(src/cache.rs:206, src/model/mod.rs:376-383): after each update_and_fetch
the last W positions are stored and visible (tail_along_time,
src/cache.rs:140-148; the sliding mask src/model/mod.rs:717-753). Here a
ring holds the window rounded up to whole head-blocks, position p at slot
p mod Ws, and the attention sees the last W positions only, by position.

  * appends (chunks shorter and longer than the ring, single tokens through
    wraps): stored codes bit-exact with the oracle at every slot, stored_len
    = min(offset, W), peek_kv the last W positions;
  * decode steps through wraps in every cache mode, sparse-V steps, and
    prefill chunks on the ring (the band j > p - W), outputs within the path
    tolerance (max-abs 2e-2, mean-abs 2e-3; bf16 outputs: 2e-2 plus half a
    bf16 ulp of the exact value) of the oracle's exact attention."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, check_codes, dev_bf16, kv_batch

pytestmark = pytest.mark.gpu


def q_rows(seed, Hq, Hkv, D):
    return synth.q_rows(seed + 100, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D))


def q_chunk(seed, L, Hq, Hkv, D):
    return synth.q_rows(seed, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D), batch=L)


@pytest.mark.parametrize("W", [5, 40, 100, 1000])
def test_odd_window_appends_bit_exact(gpu, ora, W):
    import torch

    D, bits, Hkv = 256, 4, 4
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    oc = ora.OracleCache(Hkv, D, bits, W)
    assert cache.n_slots() == oc.n_slots == (W + 15) // 16 * 16
    for i, n in enumerate([1, 7, 30, W + 3, 1, 1, 2 * W + 9, 17]):
        k, v = kv_batch(300 + 2 * i, n, Hkv, D), kv_batch(301 + 2 * i, n, Hkv, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
        torch.cuda.synchronize()
        assert cache.offset() == oc.offset
        assert cache.stored_len() == min(oc.offset, W) == oc.stored_len()
        check_codes(*cache.read_codes(), oc, what=f"W={W} after chunk {i} ({n} tokens)")
    kf, vf = cache.peek_kv(dtype=torch.float32)
    wk, wv = oc.dequant_kv()
    assert kf.shape == wk.shape and kf.shape[0] == W
    for got, want in ((kf, wk), (vf, wv)):
        g = got.cpu().numpy()
        assert np.max(np.abs(g - want)) <= 1e-5 * max(1.0, np.abs(want).max())


# mode, D, bits, Hkv, Hq, W
STEP_SHAPES = [
    (0, 256, 4, 8, 16, 40),
    (0, 512, 8, 2, 16, 100),
    (0, 128, 8, 4, 8, 23),
    (1, 512, 3, 2, 16, 72),
    (2, 256, 16, 8, 16, 24),
]


@pytest.mark.parametrize("mode,D,bits,Hkv,Hq,W", STEP_SHAPES)
def test_odd_window_decode_steps_through_wraps(gpu, ora, mode, D, bits, Hkv, Hq, W):
    """Single-token decode steps (append in the attention launch) from an
    empty cache through three wraps of the window, every step checked; the
    stored slots bit-exact at the end."""
    import torch

    cache = gpu.KVCache(gpu.make_desc(Hkv, D, bits, W, 0, mode))
    oc = ora.OracleCache(Hkv, D, bits, W, mode=mode)
    n = 3 * W + 5
    ks = kv_batch(900, n, Hkv, D, special=False)
    vs = kv_batch(901, n, Hkv, D, special=False)
    for i in range(n):
        q = q_rows(950 + i, Hq, Hkv, D)
        scale = 1.0 if i % 2 == 0 else 0.01
        dt = torch.float32 if i % 3 else torch.bfloat16
        out = cache.decode_step(dev_bf16(ks[i:i + 1]), dev_bf16(vs[i:i + 1]), dev_bf16(q), scale,
                                dtype=dt)
        oc.append(ks[i:i + 1], vs[i:i + 1])
        torch.cuda.synchronize()
        check_attention(out, oc.attention(q, scale), f"mode {mode} W={W} step {i}")
    assert cache.stored_len() == W
    check_codes(*cache.read_codes(), oc, what=f"mode {mode} W={W}")


@pytest.mark.parametrize("mode,bits", [(0, 4), (1, 3)])
def test_odd_window_sparse_v_steps(gpu, ora, mode, bits):
    """Sparse-V decode steps on a 40-token window through wraps (statistics
    pass with the appending new-token column, gated pass, combine)."""
    import torch

    D, Hkv, Hq, W, tau = 256, 8, 16, 40, 0.02
    cache = gpu.KVCache(gpu.make_desc(Hkv, D, bits, W, 0, mode))
    oc = ora.OracleCache(Hkv, D, bits, W, mode=mode)
    n = 2 * W + 7
    ks = kv_batch(700, n, Hkv, D, special=False)
    vs = kv_batch(701, n, Hkv, D, special=False)
    for i in range(n):
        q = q_rows(750 + i, Hq, Hkv, D)
        out = cache.decode_step(dev_bf16(ks[i:i + 1]), dev_bf16(vs[i:i + 1]), dev_bf16(q), 0.05,
                                sparse_v_tau=tau, dtype=torch.float32)
        oc.append(ks[i:i + 1], vs[i:i + 1])
        torch.cuda.synchronize()
        check_attention(out, oc.attention(q, 0.05, tau), f"mode {mode} sparse-V step {i}")


# mode, D, bits, Hkv, Hq, W
PREFILL_SHAPES = [
    (0, 256, 4, 8, 16, 40),
    (0, 512, 8, 2, 16, 100),
    (1, 256, 3, 2, 8, 56),
    (2, 128, 16, 4, 8, 30),
]


@pytest.mark.parametrize("mode,D,bits,Hkv,Hq,W", PREFILL_SHAPES)
def test_odd_window_prefill_chunks(gpu, ora, mode, D, bits, Hkv, Hq, W):
    """Chunks shorter and longer than the window after a 37-token prefix: each
    query sees the band p - W < j <= p (the ring read before the chunk's own
    rows overwrite it); the stored slots bit-exact afterwards."""
    import torch

    cache = gpu.KVCache(gpu.make_desc(Hkv, D, bits, W, 0, mode))
    oc = ora.OracleCache(Hkv, D, bits, W, mode=mode)
    k0, v0 = kv_batch(40, 37, Hkv, D), kv_batch(41, 37, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    for step, L in enumerate((1, 19, W + 30, 16, 2 * W + 3)):
        k, v = kv_batch(50 + 2 * step, L, Hkv, D), kv_batch(51 + 2 * step, L, Hkv, D)
        q = q_chunk(60 + step, L, Hq, Hkv, D)
        dt = torch.float32 if step % 2 == 0 else torch.bfloat16
        out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0, dtype=dt)
        want = oc.prefill(k, v, q, 1.0)
        torch.cuda.synchronize()
        check_attention(out, want, f"mode {mode} W={W} chunk {step} (L={L})")
        assert cache.offset() == oc.offset and cache.stored_len() == oc.stored_len()
        check_codes(*cache.read_codes(), oc, what=f"mode {mode} W={W} after chunk {step}")


def test_sliding_window_1000_stack_steps(gpu, ora):
    """A sliding layer of window 1000 (Hq 16, Hkv 8, head_dim 256, 4-bit):
    1100 prefill tokens then 1100 decode steps (two wraps of the 1008-slot
    ring), checked around the window's edges."""
    import torch

    from gpu_util import fast_kv, fast_q

    Hq, Hkv, D, bits, W = 16, 8, 256, 4, 1000
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    oc = ora.OracleCache(Hkv, D, bits, W)
    n0, n = 1100, 1100
    k, v = fast_kv(301, n0 + n, Hkv, D), fast_kv(302, n0 + n, Hkv, D)
    q = fast_q(301, n, Hq, Hkv, D)
    cache.append(dev_bf16(k[:n0]), dev_bf16(v[:n0]))
    kd, vd, qd = dev_bf16(k), dev_bf16(v), dev_bf16(q)
    checks = {0, 6, 7, 8, 500, 907, 908, 915, 916, 1099}
    outs = {}
    for i in range(n):
        o = cache.decode_step(kd[n0 + i:n0 + i + 1], vd[n0 + i:n0 + i + 1], qd[i], 1.0,
                              dtype=torch.float32)
        if i in checks:
            outs[i] = o
    torch.cuda.synchronize()
    done = 0
    oc.append(k[:n0], v[:n0])
    for i in sorted(checks):
        oc.append(k[n0 + done:n0 + i + 1], v[n0 + done:n0 + i + 1])
        done = i + 1
        check_attention(outs[i], oc.attention(q[i], 1.0), f"W=1000 step {i} (T={n0 + i + 1})")
    check_codes(*cache.read_codes(), oc, what="W=1000 ring")
    assert cache.stored_len() == W
