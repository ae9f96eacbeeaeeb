"""Decode step (append + attention in one call) on the GPU.

With one new token the attention launch appends it itself (its new-token
column) and adds the token's attention as one more split partial. The step
must store codes bit-identical to the oracle's and to a separate append,
attend within the path tolerance (max-abs 2e-2, mean-abs 2e-3) of the
oracle's exact attention over its dequantized cache, and agree with the two
separate calls to 1e-3 + 1e-4 relative (the same cache read; only the new
token's score is summed in a different order)."""

# fused step vs append + attention (see the module docstring)
TWO_CALLS_RTOL, TWO_CALLS_ATOL = 1e-4, 1e-3
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu


def q_rows(seed, Hq, Hkv, D):
    return synth.q_rows(seed, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D))


@pytest.mark.parametrize("D,bits,Hkv,Hq,W", [
    (512, 8, 2, 16, 0),     # global layer shape
    (256, 4, 8, 16, 64),    # sliding layer shape, ring of 64 slots
    (128, 4, 4, 4, 0),
    (256, 8, 2, 12, 32),
])
def test_step_matches_oracle_and_two_calls(gpu, ora, D, bits, Hkv, Hq, W):
    import torch

    cap = 0 if W else 400
    a = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
    b = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, W, cap)
    k0, v0 = kv_batch(1, 90, Hkv, D), kv_batch(2, 90, Hkv, D)
    for c in (a, b):
        c.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    for step in range(40):
        n = 1 if step % 7 else 3  # mostly single tokens, sometimes a few
        k = kv_batch(100 + 2 * step, n, Hkv, D, special=False)
        v = kv_batch(101 + 2 * step, n, Hkv, D, special=False)
        q = q_rows(300 + step, Hq, Hkv, D)
        out_a = a.decode_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 0.05, dtype=torch.float32)
        b.append(dev_bf16(k), dev_bf16(v))
        out_b = b.attention(dev_bf16(q), 0.05, dtype=torch.float32)
        oc.append(k, v)
        torch.cuda.synchronize()
        assert a.offset() == b.offset() == oc.offset
        assert torch.allclose(out_a, out_b, rtol=TWO_CALLS_RTOL, atol=TWO_CALLS_ATOL), \
            f"step {step}: step vs two calls"
        check_attention(out_a, oc.attention(q, 0.05), f"step {step}")
    ca, ma = a.read_codes()
    cb, mb = b.read_codes()
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(ca), host_u32(cb)) and np.array_equal(host_u16(ma), host_u16(mb))
    filled = min(oc.offset, oc.n_slots)
    assert np.array_equal(host_u32(ca)[:filled], oc.codes[:filled])
    assert np.array_equal(host_u16(ma)[:filled], oc.meta[:filled])


@pytest.mark.parametrize("D,bits,Hkv,Hq,W", [(512, 8, 2, 16, 0), (256, 4, 8, 16, 32)])
def test_steps_from_empty_cache(gpu, ora, D, bits, Hkv, Hq, W):
    """Single-token steps from position 0: the first step attends to the new
    token alone; block boundaries (16, 17) and, for the ring, the first wraps
    (32, 33) pass."""
    import torch

    cap = 0 if W else 64
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, W, cap)
    for step in range(40):
        k = kv_batch(500 + 2 * step, 1, Hkv, D, special=False)
        v = kv_batch(501 + 2 * step, 1, Hkv, D, special=False)
        q = q_rows(600 + step, Hq, Hkv, D)
        out = cache.decode_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0 / np.sqrt(D),
                                dtype=torch.float32)
        oc.append(k, v)
        torch.cuda.synchronize()
        check_attention(out, oc.attention(q, 1.0 / np.sqrt(D)), f"step {step}")
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    filled = min(oc.offset, oc.n_slots)
    assert np.array_equal(host_u32(codes)[:filled], oc.codes[:filled])
    assert np.array_equal(host_u16(meta)[:filled], oc.meta[:filled])


def test_step_validation_leaves_cache_unchanged(gpu):
    import torch

    cache = gpu.KVCache.new_quantized(256, 4, 2, capacity=32)
    k = torch.zeros((1, 2, 256), dtype=torch.bfloat16, device="cuda")
    bad_q = torch.ones((3, 256), dtype=torch.bfloat16, device="cuda")  # 3 % 2 != 0
    with pytest.raises(gpu.Exception_):
        cache.decode_step(k, k, bad_q)
    assert cache.offset() == 0
    q = torch.ones((4, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(gpu.Exception_) as ei:
        cache.decode_step(k, k, q, sparse_v_tau=-0.5)
    assert ei.value.code == gpu.FMKV_ERR_INVALID_ARG
    assert cache.offset() == 0
    out = cache.decode_step(k, k, q, dtype=torch.float32)
    torch.cuda.synchronize()
    assert cache.offset() == 1 and torch.isfinite(out).all()


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(256, 4, 8, 16), (512, 8, 2, 16)])
@pytest.mark.parametrize("bps", [0, 2, 8])
def test_paged_step_matches_oracle_and_two_calls(gpu, ora, D, bits, Hkv, Hq, bps):
    """bps: blocks per split (0: the plan's; 2 and 8 give several splits
    per sequence)."""
    import torch

    lens = [3, 40, 129, 16, 1, 250]
    n_seqs = len(lens)
    need = [(n + 2 + 15) // 16 for n in lens]
    max_blocks = max(need)
    n_blocks = sum(need) + 5
    perm = np.argsort(synth.splitmix64(55, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    desc = gpu.make_desc(Hkv, D, bits)
    pa, pb = gpu.PagedPool(desc, n_blocks), gpu.PagedPool(desc, n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, n in enumerate(lens):
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 2)
        k, v = kv_batch(20 * s, n, Hkv, D), kv_batch(20 * s + 1, n, Hkv, D)
        oc.append(k, v)
        oracles.append(oc)
        for p in (pa, pb):
            p.append(dev_bf16(k[None]), dev_bf16(v[None]), dtab[s:s + 1].contiguous(),
                     torch.zeros(1, dtype=torch.int32, device="cuda"))
    for step in range(2):
        k1 = np.stack([kv_batch(700 + 10 * step + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
        v1 = np.stack([kv_batch(800 + 10 * step + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
        start = torch.tensor([n + step for n in lens], dtype=torch.int32, device="cuda")
        seq_lens = start + 1
        mx = max(lens) + step + 1
        q = np.stack([q_rows(950 + 10 * step + s, Hq, Hkv, D) for s in range(n_seqs)])
        gpu.set_blocks_per_split(bps)
        try:
            out_a = pa.decode_step(dev_bf16(k1), dev_bf16(v1), dtab, start, seq_lens, mx, dev_bf16(q),
                                   0.05, dtype=torch.float32)
            pb.append(dev_bf16(k1), dev_bf16(v1), dtab, start)
            out_b = pb.attention(dev_bf16(q), dtab, seq_lens, mx, 0.05, dtype=torch.float32)
            torch.cuda.synchronize()
        finally:
            gpu.set_blocks_per_split(0)
        assert torch.allclose(out_a, out_b, rtol=TWO_CALLS_RTOL, atol=TWO_CALLS_ATOL), \
            f"step {step}: step vs two calls"
        for s in range(n_seqs):
            oracles[s].append(k1[s], v1[s])
            check_attention(out_a[s], oracles[s].attention(q[s], 0.05), f"step {step} seq {s}")
    ca, cb = pa.read_codes(), pb.read_codes()
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(ca[0]), host_u32(cb[0]))
    assert np.array_equal(host_u16(ca[1]), host_u16(cb[1]))
