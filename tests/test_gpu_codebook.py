"""Decode attention over codebook (TurboQuant) caches on the GPU against the
oracle: exact f64 softmax attention over the oracle's codebook dequantization
(centroid[idx] * norm / sqrt(D), un-rotated; src/cache.rs:94-129 without the
bf16 round trip). Tolerance: max-abs 2e-2, mean-abs 2e-3 (bf16 outputs: 2e-2
plus half a bf16 ulp of the exact value). Codes written by appends are checked
bit-exact by test_gpu_append.py, those written by decode steps' new-token
column here."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, fast_kv, fast_q, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu
CB = 1  # MODE_CODEBOOK


def q_batch(seed, Hq, Hkv, D):
    ch = synth.outlier_channels(seed, Hkv, D)
    return synth.q_rows(seed + 100, Hq, Hkv, D, ch)


def filled(gpu, ora, D, bits, Hkv, T, window=0, chunks=None, seed=0):
    cap = 0 if window else T + 16
    cache = gpu.KVCache.new_quantized_with_window(D, bits, window, Hkv, cap, mode=CB)
    oc = ora.OracleCache(Hkv, D, bits, window, cap, mode=CB)
    for i, n in enumerate(chunks or [T]):
        k = kv_batch(seed + 2 * i, n, Hkv, D)
        v = kv_batch(seed + 2 * i + 1, n, Hkv, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    return cache, oc


CONFIGS = [  # D, bits, Hkv, Hq
    (256, 3, 8, 16),  # the reference's default cache on a sliding layer
    (512, 3, 2, 16),  # and on a global layer
    (256, 2, 8, 16),
    (256, 4, 8, 16),
    (512, 4, 2, 16),
    (512, 2, 2, 16),
    (128, 3, 4, 4),
    (128, 4, 2, 12),
]


@pytest.mark.parametrize("D,bits,Hkv,Hq", CONFIGS)
@pytest.mark.parametrize("T", [1, 17, 300, 1500])
def test_codebook_attention_linear(gpu, ora, D, bits, Hkv, Hq, T):
    import torch

    cache, oc = filled(gpu, ora, D, bits, Hkv, T, chunks=[T // 2, T - T // 2] if T > 1 else [1])
    q = q_batch(T + bits, Hq, Hkv, D)
    for scale in (1.0, 0.03):
        ref = oc.attention(q, scale)
        out32 = cache.attention(dev_bf16(q), scale, dtype=torch.float32)
        out16 = cache.attention(dev_bf16(q), scale, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        check_attention(out32, ref, f"f32 T={T} scale={scale}")
        check_attention(out16, ref, f"bf16 T={T} scale={scale}")


@pytest.mark.parametrize("bps", [1, 2, 7, 40])
def test_codebook_split_counts_agree(gpu, ora, bps):
    import torch

    D, bits, Hkv, Hq, T = 512, 3, 2, 16, 900
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=5)
    q = q_batch(11, Hq, Hkv, D)
    ref = oc.attention(q, 0.05)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), 0.05, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, ref, f"bps={bps}")


@pytest.mark.parametrize("D,bits,W", [(256, 3, 64), (256, 4, 32), (512, 3, 48)])
def test_codebook_ring_steps_through_wraps(gpu, ora, D, bits, W):
    """Sliding ring: single-token decode steps (append, then attention) across
    several wraps, each step against the oracle."""
    import torch

    Hkv, Hq = (8, 16) if D == 256 else (2, 16)
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, mode=CB)
    oc = ora.OracleCache(Hkv, D, bits, W, mode=CB)
    n = 3 * W + 5
    k, v = kv_batch(21, n, Hkv, D), kv_batch(22, n, Hkv, D)
    q = fast_q(23, n, Hq, Hkv, D)
    kd, vd = dev_bf16(k), dev_bf16(v)
    for i in range(n):
        out = cache.decode_step(kd[i:i + 1], vd[i:i + 1], dev_bf16(q[i]), 0.02, dtype=torch.float32)
        oc.append(k[i:i + 1], v[i:i + 1])
        if i % 7 == 0 or i in (W - 1, W, 2 * W, n - 1):
            torch.cuda.synchronize()
            check_attention(out, oc.attention(q[i], 0.02), f"ring W={W} step {i}")
    assert cache.stored_len() == W


@pytest.mark.parametrize("D,bits,W", [(256, 3, 0), (512, 3, 0), (512, 2, 48), (256, 4, 32), (128, 3, 16)])
def test_codebook_decode_steps_store_append_codes(gpu, ora, D, bits, W):
    """Decode steps append their token in the attention launch's new-token
    column: after a prefill and single-token steps (linear, or a ring through
    wraps) every stored index and norm equals the oracle's round trip, and
    every step's output is within the path tolerance."""
    import torch

    Hkv, Hq = (8, 16) if D == 256 else (2, 16)
    n0, n = 37, (3 * W + 5 if W else 70)
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, 0 if W else n0 + n + 16, mode=CB)
    oc = ora.OracleCache(Hkv, D, bits, W, 0 if W else n0 + n + 16, mode=CB)
    k0, v0 = kv_batch(61, n0, Hkv, D), kv_batch(62, n0, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    k, v = kv_batch(63, n, Hkv, D), kv_batch(64, n, Hkv, D)
    q = fast_q(65, n, Hq, Hkv, D)
    kd, vd = dev_bf16(k), dev_bf16(v)
    for i in range(n):
        out = cache.decode_step(kd[i:i + 1], vd[i:i + 1], dev_bf16(q[i]), 0.02, dtype=torch.float32)
        oc.append(k[i:i + 1], v[i:i + 1])
        if i % 9 == 0 or i == n - 1:
            torch.cuda.synchronize()
            check_attention(out, oc.attention(q[i], 0.02), f"step {i}")
    torch.cuda.synchronize()
    assert cache.offset() == n0 + n
    codes, meta = cache.read_codes()
    c, m = host_u32(codes), host_u16(meta)
    bad = np.argwhere((c != oc.codes).any(-1))
    assert bad.size == 0, f"index mismatch at (slot, kv, head) {bad[:5].tolist()} of {len(bad)}"
    badm = np.argwhere((m != oc.meta).any(-1))
    assert badm.size == 0, f"norm mismatch at {badm[:5].tolist()}"


def test_codebook_trim_and_empty(gpu, ora):
    import torch

    D, bits, Hkv, Hq = 256, 3, 2, 8
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=400, mode=CB)
    q = q_batch(31, Hq, Hkv, D)
    out = cache.attention(dev_bf16(q), 1.0, dtype=torch.float32)  # empty cache
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
    cache2, oc = filled(gpu, ora, D, bits, Hkv, 350, seed=9)
    cache2.trim(100)
    oc.trim(100)
    out = cache2.attention(dev_bf16(q), 0.05, dtype=torch.float32)
    torch.cuda.synchronize()
    check_attention(out, oc.attention(q, 0.05), "trimmed")


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(256, 3, 8, 16), (512, 3, 2, 16)])
def test_codebook_paged_batch(gpu, ora, D, bits, Hkv, Hq):
    """Ragged sequences on shuffled 16-token blocks: one batched decode step
    (append + attention), every sequence against its own oracle."""
    import torch

    lens = [5, 40, 100, 17, 1, 64, 300, 700]
    n_seqs = len(lens)
    need = [(n + 1 + 15) // 16 for n in lens]
    max_blocks = max(need)
    n_blocks = sum(need) + 3
    perm = np.argsort(synth.splitmix64(81, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits, mode=CB), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    ocs = []
    for s, n in enumerate(lens):
        k, v = kv_batch(40 + 2 * s, n, Hkv, D), kv_batch(41 + 2 * s, n, Hkv, D)
        pool.append(dev_bf16(k)[None].contiguous(), dev_bf16(v)[None].contiguous(),
                    dtab[s:s + 1].contiguous(), torch.zeros(1, dtype=torch.int32, device="cuda"))
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 1, mode=CB)
        oc.append(k, v)
        ocs.append(oc)
    k1, v1 = fast_kv(90, n_seqs, Hkv, D), fast_kv(91, n_seqs, Hkv, D)
    q = fast_q(92, n_seqs, Hq, Hkv, D)
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = pool.decode_step(dev_bf16(k1)[:, None].contiguous(), dev_bf16(v1)[:, None].contiguous(), dtab,
                           start, start + 1, max(lens) + 1, dev_bf16(q), 0.02, dtype=torch.float32)
    torch.cuda.synchronize()
    for s in range(n_seqs):
        ocs[s].append(k1[s:s + 1], v1[s:s + 1])
        check_attention(out[s], ocs[s].attention(q[s], 0.02), f"paged seq {s} (T={lens[s] + 1})")
