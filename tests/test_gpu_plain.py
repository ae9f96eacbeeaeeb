"""Plain (unquantized bf16) caches on the GPU against the oracle.

KVCacheInner::Plain (src/cache.rs:174-178, :274-288) stores the K/V rows as
given; make_cache(None) (src/model/mod.rs:390-393, --no-kv-quant) builds one
per layer. Stored rows (read_codes, fetch) must equal the input bits; decode
attention must match the oracle's exact f64 attention over those rows
(max-abs 2e-2, mean-abs 2e-3; bf16 outputs: 2e-2 plus half a bf16 ulp)."""
import numpy as np
import pytest

import synth
from gpu_util import (check_attention, check_codes, dev_bf16, fast_kv, fast_q, host_u16, host_u32,
                      kv_batch)

pytestmark = pytest.mark.gpu
PLAIN = 2  # MODE_PLAIN


def q_batch(seed, Hq, Hkv, D):
    ch = synth.outlier_channels(seed, Hkv, D)
    return synth.q_rows(seed + 100, Hq, Hkv, D, ch)


def filled(gpu, ora, D, Hkv, T, window=0, chunks=None, seed=0):
    cap = 0 if window else sum(chunks or [T]) + 16
    cache = gpu.KVCache.new_with_window(D, window or None, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, 16, window, cap, mode=PLAIN)
    for i, n in enumerate(chunks or [T]):
        k = kv_batch(seed + 2 * i, n, Hkv, D)
        v = kv_batch(seed + 2 * i + 1, n, Hkv, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    return cache, oc


CONFIGS = [  # D, Hkv, Hq
    (512, 2, 16),  # the global layer
    (256, 8, 16),  # the sliding layer
    (128, 4, 4),
    (128, 2, 12),
]


@pytest.mark.parametrize("D,Hkv,Hq", CONFIGS)
def test_plain_rows_stored_as_given(gpu, ora, D, Hkv, Hq):
    """Chunked appends across block boundaries: every stored word equals the
    input bf16 bits (read_codes) and fetch returns the visible rows exactly."""
    import torch

    cache, oc = filled(gpu, ora, D, Hkv, 0, chunks=[5, 1, 30, 16, 17], seed=D)
    codes, meta = cache.read_codes()
    k, v = cache.peek_kv(dtype=torch.bfloat16)
    kf, vf = cache.peek_kv(dtype=torch.float32)
    torch.cuda.synchronize()
    n = oc.offset
    check_codes(codes, meta, oc, np.arange(n), "plain rows")
    want_k, want_v = oc.dequant_kv()
    assert np.array_equal(host_u16(k.view(torch.int16)), oc.codes[:n, 0].view(np.uint16))
    assert np.array_equal(host_u16(v.view(torch.int16)), oc.codes[:n, 1].view(np.uint16))
    assert np.array_equal(kf.cpu().numpy().astype(np.float64), want_k)
    assert np.array_equal(vf.cpu().numpy().astype(np.float64), want_v)


@pytest.mark.parametrize("D,Hkv,Hq", CONFIGS)
@pytest.mark.parametrize("T", [1, 17, 300, 1500])
def test_plain_attention_linear(gpu, ora, D, Hkv, Hq, T):
    import torch

    cache, oc = filled(gpu, ora, D, Hkv, T, chunks=[T // 2, T - T // 2] if T > 1 else [1])
    q = q_batch(T + D, Hq, Hkv, D)
    for scale in (1.0, 0.03):
        ref = oc.attention(q, scale)
        out32 = cache.attention(dev_bf16(q), scale, dtype=torch.float32)
        out16 = cache.attention(dev_bf16(q), scale, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        check_attention(out32, ref, f"f32 T={T} scale={scale}")
        check_attention(out16, ref, f"bf16 T={T} scale={scale}")


@pytest.mark.parametrize("bps", [1, 2, 7, 40])
def test_plain_split_counts_agree(gpu, ora, bps):
    import torch

    D, Hkv, Hq, T = 512, 2, 16, 900
    cache, oc = filled(gpu, ora, D, Hkv, T, seed=5)
    q = q_batch(11, Hq, Hkv, D)
    ref = oc.attention(q, 0.05)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), 0.05, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, ref, f"bps={bps}")


@pytest.mark.parametrize("D,W", [(256, 64), (512, 48), (128, 32)])
def test_plain_ring_steps_through_wraps(gpu, ora, D, W):
    """Sliding ring: single-token decode steps (append, then attention)
    across several wraps; rows and attention against the oracle."""
    import torch

    Hkv, Hq = (8, 16) if D == 256 else (2, 16)
    cache = gpu.KVCache.new_with_window(D, W, Hkv)
    oc = ora.OracleCache(Hkv, D, 16, W, mode=PLAIN)
    n = 3 * W + 5
    k, v = kv_batch(21, n, Hkv, D), kv_batch(22, n, Hkv, D)
    q = fast_q(23, n, Hq, Hkv, D)
    kd, vd = dev_bf16(k), dev_bf16(v)
    for i in range(n):
        out = cache.decode_step(kd[i:i + 1], vd[i:i + 1], dev_bf16(q[i]), 0.02, dtype=torch.float32)
        oc.append(k[i:i + 1], v[i:i + 1])
        if i % 7 == 0 or i in (W - 1, W, 2 * W, n - 1):
            codes, meta = cache.read_codes()
            torch.cuda.synchronize()
            check_codes(codes, meta, oc, None, f"ring W={W} step {i}")
            check_attention(out, oc.attention(q[i], 0.02), f"ring W={W} step {i}")
    assert cache.stored_len() == W


def test_plain_ring_chunk_overwrites_partial_blocks(gpu, ora):
    """Chunks that start and end inside blocks of a ring keep the other
    tokens of those blocks (V is dim-major: a block's dim row holds all 16
    tokens)."""
    import torch

    D, Hkv, W = 256, 2, 64
    cache = gpu.KVCache.new_with_window(D, W, Hkv)
    oc = ora.OracleCache(Hkv, D, 16, W, mode=PLAIN)
    for i, n in enumerate([40, 1, 1, 90, 3, 7, 64, 13]):
        k, v = kv_batch(50 + 2 * i, n, Hkv, D), kv_batch(51 + 2 * i, n, Hkv, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
        codes, meta = cache.read_codes()
        torch.cuda.synchronize()
        check_codes(codes, meta, oc, None, f"chunk {i} (n={n})")


def test_plain_trim_and_empty(gpu, ora):
    import torch

    D, Hkv, Hq = 256, 2, 8
    cache = gpu.KVCache.new(D, Hkv, capacity=400)
    q = q_batch(31, Hq, Hkv, D)
    out = cache.attention(dev_bf16(q), 1.0, dtype=torch.float32)  # empty cache
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
    cache2, oc = filled(gpu, ora, D, Hkv, 350, seed=9)
    cache2.trim(100)
    oc.trim(100)
    out = cache2.attention(dev_bf16(q), 0.05, dtype=torch.float32)
    k, _ = cache2.peek_kv()
    torch.cuda.synchronize()
    check_attention(out, oc.attention(q, 0.05), "trimmed")
    assert k.shape[0] == 100


@pytest.mark.parametrize("D,Hkv,Hq", [(256, 8, 16), (512, 2, 16)])
def test_plain_paged_batch(gpu, ora, D, Hkv, Hq):
    """Ragged sequences on shuffled 16-token blocks: one batched decode step
    (append + attention), every sequence against its own oracle."""
    import torch

    lens = [5, 40, 100, 17, 1, 64, 300, 700]
    n_seqs = len(lens)
    need = [(n + 1 + 15) // 16 for n in lens]
    max_blocks = max(need)
    n_blocks = sum(need) + 3
    perm = np.argsort(synth.splitmix64(83, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, 16, mode=PLAIN), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    ocs = []
    for s, n in enumerate(lens):
        k, v = kv_batch(240 + 2 * s, n, Hkv, D), kv_batch(241 + 2 * s, n, Hkv, D)
        pool.append(dev_bf16(k)[None].contiguous(), dev_bf16(v)[None].contiguous(),
                    dtab[s:s + 1].contiguous(), torch.zeros(1, dtype=torch.int32, device="cuda"))
        oc = ora.OracleCache(Hkv, D, 16, 0, n + 1, mode=PLAIN)
        oc.append(k, v)
        ocs.append(oc)
    k1, v1 = fast_kv(290, n_seqs, Hkv, D), fast_kv(291, n_seqs, Hkv, D)
    q = fast_q(292, n_seqs, Hq, Hkv, D)
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = pool.decode_step(dev_bf16(k1)[:, None].contiguous(), dev_bf16(v1)[:, None].contiguous(), dtab,
                           start, start + 1, max(lens) + 1, dev_bf16(q), 0.02, dtype=torch.float32)
    codes, _ = pool.read_codes()
    torch.cuda.synchronize()
    codes = host_u32(codes)
    for s in range(n_seqs):
        ocs[s].append(k1[s:s + 1], v1[s:s + 1])
        for p in range(lens[s] + 1):
            slot = tables[s, p // 16] * 16 + p % 16
            assert np.array_equal(codes[slot], ocs[s].codes[p]), f"seq {s} position {p}"
        check_attention(out[s], ocs[s].attention(q[s], 0.02), f"paged seq {s} (T={lens[s] + 1})")


def test_plain_make_cache_stack(gpu, ora):
    """make_cache(kv_quant_bits=None): plain caches on every layer, windowed
    on the sliding layers (src/model/mod.rs:375-396); a decode step on each
    layer kind against the oracle."""
    import torch

    types = ["sliding_attention"] * 5 + ["full_attention"]
    caches = gpu.make_cache(types, 256, 8, capacity=256, global_head_dim=512, n_global_kv_heads=2,
                            sliding_window=64, attention_k_eq_v=True, kv_quant_bits=None)
    assert [c.desc.mode for c in caches] == [PLAIN] * 6
    assert [c.desc.window for c in caches] == [64] * 5 + [0]
    for li in (0, 5):
        c = caches[li]
        D, H = c.desc.head_dim, c.desc.n_kv_heads
        oc = ora.OracleCache(H, D, 16, c.desc.window, 256, mode=PLAIN)
        k, v = kv_batch(300 + li, 100, H, D), kv_batch(301 + li, 100, H, D)
        c.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
        k1, v1 = kv_batch(302 + li, 1, H, D), kv_batch(303 + li, 1, H, D)
        q = fast_q(304 + li, 1, 16, H, D)[0]
        out = c.decode_step(dev_bf16(k1), dev_bf16(v1), dev_bf16(q), 1.0, dtype=torch.float32)
        torch.cuda.synchronize()
        oc.append(k1, v1)
        check_attention(out, oc.attention(q, 1.0), f"layer {li}")


@pytest.mark.parametrize("bps", [0, 3, 40])
def test_plain_linear_decode_steps(gpu, ora, bps):
    """Linear cache, single-token decode steps after a 3000-token prefill
    under the default plan and forced split sizes: the step's attention
    launch stores the token in its new-token column and attends it there
    (the split columns leave its slot out); rows and attention against the
    oracle."""
    import torch

    D, Hkv, Hq, T0, n = 512, 2, 16, 3000, 6
    cache = gpu.KVCache.new(D, Hkv, capacity=T0 + 16)
    oc = ora.OracleCache(Hkv, D, 16, 0, T0 + 16, mode=PLAIN)
    k0, v0 = kv_batch(41, T0, Hkv, D), kv_batch(42, T0, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    k, v = kv_batch(43, n, Hkv, D), kv_batch(44, n, Hkv, D)
    q = fast_q(45, n, Hq, Hkv, D)
    kd, vd = dev_bf16(k), dev_bf16(v)
    gpu.set_blocks_per_split(bps)
    try:
        for i in range(n):
            scale = 1.0 if i % 2 == 0 else 0.02
            out = cache.decode_step(kd[i:i + 1], vd[i:i + 1], dev_bf16(q[i]), scale,
                                    dtype=torch.float32)
            oc.append(k[i:i + 1], v[i:i + 1])
            torch.cuda.synchronize()
            check_attention(out, oc.attention(q[i], scale), f"bps={bps} step {i}")
    finally:
        gpu.set_blocks_per_split(0)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    check_codes(codes, meta, oc, None, f"bps={bps} rows")
