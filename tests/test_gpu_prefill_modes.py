"""Prefill (chunked) attention over codebook (TurboQuant) and plain caches on
the GPU against the oracle.

The reference's default cache is 3-bit TurboQuant (src/main.rs:84) and
--no-kv-quant gives plain bf16 (src/main.rs:87, :149); its prefill runs the
fused SDPA with the causal or sliding mask over whatever update_and_fetch
returns (src/model/gemma4_attention.rs:84-104, masks src/model/mod.rs
:682-753). fmkv_prefill_step and fmkv_paged_prefill_step do the same over
the stored indices (centroid * norm / sqrt(D) in the rotated domain) or
the stored bf16 rows. Outputs within the path tolerance (max-abs 2e-2,
mean-abs 2e-3; bf16 outputs compared in bf16) of the oracle's exact
attention; stored indices, norms and rows bit-exact."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, check_codes, dev_bf16, fast_kv, fast_q, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu

CB, PLAIN = 1, 2

CONFIGS = [  # mode, D, bits, Hkv, Hq, W
    (CB, 512, 3, 2, 16, 0),
    (CB, 256, 2, 8, 16, 64),
    (CB, 256, 3, 2, 4, 0),
    (CB, 128, 4, 4, 4, 32),
    (PLAIN, 512, 16, 2, 16, 0),
    (PLAIN, 256, 16, 8, 16, 64),
    (PLAIN, 128, 16, 1, 8, 48),
]


def q_chunk(seed, L, Hq, Hkv, D):
    return synth.q_rows(seed, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D), batch=L)


def make(gpu, ora, mode, D, bits, Hkv, W, cap):
    return (gpu.KVCache(gpu.make_desc(Hkv, D, bits, W, cap, mode)),
            ora.OracleCache(Hkv, D, bits, W, cap, mode=mode))


def codes_equal(cache, oc):
    import torch

    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    n = oc.codes.shape[0] if oc.W else oc.offset
    assert np.array_equal(host_u32(codes)[:n], oc.codes[:n])
    assert np.array_equal(host_u16(meta)[:n], oc.meta[:n])


@pytest.mark.parametrize("mode,D,bits,Hkv,Hq,W", CONFIGS)
def test_prefill_modes_chunks_match_oracle(gpu, ora, mode, D, bits, Hkv, Hq, W):
    """Chunks of 1, 19, 70 and 16 tokens after a 37-token prefix: unaligned
    chunk starts, a ring's band across wraps (70 > W), f32 and bf16 outputs,
    Gemma-4's scale 1.0 and a soft scale."""
    import torch

    cap = 0 if W else 400
    cache, oc = make(gpu, ora, mode, D, bits, Hkv, W, cap)
    k0, v0 = kv_batch(1, 37, Hkv, D), kv_batch(2, 37, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    for step, L in enumerate((1, 19, 70, 16)):
        k, v = kv_batch(10 + step, L, Hkv, D), kv_batch(20 + step, L, Hkv, D)
        q = q_chunk(30 + step, L, Hq, Hkv, D)
        dtype = torch.float32 if step % 2 else torch.bfloat16
        scale = 1.0 if step < 2 else 0.02
        out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), scale, dtype=dtype)
        want = oc.prefill(k, v, q, scale)
        torch.cuda.synchronize()
        check_attention(out, want, f"mode {mode} prefill step {step} (L={L}, scale {scale})")
    assert cache.offset() == oc.offset
    codes_equal(cache, oc)


@pytest.mark.parametrize("mode,D,bits,Hkv,Hq", [(CB, 512, 3, 2, 16), (CB, 256, 4, 8, 16),
                                                (PLAIN, 512, 16, 2, 16), (PLAIN, 256, 16, 8, 16)])
def test_prefill_modes_long_context(gpu, ora, mode, D, bits, Hkv, Hq):
    """A 96-token chunk over a 1500-token linear cache, then a trim and a
    33-token chunk (the hidden positions stay hidden)."""
    import torch

    cache, oc = make(gpu, ora, mode, D, bits, Hkv, 0, 1700)
    k0, v0 = kv_batch(3, 1500, Hkv, D), kv_batch(4, 1500, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    k, v = kv_batch(5, 96, Hkv, D), kv_batch(6, 96, Hkv, D)
    q = q_chunk(7, 96, Hq, Hkv, D)
    out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 0.05, dtype=torch.float32)
    want = oc.prefill(k, v, q, 0.05)
    torch.cuda.synchronize()
    check_attention(out, want, f"mode {mode} long-context prefill")
    cache.trim(200)
    oc.trim(200)
    k, v = kv_batch(8, 33, Hkv, D), kv_batch(9, 33, Hkv, D)
    q = q_chunk(10, 33, Hq, Hkv, D)
    out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0, dtype=torch.bfloat16)
    want = oc.prefill(k, v, q, 1.0)
    torch.cuda.synchronize()
    check_attention(out, want, f"mode {mode} prefill after trim")
    codes_equal(cache, oc)


@pytest.mark.parametrize("mode,bits", [(CB, 3), (PLAIN, 16)])
def test_paged_prefill_modes_ragged_starts(gpu, ora, mode, bits):
    """fmkv_paged_prefill_step: four sequences with prefixes of 0, 21, 64 and
    150 tokens on shuffled blocks take a 40-token chunk each in one call."""
    import torch

    D, Hkv, Hq = 256, 8, 16
    starts, n_new = [0, 21, 64, 150], 40
    n_seqs = len(starts)
    need = [(p0 + n_new + 15) // 16 for p0 in starts]
    n_blocks = sum(need) + 5
    perm = np.argsort(synth.splitmix64(91 + mode, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max(need)), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits, mode=mode), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, p0 in enumerate(starts):
        oc = ora.OracleCache(Hkv, D, bits, 0, p0 + n_new, mode=mode)
        if p0:
            k0, v0 = kv_batch(200 + s, p0, Hkv, D), kv_batch(300 + s, p0, Hkv, D)
            oc.append(k0, v0)
            pool.append(dev_bf16(k0[None]), dev_bf16(v0[None]), dtab[s:s + 1].contiguous(),
                        torch.zeros(1, dtype=torch.int32, device="cuda"))
        oracles.append(oc)
    k = np.stack([kv_batch(400 + s, n_new, Hkv, D) for s in range(n_seqs)])
    v = np.stack([kv_batch(500 + s, n_new, Hkv, D) for s in range(n_seqs)])
    q = np.stack([q_chunk(600 + s, n_new, Hq, Hkv, D) for s in range(n_seqs)])
    out = pool.prefill_step(dev_bf16(k), dev_bf16(v), dtab,
                            torch.tensor(starts, dtype=torch.int32, device="cuda"), dev_bf16(q),
                            1.0, dtype=torch.float32)
    codes, meta = pool.read_codes()
    torch.cuda.synchronize()
    c, m = host_u32(codes), host_u16(meta)
    for s, p0 in enumerate(starts):
        check_attention(out[s], oracles[s].prefill(k[s], v[s], q[s], 1.0), f"seq {s}")
        p = np.arange(p0 + n_new)
        slots = tables[s, p // 16].astype(np.int64) * 16 + p % 16
        assert np.array_equal(c[slots], oracles[s].codes[p]), f"seq {s} codes"
        assert np.array_equal(m[slots], oracles[s].meta[p]), f"seq {s} norms"


@pytest.mark.parametrize("mode,bits", [(CB, 3), (PLAIN, 16)])
def test_prefill_modes_2048_chunk_after_32k(gpu, ora, mode, bits):
    """The benchmarked prefill shape on the reference's default cache kinds: a
    2048-token chunk after a 32768-token global prefill (Hq 16, Hkv 2,
    head_dim 512); sampled rows of the chunk (its first and last among them)
    against the oracle, the chunk's stored rows bit-exact."""
    import torch

    Hq, Hkv, D, T0, L = 16, 2, 512, 32768, 2048
    cap = T0 + L
    cache, oc = make(gpu, ora, mode, D, bits, Hkv, 0, cap)
    for c0 in range(0, T0, L):
        k = fast_kv(510 + c0, L, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(100510 + c0, L, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    k = fast_kv(595, L, Hkv, D, dist="t3", outliers=False)
    v = fast_kv(596, L, Hkv, D, outliers=False)
    q = fast_q(597, L, Hq, Hkv, D, outliers=False)
    out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 0.05, dtype=torch.float32)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    rows = sorted({0, 1, 2, 17, L // 2 - 1, L // 2, L - 2, L - 1})
    ref = oc.prefill(k, v, q, 0.05, rows=rows)
    check_codes(codes, meta, oc, slots=np.arange(T0 - 16, T0 + L), what=f"mode {mode} chunk rows")
    check_attention(out[rows], ref, f"mode {mode} 2048-token chunk after 32K")
