"""Prefill (chunked) attention on the GPU against the oracle.

fmkv_prefill_step appends an L-token chunk and attends its L queries with
the causal mask of global layers or the sliding band of rings, as
Gemma4Attention::forward does for L > 1 (src/model/gemma4_attention.rs
:84-104, masks src/model/mod.rs:682-753). Outputs must lie within the path
tolerance (max-abs 2e-2, mean-abs 2e-3; bf16 outputs compared in bf16) of
the oracle's exact attention, and the stored codes must be bit-exact."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu

CONFIGS = [  # D, bits, Hkv, Hq, W
    (512, 8, 2, 16, 0),
    (512, 4, 2, 8, 0),
    (256, 4, 8, 16, 64),
    (256, 8, 2, 4, 0),
    (128, 4, 4, 4, 32),
    (128, 8, 1, 8, 48),
]


def q_chunk(seed, L, Hq, Hkv, D):
    return synth.q_rows(seed, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D), batch=L)


def check_codes(cache, oc):
    import torch

    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    n = oc.codes.shape[0] if oc.W else oc.offset
    assert np.array_equal(host_u32(codes)[:n], oc.codes[:n])
    assert np.array_equal(host_u16(meta)[:n], oc.meta[:n])


@pytest.mark.parametrize("D,bits,Hkv,Hq,W", CONFIGS)
def test_prefill_chunks_match_oracle(gpu, ora, D, bits, Hkv, Hq, W):
    """Chunks of 1, 19, 70 and 16 tokens after a 37-token prefix: unaligned
    chunk starts, a ring's band across wraps (70 > W), f32 and bf16 outputs."""
    import torch

    cap = 0 if W else 400
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, W, cap)
    k0, v0 = kv_batch(1, 37, Hkv, D), kv_batch(2, 37, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    for step, L in enumerate((1, 19, 70, 16)):
        k, v = kv_batch(10 + step, L, Hkv, D), kv_batch(20 + step, L, Hkv, D)
        q = q_chunk(30 + step, L, Hq, Hkv, D)
        dtype = torch.float32 if step % 2 else torch.bfloat16
        out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0, dtype=dtype)
        want = oc.prefill(k, v, q, 1.0)
        torch.cuda.synchronize()
        check_attention(out, want, f"prefill step {step} (L={L})")
    assert cache.offset() == oc.offset
    check_codes(cache, oc)


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(512, 8, 2, 16), (256, 4, 8, 16)])
def test_prefill_long_context(gpu, ora, D, bits, Hkv, Hq):
    """A 96-token chunk over a 1500-token linear cache: most blocks take the
    unmasked path, the last ones the causal edge."""
    import torch

    cache = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, 1700)
    oc = ora.OracleCache(Hkv, D, bits, 0, 1700)
    k0, v0 = kv_batch(3, 1500, Hkv, D), kv_batch(4, 1500, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    k, v = kv_batch(5, 96, Hkv, D), kv_batch(6, 96, Hkv, D)
    q = q_chunk(7, 96, Hq, Hkv, D)
    out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0, dtype=torch.float32)
    want = oc.prefill(k, v, q, 1.0)
    torch.cuda.synchronize()
    check_attention(out, want, "long-context prefill")
    check_codes(cache, oc)


def test_prefill_after_trim_and_from_empty(gpu, ora):
    """A first chunk into an empty cache (every query sees only the chunk),
    then a chunk after trim(keep_last) (the hidden positions stay hidden)."""
    import torch

    D, bits, Hkv, Hq = 256, 8, 2, 8
    cache = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, 300)
    oc = ora.OracleCache(Hkv, D, bits, 0, 300)
    for step, L in enumerate((50, 33)):
        if step == 1:
            cache.trim(20)
            oc.trim(20)
        k, v = kv_batch(60 + step, L, Hkv, D), kv_batch(70 + step, L, Hkv, D)
        q = q_chunk(80 + step, L, Hq, Hkv, D)
        out = cache.prefill_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 1.0, dtype=torch.float32)
        want = oc.prefill(k, v, q, 1.0)
        torch.cuda.synchronize()
        check_attention(out, want, f"prefill step {step}")
    check_codes(cache, oc)


def test_prefill_rejects_bad_arguments(gpu):
    import torch

    D = 256
    cache = gpu.KVCache.new_quantized_with_window(D, 4, 0, 2, 64)
    k = torch.zeros((4, 2, D), dtype=torch.bfloat16, device="cuda")
    q = torch.zeros((4, 6, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((4, 6, D), dtype=torch.float32, device="cuda")
    lib = gpu.load_library()
    for args, code in [
        ((4, q.data_ptr(), 5), gpu.FMKV_ERR_INVALID_ARG),    # 5 q heads over 2 KV heads
        ((4, q.data_ptr(), 18), gpu.FMKV_ERR_UNSUPPORTED),   # 9 q heads per KV head
        ((0, q.data_ptr(), 6), gpu.FMKV_ERR_INVALID_ARG),    # empty chunk
        ((4, None, 6), gpu.FMKV_ERR_INVALID_ARG),            # no q
    ]:
        n, qp, hq = args
        rc = lib.fmkv_prefill_step(cache._h, k.data_ptr(), k.data_ptr(), n, qp, hq, 1.0,
                                   out.data_ptr(), gpu.DTYPE_F32, None)
        assert rc == code
    assert cache.offset() == 0


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(512, 8, 2, 16), (256, 4, 8, 16)])
def test_paged_prefill_ragged_starts(gpu, ora, D, bits, Hkv, Hq):
    """fmkv_paged_prefill_step: four sequences with prefixes of 0, 21, 64 and
    150 tokens on shuffled blocks take a 40-token chunk each in one call;
    every sequence's outputs match its own oracle, its codes sit at the
    block-table addresses."""
    import torch

    starts, n_new = [0, 21, 64, 150], 40
    n_seqs = len(starts)
    need = [(p0 + n_new + 15) // 16 for p0 in starts]
    n_blocks = sum(need) + 5
    perm = np.argsort(synth.splitmix64(91, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max(need)), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, p0 in enumerate(starts):
        oc = ora.OracleCache(Hkv, D, bits, 0, p0 + n_new)
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
        assert np.array_equal(m[slots], oracles[s].meta[p]), f"seq {s} scales"
