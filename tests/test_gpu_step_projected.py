"""The decode step from raw projections (fmkv_decode_step_projected,
fmkv_paged_decode_step_projected) on the GPU against the oracle.

One token per step with sparse_v_tau == 0 runs the layer's prologue
(k_norm + RoPE on K, v_norm on V; src/model/gemma4_attention.rs:52-81),
the quantization and the slot write inside the attention launch's
new-token column; other steps run the projected append, then attention.
Either way the stored codes and scale/bias must equal the oracle's
OracleCache.append_projected bit for bit, and the step's attention output
the oracle's exact attention over the stored codes (max-abs 2e-2, mean-abs
2e-3; bf16 outputs: 2e-2 plus half a bf16 ulp)."""
import numpy as np
import pytest

import synth
from gpu_util import (check_attention, check_codes, dev_bf16, fast_kv, fast_q, host_u16, host_u32,
                      kv_batch)

pytestmark = pytest.mark.gpu

CONFIGS = [  # D, bits, Hkv, Hq, rope_dims, theta
    (512, 8, 2, 16, 128, 1e6),    # the global layer (partial rotary 0.25)
    (512, 4, 2, 16, 512, 1e6),
    (256, 4, 8, 16, 256, 10000.0),  # the sliding layer
    (256, 8, 8, 16, 64, 10000.0),
    (128, 8, 4, 8, 4, 500.0),
    (128, 4, 2, 12, 128, 10000.0),
]


def weight(seed, D):
    rng = np.random.default_rng(seed)
    return synth.f32_to_bf16_bits((1.0 + 0.5 * rng.standard_normal(D)).astype(np.float32))


@pytest.mark.parametrize("D,bits,Hkv,Hq,rope_dims,theta", CONFIGS)
@pytest.mark.parametrize("k_eq_v", [False, True])
def test_projected_step_linear(gpu, ora, D, bits, Hkv, Hq, rope_dims, theta, k_eq_v):
    """A projected prefill of 300 tokens, then single-token fused steps and
    one 3-token step; codes after every step, attention at scales 1.0 and
    0.03 in f32 and bf16."""
    import torch

    eps = 1e-6
    w = weight(D + rope_dims + bits, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta, v_from_k=k_eq_v)
    cap = 340
    cache = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap)
    k = kv_batch(D + 1, 300, Hkv, D)
    v = kv_batch(D + 2, 300, Hkv, D)
    cache.append_projected(dev_bf16(k), None if k_eq_v else dev_bf16(v), pro)
    oc.append_projected(k, None if k_eq_v else v, w, eps, rope_dims, theta)
    for step, n in enumerate((1, 1, 3, 1, 1)):
        kn, vn = kv_batch(900 + 2 * step, n, Hkv, D), kv_batch(901 + 2 * step, n, Hkv, D)
        q = fast_q(950 + step, 1, Hq, Hkv, D)[0]
        scale = 1.0 if step % 2 == 0 else 0.03
        dt = torch.float32 if step < 3 else torch.bfloat16
        out = cache.decode_step_projected(dev_bf16(kn), None if k_eq_v else dev_bf16(vn), pro,
                                          dev_bf16(q), scale, dtype=dt)
        oc.append_projected(kn, None if k_eq_v else vn, w, eps, rope_dims, theta)
        codes, meta = cache.read_codes()
        torch.cuda.synchronize()
        assert cache.offset() == oc.offset
        check_codes(codes, meta, oc, np.arange(oc.offset), f"step {step} (n={n})")
        check_attention(out, oc.attention(q, scale), f"step {step} (n={n}) scale={scale}")


def test_projected_step_fused_equals_unfused(gpu, ora):
    """The fused column (tau 0) and the append-then-attend path (tau > 0
    forces it) store identical codes for the same projected rows."""
    import torch

    D, bits, Hkv, Hq, eps, rope_dims, theta = 512, 8, 2, 16, 1e-6, 128, 1e6
    w = dev_bf16(weight(3, D))
    pro = gpu.make_prologue(w, eps, rope_dims, theta, v_from_k=True)
    a = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, 64)
    b = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, 64)
    k = dev_bf16(kv_batch(5, 40, Hkv, D))
    q = dev_bf16(fast_q(6, 1, Hq, Hkv, D)[0])
    for c in (a, b):
        c.append_projected(k[:20], None, pro)
    for t in range(20, 40):
        a.decode_step_projected(k[t:t + 1], None, pro, q, 1.0)
        b.decode_step_projected(k[t:t + 1], None, pro, q, 1.0, sparse_v_tau=1e-9)
    ca, ma = a.read_codes()
    cb, mb = b.read_codes()
    torch.cuda.synchronize()
    assert torch.equal(ca, cb) and torch.equal(ma, mb)


@pytest.mark.parametrize("D,bits,W", [(256, 4, 64), (256, 8, 32), (512, 8, 48)])
def test_projected_step_ring_wraps(gpu, ora, D, bits, W):
    """Sliding ring: fused single-token projected steps across several wraps."""
    import torch

    Hkv, Hq = (8, 16) if D == 256 else (2, 16)
    eps, rope_dims, theta = 1e-6, D, 10000.0
    w = weight(17 + D, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta)
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, 0)
    oc = ora.OracleCache(Hkv, D, bits, W, 0)
    n = 3 * W + 5
    k, v = kv_batch(71, n, Hkv, D), kv_batch(72, n, Hkv, D)
    q = fast_q(73, n, Hq, Hkv, D)
    kd, vd = dev_bf16(k), dev_bf16(v)
    for i in range(n):
        out = cache.decode_step_projected(kd[i:i + 1], vd[i:i + 1], pro, dev_bf16(q[i]), 0.05,
                                          dtype=torch.float32)
        oc.append_projected(k[i:i + 1], v[i:i + 1], w, eps, rope_dims, theta)
        if i % 9 == 0 or i in (W - 1, W, 2 * W, n - 1):
            codes, meta = cache.read_codes()
            torch.cuda.synchronize()
            check_codes(codes, meta, oc, None, f"ring W={W} step {i}")
            check_attention(out, oc.attention(q[i], 0.05), f"ring W={W} step {i}")
    assert cache.stored_len() == W


def test_projected_step_large_positions(gpu, ora):
    """A ring at positions past 100000: the new token's f32 RoPE angle
    (position * inverse frequency) in the fused column matches the oracle
    bit for bit. The device ring is filled up to the window's start with
    plain appends; the oracle, whose slots the same 64 projected rows then
    overwrite, starts at that position."""
    import torch

    D, bits, Hkv, Hq, W = 256, 8, 8, 16, 64
    eps, rope_dims, theta = 1e-6, 256, 1e6
    w = weight(23, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta)
    p0 = 100003 - W
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, 0)
    filler = torch.zeros((4096, Hkv, D), dtype=torch.bfloat16, device="cuda")
    left = p0
    while left > 0:
        n = min(left, 4096)
        cache.append(filler[:n], filler[:n])
        left -= n
    oc = ora.OracleCache(Hkv, D, bits, W, 0)
    oc.offset = p0
    k, v = kv_batch(81, W, Hkv, D), kv_batch(82, W, Hkv, D)
    cache.append_projected(dev_bf16(k), dev_bf16(v), pro)
    oc.append_projected(k, v, w, eps, rope_dims, theta)
    for i in range(6):
        kn, vn = kv_batch(83 + 2 * i, 1, Hkv, D), kv_batch(84 + 2 * i, 1, Hkv, D)
        q = fast_q(95 + i, 1, Hq, Hkv, D)[0]
        out = cache.decode_step_projected(dev_bf16(kn), dev_bf16(vn), pro, dev_bf16(q), 0.05,
                                          dtype=torch.float32)
        oc.append_projected(kn, vn, w, eps, rope_dims, theta)
        codes, meta = cache.read_codes()
        torch.cuda.synchronize()
        assert cache.offset() == oc.offset
        check_codes(codes, meta, oc, None, f"position {oc.offset - 1}")
        check_attention(out, oc.attention(q, 0.05), f"position {oc.offset - 1}")


@pytest.mark.parametrize("k_eq_v", [False, True])
def test_projected_step_paged(gpu, ora, k_eq_v):
    """Ragged sequences on shuffled 16-token blocks: projected prefill, then
    one batched fused projected step; every sequence against its own oracle."""
    import torch

    D, bits, Hkv, Hq, eps, rope_dims, theta = 512, 8, 2, 16, 1e-6, 128, 1e6
    lens = [5, 40, 100, 17, 1, 64, 300, 0]
    n_seqs = len(lens)
    need = [(n + 1 + 15) // 16 for n in lens]
    max_blocks = max(need)
    n_blocks = sum(need) + 3
    perm = np.argsort(synth.splitmix64(181, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    w = weight(29, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta, v_from_k=k_eq_v)
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    ocs = []
    for s, n in enumerate(lens):
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 1)
        if n:
            k, v = kv_batch(140 + 2 * s, n, Hkv, D), kv_batch(141 + 2 * s, n, Hkv, D)
            pool.append_projected(dev_bf16(k)[None].contiguous(),
                                  None if k_eq_v else dev_bf16(v)[None].contiguous(),
                                  dtab[s:s + 1].contiguous(),
                                  torch.zeros(1, dtype=torch.int32, device="cuda"), pro)
            oc.append_projected(k, None if k_eq_v else v, w, eps, rope_dims, theta)
        ocs.append(oc)
    k1, v1 = fast_kv(190, n_seqs, Hkv, D), fast_kv(191, n_seqs, Hkv, D)
    q = fast_q(192, n_seqs, Hq, Hkv, D)
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = pool.decode_step_projected(dev_bf16(k1)[:, None].contiguous(),
                                     None if k_eq_v else dev_bf16(v1)[:, None].contiguous(),
                                     dtab, start, start + 1, max(lens) + 1, pro, dev_bf16(q), 0.05,
                                     dtype=torch.float32)
    codes, meta = pool.read_codes()
    torch.cuda.synchronize()
    codes, meta = host_u32(codes), host_u16(meta)
    for s in range(n_seqs):
        ocs[s].append_projected(k1[s:s + 1], None if k_eq_v else v1[s:s + 1], w, eps, rope_dims,
                                theta)
        for p in range(lens[s] + 1):
            slot = tables[s, p // 16] * 16 + p % 16
            assert np.array_equal(codes[slot], ocs[s].codes[p]), f"seq {s} position {p} codes"
            assert np.array_equal(meta[slot], ocs[s].meta[p]), f"seq {s} position {p} meta"
        check_attention(out[s], ocs[s].attention(q[s], 0.05), f"paged seq {s} (T={lens[s] + 1})")


def test_projected_step_rejections(gpu):
    """Null prologue and bad prologue fields fail before anything is
    launched or changed."""
    import torch

    D = 256
    wd = dev_bf16(weight(1, D))
    cache = gpu.KVCache.new_quantized_with_window(D, 4, 0, 2, 32)
    k = torch.zeros((1, 2, D), dtype=torch.bfloat16, device="cuda")
    q = torch.zeros((4, D), dtype=torch.bfloat16, device="cuda")
    lib = gpu.load_library()
    out = torch.empty((4, D), dtype=torch.bfloat16, device="cuda")
    rc = lib.fmkv_decode_step_projected(cache._h, k.data_ptr(), k.data_ptr(), 1, None,
                                        q.data_ptr(), 4, 1.0, 0.0, out.data_ptr(), gpu.DTYPE_BF16,
                                        None)
    assert rc == gpu.FMKV_ERR_INVALID_ARG
    with pytest.raises(gpu.Exception_) as e:
        cache.decode_step_projected(k, k, gpu.make_prologue(wd, 1e-6, 96, 1e4), q)
    assert e.value.code == gpu.FMKV_ERR_UNSUPPORTED
    with pytest.raises(gpu.Exception_) as e:
        cache.decode_step_projected(k, k, gpu.make_prologue(wd, 0.0, 256, 1e4), q)
    assert e.value.code == gpu.FMKV_ERR_INVALID_ARG
    assert cache.offset() == 0
