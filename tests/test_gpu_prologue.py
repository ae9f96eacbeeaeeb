"""The layer prologue fused into the append, on the GPU against the oracle.

fmkv_cache_append_projected / fmkv_paged_append_projected take raw k_proj /
v_proj rows and apply the layer's k_norm + RoPE (K) and v_norm (V) before
rotating and quantizing (src/model/gemma4_attention.rs:52-81). The stored
codes and scale/bias must be bit-identical to the oracle's kv_prologue
followed by its quantizer, at small and large positions, with and without
K==V, through ring wraps; attention over the result stays within the path
tolerance."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu

CONFIGS = [  # D, bits, rope_dims, theta
    (512, 8, 128, 1e6),
    (512, 8, 512, 10000.0),
    (256, 4, 256, 10000.0),
    (256, 8, 64, 10000.0),
    (128, 4, 128, 10000.0),
    (128, 8, 4, 500.0),
]


def weight(seed, D):
    rng = np.random.default_rng(seed)
    return synth.f32_to_bf16_bits((1.0 + 0.5 * rng.standard_normal(D)).astype(np.float32))


@pytest.mark.parametrize("D,bits,rope_dims,theta", CONFIGS)
@pytest.mark.parametrize("k_eq_v", [False, True])
def test_projected_append_bit_exact(gpu, ora, D, bits, rope_dims, theta, k_eq_v):
    import torch

    Hkv, eps = 2, 1e-6
    w = weight(D + rope_dims, D)
    wd = dev_bf16(w)
    pro = gpu.make_prologue(wd, eps, rope_dims, theta, v_from_k=k_eq_v)
    cache = gpu.KVCache.new_quantized_with_window(D, bits, 0, Hkv, 200)
    oc = ora.OracleCache(Hkv, D, bits, 0, 200)
    for i, n in enumerate((37, 1, 20, 16)):
        k = kv_batch(3 * i + D, n, Hkv, D)
        v = kv_batch(3 * i + D + 1, n, Hkv, D)
        cache.append_projected(dev_bf16(k), None if k_eq_v else dev_bf16(v), pro)
        oc.append_projected(k, None if k_eq_v else v, w, eps, rope_dims, theta)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    n = oc.offset
    assert np.array_equal(host_u32(codes)[:n], oc.codes[:n])
    assert np.array_equal(host_u16(meta)[:n], oc.meta[:n])
    q = synth.q_rows(D + 5, 16, Hkv, D, None)
    out = cache.attention(dev_bf16(q), 1.0, dtype=torch.float32)
    torch.cuda.synchronize()
    check_attention(out, oc.attention(q, 1.0), "attention over projected rows")


@pytest.mark.parametrize("D,bits", [(256, 4), (256, 8)])
def test_projected_append_ring(gpu, ora, D, bits):
    """Sliding ring W = 64: single-token and chunked appends through wraps.
    The weight tensor is a temporary: the prologue keeps it alive."""
    import torch

    Hkv, W, eps, rope_dims, theta = 8, 64, 1e-6, 256, 10000.0
    w = weight(9, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta)
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, 0)
    oc = ora.OracleCache(Hkv, D, bits, W, 0)
    for i, n in enumerate([40, 1, 1, 90, 1, 7, 64, 1]):
        k = kv_batch(50 + 2 * i, n, Hkv, D)
        v = kv_batch(51 + 2 * i, n, Hkv, D)
        cache.append_projected(dev_bf16(k), dev_bf16(v), pro)
        oc.append_projected(k, v, w, eps, rope_dims, theta)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(codes), oc.codes)
    assert np.array_equal(host_u16(meta), oc.meta)


def test_projected_paged_large_positions(gpu, ora):
    """Paged pool, two sequences starting at positions 100003 and 7: the
    f32 RoPE angle at large positions matches the oracle bit for bit."""
    import torch

    D, bits, Hkv, eps, rope_dims, theta = 512, 8, 2, 1e-6, 128, 1e6
    w = weight(11, D)
    pro = gpu.make_prologue(dev_bf16(w), eps, rope_dims, theta)
    starts, n = [100003, 7], 21
    width = (max(starts) + n) // 16 + 1
    tables = np.full((2, width), -1, np.int32)
    phys = 0
    for s, p0 in enumerate(starts):
        for lb in range(p0 // 16, (p0 + n - 1) // 16 + 1):
            tables[s, lb] = phys
            phys += 1
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), phys)
    dtab = torch.from_numpy(tables).cuda()
    k = np.stack([kv_batch(60 + s, n, Hkv, D) for s in range(2)])
    v = np.stack([kv_batch(70 + s, n, Hkv, D) for s in range(2)])
    pool.append_projected(dev_bf16(k), dev_bf16(v), dtab,
                          torch.tensor(starts, dtype=torch.int32, device="cuda"), pro)
    codes, meta = pool.read_codes()
    torch.cuda.synchronize()
    codes, meta = host_u32(codes), host_u16(meta)
    qz = ora.OracleCache(Hkv, D, bits, 0, 1)
    for s, p0 in enumerate(starts):
        ko, vo = ora.kv_prologue(k[s], v[s], p0, w, eps, rope_dims, theta)
        kp, km = qz.quantize_rows(ko)
        vp, vm = qz.quantize_rows_f32(vo)
        for t in range(n):
            p = p0 + t
            slot = tables[s, p // 16] * 16 + p % 16
            assert np.array_equal(codes[slot, 0], kp[t]) and np.array_equal(meta[slot, 0], km[t])
            assert np.array_equal(codes[slot, 1], vp[t]) and np.array_equal(meta[slot, 1], vm[t])


def test_projected_append_rejects_bad_prologue(gpu):
    import torch

    D = 256
    wd = dev_bf16(weight(1, D))
    cache = gpu.KVCache.new_quantized_with_window(D, 4, 0, 2, 32)
    k = torch.zeros((2, 2, D), dtype=torch.bfloat16, device="cuda")
    bad = [
        (gpu.make_prologue(wd, 1e-6, 96, 1e4), gpu.FMKV_ERR_UNSUPPORTED),   # not a power of 2
        (gpu.make_prologue(wd, 1e-6, 4, 1e4), gpu.FMKV_ERR_UNSUPPORTED),    # < 2 * D / 64
        (gpu.make_prologue(wd, 1e-6, 512, 1e4), gpu.FMKV_ERR_UNSUPPORTED),  # > D
        (gpu.make_prologue(wd, 0.0, 256, 1e4), gpu.FMKV_ERR_INVALID_ARG),
        (gpu.make_prologue(wd, 1e-6, 256, -1.0), gpu.FMKV_ERR_INVALID_ARG),
        (gpu.KvPrologue(None, 1e-6, 256, 1e4, 0), gpu.FMKV_ERR_INVALID_ARG),
    ]
    for pro, code in bad:
        with pytest.raises(gpu.Exception_) as e:
            cache.append_projected(k, k, pro)
        assert e.value.code == code
    with pytest.raises(ValueError):  # weight length != head_dim
        cache.append_projected(k, k, gpu.make_prologue(dev_bf16(weight(1, 128)), 1e-6, 256, 1e4))
    assert cache.offset() == 0
