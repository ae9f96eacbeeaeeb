"""Append path on the GPU: stored codes, f16 scale/bias (or norms) and ring
slots are bit-exact against the oracle; fetch (peek_kv) matches the oracle's
dequantized, un-rotated rows."""
import numpy as np
import pytest

from gpu_util import dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu


def run_appends(gpu, ora, D, bits, window, capacity, chunks, mode=0, H=2, seed=0):
    import torch

    cache = gpu.KVCache.new_quantized_with_window(D, bits, window, H, capacity, mode=mode)
    oc = ora.OracleCache(H, D, bits, window, capacity, mode=mode)
    for i, n in enumerate(chunks):
        k = kv_batch(seed + 2 * i, n, H, D)
        v = kv_batch(seed + 2 * i + 1, n, H, D)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    torch.cuda.synchronize()
    return cache, oc


def assert_codes_equal(cache, oc):
    codes, meta = cache.read_codes()
    c, m = host_u32(codes), host_u16(meta)
    bad = np.argwhere((c != oc.codes).any(-1))
    assert bad.size == 0, f"code mismatch at (slot, kv, head) {bad[:5].tolist()} of {len(bad)}"
    badm = np.argwhere((m != oc.meta).any(-1))
    assert badm.size == 0, f"scale/bias mismatch at {badm[:5].tolist()}"


@pytest.mark.parametrize("D,bits", [(128, 4), (128, 8), (256, 4), (256, 8), (512, 4), (512, 8)])
def test_append_linear_bit_exact(gpu, ora, D, bits):
    cache, oc = run_appends(gpu, ora, D, bits, 0, 200, [1, 5, 16, 37, 3, 60, 1])
    assert cache.offset() == oc.offset == 123
    assert cache.stored_len() == 123
    assert_codes_equal(cache, oc)


@pytest.mark.parametrize("D,bits", [(256, 4), (512, 8), (256, 8)])
def test_append_ring_bit_exact(gpu, ora, D, bits):
    # W = 64: chunks cross block edges, wrap, and one chunk exceeds the window
    cache, oc = run_appends(gpu, ora, D, bits, 64, 0, [1, 7, 30, 50, 100, 1, 1, 64, 17], seed=5)
    assert cache.offset() == oc.offset
    assert cache.stored_len() == 64
    assert_codes_equal(cache, oc)


def test_append_ring_single_tokens_through_wraps(gpu, ora):
    cache, oc = run_appends(gpu, ora, 256, 4, 32, 0, [1] * 75, H=8, seed=11)
    assert_codes_equal(cache, oc)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("D", [256, 512])
def test_append_codebook_bit_exact_and_round_trip(gpu, ora, D, bits):
    import torch

    cache, oc = run_appends(gpu, ora, D, bits, 0, 100, [3, 40, 1, 20], mode=1, seed=3)
    assert_codes_equal(cache, oc)
    # fetch = the reference's round trip output (src/cache.rs:119-125), bf16, bit-exact
    k, v = cache.peek_kv(dtype=torch.bfloat16)
    pos = oc.visible_positions()
    for kv, got in ((0, k), (1, v)):
        want = ora.codebook_round_trip(oc.codes[pos, kv], np.ascontiguousarray(oc.meta[pos, kv, :, 0]),
                                       D, bits, oc.sgn)
        assert np.array_equal(host_u16(got.view(torch.int16)), want)


@pytest.mark.parametrize("D,bits,window", [(256, 4, 0), (512, 8, 0), (256, 4, 48)])
def test_fetch_matches_oracle_dequant(gpu, ora, D, bits, window):
    import torch

    cache, oc = run_appends(gpu, ora, D, bits, window, 0 if window else 150, [20, 33, 1, 40], seed=7)
    k, v = cache.peek_kv(dtype=torch.float32)
    wk, wv = oc.dequant_kv()
    assert k.shape == wk.shape
    for got, want in ((k, wk), (v, wv)):
        g = got.cpu().numpy()
        assert np.max(np.abs(g - want)) <= 1e-5 * max(1.0, np.abs(want).max())


def test_capacity_error(gpu):
    import torch

    cache = gpu.KVCache.new_quantized(256, 4, 2, capacity=20)
    k = torch.zeros((16, 2, 256), dtype=torch.bfloat16, device="cuda")
    cache.append(k, k)
    with pytest.raises(gpu.Exception_) as ei:
        cache.append(k, k)
    assert ei.value.code == gpu.FMKV_ERR_CAPACITY
    assert cache.offset() == 16
