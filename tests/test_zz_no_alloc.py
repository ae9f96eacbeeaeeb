"""fmkv_decode_step_noalloc (the decode step with its split partials in the
library's fixed per-GPU scratch instead of the handle's workspace) against
fmkv_decode_step, through the C ABI: two twin caches take the same appends
and steps, and every step's output and the stored codes must be identical
bit for bit (the same kernels on the same inputs). Two calls in a row, the
second on a smaller cache, so the scratch still holds the larger call's
contents; a call needing more than the scratch holds is rejected with
nothing launched."""
import ctypes

import numpy as np
import pytest

from gpu_util import dev_bf16, fast_kv, fast_q, host_u16, host_u32

pytestmark = pytest.mark.gpu


def step(lib, fn, cache, k, v, q, Hq, scale, tau, out):
    import torch

    rc = fn(cache._h, k.data_ptr(), v.data_ptr(), k.shape[0], q.data_ptr(), Hq, scale, tau,
            out.data_ptr(), 1 if out.dtype == torch.float32 else 0,
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.fmkv_last_error().decode()


@pytest.mark.parametrize("case", [
    # (D, bits, Hkv, Hq, window, prefill tokens, new tokens per step, tau)
    [(512, 8, 2, 16, 0, 6000, 1, 0.0), (256, 4, 8, 16, 1024, 300, 1, 0.0)],
    [(256, 4, 8, 16, 0, 3000, 1, 1e-3), (128, 8, 2, 8, 0, 40, 3, 0.0)],
])
def test_noalloc_step_matches_decode_step(gpu, case):
    import torch

    lib = gpu.load_library()
    for i, (D, bits, Hkv, Hq, W, T0, n, tau) in enumerate(case):
        cap = 0 if W else T0 + 16
        a = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
        b = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap)
        k, v = dev_bf16(fast_kv(10 + i, T0, Hkv, D)), dev_bf16(fast_kv(20 + i, T0, Hkv, D))
        a.append(k, v)
        b.append(k, v)
        kn, vn = dev_bf16(fast_kv(30 + i, 2 * n, Hkv, D)), dev_bf16(fast_kv(40 + i, 2 * n, Hkv, D))
        q = dev_bf16(fast_q(50 + i, 2, Hq, Hkv, D))
        for s in range(2):
            oa = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
            ob = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
            ks, vs = kn[s * n:(s + 1) * n].contiguous(), vn[s * n:(s + 1) * n].contiguous()
            step(lib, lib.fmkv_decode_step, a, ks, vs, q[s], Hq, 0.05, tau, oa)
            # the entry point's contract: no device memory is taken (b is a
            # fresh handle that never ran fmkv_decode_step; the scratch's
            # device address was set up when a handle was created, and the
            # same kernels already ran for a, so nothing loads lazily either)
            torch.cuda.synchronize()
            free0 = torch.cuda.mem_get_info()[0]
            step(lib, lib.fmkv_decode_step_noalloc, b, ks, vs, q[s], Hq, 0.05, tau, ob)
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, f"call {i} step {s}: device memory taken"
            assert torch.isfinite(ob).all()
            assert torch.equal(oa, ob), f"call {i} step {s}: outputs differ"
        assert a.offset() == b.offset() == T0 + 2 * n
        ca, ma = a.read_codes()
        cb, mb = b.read_codes()
        torch.cuda.synchronize()
        assert np.array_equal(host_u32(ca), host_u32(cb)) and np.array_equal(host_u16(ma), host_u16(mb))


def test_noalloc_rejects_partials_beyond_the_scratch(gpu):
    """A single-split-per-block plan over a long cache needs more partials than
    the scratch holds: FMKV_ERR_CAPACITY, offset unchanged, nothing written."""
    import torch

    lib = gpu.load_library()
    D, bits, Hkv, Hq, T0 = 512, 8, 2, 16, 20000
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=T0 + 16)
    k = dev_bf16(fast_kv(60, T0 + 1, Hkv, D))
    cache.append(k[:T0].contiguous(), k[:T0].contiguous())
    q = dev_bf16(fast_q(61, 1, Hq, Hkv, D))[0]
    out = torch.zeros((Hq, D), dtype=torch.float32, device="cuda")
    gpu.set_blocks_per_split(1)  # 1250 splits x 16 heads x 514 floats = 41 MB of partials
    try:
        kk = k[T0:].contiguous()
        rc = lib.fmkv_decode_step_noalloc(cache._h, kk.data_ptr(), kk.data_ptr(), 1, q.data_ptr(), Hq,
                                          1.0, 0.0, out.data_ptr(), 1,
                                          torch.cuda.current_stream().cuda_stream)
    finally:
        gpu.set_blocks_per_split(0)
    torch.cuda.synchronize()
    assert rc == gpu.FMKV_ERR_CAPACITY
    assert b"scratch" in lib.fmkv_last_error()
    assert cache.offset() == T0
    assert torch.count_nonzero(out) == 0
