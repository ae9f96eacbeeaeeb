"""The HIP library against the frozen fixtures (tests/golden/*.npz): the
same two appends stored bit for bit (codes and scale/bias or norms), and
the decode attention of affine caches within the path tolerance of the
fixture's f64 attention."""
from pathlib import Path

import numpy as np
import pytest

from gpu_util import check_attention, dev_bf16, host_u16, host_u32

pytestmark = pytest.mark.gpu
GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.npz"))


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_gpu_reproduces_fixture(gpu, path):
    import torch

    f = np.load(path)
    D, bits, mode, H, W, n = (int(x) for x in f["spec"])
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, H, 0 if W else n, mode)
    k, v = dev_bf16(f["k"]), dev_bf16(f["v"])
    cache.append(k[:n // 2].contiguous(), v[:n // 2].contiguous())
    cache.append(k[n // 2:].contiguous(), v[n // 2:].contiguous())
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(codes), f["codes"])
    assert np.array_equal(host_u16(meta), f["meta"])
    if mode == gpu.MODE_AFFINE:
        for scale in (1.0, 0.01):
            out = cache.attention(dev_bf16(f["q"]), scale, dtype=torch.float32)
            torch.cuda.synchronize()
            check_attention(out, f[f"attn_{scale}"], f"{path.stem} scale {scale}")
