"""Helpers shared by the GPU parity tests."""
import numpy as np

import synth


def dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def host_u32(t) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


def host_u16(t) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def kv_batch(seed: int, n: int, H: int, D: int, outliers=True, special=True) -> np.ndarray:
    """bf16 bits [n, H, D]: N(0,1) with x20 outlier channels, per-row random
    scale, and a few adversarial rows (zeros, constants, tiny values)."""
    ch = synth.outlier_channels(seed, H, D) if outliers else None
    x = synth.bf16_bits_to_f32(synth.kv_rows(seed, n, H, D, ch)).astype(np.float32)
    scale = (0.05 + 3.0 * synth.uniform(seed + 1, n)).astype(np.float32)
    x = x * scale[:, None, None]
    if special and n >= 4:
        x[1, 0] = 0.0
        x[2, -1] = 1.5
        x[3, 0] *= np.float32(1e-3)
    return synth.f32_to_bf16_bits(x)


def check_attention(out, ref, what=""):
    """Tolerance of the path: max-abs 2e-2 and mean-abs 2e-3.

    f32 outputs are compared with the exact (f64) reference. bf16 outputs
    are held to the same 2e-2 before their own rounding: each element lies
    within 2e-2 plus half a bf16 ulp of the exact value (half an ulp being
    what rounding a value already within 2e-2 can add; one ulp is 0.031 at
    |x| in [4, 8)). Their mean error is taken against the reference rounded
    to bf16, so that the format's own rounding does not count against it."""
    import torch

    o = out.float().cpu().numpy().astype(np.float64)
    if out.dtype == torch.bfloat16:
        exact = ref.astype(np.float64)
        r = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
        # (the binade of a value up to 2e-2 above |exact|)
        half_ulp = np.exp2(np.floor(np.log2(np.abs(exact) + 2e-2)) - 8)
        allow = 2e-2 + half_ulp * (1 + 1e-9)
        err_max = np.abs(o - exact)
    else:
        r = ref
        allow = np.full(ref.shape, 2e-2)
        err_max = np.abs(o - r)
    err = np.abs(o - r)
    worst = np.unravel_index(np.argmax(err_max - allow), err_max.shape)
    assert np.all(err_max <= allow), (f"{what}: max err {err_max.max():.3e} at {worst} "
                                      f"(ref {ref[worst]:.4f})")
    assert err.mean() <= 2e-3, f"{what}: mean err {err.mean():.3e}"
    return err_max.max(), err.mean()


def _randn(seed: int, shape):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def _bf16_bits(x) -> np.ndarray:
    import torch

    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # RNE


def _outlier_gain(ch, H: int, D: int):
    import torch

    g = torch.ones((H, D), dtype=torch.float32)
    for h in range(H):
        g[h, torch.from_numpy(ch[h])] = 20.0
    return g


def fast_kv(seed: int, n: int, H: int, D: int, dist: str = "normal", outliers: bool = True) -> np.ndarray:
    """bf16 bits [n, H, D] for config-sized tests: torch's CPU normals
    (Student-t(3) as Z / sqrt(chi2_3 / 3) for dist="t3"), with 4 outlier
    channels per head x20 when asked (synth's channel choice)."""
    x = _randn(seed, (n, H, D))
    if dist == "t3":
        chi = _randn(seed + 1000003, (3, n, H, D))
        x /= ((chi * chi).sum(0) / 3.0).sqrt()
    if outliers:
        x *= _outlier_gain(synth.outlier_channels(seed, H, D), H, D)
    return _bf16_bits(x)


def fast_q(seed: int, n: int, Hq: int, Hkv: int, D: int, outliers: bool = True) -> np.ndarray:
    """bf16 bits [n, Hq, D]; q head h shares the outlier channels of KV head
    h / (Hq / Hkv) (the K/V made by fast_kv with the same seed)."""
    x = _randn(seed + 7919, (n, Hq, D))
    if outliers:
        g = _outlier_gain(synth.outlier_channels(seed, Hkv, D), Hkv, D)
        x *= g.repeat_interleave(Hq // Hkv, dim=0)
    return _bf16_bits(x)


def check_codes(codes, meta, oc, slots=None, what=""):
    """Device codes/meta (read_codes) bit-exact against an OracleCache, over
    `slots` (default: all)."""
    c = host_u32(codes)
    m = host_u16(meta)
    if slots is None:
        slots = np.arange(oc.codes.shape[0])
    bad = np.nonzero(np.any(c[slots] != oc.codes[slots], axis=(1, 2, 3)))[0]
    assert bad.size == 0, f"{what}: codes differ at {bad.size} slots, first {slots[bad[0]]}"
    bad = np.nonzero(np.any(m[slots] != oc.meta[slots], axis=(1, 2, 3)))[0]
    assert bad.size == 0, f"{what}: scale/bias differ at {bad.size} slots, first {slots[bad[0]]}"
