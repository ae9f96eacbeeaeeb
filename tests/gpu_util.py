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

    f32 outputs are compared with the exact (f64) reference. bf16 outputs are
    compared in bf16: against the reference rounded to bf16, where an element
    may also differ by one bf16 ulp (a rounding flip of a value that sits on a
    rounding boundary, which is larger than 2e-2 once |x| >= 4)."""
    import torch

    o = out.float().cpu().numpy().astype(np.float64)
    if out.dtype == torch.bfloat16:
        r = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(r), 1e-30))) - 7)
        allow = np.maximum(2e-2, ulp * (1 + 1e-9))
    else:
        r = ref
        allow = np.full(ref.shape, 2e-2)
    err = np.abs(o - r)
    worst = np.unravel_index(np.argmax(err - allow), err.shape)
    assert np.all(err <= allow), f"{what}: max err {err.max():.3e} at {worst} (ref {r[worst]:.4f})"
    assert err.mean() <= 2e-3, f"{what}: mean err {err.mean():.3e}"
    return err.max(), err.mean()
