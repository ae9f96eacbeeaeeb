"""Write the golden fixtures of the quantized KV path (tests/golden/*.npz).

Seeded inputs and the oracle's outputs for them, frozen as regression pins:
tests/test_golden.py checks that the oracle still produces these exact
bytes (so an edit of the oracle cannot silently move the contract), and
tests/test_gpu_golden.py that the HIP library does. Run from the repository
root: python tests/golden/make_golden.py. The reference (Rust + MLX) has no
tests or fixtures of its own for this path, so these come from the oracle,
whose functions are pinned by tests/test_oracle_pins.py.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "gemma4-moe-flash-mlx-turbo_amd"), str(ROOT / "oracle")]

import oracle  # noqa: E402
import synth  # noqa: E402

OUT = Path(__file__).resolve().parent

# (head_dim, bits, mode, n_kv_heads, window): the affine layouts the
# attention kernels read, and the TurboQuant codebook widths
CASES = [
    (128, 4, 0, 2, 0), (128, 8, 0, 2, 0), (256, 4, 0, 2, 0), (256, 8, 0, 2, 0),
    (512, 4, 0, 2, 0), (512, 8, 0, 2, 0), (256, 4, 0, 2, 16),
    (256, 2, 1, 2, 0), (256, 3, 1, 2, 0), (256, 4, 1, 2, 0), (512, 3, 1, 2, 0),
]
N_TOK = 24  # > W for the ring case: its early slots are overwritten
HQ_PER_KV = 2


def case_name(D, bits, mode, H, W):
    return f"{'affine' if mode == 0 else 'codebook'}_d{D}_b{bits}_h{H}_w{W}"


def make_case(D, bits, mode, H, W):
    seed = 1000 + D + 10 * bits + 100 * mode + W
    ch = synth.outlier_channels(seed, H, D)
    k = synth.kv_rows(seed, N_TOK, H, D, ch)
    v = synth.kv_rows(seed + 1, N_TOK, H, D, ch)
    q = synth.q_rows(seed + 2, H * HQ_PER_KV, H, D, ch)
    oc = oracle.OracleCache(H, D, bits, W, 0 if W else N_TOK, mode)
    oc.append(k[:N_TOK // 2], v[:N_TOK // 2])
    oc.append(k[N_TOK // 2:], v[N_TOK // 2:])
    out = {"k": k, "v": v, "q": q, "codes": oc.codes, "meta": oc.meta,
           "spec": np.array([D, bits, mode, H, W, N_TOK], np.int64)}
    for scale in (1.0, 0.01):
        out[f"attn_{scale}"] = oc.attention(q, scale)
    return out


def main() -> int:
    for case in CASES:
        path = OUT / f"{case_name(*case)}.npz"
        np.savez_compressed(path, **make_case(*case))
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
