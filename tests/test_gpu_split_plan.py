"""The one-sequence split plan for two KV heads (the global-layer shape, Hq
16, Hkv 2, head_dim 512) against the oracle. With one work-group per CU the
plan gives every CU a split of b blocks and deals the nblk - n_s * b blocks
left over one each to the splits s = 0 mod 4 when they fit there, else to
the splits s = 0 mod 2, else to the first splits. The context lengths below
put the plan in each of the three cases, for the decode step (127 split
columns and the new-token column per KV head on 256 CUs) and for the plain
attention read (128 split columns):

  T     blocks  step: b, left over   read: b, left over
  8200  513     4, 5  (mod 4)        4, 1  (mod 4)
  8900  557     4, 49 (mod 2)        4, 45 (mod 2)
  9700  607     4, 99 (first)        4, 95 (first)

(b is at least 4, one block for each of a work-group's four block streams.)

Checked: each output within max-abs 2e-2 / mean-abs 2e-3 of the exact f64
oracle (src/model/gemma4_attention.rs:84-103) at scale 1.0 and at a soft
scale, and the codes the steps stored bit-exact (src/cache.rs:266-310)."""
import numpy as np
import pytest

from gpu_util import check_attention, check_codes, dev_bf16, fast_kv, fast_q, host_u16, host_u32

pytestmark = pytest.mark.gpu

Hq, Hkv, D = 16, 2, 512


def plan_columns(nblk: int, cus: int, new_col: int) -> int:
    """Split columns per KV head of the XCD-aware plan (n_s = the CUs left
    after the new-token columns, over the two KV heads)."""
    n_s = (cus - new_col * Hkv) // Hkv
    assert nblk // n_s >= 4, "the plan needs at least four blocks per split"
    return n_s


@pytest.mark.parametrize("mode,bits", [(0, 8), (1, 3)])
@pytest.mark.parametrize("T", [8200, 8900, 9700])
def test_one_sequence_split_plan(gpu, ora, mode, bits, T):
    import torch

    steps = 2
    T0 = T - steps
    cap = T + 16
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap, mode=mode)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap, mode=mode)
    for c0 in range(0, T0, 2048):
        n = min(2048, T0 - c0)
        k = fast_kv(700 + c0, n, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(900 + c0, n, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"the table of cases is for 256 CUs (this GPU has {cus})")
    k1 = fast_kv(771, steps, Hkv, D, dist="t3", outliers=False)
    v1 = fast_kv(772, steps, Hkv, D, outliers=False)
    q = fast_q(773, steps + 1, Hq, Hkv, D, outliers=False)
    outs = []
    for i in range(steps):
        scale = 1.0 if i == 0 else 0.02
        dt = torch.float32 if i == 0 else torch.bfloat16
        outs.append((scale, cache.decode_step(dev_bf16(k1[i:i + 1]), dev_bf16(v1[i:i + 1]),
                                              dev_bf16(q[i]), scale, dtype=dt)))
    nblk = (T + 15) // 16
    assert cache.decode_splits() == plan_columns(nblk, cus, 0)
    read = cache.attention(dev_bf16(q[steps]), 0.02, dtype=torch.float32)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    plan_columns(nblk, cus, 1)
    for i in range(steps):
        oc.append(k1[i:i + 1], v1[i:i + 1])
        scale, out = outs[i]
        check_attention(out, oc.attention(q[i], scale), f"step {i} (T={T0 + i + 1}) scale {scale}")
    check_attention(read, oc.attention(q[steps], 0.02), f"attention read (T={T})")
    if mode == 0:
        check_codes(codes, meta, oc, slots=np.arange(T - 40, T), what="codes")
    else:
        c, m = host_u32(codes), host_u16(meta)
        assert not (c[T - 40:T] != oc.codes[T - 40:T]).any(), "codebook indices differ"
        assert not (m[T - 40:T] != oc.meta[T - 40:T]).any(), "codebook norms differ"
