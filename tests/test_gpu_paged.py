"""Paged pool on the GPU: ragged sequences on shuffled 16-token blocks. Codes
at each (sequence, position) equal the oracle's bit for bit at the block-table
address; batched decode attention matches each sequence's oracle."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(256, 4, 8, 16), (512, 8, 2, 16)])
@pytest.mark.parametrize("bps", [0, 1, 3, 8])
def test_paged_ragged_decode(gpu, ora, D, bits, Hkv, Hq, bps):
    """bps: blocks per split (0: the plan's); 1, 3 and 8 give several splits
    per sequence (8: single-wave streams at 4-bit D=256). A paged
    sequence's first split takes 4 x bps blocks when the grid holds at least
    four work-groups per CU: here bps 1 on the 8-head shape (both split
    sizes), equal splits otherwise."""
    import torch

    lens = [5, 40, 100, 17, 1, 64, 300, 700]
    n_seqs = len(lens)
    need = [(n + 1 + 15) // 16 for n in lens]
    max_blocks = max(need)
    n_blocks = sum(need) + 9
    perm = np.argsort(synth.splitmix64(77, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    desc = gpu.make_desc(Hkv, D, bits)
    pool = gpu.PagedPool(desc, n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, n in enumerate(lens):  # ragged prefill, one call per sequence
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 1)
        k = kv_batch(10 * s, n, Hkv, D)
        v = kv_batch(10 * s + 1, n, Hkv, D)
        oc.append(k, v)
        oracles.append(oc)
        pool.append(dev_bf16(k[None]), dev_bf16(v[None]), dtab[s:s + 1].contiguous(),
                    torch.zeros(1, dtype=torch.int32, device="cuda"))
    # one decode step: one new token per sequence in a single call
    k1 = np.stack([kv_batch(500 + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
    v1 = np.stack([kv_batch(600 + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
    for s in range(n_seqs):
        oracles[s].append(k1[s], v1[s])
    pool.append(dev_bf16(k1), dev_bf16(v1), dtab, torch.tensor(lens, dtype=torch.int32, device="cuda"))
    seq_lens = torch.tensor([n + 1 for n in lens], dtype=torch.int32, device="cuda")
    q = np.stack([synth.q_rows(900 + s, Hq, Hkv, D, synth.outlier_channels(10 * s, Hkv, D))
                  for s in range(n_seqs)])
    gpu.set_blocks_per_split(bps)
    try:
        out = pool.attention(dev_bf16(q), dtab, seq_lens, max(lens) + 1, 0.05, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    codes, meta = pool.read_codes()
    torch.cuda.synchronize()
    c, m = host_u32(codes), host_u16(meta)
    for s, n in enumerate(lens):
        p = np.arange(n + 1)
        slots = tables[s, p // 16].astype(np.int64) * 16 + p % 16
        assert np.array_equal(c[slots], oracles[s].codes[p]), f"seq {s} codes"
        assert np.array_equal(m[slots], oracles[s].meta[p]), f"seq {s} scales"
        check_attention(out[s], oracles[s].attention(q[s], 0.05), f"seq {s}")
