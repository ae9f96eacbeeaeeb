"""Every benchmark configuration at its own full workload, checked against
the oracle: codes and f16 scale/bias bit-exact at every stored slot, attention
within max-abs 2e-2 / mean-abs 2e-3 (bf16 outputs: 2e-2 plus half a bf16 ulp
of the exact value) at Gemma-4's scale 1.0 and at a soft scale whose softmax is
checked to spread over many keys.

  C1  linear cache, Hq 16, Hkv 8, head_dim 256, 4-bit: 4096 single-token
      appends, then one decode step;
  C2  sliding ring W 1024, same shape: 8192 decode steps (8 wraps), outputs
      checked at steps around every wrap;
  C3  global layer, Hq 16, Hkv 2, head_dim 512, 8-bit: 32768 tokens in
      2048-token chunks with Student-t(3) K, then 8 decode steps under the
      default split plan (about 120 splits of 17 blocks), soft scale 0.01;
  C4  32 ragged sequences (the benchmark's seeded lengths in [512, 16384]) in a
      paged pool on shuffled blocks, one batched decode step, each sequence
      against its own oracle;
  C5  the 30-layer stack built by fmkv.make_cache: 64 chunks of 2048 into every
      layer (131072 positions on the 5 global layers, 64 wraps on the 25
      sliding rings), then one decode step of all 30 layers.

Reference semantics: src/cache.rs:266-310 (update_and_fetch: append, then the
fetch the attention reads), src/model/gemma4_attention.rs:84-103 (decode
attention, scale 1.0), src/model/mod.rs:375-396 (make_cache)."""
import copy

import numpy as np
import pytest

import synth
from gpu_util import check_attention, check_codes, dev_bf16, fast_kv, fast_q

pytestmark = pytest.mark.gpu


def softmax_spread(oc, q, scale, limit=0.99):
    """Largest softmax weight over the heads; asserts it is below `limit`
    (the soft-scale check is not a one-hot read of a single V row)."""
    w = oc.attention_weights(q, scale).max(axis=1).max()
    assert w < limit, f"softmax at scale {scale} is one-hot ({w:.4f})"
    return w


def test_c1_single_appends_then_decode(gpu, ora):
    import torch

    Hq, Hkv, D, bits, T = 16, 8, 256, 4, 4096
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=T + 16)
    oc = ora.OracleCache(Hkv, D, bits, 0, T + 16)
    k, v = fast_kv(101, T + 1, Hkv, D), fast_kv(102, T + 1, Hkv, D)
    q = fast_q(103, 1, Hq, Hkv, D)[0]
    kd, vd = dev_bf16(k), dev_bf16(v)
    for i in range(T):  # one token per append, as the reference's decode loop stores them
        cache.append(kd[i:i + 1], vd[i:i + 1])
    oc.append(k[:T], v[:T])
    assert cache.offset() == T and cache.stored_len() == T
    out = cache.decode_step(kd[T:T + 1], vd[T:T + 1], dev_bf16(q), 1.0, dtype=torch.float32)
    soft = cache.attention(dev_bf16(q), 0.002, dtype=torch.bfloat16)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    oc.append(k[T:], v[T:])
    check_codes(codes, meta, oc, what="C1")
    check_attention(out, oc.attention(q, 1.0), "C1 decode step, scale 1")
    softmax_spread(oc, q, 0.002)
    check_attention(soft, oc.attention(q, 0.002), "C1 attention, scale 0.002")


def test_c2_sliding_ring_8192_steps(gpu, ora):
    import torch

    Hq, Hkv, D, bits, W, n = 16, 8, 256, 4, 1024, 8192
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv)
    oc = ora.OracleCache(Hkv, D, bits, W)
    k, v = fast_kv(201, n, Hkv, D), fast_kv(202, n, Hkv, D)
    q = fast_q(201, n, Hq, Hkv, D)
    kd, vd, qd = dev_bf16(k), dev_bf16(v), dev_bf16(q)
    # steps (0-based; step i appends position i and attends) around every wrap
    checks = sorted({0, 15, 16, 1022, 1023, 1024, 1025, 1039, 2047, 2048, 3000, 4095, 4096, 5121,
                     6143, 7168, 8190, 8191})
    code_checks = {1025, 8191}
    scratch = torch.empty((Hq, D), dtype=torch.bfloat16, device="cuda")
    outs, done = {}, 0
    for i in range(n):
        if i in checks:
            j = checks.index(i)
            scale = 1.0 if j % 2 == 0 else 0.002
            dt = torch.float32 if (j // 2) % 2 == 0 else torch.bfloat16
            outs[i] = (scale, cache.decode_step(kd[i:i + 1], vd[i:i + 1], qd[i], scale, dtype=dt))
        else:
            cache.decode_step(kd[i:i + 1], vd[i:i + 1], qd[i], 1.0, out=scratch)
        if i in code_checks:
            codes, meta = cache.read_codes()
            torch.cuda.synchronize()
            oc.append(k[done:i + 1], v[done:i + 1])
            done = i + 1
            check_codes(codes, meta, oc, what=f"C2 ring after step {i}")
    torch.cuda.synchronize()
    assert cache.offset() == n and cache.stored_len() == W
    # replay the oracle to each checked step
    oc2 = ora.OracleCache(Hkv, D, bits, W)
    done = 0
    for i in checks:
        oc2.append(k[done:i + 1], v[done:i + 1])
        done = i + 1
        scale, out = outs[i]
        if scale != 1.0:
            softmax_spread(oc2, q[i], scale)
        check_attention(out, oc2.attention(q[i], scale), f"C2 step {i} (T={i + 1}) scale {scale}")


def test_c3_global_32k_decode_steps(gpu, ora):
    import torch

    Hq, Hkv, D, bits, T0, L, steps = 16, 2, 512, 8, 32768, 2048, 8
    cap = T0 + 64
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap)
    for c0 in range(0, T0, L):
        k = fast_kv(300 + c0, L, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(100300 + c0, L, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    check_codes(codes, meta, oc, what="C3 prefill")
    splits = cache.decode_splits()
    assert splits > 64, f"C3 runs the many-split plan (got {splits} splits)"
    k1 = fast_kv(391, steps, Hkv, D, dist="t3", outliers=False)
    v1 = fast_kv(392, steps, Hkv, D, outliers=False)
    q = fast_q(393, steps, Hq, Hkv, D, outliers=False)
    outs = []
    for i in range(steps):
        scale = 1.0 if i % 2 == 0 else 0.01
        dt = torch.float32 if (i // 2) % 2 == 0 else torch.bfloat16
        outs.append((scale, cache.decode_step(dev_bf16(k1[i:i + 1]), dev_bf16(v1[i:i + 1]),
                                              dev_bf16(q[i]), scale, dtype=dt)))
    # the attention entry point on the same state (split columns only)
    read = cache.attention(dev_bf16(q[0]), 0.01, dtype=torch.float32)
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    for i in range(steps):
        oc.append(k1[i:i + 1], v1[i:i + 1])
        scale, out = outs[i]
        if scale != 1.0:
            softmax_spread(oc, q[i], scale)
        check_attention(out, oc.attention(q[i], scale), f"C3 step {i} (T={T0 + i + 1}) scale {scale}")
    check_codes(codes, meta, oc, slots=np.arange(T0 - 64, T0 + steps), what="C3 after the steps")
    check_attention(read, oc.attention(q[0], 0.01), "C3 attention read")


def c4_lengths():
    """The benchmark's 32 seeded lengths in [512, 16384]."""
    return (512 + (synth.splitmix64(404, 32) % np.uint64(16384 - 512 + 1))).astype(np.int64)


def test_c4_ragged_paged_step(gpu, ora):
    import torch

    Hq, Hkv, D, bits, n_seqs = 16, 8, 256, 4, 32
    lens = c4_lengths()
    need = (lens + 1 + 15) // 16
    max_blocks, n_blocks = int(need.max()), int(need.sum())
    perm = np.argsort(synth.splitmix64(405, n_blocks)).astype(np.int32)  # shuffled block ids
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += int(nb)
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    ocs = []
    for s in range(n_seqs):
        T = int(lens[s])
        k, v = fast_kv(4000 + s, T, Hkv, D), fast_kv(5000 + s, T, Hkv, D)
        kd, vd = dev_bf16(k), dev_bf16(v)
        for p0 in range(0, T, 2048):
            n = min(2048, T - p0)
            pool.append(kd[None, p0:p0 + n].contiguous(), vd[None, p0:p0 + n].contiguous(),
                        dtab[s:s + 1].contiguous(), torch.tensor([p0], dtype=torch.int32, device="cuda"))
        oc = ora.OracleCache(Hkv, D, bits, 0, T + 1)
        oc.append(k, v)
        ocs.append(oc)
    k1, v1 = fast_kv(4400, n_seqs, Hkv, D), fast_kv(4401, n_seqs, Hkv, D)
    q = fast_q(4400, n_seqs, Hq, Hkv, D)
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    slen = start + 1
    mx = int(lens.max()) + 1
    out = pool.decode_step(dev_bf16(k1)[:, None].contiguous(), dev_bf16(v1)[:, None].contiguous(), dtab,
                           start, slen, mx, dev_bf16(q), 1.0, dtype=torch.float32)
    soft = pool.attention(dev_bf16(q), dtab, slen, mx, 0.002, dtype=torch.bfloat16)
    codes, meta = pool.read_codes()
    torch.cuda.synchronize()
    c, m = codes.cpu().numpy().view(np.uint32), meta.cpu().numpy().view(np.uint16)
    for s in range(n_seqs):
        ocs[s].append(k1[s:s + 1], v1[s:s + 1])
        pos = np.arange(int(lens[s]) + 1)
        phys = tables[s, pos // 16].astype(np.int64) * 16 + pos % 16
        assert np.array_equal(c[phys], ocs[s].codes[pos]), f"C4 seq {s}: codes differ"
        assert np.array_equal(m[phys], ocs[s].meta[pos]), f"C4 seq {s}: scale/bias differ"
        check_attention(out[s], ocs[s].attention(q[s], 1.0), f"C4 seq {s} (T={lens[s] + 1}) scale 1")
        check_attention(soft[s], ocs[s].attention(q[s], 0.002), f"C4 seq {s} scale 0.002")
    softmax_spread(ocs[int(np.argmax(lens))], q[int(np.argmax(lens))], 0.002)


def test_c5_stack_through_make_cache(gpu, ora):
    import torch

    Hq, L, n_chunks = 16, 2048, 64
    T0 = L * n_chunks  # 131072
    types = (["sliding_attention"] * 5 + ["full_attention"]) * 5
    caches = gpu.make_cache(types, 256, 8, capacity=T0 + 16, global_head_dim=512, n_global_kv_heads=2,
                            sliding_window=1024, attention_k_eq_v=True, kv_quant_bits=4,
                            global_kv_quant_bits=8, mode=gpu.MODE_AFFINE)
    assert len(caches) == 30
    for i, c in enumerate(caches):
        glob = i % 6 == 5
        assert (c.desc.window, c.desc.head_dim, c.desc.n_kv_heads, c.desc.bits) == \
            ((0, 512, 2, 8) if glob else (1024, 256, 8, 4)), f"layer {i}: {c.spec}"
    shape = {True: (2, 512, 8, 0), False: (8, 256, 4, 1024)}
    # chunks 0..62 are shared by the layers of a type; chunk 63 and the decode
    # token are each layer's own, so a layer reading another's arena fails
    base = {}
    for glob, (Hkv, D, bits, W) in shape.items():
        oc = ora.OracleCache(Hkv, D, bits, W, 0 if W else T0 + 16)
        for c in range(n_chunks - 1):
            seed = 60000 + 1000 * D + c
            k, v = fast_kv(seed, L, Hkv, D), fast_kv(seed + 500, L, Hkv, D)
            kd, vd = dev_bf16(k), dev_bf16(v)
            for i, cache in enumerate(caches):
                if (i % 6 == 5) == glob:
                    cache.append(kd, vd)
            oc.append(k, v)
        base[glob] = oc
    outs, ocs, qs = [], [], []
    for i, cache in enumerate(caches):
        glob = i % 6 == 5
        Hkv, D, bits, W = shape[glob]
        k, v = fast_kv(70000 + i, L + 1, Hkv, D), fast_kv(71000 + i, L + 1, Hkv, D)
        q = fast_q(72000 + i, 1, Hq, Hkv, D)[0]
        cache.append(dev_bf16(k[:L]), dev_bf16(v[:L]))
        outs.append(cache.decode_step(dev_bf16(k[L:]), dev_bf16(v[L:]), dev_bf16(q), 1.0,
                                      dtype=torch.float32))
        oc = copy.deepcopy(base[glob])
        oc.append(k, v)
        ocs.append(oc)
        qs.append(q)
    torch.cuda.synchronize()
    for i in (0, 5, 28, 29):  # codes of both kinds, first and last layers
        codes, meta = caches[i].read_codes()
        torch.cuda.synchronize()
        check_codes(codes, meta, ocs[i], what=f"C5 layer {i}")
    for i, cache in enumerate(caches):
        assert cache.offset() == T0 + 1
        check_attention(outs[i], ocs[i].attention(qs[i], 1.0), f"C5 layer {i} decode step")
    for c in caches:
        c.close()
