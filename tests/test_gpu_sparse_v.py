"""Sparse-V decode attention on the GPU against the oracle.

src/model/gemma4_attention.rs:196-234: at decode with tau > 0 the softmax
weights below tau are zeroed without renormalisation before the product
with V. The oracle (ora_attention_f64) applies the same rule to the exact
f64 weights; the kernels compare their f32 scores with the base-2 threshold
M + log2(tau * L) of a statistics pass. Each test runs on both second
halves: the gather (one work-group per q head reads the kept tokens' V rows;
with more than 64 candidate blocks a head's parts merge through a counter)
and the gated pass with the split merge. Tolerance: max-abs 2e-2, mean-abs
2e-3 (bf16 outputs: 2e-2 plus half a bf16 ulp of the exact value)."""
import numpy as np
import pytest

import synth
from gpu_util import check_attention, dev_bf16, host_u16, host_u32, kv_batch

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["gather", "gated"], autouse=True)
def sparse_path(request, gpu):
    """Every test on both second halves of sparse-V: the gather of the kept V
    rows (the default) and the gated pass with the split merge."""
    gpu.set_sparse_v_gather(request.param == "gather")
    yield request.param
    gpu.set_sparse_v_gather(True)


def q_batch(seed, Hq, Hkv, D):
    return synth.q_rows(seed + 100, Hq, Hkv, D, synth.outlier_channels(seed, Hkv, D))


def filled(gpu, ora, D, bits, Hkv, T, window=0, seed=0):
    cap = 0 if window else T + 16
    cache = gpu.KVCache.new_quantized_with_window(D, bits, window, Hkv, cap)
    oc = ora.OracleCache(Hkv, D, bits, window, cap)
    k, v = kv_batch(seed, T, Hkv, D), kv_batch(seed + 1, T, Hkv, D)
    cache.append(dev_bf16(k), dev_bf16(v))
    oc.append(k, v)
    return cache, oc


def kept_fraction(oc, q, scale, tau):
    """Share of (head, token) weights at or above tau (so a test is known to
    exercise the gate rather than keep or drop everything)."""
    w = oc.attention_weights(q, scale)
    return float(np.mean(w >= tau))


@pytest.mark.parametrize("D,bits,Hkv,Hq", [(512, 8, 2, 16), (256, 4, 8, 16), (128, 4, 4, 4),
                                           (256, 8, 2, 12)])
@pytest.mark.parametrize("T", [1, 33, 700, 1500])
def test_sparse_v_matches_oracle(gpu, ora, D, bits, Hkv, Hq, T):
    import torch

    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=T)
    q = q_batch(T, Hq, Hkv, D)
    # peaked (Gemma-4 scale 1.0) to soft: with the x20 outlier channels only
    # scale 0.003 leaves many weights near the thresholds
    for scale, tau in ((1.0, 1e-3), (1.0, 0.05), (0.05, 1.0 / (2 * T)), (0.05, 0.02), (0.003, 1e-3)):
        ref = oc.attention(q, scale, tau)
        out32 = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
        out16 = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        check_attention(out32, ref, f"f32 scale={scale} tau={tau}")
        check_attention(out16, ref, f"bf16 scale={scale} tau={tau}")


def test_sparse_v_gate_is_exercised(gpu, ora):
    """A soft softmax with tau at the 99th percentile of the weights: about 1%
    of the weights are kept, and the result differs from dense attention by
    far more than the tolerance."""
    import torch

    D, bits, Hkv, Hq, T = 512, 8, 2, 16, 1500
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=5)
    q = q_batch(5, Hq, Hkv, D)
    scale = 0.003
    tau = float(np.quantile(oc.attention_weights(q, scale), 0.99))
    frac = kept_fraction(oc, q, scale, tau)
    assert 0.005 < frac < 0.05, frac
    dense = oc.attention(q, scale)
    ref = oc.attention(q, scale, tau)
    assert np.abs(dense - ref).max() > 0.1
    out = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
    torch.cuda.synchronize()
    check_attention(out, ref, "gated")


def test_sparse_v_limits(gpu, ora):
    """tau above every weight: zero output; a tau below every weight: dense."""
    import torch

    D, bits, Hkv, Hq, T = 256, 4, 8, 16, 300
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=7)
    q = q_batch(7, Hq, Hkv, D)
    out = cache.attention(dev_bf16(q), 1.0, sparse_v_tau=1.5, dtype=torch.float32)
    tiny = cache.attention(dev_bf16(q), 1.0, sparse_v_tau=1e-30, dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
    check_attention(tiny, oc.attention(q, 1.0), "tau 1e-30 vs dense")


@pytest.mark.parametrize("bps", [1, 2, 3, 5])
def test_sparse_v_split_counts_agree(gpu, ora, bps):
    import torch

    D, bits, Hkv, Hq, T = 512, 8, 2, 16, 700
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=4)
    q = q_batch(9, Hq, Hkv, D)
    tau = 1.0 / 1400
    ref = oc.attention(q, 0.05, tau)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), 0.05, sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, ref, f"bps={bps}")


@pytest.mark.parametrize("bps", [40, 300])
@pytest.mark.parametrize("scale,tau", [(1.0, 1e-3), (0.05, 1.0 / 12000)])
def test_sparse_v_block_skip_long_splits(gpu, ora, bps, scale, tau):
    """The gated pass visits only the blocks in which some head's largest
    score reaches its threshold (each of a work-group's four block streams
    tests up to 64 of its blocks at once; bps 300 gives streams of 75 blocks,
    whose blocks past the 64th are always visited): peaked weights (most
    blocks skipped) and soft ones, both within tolerance."""
    import torch

    D, bits, Hkv, Hq, T = 512, 8, 2, 16, 6000
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=12)
    q = q_batch(13, Hq, Hkv, D)
    ref = oc.attention(q, scale, tau)
    gpu.set_blocks_per_split(bps)
    try:
        out = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        gpu.set_blocks_per_split(0)
    check_attention(out, ref, f"bps={bps} scale={scale} tau={tau}")


def test_sparse_v_32k_decode_steps(gpu, ora):
    """Global-layer shape at 32K context (Hq 16, Hkv 2, head_dim 512, 8-bit):
    decode steps with tau 1e-3 at scale 1.0 and at a soft scale whose tau is
    the weights' 99.9th percentile, against the oracle; the codes the steps
    stored bit-exact."""
    import torch
    from gpu_util import check_codes, fast_kv, fast_q

    Hq, Hkv, D, bits, T0, L, steps = 16, 2, 512, 8, 32768, 2048, 4
    cap = T0 + 16
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap)
    for c0 in range(0, T0, L):
        k = fast_kv(600 + c0, L, Hkv, D, dist="t3", outliers=False)
        v = fast_kv(100600 + c0, L, Hkv, D, outliers=False)
        cache.append(dev_bf16(k), dev_bf16(v))
        oc.append(k, v)
    k1 = fast_kv(691, steps, Hkv, D, dist="t3", outliers=False)
    v1 = fast_kv(692, steps, Hkv, D, outliers=False)
    q = fast_q(693, steps, Hq, Hkv, D, outliers=False)
    soft = 0.01
    outs = []
    for i in range(steps):
        oc.append(k1[i:i + 1], v1[i:i + 1])
        scale = 1.0 if i % 2 == 0 else soft
        tau = 1e-3 if i % 2 == 0 else float(np.quantile(oc.attention_weights(q[i], soft), 0.999))
        ref = oc.attention(q[i], scale, tau)
        out = cache.decode_step(dev_bf16(k1[i:i + 1]), dev_bf16(v1[i:i + 1]), dev_bf16(q[i]),
                                scale, sparse_v_tau=tau, dtype=torch.float32)
        outs.append((out, ref, scale, tau))
    codes, meta = cache.read_codes()
    torch.cuda.synchronize()
    for i, (out, ref, scale, tau) in enumerate(outs):
        check_attention(out, ref, f"step {i} scale {scale} tau {tau:.3g}")
    check_codes(codes, meta, oc, slots=np.arange(T0 - 16, T0 + steps), what="32K sparse-V steps")


@pytest.mark.parametrize("D,bits", [(256, 4), (256, 8)])
def test_sparse_v_ring_steps(gpu, ora, D, bits):
    """Sliding layer W = 64: decode steps through two wraps with tau > 0 (the
    statistics pass's new-token column appends the token, the gated pass
    reads it back): every checked output within tolerance, and the stored
    codes and scale/bias bit-exact with the oracle's at the end."""
    import torch

    Hkv, Hq, W = 8, 16, 64
    cache = gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, 0)
    oc = ora.OracleCache(Hkv, D, bits, W, 0)
    k0, v0 = kv_batch(1, 40, Hkv, D), kv_batch(2, 40, Hkv, D)
    cache.append(dev_bf16(k0), dev_bf16(v0))
    oc.append(k0, v0)
    for step in range(100):
        k = kv_batch(100 + 2 * step, 1, Hkv, D, special=False)
        v = kv_batch(101 + 2 * step, 1, Hkv, D, special=False)
        q = q_batch(300 + step, Hq, Hkv, D)
        out = cache.decode_step(dev_bf16(k), dev_bf16(v), dev_bf16(q), 0.05, sparse_v_tau=0.01,
                                dtype=torch.float32)
        oc.append(k, v)
        torch.cuda.synchronize()
        if step % 9 == 0 or step > 90:
            check_attention(out, oc.attention(q, 0.05, 0.01), f"step {step}")
    codes, meta = cache.read_codes()
    assert np.array_equal(host_u32(codes), oc.codes), "codes written by sparse-V steps"
    assert np.array_equal(host_u16(meta), oc.meta), "scale/bias written by sparse-V steps"


def test_sparse_v_paged(gpu, ora):
    """Paged pool, ragged sequences, shuffled block ids: gated decode step."""
    import torch

    D, bits, Hkv, Hq = 256, 4, 8, 16
    lens = [37, 300, 16, 901]
    n_seqs = len(lens)
    need = [(n + 2 + 15) // 16 for n in lens]
    max_blocks, n_blocks = max(need), sum(need)
    perm = np.argsort(synth.splitmix64(77, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, n in enumerate(lens):
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 2)
        k, v = kv_batch(20 * s, n, Hkv, D), kv_batch(20 * s + 1, n, Hkv, D)
        oc.append(k, v)
        oracles.append(oc)
        pool.append(dev_bf16(k[None]), dev_bf16(v[None]), dtab[s:s + 1].contiguous(),
                    torch.zeros(1, dtype=torch.int32, device="cuda"))
    k1 = np.stack([kv_batch(700 + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
    v1 = np.stack([kv_batch(800 + s, 1, Hkv, D, special=False) for s in range(n_seqs)])
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    q = np.stack([q_batch(950 + s, Hq, Hkv, D) for s in range(n_seqs)])
    tau = 2e-3
    out = pool.decode_step(dev_bf16(k1), dev_bf16(v1), dtab, start, start + 1, max(lens) + 1,
                           dev_bf16(q), 0.05, sparse_v_tau=tau, dtype=torch.float32)
    torch.cuda.synchronize()
    for s in range(n_seqs):
        oracles[s].append(k1[s], v1[s])
        check_attention(out[s], oracles[s].attention(q[s], 0.05, tau), f"seq {s}")


def test_sparse_v_gated_grid_beyond_resident(gpu, ora):
    """One cache split one block per work-group (Hkv 8, 6000 tokens: 3000
    gated work-groups, several waves of them per CU): every gated work-group
    derives its thresholds from the statistics pass's (m, l), which no gated
    work-group overwrites, however early its siblings finish. tau is the
    weights' 99th percentile at a soft scale, so about 1% of the weights sit
    above it and many near it."""
    import torch

    D, bits, Hkv, Hq, T = 256, 4, 8, 16, 6000
    cache, oc = filled(gpu, ora, D, bits, Hkv, T, seed=31)
    q = q_batch(31, Hq, Hkv, D)
    for scale in (1.0, 0.003):
        tau = 1e-3 if scale == 1.0 else float(np.quantile(oc.attention_weights(q, scale), 0.99))
        ref = oc.attention(q, scale, tau)
        gpu.set_blocks_per_split(1)
        try:
            out = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
            torch.cuda.synchronize()
        finally:
            gpu.set_blocks_per_split(0)
        check_attention(out, ref, f"bps=1 scale={scale} tau={tau:.3g}")


def test_sparse_v_paged_batch_beyond_resident(gpu, ora):
    """Sixteen ragged sequences of 2048..6144 tokens in a paged pool (Hkv 8,
    head_dim 256, 4-bit, shuffled blocks): the batched plan puts several
    work-groups on every CU, so gated work-groups start after others of the
    same sequence have finished. Sparse-V decode steps against the oracle's
    gated attention at tau 1e-3 (scale 1.0) and at the 99th-percentile weight
    of a soft scale."""
    import torch

    from gpu_util import fast_kv, fast_q

    D, bits, Hkv, Hq, n_seqs = 256, 4, 8, 16, 16
    lens = (2048 + np.floor(synth.uniform(41, n_seqs) * 4096)).astype(int).tolist()
    need = [(n + 2 + 15) // 16 for n in lens]
    max_blocks, n_blocks = max(need), sum(need)
    perm = np.argsort(synth.splitmix64(43, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, n in enumerate(lens):
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 2)
        k, v = fast_kv(1000 + s, n, Hkv, D), fast_kv(2000 + s, n, Hkv, D)
        oc.append(k, v)
        oracles.append(oc)
        pool.append(dev_bf16(k[None]), dev_bf16(v[None]), dtab[s:s + 1].contiguous(),
                    torch.zeros(1, dtype=torch.int32, device="cuda"))
    k1 = np.stack([fast_kv(3000 + s, 1, Hkv, D) for s in range(n_seqs)])
    v1 = np.stack([fast_kv(4000 + s, 1, Hkv, D) for s in range(n_seqs)])
    q = np.stack([fast_q(5000 + s, 1, Hq, Hkv, D)[0] for s in range(n_seqs)])
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    for s in range(n_seqs):
        oracles[s].append(k1[s], v1[s])
    soft = 0.003
    taus = [float(np.quantile(oracles[s].attention_weights(q[s], soft), 0.99)) for s in range(n_seqs)]
    tau_soft = float(np.median(taus))
    out1 = pool.decode_step(dev_bf16(k1), dev_bf16(v1), dtab, start, start + 1, max(lens) + 1,
                            dev_bf16(q), 1.0, sparse_v_tau=1e-3, dtype=torch.float32)
    out2 = pool.attention(dev_bf16(q), dtab, start + 1, max(lens) + 1, soft,
                          sparse_v_tau=tau_soft, dtype=torch.float32)
    torch.cuda.synchronize()
    for s in range(n_seqs):
        check_attention(out1[s], oracles[s].attention(q[s], 1.0, 1e-3), f"seq {s} scale 1.0")
        check_attention(out2[s], oracles[s].attention(q[s], soft, tau_soft),
                        f"seq {s} scale {soft} tau {tau_soft:.3g}")


def test_sparse_v_rejects_bad_tau(gpu):
    import torch

    cache = gpu.KVCache.new_quantized_with_window(256, 4, 0, 8, 64)
    k = torch.zeros((4, 8, 256), dtype=torch.bfloat16, device="cuda")
    cache.append(k, k)
    q = torch.zeros((16, 256), dtype=torch.bfloat16, device="cuda")
    for bad in (-1e-3, float("nan"), float("inf")):
        with pytest.raises(gpu.Exception_) as e:
            cache.attention(q, 1.0, sparse_v_tau=bad)
        assert e.value.code == gpu.FMKV_ERR_INVALID_ARG


def test_sparse_v_many_candidates_with_new_token(gpu, ora):
    """Soft weights and tau at the median weight, so that about half the
    weights are kept and almost every block holds one: the gather splits
    each head's candidate blocks over several parts that merge through the
    head's counter, and part 0 also takes the decode step's new token, whose
    K row is a q of its group scaled so that its weight is kept. Three
    decode steps against the oracle's gated attention."""
    import torch

    from gpu_util import fast_kv, fast_q

    D, bits, Hkv, Hq, T0, steps = 256, 4, 2, 16, 4000, 3
    cap = T0 + 16
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=cap)
    oc = ora.OracleCache(Hkv, D, bits, 0, cap)
    k, v = fast_kv(71, T0, Hkv, D), fast_kv(72, T0, Hkv, D)
    cache.append(dev_bf16(k), dev_bf16(v))
    oc.append(k, v)
    q = fast_q(73, steps, Hq, Hkv, D)
    v1 = fast_kv(74, steps, Hkv, D)
    scale = 0.003
    G = Hq // Hkv
    for i in range(steps):
        # the new K row of KV head h: q of head h G, scaled so that its score
        # sits four standard deviations above that head's other scores
        qf = synth.bf16_bits_to_f32(q[i]).astype(np.float64)
        kd, _ = oc.dequant_kv()
        kf = np.zeros((1, Hkv, D), np.float32)
        for h in range(Hkv):
            sc = scale * (kd[:, h] @ qf[h * G])
            kf[0, h] = qf[h * G] * ((sc.mean() + 4 * sc.std()) / (scale * qf[h * G] @ qf[h * G]))
        k1 = synth.f32_to_bf16_bits(kf)
        oc.append(k1, v1[i:i + 1])
        w = oc.attention_weights(q[i], scale)
        tau = float(np.quantile(w, 0.5))
        assert w[0, -1] >= tau and w[G, -1] >= tau, "the new token is kept"
        assert 0.3 < np.mean(w >= tau) < 0.7, "about half the weights kept"
        ref = oc.attention(q[i], scale, tau)
        out = cache.decode_step(dev_bf16(k1), dev_bf16(v1[i:i + 1]), dev_bf16(q[i]), scale,
                                sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
        check_attention(out, ref, f"step {i}")


def test_sparse_v_beyond_8192_blocks(gpu, ora):
    """140000 visible tokens (8750 blocks of 16): each gather thread scans
    more than 32 block rows, so candidates sit in both halves of its row
    flags. Soft weights with tau at the 99.9th percentile (kept tokens spread
    over the whole context) and a peaked step at tau 1e-3, against the
    oracle."""
    import torch

    from gpu_util import fast_kv, fast_q

    D, bits, Hkv, Hq, T = 128, 4, 1, 4, 140000
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=T + 16)
    oc = ora.OracleCache(Hkv, D, bits, 0, T + 16)
    k, v = fast_kv(81, T, Hkv, D), fast_kv(82, T, Hkv, D)
    cache.append(dev_bf16(k), dev_bf16(v))
    oc.append(k, v)
    q = fast_q(83, 1, Hq, Hkv, D)[0]
    for scale in (0.003, 1.0):
        w = oc.attention_weights(q, scale)
        tau = float(np.quantile(w, 0.999)) if scale < 1.0 else 1e-3
        kept = np.nonzero(w >= tau)[1]
        if scale < 1.0:
            assert kept.min() < 16 * 8192 <= kept.max(), "kept tokens on both sides of row 8192"
        ref = oc.attention(q, scale, tau)
        out = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
        check_attention(out, ref, f"scale={scale} tau={tau:.3g}")


@pytest.mark.parametrize("T", [4096, 4112, 40000, 70000])
def test_sparse_v_gather_row_instances(gpu, ora, T):
    """Contexts at the gather's instance boundaries (256 and 257 block rows)
    and inside the 4096- and 8192-row instances (2500 and 4375 rows): a soft
    step with tau at the 99.9th percentile (kept tokens spread over every
    row) and a peaked one at tau 1e-3, against the oracle."""
    import torch

    from gpu_util import fast_kv, fast_q

    D, bits, Hkv, Hq = 128, 4, 1, 4
    cache = gpu.KVCache.new_quantized(D, bits, Hkv, capacity=T + 16)
    oc = ora.OracleCache(Hkv, D, bits, 0, T + 16)
    k, v = fast_kv(91 + T, T, Hkv, D), fast_kv(92 + T, T, Hkv, D)
    cache.append(dev_bf16(k), dev_bf16(v))
    oc.append(k, v)
    q = fast_q(93 + T, 1, Hq, Hkv, D)[0]
    for scale in (0.003, 1.0):
        w = oc.attention_weights(q, scale)
        tau = float(np.quantile(w, 0.999)) if scale < 1.0 else 1e-3
        if scale < 1.0:
            kept = np.nonzero(w >= tau)[1]
            assert kept.max() >= T - T // 8, "kept tokens reach the last rows"
        ref = oc.attention(q, scale, tau)
        out = cache.attention(dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
        torch.cuda.synchronize()
        check_attention(out, ref, f"T={T} scale={scale} tau={tau:.3g}")


def test_sparse_v_paged_long_ragged(gpu, ora):
    """Paged pool, shuffled block ids, ragged sequences up to 70000 tokens
    (the gather's 8192-row instance, reading through block tables): one
    decode step at scale 0.05 with tau 1e-3, against the oracle."""
    import torch

    from gpu_util import fast_kv, fast_q

    D, bits, Hkv, Hq = 128, 4, 1, 4
    lens = [70000, 300, 40000, 5000]
    n_seqs = len(lens)
    need = [(n + 2 + 15) // 16 for n in lens]
    max_blocks, n_blocks = max(need), sum(need)
    perm = np.argsort(synth.splitmix64(78, n_blocks)).astype(np.int32)
    tables = np.zeros((n_seqs, max_blocks), np.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb]
        o += nb
    pool = gpu.PagedPool(gpu.make_desc(Hkv, D, bits), n_blocks)
    dtab = torch.from_numpy(tables).cuda()
    oracles = []
    for s, n in enumerate(lens):
        oc = ora.OracleCache(Hkv, D, bits, 0, n + 2)
        k, v = fast_kv(30 * s + 5, n, Hkv, D), fast_kv(30 * s + 6, n, Hkv, D)
        oc.append(k, v)
        oracles.append(oc)
        pool.append(dev_bf16(k[None]), dev_bf16(v[None]), dtab[s:s + 1].contiguous(),
                    torch.zeros(1, dtype=torch.int32, device="cuda"))
    k1 = np.stack([fast_kv(710 + s, 1, Hkv, D) for s in range(n_seqs)])
    v1 = np.stack([fast_kv(810 + s, 1, Hkv, D) for s in range(n_seqs)])
    start = torch.tensor(lens, dtype=torch.int32, device="cuda")
    q = np.stack([fast_q(960 + s, 1, Hq, Hkv, D)[0] for s in range(n_seqs)])
    scale, tau = 0.05, 1e-3  # kept fractions 0.13%, 22%, 0.27%, 0.12%
    out = pool.decode_step(dev_bf16(k1), dev_bf16(v1), dtab, start, start + 1, max(lens) + 1,
                           dev_bf16(q), scale, sparse_v_tau=tau, dtype=torch.float32)
    torch.cuda.synchronize()
    for s in range(n_seqs):
        oracles[s].append(k1[s], v1[s])
        w = oracles[s].attention_weights(q[s], scale)
        assert 0 < np.mean(w >= tau) < 1, f"seq {s}: the gate keeps some weights and drops some"
        check_attention(out[s], oracles[s].attention(q[s], scale, tau), f"seq {s} (T={lens[s] + 1})")
