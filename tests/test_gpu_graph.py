"""Decode steps captured in a HIP graph replay exactly the eager results.

A graph of n consecutive `fmkv_decode_step` calls repeats, on every replay,
the same appends (the same codes into the same slots) and the same
attention reads. Linear cache: a replay rewrites positions nobody beyond
them reads, so every replay reproduces the eager outputs of those steps
bit for bit. Ring of W slots: the graph spans one whole wrap (n = W), and
replay r reproduces the r-th eager pass over the same inputs (from the
second pass on, every slot holds what the previous pass wrote). The
workspace is sized by an eager step before the capture (nothing may
allocate inside it), and the steps stay inside one split plan. Each replay
is followed by unrelated eager work and a synchronisation, and every
replay is checked; the same for sparse-V steps (tau > 0)."""
import pytest

from gpu_util import dev_bf16, kv_batch
import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tau", [0.0, 0.01])  # dense; sparse-V (stats, gated, combine)
@pytest.mark.parametrize("D,bits,Hkv,Hq,W,T0", [
    (512, 8, 2, 16, 0, 295),   # global layer: positions 296..304 stay in 19 blocks
    (256, 4, 8, 16, 64, 200),  # sliding ring: 4 blocks once full
])
def test_graph_replays_match_eager(gpu, D, bits, Hkv, Hq, W, T0, tau):
    import torch

    cap = 0 if W else T0 + 32
    caches = [gpu.KVCache.new_quantized_with_window(D, bits, W, Hkv, cap) for _ in range(2)]
    k0, v0 = dev_bf16(kv_batch(1, T0, Hkv, D)), dev_bf16(kv_batch(2, T0, Hkv, D))
    n = W if W else 8
    ks = [dev_bf16(kv_batch(10 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    vs = [dev_bf16(kv_batch(40 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    qs = [dev_bf16(synth.q_rows(70 + j, Hq, Hkv, D, None)) for j in range(n + 1)]
    for c in caches:
        c.append(k0, v0)
        # sizes the workspace
        c.decode_step(ks[0], vs[0], qs[0], 1.0, sparse_v_tau=tau, dtype=torch.float32)
    eager, graphed = caches
    passes = 3 if W else 1
    want = [[eager.decode_step(ks[j], vs[j], qs[j], 1.0, sparse_v_tau=tau, dtype=torch.float32)
             for j in range(1, n + 1)] for _ in range(passes)]
    torch.cuda.synchronize()

    outs = [torch.empty((Hq, D), dtype=torch.float32, device="cuda") for _ in range(n)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for j in range(n):
            graphed.decode_step(ks[j + 1], vs[j + 1], qs[j + 1], 1.0, sparse_v_tau=tau, out=outs[j],
                                stream=s)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 16, device="cuda").sum()  # unrelated eager work
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        w = want[min(rep, passes - 1)]
        for j in range(n):
            assert torch.equal(outs[j], w[j]), f"replay {rep} step {j}"
    ca, ma = eager.read_codes()
    cb, mb = graphed.read_codes()
    torch.cuda.synchronize()
    assert torch.equal(ca, cb) and torch.equal(ma, mb)


@pytest.mark.parametrize("mode,bits", [(0, 8), (1, 3), (2, 16)])
def test_graph_steps_across_split_plans(gpu, mode, bits):
    """A cache's workspace is sized for the largest plan its capacity allows:
    after one eager step, a graph of 40 decode steps whose context crosses
    three block boundaries (the split count grows with each) captures with
    no allocation, and every replay equals the eager steps bit for bit."""
    import torch

    D, Hkv, Hq, T0, n = 512, 2, 16, 100, 40
    caches = [gpu.KVCache(gpu.make_desc(Hkv, D, bits, 0, T0 + n + 16, mode)) for _ in range(2)]
    k0, v0 = dev_bf16(kv_batch(3, T0, Hkv, D)), dev_bf16(kv_batch(4, T0, Hkv, D))
    ks = [dev_bf16(kv_batch(100 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    vs = [dev_bf16(kv_batch(200 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    qs = [dev_bf16(synth.q_rows(300 + j, Hq, Hkv, D, None)) for j in range(n + 1)]
    for c in caches:
        c.append(k0, v0)
        c.decode_step(ks[0], vs[0], qs[0], 1.0, dtype=torch.float32)
    eager, graphed = caches
    splits0 = eager.decode_splits()
    want = [eager.decode_step(ks[j], vs[j], qs[j], 1.0, dtype=torch.float32) for j in range(1, n + 1)]
    assert eager.decode_splits() > splits0, "the steps cross split plans"
    torch.cuda.synchronize()
    outs = [torch.empty((Hq, D), dtype=torch.float32, device="cuda") for _ in range(n)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for j in range(n):
            graphed.decode_step(ks[j + 1], vs[j + 1], qs[j + 1], 1.0, out=outs[j], stream=s)
    for rep in range(2):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for j in range(n):
            assert torch.equal(outs[j], want[j]), f"mode {mode} replay {rep} step {j}"


def test_graph_replays_sparse_gather_merge(gpu):
    """Sparse-V steps whose heads have more candidate blocks than one
    work-group takes (soft weights, tau 1e-4 on a 1500-token global layer:
    most tokens kept, about 94 candidate blocks, so several parts merge
    through the head's counter, which the statistics pass zeroes): every
    replay equals the eager steps bit for bit (the parts' rows are summed in
    part order whatever order they arrive in)."""
    import torch

    D, bits, Hkv, Hq, T0, n = 512, 8, 2, 16, 1500, 6
    scale, tau = 0.003, 1e-4
    caches = [gpu.KVCache.new_quantized(D, bits, Hkv, capacity=T0 + 32) for _ in range(2)]
    k0, v0 = dev_bf16(kv_batch(3, T0, Hkv, D)), dev_bf16(kv_batch(4, T0, Hkv, D))
    ks = [dev_bf16(kv_batch(110 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    vs = [dev_bf16(kv_batch(140 + j, 1, Hkv, D, special=False)) for j in range(n + 1)]
    qs = [dev_bf16(synth.q_rows(170 + j, Hq, Hkv, D, None)) for j in range(n + 1)]
    for c in caches:
        c.append(k0, v0)
        c.decode_step(ks[0], vs[0], qs[0], scale, sparse_v_tau=tau, dtype=torch.float32)
    eager, graphed = caches
    want = [eager.decode_step(ks[j], vs[j], qs[j], scale, sparse_v_tau=tau, dtype=torch.float32)
            for j in range(1, n + 1)]
    torch.cuda.synchronize()
    outs = [torch.empty((Hq, D), dtype=torch.float32, device="cuda") for _ in range(n)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for j in range(n):
            graphed.decode_step(ks[j + 1], vs[j + 1], qs[j + 1], scale, sparse_v_tau=tau,
                                out=outs[j], stream=s)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 16, device="cuda").sum()  # unrelated eager work
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        for j in range(n):
            assert torch.equal(outs[j], want[j]), f"replay {rep} step {j}"
