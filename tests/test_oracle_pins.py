"""Pins of the CPU oracle (no GPU).

The reference ships no tests or golden vectors for its KV path, so every
oracle function is pinned here by something outside its own formula: known
answers copied from src/cache.rs, closed forms (Sylvester entries, Lloyd-Max
conditional means), invariants (orthogonality, involution), brute force on
tiny inputs, and independent numpy restatements in IEEE single precision.
"""
import math

import numpy as np
import pytest
from scipy.special import erf, logsumexp

import synth


# --------------------------------------------------------------------------
# scalar conversions
# --------------------------------------------------------------------------
def test_f16_conversion_matches_numpy(ora):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1e-7, -1e-7, np.inf, -np.inf],
                 dtype=np.float32),
    ]).astype(np.float32)
    got = ora.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = ora.f16_to_f32(want)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch(ora):
    import torch

    rng = np.random.default_rng(2)
    x = (rng.standard_normal(50000) * 10.0 ** rng.integers(-30, 30, 50000)).astype(np.float32)
    got = ora.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(synth.f32_to_bf16_bits(x), want)


# --------------------------------------------------------------------------
# src/cache.rs:6-62 -- Hadamard, LCG signs, RHT
# --------------------------------------------------------------------------
@pytest.mark.parametrize("n", [2, 8, 64, 256, 512])
def test_hadamard_closed_form(ora, n):
    h = ora.hadamard(n)
    i = np.arange(n)
    pop = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    want = np.where(pop % 2 == 0, 1.0, -1.0) * np.float32(1.0 / math.sqrt(n))
    assert np.array_equal(h, want.astype(np.float32))
    assert np.allclose(h.astype(np.float64) @ h.T.astype(np.float64), np.eye(n), atol=1e-6)


def test_signs_known_answer(ora):
    # first 32 signs for seed 42 (SplitMix-free MMIX LCG of src/cache.rs:29-43)
    s = ora.signs(512, 42)
    text = "".join("+" if v > 0 else "-" for v in s[:32])
    assert text == "-++--++++++--+-+-++-+++++--++---"
    assert int(s[:256].sum()) == -20
    assert int(s.sum()) == -24
    # independent big-integer evaluation of the LCG
    st, ref = 42, []
    for _ in range(512):
        st = (st * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        ref.append(1.0 if (st >> 63) == 0 else -1.0)
    assert np.array_equal(s, np.array(ref, np.float32))


@pytest.mark.parametrize("d", [128, 256, 512])
def test_rht_orthogonal_and_transpose(ora, d):
    r, rt = ora.build_rht(d, 42)
    assert np.array_equal(rt, r.T)
    assert np.allclose(r.astype(np.float64) @ rt.astype(np.float64), np.eye(d), atol=1e-6)


# --------------------------------------------------------------------------
# src/cache.rs:67-89 -- Lloyd-Max tables
# --------------------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_lloyd_max_tables_are_lloyd_max(ora, bits):
    c, b = ora.codebook(bits)
    assert len(c) == 1 << bits and len(b) == (1 << bits) - 1
    assert np.allclose(c, -c[::-1]) and np.allclose(b, -b[::-1])
    # boundaries are midpoints of neighbouring centroids (nearest-neighbour rule)
    assert np.max(np.abs(b - (c[:-1] + c[1:]) / 2)) <= 1.5e-3
    # centroids are N(0,1) conditional means of their cells (centroid rule)
    edges = np.concatenate([[-np.inf], b.astype(np.float64), [np.inf]])
    phi = lambda x: np.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)
    Phi = lambda x: 0.5 * (1 + erf(x / math.sqrt(2)))
    cm = (phi(edges[:-1]) - phi(edges[1:])) / (Phi(edges[1:]) - Phi(edges[:-1]))
    assert np.max(np.abs(cm - c)) <= 6e-3


def test_codebook_rejects_other_bits(ora):
    with pytest.raises(ValueError):
        ora.codebook(5)


# --------------------------------------------------------------------------
# canonical FWHT rotation vs the reference's dense x.R
# --------------------------------------------------------------------------
def np_fwht_f32(x):
    """Independent numpy FWHT in the canonical stage order (f32 per op)."""
    y = np.array(x, dtype=np.float32).copy()
    n = y.shape[-1]
    h = 1
    while h < n:
        y = y.reshape(y.shape[:-1] + (n // (2 * h), 2, h))
        a, b = y[..., 0, :].copy(), y[..., 1, :].copy()
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        y = y.reshape(y.shape[:-3] + (n,))
        h *= 2
    return y


@pytest.mark.parametrize("d", [128, 256, 512])
def test_fwht_matches_dense_and_numpy(ora, d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal(d).astype(np.float32)
    got = ora.fwht(x)
    assert np.array_equal(got, np_fwht_f32(x))
    h = ora.hadamard(d).astype(np.float64) * math.sqrt(d)
    assert np.allclose(got, x.astype(np.float64) @ h, rtol=0, atol=1e-4 * math.sqrt(d))
    # one-hot rows map to Hadamard rows exactly; FWHT twice is d * identity
    e = np.zeros(d, np.float32)
    e[d // 3] = 1.0
    assert np.array_equal(ora.fwht(e), np.round(h[d // 3]).astype(np.float32))
    assert np.allclose(ora.fwht(ora.fwht(x)), d * x, atol=1e-3)


@pytest.mark.parametrize("d", [256, 512])
def test_rotate_rows_is_x_times_r(ora, d):
    rng = np.random.default_rng(7 + d)
    xb = synth.f32_to_bf16_bits(rng.standard_normal((8, d)).astype(np.float32) * 3)
    s = ora.signs(d, 42)
    y = ora.rotate_rows(xb, s)
    r, _ = ora.build_rht(d, 42)
    x = ora.bf16_to_f32(xb).astype(np.float64)
    assert np.allclose(y, x @ r.astype(np.float64), atol=2e-5 * np.abs(x).max() * math.sqrt(d))
    # canonical order, restated with numpy f32 ops
    c = np.float32(1.0) / np.sqrt(np.float32(d))
    want = (np_fwht_f32(ora.bf16_to_f32(xb)) * c) * s
    assert np.array_equal(y, want.astype(np.float32))
    # inverse rotation (f64) recovers x
    assert np.allclose(ora.unrotate_rows_f64(y.astype(np.float64), s), x, atol=1e-4)


# --------------------------------------------------------------------------
# MLX affine quantizer (A16)
# --------------------------------------------------------------------------
def np_affine(y, bits):
    """numpy f32 restatement of MLX affine_quantize for groups of 64."""
    y = np.asarray(y, np.float32).reshape(-1, 64)
    nb = np.float32((1 << bits) - 1)
    mx, mn = y.max(1), y.min(1)
    scale = np.maximum((mx - mn) / nb, np.float32(1e-7))
    side = np.abs(mn) > np.abs(mx)
    scale = np.where(side, scale, -scale).astype(np.float32)
    edge = np.where(side, mn, mx).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nz = q0 != 0
    scale = np.where(nz, edge / np.where(nz, q0, 1), scale).astype(np.float32)
    bias = np.where(nz, edge, 0).astype(np.float32)
    q = np.clip(np.rint((y - bias[:, None]) / scale[:, None]), 0, nb).astype(np.int64)
    return q, scale, bias


def test_affine_known_answers(ora):
    # 4-bit, values 0..15 (+ pad with 0..15 repeated): scale -1, bias 15, code 15 - w
    w = np.tile(np.arange(16, dtype=np.float32), 4)
    p, sc, bi = ora.affine_quantize(w[None, :], 4)
    codes = ora.unpack_codes(p, 64, 4)[0]
    assert np.array_equal(codes, 15 - w.astype(np.int64))
    assert ora.f16_to_f32(sc)[0, 0] == -1.0 and ora.f16_to_f32(bi)[0, 0] == 15.0
    # 4-bit, values -8..7: scale 1, bias -8, code w + 8
    w = np.tile(np.arange(-8, 8, dtype=np.float32), 4)
    p, sc, bi = ora.affine_quantize(w[None, :], 4)
    assert np.array_equal(ora.unpack_codes(p, 64, 4)[0], (w + 8).astype(np.int64))
    # half-way cases round to even: (2.5-15)/-1 = 12.5 -> 12 ; (3.5-15)/-1 = 11.5 -> 12
    w = np.zeros(64, np.float32)
    w[1], w[2], w[3] = 15.0, 2.5, 3.5
    codes = ora.unpack_codes(ora.affine_quantize(w[None, :], 4)[0], 64, 4)[0]
    assert codes[2] == 12 and codes[3] == 12 and codes[1] == 0 and codes[0] == 15
    # constant group -> code 0, bias = the constant
    w = np.full(64, 3.0, np.float32)
    p, sc, bi = ora.affine_quantize(w[None, :], 8)
    assert not ora.unpack_codes(p, 64, 8).any() and ora.f16_to_f32(bi)[0, 0] == 3.0
    # packing: element k of a word at bits [4k, 4k+4)
    w = np.tile(np.arange(-8, 8, dtype=np.float32), 4)
    p, _, _ = ora.affine_quantize(w[None, :], 4)  # -8..7 -> code k at element k
    assert p[0, 0] == 0x76543210 and p[0, 1] == 0xFEDCBA98
    p, _, _ = ora.affine_quantize(np.tile(np.arange(-128, 128, 4, dtype=np.float32), 1)[None, :], 8)
    # 8-bit, -128..124 step 4: q0 = rint(-128 / (252/255)) = -130, scale = 128/130,
    # code_k = rint(4k * 130/128) = 0, 4, 8, 12 -> byte k of the word is element k
    assert p[0, 0] == 0x0C080400


@pytest.mark.parametrize("bits", [4, 8])
def test_affine_matches_numpy_and_error_bound(ora, bits):
    rng = np.random.default_rng(bits)
    y = (rng.standard_normal((300, 256)) * rng.uniform(0.01, 30, (300, 1))).astype(np.float32)
    y[5] = 0.0
    y[6, :64] = -2.0
    p, sc, bi = ora.affine_quantize(y, bits)
    codes = ora.unpack_codes(p, 256, bits).reshape(-1, 64)
    q, scale, bias = np_affine(y, bits)
    assert np.array_equal(codes, q)
    assert np.array_equal(sc.reshape(-1), scale.astype(np.float16).view(np.uint16))
    assert np.array_equal(bi.reshape(-1), bias.astype(np.float16).view(np.uint16))
    assert codes.min() >= 0 and codes.max() <= (1 << bits) - 1
    # unclipped codes: |dequant - w| <= |scale|/2 (+ f16 storage of scale and
    # bias). MLX's edge rule (scale = edge / q0) can shrink |scale| so the far
    # end of the range clips; those codes sit at 0 or n_bins.
    yg = y.reshape(-1, 64).astype(np.float64)
    raw = np.rint((y.reshape(-1, 64) - bias[:, None]) / scale[:, None])
    clipped = (raw < 0) | (raw > (1 << bits) - 1)
    assert np.all(np.isin(codes[clipped], [0, (1 << bits) - 1]))
    deq = ora.affine_dequantize(p, sc, bi, 256, bits).reshape(-1, 64)
    s16 = ora.f16_to_f32(sc).reshape(-1).astype(np.float64)
    b16 = ora.f16_to_f32(bi).reshape(-1).astype(np.float64)
    bound = (np.abs(scale) / 2 + q.max(1) * np.abs(s16 - scale) + np.abs(b16 - bias)) * (1 + 1e-6) + 1e-12
    ok = np.abs(deq - yg) <= bound[:, None]
    assert np.all(ok | clipped)
    assert clipped.mean() < 0.02


# --------------------------------------------------------------------------
# TurboQuant round trip (A7), dense reference order and canonical order
# --------------------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_turbo_round_trip_known_answers(ora, bits):
    d = 256
    c, _ = ora.codebook(bits)
    x = np.zeros((3, d), np.float32)
    x[1, 17] = 1.0  # one-hot: z = +-1 in every coordinate -> +-centroid for +-1
    x[2, 200] = -4.0
    xb = synth.f32_to_bf16_bits(x)
    out = ora.bf16_to_f32(ora.turbo_round_trip_dense(xb, bits))
    assert not out[0].any()  # zero row: norm 0, output 0
    top = c[np.searchsorted(ora.codebook(bits)[1], 1.0 - 1e-6, side="right")]
    want1 = np.zeros(d)
    want1[17] = top
    want2 = np.zeros(d)
    want2[200] = -4.0 * top
    assert np.allclose(out[1], want1, atol=2e-2 * top)
    assert np.allclose(out[2], want2, atol=8e-2 * top)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [256, 512])
def test_codebook_canonical_vs_dense_reference(ora, bits, d):
    rng = np.random.default_rng(bits * d)
    x = rng.standard_normal((64, d)).astype(np.float32)
    x[:, :4] *= 20
    xb = synth.f32_to_bf16_bits(x)
    s = ora.signs(d, 42)
    packed, norms = ora.codebook_quantize(xb, bits, s)
    # indices vs exact math: bins of (x/|x|).R.sqrt(d) computed in f64
    xf = ora.bf16_to_f32(xb).astype(np.float64)
    r, _ = ora.build_rht(d, 42)
    z = (xf / np.linalg.norm(xf, axis=1, keepdims=True)) @ r.astype(np.float64) * math.sqrt(d)
    idx_exact = np.searchsorted(ora.codebook(bits)[1].astype(np.float64), z, side="right")
    idx = ora.unpack_codes(packed, d, bits)
    assert np.mean(idx != idx_exact) < 1e-3
    assert np.allclose(ora.f16_to_f32(norms), np.linalg.norm(xf, axis=1), rtol=1e-3)
    # canonical round trip stays close to the reference-order dense round trip
    rt = ora.bf16_to_f32(ora.codebook_round_trip(packed, norms, d, bits, s))
    dense = ora.bf16_to_f32(ora.turbo_round_trip_dense(xb, bits))
    err = np.abs(rt - dense)
    assert np.mean(err) <= 2e-3 * np.abs(dense).mean() + 1e-3


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [256, 512])
def test_codebook_quantize_f32_rows(ora, bits, d):
    """ora_codebook_quantize_f32 (f32 rows: V after v_norm) bins exactly as
    ora_codebook_quantize on bf16-representable rows, and on general f32 rows
    follows the exact binning of (x/|x|) . R . sqrt(d) (src/cache.rs:104-118,
    f64) up to boundary flips of the f32 rounding."""
    rng = np.random.default_rng(7 * bits + d)
    x = rng.standard_normal((64, d)).astype(np.float32)
    x /= np.sqrt(np.mean(x * x, axis=1, keepdims=True))
    x[:, 3] *= 20
    s = ora.signs(d, 42)
    xb = synth.f32_to_bf16_bits(x)
    pb, nb = ora.codebook_quantize(xb, bits, s)
    pf, nf = ora.codebook_quantize_f32(ora.bf16_to_f32(xb), bits, s)
    assert np.array_equal(pb, pf) and np.array_equal(nb, nf)
    packed, norms = ora.codebook_quantize_f32(x, bits, s)
    r, _ = ora.build_rht(d, 42)
    xf = x.astype(np.float64)
    z = (xf / np.linalg.norm(xf, axis=1, keepdims=True)) @ r.astype(np.float64) * math.sqrt(d)
    idx_exact = np.searchsorted(ora.codebook(bits)[1].astype(np.float64), z, side="right")
    assert np.mean(ora.unpack_codes(packed, d, bits) != idx_exact) < 1e-3
    assert np.array_equal(norms, ora.f32_to_f16(np.sqrt(np.sum(xf * xf, axis=1)).astype(np.float32))) or \
        np.allclose(ora.f16_to_f32(norms), np.linalg.norm(xf, axis=1), rtol=1e-3)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [128, 256, 512])
def test_codebook_dequant_rotated_is_reference_dequant(ora, bits, d):
    """ora_codebook_dequant_rotated (the rotated-domain row every codebook
    attention check reads) composed with the f64 inverse rotation equals the
    reference's dequantization written as src/cache.rs:119-125 does it:
    (centroid[idx] / sqrt(d)) . R^T . norm, with the dense R^T of
    build_rht (src/cache.rs:47-62) in f64 -- to 1e-12. The canonical f32
    round trip from the same codes (ora_codebook_round_trip) lies within one
    bf16 rounding of it. A row whose indices are all one value k is
    centroid[k] * norm / sqrt(d) in every coordinate."""
    rng = np.random.default_rng(100 * bits + d)
    x = (rng.standard_normal((24, d)) * rng.uniform(0.1, 30, (24, 1))).astype(np.float32)
    x[:, :4] *= 20
    x[3] = 0.0
    xb = synth.f32_to_bf16_bits(x)
    s = ora.signs(d, 42)
    packed, norms = ora.codebook_quantize(xb, bits, s)
    y = ora.codebook_dequant_rotated(packed, norms, d, bits)
    got = ora.unrotate_rows_f64(y, s)
    # the reference order, dense and in f64, from the same stored codes
    c, _ = ora.codebook(bits)
    idx = ora.unpack_codes(packed, d, bits)
    _, rt = ora.build_rht(d, 42)
    nrm = ora.f16_to_f32(norms).astype(np.float64)
    inv = np.float64(np.float32(1.0) / np.sqrt(np.float32(d)))
    want = ((c.astype(np.float64)[idx] * inv) @ rt.astype(np.float64)) * nrm[:, None]
    assert np.allclose(got, want, rtol=0, atol=1e-12 * max(1.0, np.abs(want).max()))
    assert not got[3].any()  # zero row: norm 0
    # canonical f32 round trip (bf16 output) from the same codes
    rt_bf16 = ora.bf16_to_f32(ora.codebook_round_trip(packed, norms, d, bits, s)).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    assert np.all(np.abs(rt_bf16 - want) <= ulp * 1.01 + 1e-6 * nrm[:, None])
    # constant indices: every rotated coordinate is centroid[k] * norm / sqrt(d)
    for k in (0, (1 << bits) - 1, 1 << (bits - 1)):
        row = np.zeros((1, packed.shape[1]), np.uint32)
        for j in range(d):
            bit = j * bits
            row[0, bit // 32] |= np.uint32((k << (bit % 32)) & 0xFFFFFFFF)
            if bit % 32 + bits > 32:
                row[0, bit // 32 + 1] |= np.uint32(k >> (32 - bit % 32))
        n16 = ora.f32_to_f16(np.array([2.5], np.float32))
        yk = ora.codebook_dequant_rotated(row, n16, d, bits)
        assert np.all(yk == np.float64(c[k]) * inv * 2.5)


@pytest.mark.parametrize("d", [128, 256, 512])
def test_rotate_rows_f32_is_x_times_r(ora, d):
    """ora_rotate_rows_f32 (the rotation of f32 rows -- v_norm output -- behind
    every projected-V code) is x . R (src/cache.rs:47-62, 109-112) within f32
    FWHT rounding of the dense f64 product, bit-identical to rotate_rows on
    bf16-representable rows and to the canonical order restated in numpy,
    and maps the one-hot row e_k to (-1)^popcount(k & j) * c * s_j exactly."""
    rng = np.random.default_rng(3 * d)
    x = rng.standard_normal((16, d)).astype(np.float32)
    x /= np.sqrt(np.mean(x * x, axis=1, keepdims=True))  # unit RMS, as v_norm leaves a row
    x[:, 5] *= 20
    s = ora.signs(d, 42)
    r, _ = ora.build_rht(d, 42)
    y = ora.rotate_rows_f32(x, s)
    dense = ora.rotate_rows_dense_f64(x, r)
    assert np.allclose(y, dense, rtol=0, atol=4 * math.log2(d) * 2.0 ** -24 * np.abs(x).sum(1).max())
    c = np.float32(1.0) / np.sqrt(np.float32(d))
    assert np.array_equal(y, ((np_fwht_f32(x) * c) * s).astype(np.float32))
    xb = synth.f32_to_bf16_bits(x)
    assert np.array_equal(ora.rotate_rows_f32(ora.bf16_to_f32(xb), s), ora.rotate_rows(xb, s))
    for k in (0, 1, d // 2 + 3, d - 1):
        e = np.zeros((1, d), np.float32)
        e[0, k] = 1.0
        j = np.arange(d)
        par = np.vectorize(lambda v: bin(v).count("1") & 1)(k & j)
        want = np.where(par == 0, c, -c).astype(np.float32) * s
        assert np.array_equal(ora.rotate_rows_f32(e, s)[0], want)


@pytest.mark.parametrize("W", [5, 40, 100])
def test_ring_of_any_window_is_concat_then_tail(ora, W):
    """A window that is not a multiple of 16: the ring holds Ws = W rounded up
    to whole 16-token blocks, position p at slot p mod Ws, so after any
    sequence of chunks it holds the last Ws positions, and the visible ones
    are exactly the last W -- the rows concat-then-tail keeps
    (src/cache.rs:132-148) -- in chronological order."""
    rng = np.random.default_rng(W)
    D, H = 128, 2
    c = ora.OracleCache(H, D, 16, W, 0, mode=2)
    assert c.n_slots == c.Ws == (W + 15) // 16 * 16
    rows = []
    for n in (3, W + 17, 1, 2 * W + 5, 7):
        k = synth.f32_to_bf16_bits(rng.standard_normal((n, H, D)).astype(np.float32))
        v = synth.f32_to_bf16_bits(rng.standard_normal((n, H, D)).astype(np.float32))
        c.append(k, v)
        rows += list(zip(k, v))
        T = len(rows)
        assert list(c.visible_positions()) == list(range(max(0, T - W), T))
        for p in range(max(0, T - c.Ws), T):  # every slot holds its latest position
            assert np.array_equal(c.codes[p % c.Ws, 0].view(np.uint16), rows[p][0])
            assert np.array_equal(c.codes[p % c.Ws, 1].view(np.uint16), rows[p][1])
        kf, vf = c.dequant_kv()
        tail = rows[-W:]
        assert np.array_equal(kf, ora.bf16_to_f32(np.stack([r[0] for r in tail])).astype(np.float64))
        assert np.array_equal(vf, ora.bf16_to_f32(np.stack([r[1] for r in tail])).astype(np.float64))


# --------------------------------------------------------------------------
# cache index semantics (A8, A9, A14)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("window", [4, 16, 48])
def test_ring_equals_concat_then_tail(ora, window):
    """Brute force: the reference keeps tail_along_time(concat(...), W); a ring
    that overwrites slot p % W holds exactly those positions."""
    stored = []  # positions, chronological (reference model)
    rng = np.random.default_rng(window)
    offset = 0
    for _ in range(40):
        n = int(rng.integers(1, 2 * window))
        stored = (stored + list(range(offset, offset + n)))[-window:]
        offset += n
        held = sorted(p for p in (ora.slot_position(s, offset, window) for s in range(window)) if p >= 0)
        assert held == stored
        assert all(ora.ring_slot(p, window) == p % window for p in stored)


def test_sliding_mask_decode_sees_last_w(ora):
    W = 8
    for stored in range(0, 3 * W):
        st = min(stored, W)
        m = ora.sliding_mask(st, 1, W)
        vis = np.flatnonzero(m[0] == 0)
        # columns are [stored cache ..., current]; visible = last min(st+1, W)
        assert list(vis) == list(range(st + 1 - min(st + 1, W), st + 1))
    # prefill rows: causal band
    m = ora.sliding_mask(3, 5, 4)
    for i in range(5):
        row = 3 + i
        want = [j for j in range(8) if j <= row and row - j < 4]
        assert list(np.flatnonzero(m[i] == 0)) == want
    cm = ora.causal_mask(2, 3)
    assert [list(np.flatnonzero(r == 0)) for r in cm] == [[0, 1, 2], [0, 1, 2, 3], [0, 1, 2, 3, 4]]


def test_paged_address(ora):
    table = np.array([7, 2, 9], np.int32)
    assert [ora.paged_address(table, p, 16) for p in (0, 15, 16, 40)] == [112, 127, 32, 152]


# --------------------------------------------------------------------------
# attention (A12, A13) and the split merge (A17)
# --------------------------------------------------------------------------
def np_attention(q, k, v, scale=1.0, tau=0.0):
    hq, d = q.shape
    hkv = k.shape[1]
    rep = hq // hkv
    out = np.zeros((hq, d))
    for h in range(hq):
        s = k[:, h // rep] @ q[h] * scale
        w = np.exp(s - logsumexp(s))
        if tau > 0:
            w = np.where(w >= tau, w, 0)
        out[h] = w @ v[:, h // rep]
    return out


def test_attention_special_cases(ora):
    rng = np.random.default_rng(3)
    d = 64
    q = rng.standard_normal((4, d))
    v = rng.standard_normal((1, 2, d))
    k = rng.standard_normal((1, 2, d))
    assert np.allclose(ora.attention_f64(q, k, v), v[0][[0, 0, 1, 1]])  # T = 1 -> v
    k = np.repeat(rng.standard_normal((1, 2, d)), 9, axis=0)
    v = rng.standard_normal((9, 2, d))
    assert np.allclose(ora.attention_f64(q, k, v), v.mean(0)[[0, 0, 1, 1]])  # equal keys -> mean
    valid = np.zeros(9, np.uint8)
    valid[4] = 1
    assert np.allclose(ora.attention_f64(q, k, v, valid), v[4][[0, 0, 1, 1]])


@pytest.mark.parametrize("tau", [0.0, 1e-3, 5e-2])
def test_attention_matches_numpy(ora, tau):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((8, 32)) * 0.5
    k = rng.standard_normal((50, 2, 32))
    v = rng.standard_normal((50, 2, 32))
    assert np.allclose(ora.attention_f64(q, k, v, None, 0.7, tau), np_attention(q, k, v, 0.7, tau),
                       atol=1e-12)


def test_cache_attention_weights_agree_with_attention(ora):
    """OracleCache.attention_weights (used to size the sparse-V tests) gives the
    weights that OracleCache.attention applies: rows sum to 1, w @ V is the
    dense result and (w * [w >= tau]) @ V the gated one."""
    H, D, hq = 2, 128, 4
    oc = ora.OracleCache(H, D, 4, 0, 80)
    rng = np.random.default_rng(11)
    kv = [synth.f32_to_bf16_bits(rng.standard_normal((70, H, D)).astype(np.float32)) for _ in range(2)]
    oc.append(kv[0], kv[1])
    q = synth.f32_to_bf16_bits(rng.standard_normal((hq, D)).astype(np.float32))
    w = oc.attention_weights(q, 0.2)
    assert w.shape == (hq, 70) and np.allclose(w.sum(axis=1), 1.0, atol=1e-12)
    _, v = oc.dequant_kv()
    vh = np.repeat(v, hq // H, axis=1)  # [t, hq, d]
    assert np.allclose(np.einsum("ht,thd->hd", w, vh), oc.attention(q, 0.2), atol=1e-10)
    tau = np.median(w)
    wg = np.where(w >= tau, w, 0.0)
    assert np.allclose(np.einsum("ht,thd->hd", wg, vh), oc.attention(q, 0.2, tau), atol=1e-10)


def test_lse_merge_equals_full_softmax(ora):
    rng = np.random.default_rng(5)
    s = rng.standard_normal(40) * 5
    v = rng.standard_normal((40, 16))
    parts = np.split(np.arange(40), [7, 20, 21])
    m = np.array([s[p].max() for p in parts])
    l = np.array([np.exp(s[p] - s[p].max()).sum() for p in parts])
    o = np.stack([np.exp(s[p] - s[p].max()) @ v[p] for p in parts])
    w = np.exp(s - logsumexp(s))
    assert np.allclose(ora.lse_merge(m, l, o), w @ v, atol=1e-12)


def test_sdpa_bf16_baseline_close_to_exact(ora):
    rng = np.random.default_rng(6)
    q = synth.f32_to_bf16_bits(rng.standard_normal((4, 64)).astype(np.float32) * 0.2)
    k = synth.f32_to_bf16_bits(rng.standard_normal((100, 2, 64)).astype(np.float32))
    v = synth.f32_to_bf16_bits(rng.standard_normal((100, 2, 64)).astype(np.float32))
    got = ora.bf16_to_f32(ora.sdpa_bf16_decode(q, k, v, 1.0, 2))
    want = ora.attention_f64(ora.bf16_to_f32(q), ora.bf16_to_f32(k), ora.bf16_to_f32(v))
    assert np.max(np.abs(got - want)) < 2e-2


def test_sdpa_bf16_baseline_same_bits_on_any_thread_count(ora):
    """The CPU baseline splits scores, sums and output slices over threads;
    every element keeps its serial summation order, so the bits cannot
    depend on the thread count (head_dim 96 also covers a partial slice)."""
    rng = np.random.default_rng(16)
    q = synth.f32_to_bf16_bits(rng.standard_normal((6, 96)).astype(np.float32) * 0.3)
    k = synth.f32_to_bf16_bits(rng.standard_normal((1000, 3, 96)).astype(np.float32))
    v = synth.f32_to_bf16_bits(rng.standard_normal((1000, 3, 96)).astype(np.float32))
    one = ora.sdpa_bf16_decode(q, k, v, 0.7, 1)
    for n in (2, 3, 8):
        assert np.array_equal(ora.sdpa_bf16_decode(q, k, v, 0.7, n), one)
    # the op order, restated in numpy for one head: bf16(q * scale), f32
    # products summed in key order, bf16 scores; the output of a constant-V
    # column is that constant whatever the weights
    v2 = v.copy()
    v2[:, 0, 5] = synth.f32_to_bf16_bits(np.float32([1.5]))[0]
    out = ora.bf16_to_f32(ora.sdpa_bf16_decode(q, k, v2, 0.7, 4))
    assert np.all(np.abs(out[:2, 5] - 1.5) <= 1.5 * 2.0 ** -7)


def test_reference_round_trip_with_prebuilt_rotation(ora):
    """turbo_round_trip_rt (R built once, rows in parallel) == the
    per-call form (src/cache.rs:94-129), bit for bit."""
    rng = np.random.default_rng(17)
    x = synth.f32_to_bf16_bits(rng.standard_normal((70, 128)).astype(np.float32))
    r, rt = ora.build_rht(128)
    for bits in (2, 3, 4):
        assert np.array_equal(ora.turbo_round_trip_rt(x, bits, r, rt),
                              ora.turbo_round_trip_dense(x, bits))


def test_concat_rows_is_concatenate(ora):
    rng = np.random.default_rng(18)
    old = rng.integers(0, 65535, (300000, 2, 3), dtype=np.uint16)
    new = rng.integers(0, 65535, (5, 2, 3), dtype=np.uint16)
    out = np.zeros((300005, 2, 3), np.uint16)
    for t in (0, 1, 299999):
        out[:] = 0
        ora.concat_rows(old, t, new, out, 4)
        assert np.array_equal(out[:t + 5], np.concatenate([old[:t], new]))


# --------------------------------------------------------------------------
# cache model: append with ring semantics, trim, stored_len
# --------------------------------------------------------------------------
def test_oracle_cache_ring_and_trim(ora):
    c = ora.OracleCache(2, 128, 4, window=32)
    rng = np.random.default_rng(9)
    total = 0
    for n in (5, 30, 1, 40, 16):
        k = synth.f32_to_bf16_bits(rng.standard_normal((n, 2, 128)).astype(np.float32))
        c.append(k, k)
        total += n
        assert c.offset == total and c.stored_len() == min(total, 32)
    c.trim(10)
    assert c.stored_len() == 10
    assert list(c.visible_positions()) == list(range(total - 10, total))
    k, v = c.dequant_kv()
    assert k.shape == (10, 2, 128) and np.allclose(k, v)


# ------------------------------------------------------------ layer prologue
def _bf16_rows(seed, shape, scale=1.0):
    rng = np.random.default_rng(seed)
    return synth.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("d,rope_dims,theta", [(256, 256, 10000.0), (512, 128, 1e6), (128, 32, 10000.0)])
def test_rope_is_the_textbook_rotation(ora, d, rope_dims, theta):
    """K at position p is the position-0 K (k_norm only: RoPE at 0 turns by 0)
    with each pair (i, i + rope_dims/2) turned by a = f32(p) * f32(theta^(-2i/
    rope_dims)), computed here in f64; dims past rope_dims are unchanged.
    Interleaved pairs, a flipped sign or another frequency law fail."""
    x = _bf16_rows(21, (d,))
    w = _bf16_rows(22, (d,), 0.3)
    k0 = np.empty(d, np.uint16)
    ora.lib().ora_k_prologue(ora._p(x), d, ora._p(w), 1e-6, 0, rope_dims, theta, ora._p(k0))
    y0 = ora.bf16_to_f32(k0).astype(np.float64)
    half = rope_dims // 2
    i = np.arange(half)
    f = (np.float64(theta) ** (-2.0 * i / rope_dims)).astype(np.float32)
    for p in (1, 7, 1000, 100003):
        kp = np.empty(d, np.uint16)
        ora.lib().ora_k_prologue(ora._p(x), d, ora._p(w), 1e-6, p, rope_dims, theta, ora._p(kp))
        got = ora.bf16_to_f32(kp).astype(np.float64)
        a = (np.float32(p) * f).astype(np.float64)
        x1, x2 = y0[:half], y0[half:rope_dims]
        want = np.concatenate([x1 * np.cos(a) - x2 * np.sin(a), x1 * np.sin(a) + x2 * np.cos(a),
                               y0[rope_dims:]])
        # one bf16 rounding of the result (2^-8 relative) on top of exact math
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-30), p
        assert np.array_equal(got[rope_dims:], y0[rope_dims:])


def test_k_norm_closed_forms(ora):
    """fast::rms_norm: a constant row c gives w * c / sqrt(c^2 + eps); a random
    row gives x * w / sqrt(mean(x^2) + eps) (one bf16 rounding)."""
    d = 256
    w = _bf16_rows(23, (d,))
    wf = ora.bf16_to_f32(w).astype(np.float64)
    for c, eps in ((0.75, 1e-6), (-3.0, 1e-2)):
        x = synth.f32_to_bf16_bits(np.full(d, c, np.float32))
        out = np.empty(d, np.uint16)
        ora.lib().ora_k_prologue(ora._p(x), d, ora._p(w), eps, 0, d, 10000.0, ora._p(out))
        want = wf * c / math.sqrt(c * c + eps)
        assert np.allclose(ora.bf16_to_f32(out), want, rtol=2.0 ** -8, atol=0)
    x = _bf16_rows(24, (d,), 2.0)
    xf = ora.bf16_to_f32(x).astype(np.float64)
    out = np.empty(d, np.uint16)
    ora.lib().ora_k_prologue(ora._p(x), d, ora._p(w), 1e-6, 0, d, 10000.0, ora._p(out))
    want = xf * wf / math.sqrt(np.mean(xf * xf) + 1e-6)
    assert np.allclose(ora.bf16_to_f32(out), want, rtol=2.0 ** -7, atol=1e-30)


def test_v_norm_closed_forms(ora):
    """RMSNormNoScale (norm.rs:16-29): x / sqrt(mean(bf16(x^2)) + eps) with the
    mean rounded to bf16; unit RMS for any row; a zero row stays zero."""
    d = 512
    x = _bf16_rows(25, (d,), 5.0)
    xf = ora.bf16_to_f32(x).astype(np.float64)
    out = np.empty(d, np.float32)
    ora.lib().ora_v_prologue(ora._p(x), d, 1e-6, ora._p(out))
    x2 = ora.bf16_to_f32(synth.f32_to_bf16_bits((xf * xf).astype(np.float32))).astype(np.float64)
    mean = float(ora.bf16_to_f32(synth.f32_to_bf16_bits(np.array([np.mean(x2)], np.float32)))[0])
    assert np.allclose(out, xf / math.sqrt(mean + 1e-6), rtol=1e-5, atol=0)
    assert abs(math.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-2
    z = np.zeros(d, np.uint16)
    ora.lib().ora_v_prologue(ora._p(z), d, 1e-6, ora._p(out))
    assert np.all(out == 0)


def test_kv_prologue_rows_and_k_eq_v(ora):
    """Rows [n, h, d] take position pos0 + token; with no v_proj the V rows are
    v_norm of the raw K rows (gemma4_attention.rs:54-59)."""
    n, h, d = 3, 2, 128
    k = _bf16_rows(26, (n, h, d))
    v = _bf16_rows(27, (n, h, d))
    w = _bf16_rows(28, (d,))
    ko, vo = ora.kv_prologue(k, v, 40, w, 1e-6, 64, 10000.0)
    ko2, vo2 = ora.kv_prologue(k, None, 40, w, 1e-6, 64, 10000.0)
    assert np.array_equal(ko, ko2)
    for t in range(n):
        for hh in range(h):
            one = np.empty(d, np.uint16)
            ora.lib().ora_k_prologue(ora._p(np.ascontiguousarray(k[t, hh])), d, ora._p(w), 1e-6,
                                     40 + t, 64, 10000.0, ora._p(one))
            assert np.array_equal(ko[t, hh], one)
            vv = np.empty(d, np.float32)
            ora.lib().ora_v_prologue(ora._p(np.ascontiguousarray(v[t, hh])), d, 1e-6, ora._p(vv))
            assert np.array_equal(vo[t, hh], vv)
            ora.lib().ora_v_prologue(ora._p(np.ascontiguousarray(k[t, hh])), d, 1e-6, ora._p(vv))
            assert np.array_equal(vo2[t, hh], vv)


@pytest.mark.parametrize("W,keep", [(0, 0), (0, 30), (32, 0), (48, 0)])
def test_prefill_equals_token_by_token_decode(ora, W, keep):
    """A chunk's prefill attention (src/model/gemma4_attention.rs:84-104 with
    L > 1, masks src/model/mod.rs:682-753) equals decoding its tokens one at
    a time: causal on linear caches; on a ring the band j > p - W is exactly
    the last W positions a ring holds at decode. A mask edge off by one, a
    ring read after the chunk overwrote its slots, a lost trim or a wrong
    position offset fails this; the stored codes are the same as well."""
    H, D, bits, Hq = 2, 128, 4, 4
    cap = 0 if W else 200
    a = ora.OracleCache(H, D, bits, W, cap)
    b = ora.OracleCache(H, D, bits, W, cap)
    k0, v0 = _bf16_rows(40, (37, H, D)), _bf16_rows(41, (37, H, D))
    for c in (a, b):
        c.append(k0, v0)
        if keep:
            c.trim(keep)
    L = 45
    k, v, q = _bf16_rows(42, (L, H, D)), _bf16_rows(43, (L, H, D)), _bf16_rows(44, (L, Hq, D))
    got = a.prefill(k, v, q, 0.7)
    for i in range(L):
        b.append(k[i:i + 1], v[i:i + 1])
        want = b.attention(q[i], 0.7)
        assert np.allclose(got[i], want, rtol=1e-10, atol=1e-12), i
    assert np.array_equal(a.codes, b.codes) and np.array_equal(a.meta, b.meta)
    assert a.offset == b.offset


# ------------------------------------------------------------ plain caches
def test_oracle_plain_cache_stores_rows_as_given(ora):
    """Plain mode (src/cache.rs:274-288: concatenate, then keep the last W on
    a ring): the stored words are the input bf16 bits, dequant_kv returns the
    rows in chronological order, and attention equals a numpy softmax over
    the visible rows."""
    rng = np.random.default_rng(12)
    D, H, W = 128, 2, 32
    c = ora.OracleCache(H, D, 16, W, 0, mode=2)
    rows = []
    for n in (5, 30, 1, 40):
        k = synth.f32_to_bf16_bits(rng.standard_normal((n, H, D)).astype(np.float32))
        v = synth.f32_to_bf16_bits(rng.standard_normal((n, H, D)).astype(np.float32))
        c.append(k, v)
        rows += list(zip(k, v))
    assert c.meta.shape[-1] == 0 and c.words == D // 2
    pos = c.visible_positions()
    assert list(pos) == list(range(76 - W, 76))
    k_all = np.stack([r[0] for r in rows])
    v_all = np.stack([r[1] for r in rows])
    slot = pos[0] % W
    assert np.array_equal(c.codes[slot, 0].view(np.uint16), k_all[pos[0]])
    kf, vf = c.dequant_kv()
    want_k = ora.bf16_to_f32(k_all[pos]).astype(np.float64)
    want_v = ora.bf16_to_f32(v_all[pos]).astype(np.float64)
    assert np.array_equal(kf, want_k) and np.array_equal(vf, want_v)
    q = synth.f32_to_bf16_bits(rng.standard_normal((4, D)).astype(np.float32))
    qf = ora.bf16_to_f32(q).astype(np.float64)
    assert np.allclose(c.attention(q, 0.1), np_attention(qf, want_k, want_v, 0.1, 0.0), atol=1e-12)
