"""numpy/ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and
only as the checker (or as the timed CPU baseline). The product never imports
it. Each wrapper names the C function it calls; the C file cites the
reference lines each one restates.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None
_vp = ctypes.c_void_p


def build() -> Path:
    subprocess.run(["make", "-C", str(ORACLE_DIR), "-s"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        i32, i64, u64, f32, f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_double
        sig = {
            "ora_f32_to_f16": ([f32], ctypes.c_uint16),
            "ora_f16_to_f32": ([ctypes.c_uint16], f32),
            "ora_f32_to_bf16": ([f32], ctypes.c_uint16),
            "ora_bf16_to_f32": ([ctypes.c_uint16], f32),
            "ora_f32_to_f16_array": ([_vp, _vp, i64], None),
            "ora_f16_to_f32_array": ([_vp, _vp, i64], None),
            "ora_f32_to_bf16_array": ([_vp, _vp, i64], None),
            "ora_bf16_to_f32_array": ([_vp, _vp, i64], None),
            "ora_generate_hadamard": ([i32, _vp], None),
            "ora_deterministic_signs": ([i32, u64, _vp], None),
            "ora_build_rht": ([i32, u64, _vp, _vp], None),
            "ora_lloyd_max_codebook": ([i32, _vp, _vp], i32),
            "ora_turbo_round_trip_dense": ([_vp, i64, i32, i32, u64, _vp], None),
            "ora_turbo_round_trip_rt": ([_vp, i64, i32, i32, _vp, _vp, _vp], None),
            "ora_concat_rows": ([_vp, i64, _vp, i64, i64, _vp, i32], None),
            "ora_inv_sqrt": ([i32], f32),
            "ora_fwht": ([_vp, i32], None),
            "ora_rotate_rows": ([_vp, i64, i32, _vp, _vp], None),
            "ora_rotate_rows_f32": ([_vp, i64, i32, _vp, _vp], None),
            "ora_unrotate_rows_f64": ([_vp, i64, i32, _vp, _vp], None),
            "ora_rotate_rows_dense_f64": ([_vp, i64, i32, _vp, _vp], None),
            "ora_affine_quantize": ([_vp, i64, i32, i32, i32, _vp, _vp, _vp], None),
            "ora_affine_dequantize": ([_vp, _vp, _vp, i64, i32, i32, i32, _vp], None),
            "ora_codebook_quantize": ([_vp, i64, i32, i32, _vp, _vp, _vp], None),
            "ora_codebook_quantize_f32": ([_vp, i64, i32, i32, _vp, _vp, _vp], None),
            "ora_codebook_dequant_rotated": ([_vp, _vp, i64, i32, i32, _vp], None),
            "ora_codebook_round_trip": ([_vp, _vp, i64, i32, i32, _vp, _vp], None),
            "ora_rope_inv_freq": ([i32, i32, f32], f32),
            "ora_rope_cos_sin": ([i64, i32, i32, f32, ctypes.POINTER(f32), ctypes.POINTER(f32)], None),
            "ora_k_prologue": ([_vp, i32, _vp, f32, i64, i32, f32, _vp], None),
            "ora_v_prologue": ([_vp, i32, f32, _vp], None),
            "ora_kv_prologue": ([_vp, _vp, i64, i32, i32, i64, _vp, f32, i32, f32, _vp, _vp], None),
            "ora_ring_slot": ([i64, i64], i64),
            "ora_slot_position": ([i64, i64, i64], i64),
            "ora_causal_mask": ([i64, i64, _vp], None),
            "ora_sliding_mask": ([i64, i64, i64, _vp], None),
            "ora_paged_address": ([_vp, i64, i32], i64),
            "ora_attention_f64": ([_vp, _vp, _vp, _vp, i64, i32, i32, i32, f64, f64, _vp], None),
            "ora_lse_merge": ([_vp, _vp, _vp, i32, i32, _vp], None),
            "ora_sdpa_bf16_decode": ([_vp, _vp, _vp, i64, i32, i32, i32, f32, _vp, i32], None),
            "ora_splitmix64": ([ctypes.POINTER(u64)], u64),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_vp)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ----------------------------------------------------------------- conversions
def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().ora_f32_to_f16_array(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().ora_f16_to_f32_array(_p(h), _p(y), h.size)
    return y


def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().ora_f32_to_bf16_array(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().ora_bf16_to_f32_array(_p(h), _p(y), h.size)
    return y


# ------------------------------------------------- reference restatements
def hadamard(n: int) -> np.ndarray:
    h = np.empty((n, n), np.float32)
    lib().ora_generate_hadamard(n, _p(h))
    return h


def signs(n: int, seed: int = 42) -> np.ndarray:
    s = np.empty(n, np.float32)
    lib().ora_deterministic_signs(n, seed, _p(s))
    return s


def build_rht(dim: int, seed: int = 42):
    r = np.empty((dim, dim), np.float32)
    rt = np.empty((dim, dim), np.float32)
    lib().ora_build_rht(dim, seed, _p(r), _p(rt))
    return r, rt


def codebook(bits: int):
    c = np.zeros(16, np.float32)
    b = np.zeros(15, np.float32)
    n = lib().ora_lloyd_max_codebook(bits, _p(c), _p(b))
    if n == 0:
        raise ValueError(f"TurboQuant supports 2, 3, or 4 bits, got {bits}")
    return c[:n].copy(), b[: n - 1].copy()


def turbo_round_trip_dense(x_bf16, bits: int, seed: int = 42) -> np.ndarray:
    x = _c(x_bf16, np.uint16)
    d = x.shape[-1]
    out = np.empty(x.shape, np.uint16)
    lib().ora_turbo_round_trip_dense(_p(x), x.size // d, d, bits, seed, _p(out))
    return out


def turbo_round_trip_rt(x_bf16, bits: int, r, rt, out=None) -> np.ndarray:
    """turbo_round_trip_dense with R / Rt built once (rows in parallel)."""
    x = _c(x_bf16, np.uint16)
    d = x.shape[-1]
    out = np.empty(x.shape, np.uint16) if out is None else out
    lib().ora_turbo_round_trip_rt(_p(x), x.size // d, d, bits, _p(r), _p(rt), _p(out))
    return out


def concat_rows(old, t: int, new, out, n_threads: int = 0) -> np.ndarray:
    """out[:t + n] = concat(old[:t], new) along the first axis (the reference's
    per-append concatenate); rows are the trailing dims."""
    row = int(np.prod(new.shape[1:]))
    lib().ora_concat_rows(_p(old), t, _p(new), new.shape[0], row, _p(out), n_threads)
    return out


# ------------------------------------------------------- canonical rotation
def inv_sqrt(n: int) -> float:
    return lib().ora_inv_sqrt(n)


def fwht(x) -> np.ndarray:
    y = _c(x, np.float32).copy()
    lib().ora_fwht(_p(y), y.size)
    return y


def rotate_rows(x_bf16, sgn) -> np.ndarray:
    x = _c(x_bf16, np.uint16)
    d = x.shape[-1]
    y = np.empty(x.shape, np.float32)
    lib().ora_rotate_rows(_p(x), x.size // d, d, _p(_c(sgn, np.float32)), _p(y))
    return y


def rotate_rows_f32(x, sgn) -> np.ndarray:
    x = _c(x, np.float32)
    d = x.shape[-1]
    y = np.empty(x.shape, np.float32)
    lib().ora_rotate_rows_f32(_p(x), x.size // d, d, _p(_c(sgn, np.float32)), _p(y))
    return y


def kv_prologue(k_bf16, v_bf16, pos0: int, w_bf16, eps: float, rope_dims: int, theta: float):
    """K = RoPE(k_norm(k)) (bf16) and V = v_norm(v) (f32) of rows [n, h, d]
    at positions pos0.. (src/model/gemma4_attention.rs:52-81, norm.rs:5-29);
    v_bf16 None: V from the raw K (K==V layers)."""
    k = _c(k_bf16, np.uint16)
    n, h, d = k.shape
    v = None if v_bf16 is None else _c(v_bf16, np.uint16)
    ko = np.empty(k.shape, np.uint16)
    vo = np.empty(k.shape, np.float32)
    lib().ora_kv_prologue(_p(k), None if v is None else _p(v), n, h, d, pos0, _p(_c(w_bf16, np.uint16)),
                          eps, rope_dims, theta, _p(ko), _p(vo))
    return ko, vo


def unrotate_rows_f64(y, sgn) -> np.ndarray:
    y = _c(y, np.float64)
    d = y.shape[-1]
    x = np.empty(y.shape, np.float64)
    lib().ora_unrotate_rows_f64(_p(y), y.size // d, d, _p(_c(sgn, np.float32)), _p(x))
    return x


def rotate_rows_dense_f64(x, r) -> np.ndarray:
    x = _c(x, np.float32)
    d = x.shape[-1]
    y = np.empty(x.shape, np.float64)
    lib().ora_rotate_rows_dense_f64(_p(x), x.size // d, d, _p(_c(r, np.float32)), _p(y))
    return y


# --------------------------------------------------------- quantizers
def affine_quantize(y, bits: int, gs: int = 64):
    y = _c(y, np.float32)
    d = y.shape[-1]
    rows = y.size // d
    words = (d * bits + 31) // 32
    packed = np.empty(y.shape[:-1] + (words,), np.uint32)
    sc = np.empty(y.shape[:-1] + (d // gs,), np.uint16)
    bi = np.empty(y.shape[:-1] + (d // gs,), np.uint16)
    lib().ora_affine_quantize(_p(y), rows, d, bits, gs, _p(packed), _p(sc), _p(bi))
    return packed, sc, bi


def affine_dequantize(packed, scales, biases, d: int, bits: int, gs: int = 64) -> np.ndarray:
    packed = _c(packed, np.uint32)
    scales = _c(scales, np.uint16)
    biases = _c(biases, np.uint16)
    rows = scales.size // (d // gs)
    y = np.empty(scales.shape[:-1] + (d,), np.float64)
    lib().ora_affine_dequantize(_p(packed), _p(scales), _p(biases), rows, d, bits, gs, _p(y))
    return y


def codebook_quantize(x_bf16, bits: int, sgn):
    x = _c(x_bf16, np.uint16)
    d = x.shape[-1]
    rows = x.size // d
    words = (d * bits + 31) // 32
    packed = np.empty(x.shape[:-1] + (words,), np.uint32)
    norms = np.empty(x.shape[:-1], np.uint16)
    lib().ora_codebook_quantize(_p(x), rows, d, bits, _p(_c(sgn, np.float32)), _p(packed), _p(norms))
    return packed, norms


def codebook_quantize_f32(x, bits: int, sgn):
    """codebook_quantize of f32 rows (a V row after v_norm)."""
    x = _c(x, np.float32)
    d = x.shape[-1]
    rows = x.size // d
    words = (d * bits + 31) // 32
    packed = np.empty(x.shape[:-1] + (words,), np.uint32)
    norms = np.empty(x.shape[:-1], np.uint16)
    lib().ora_codebook_quantize_f32(_p(x), rows, d, bits, _p(_c(sgn, np.float32)), _p(packed),
                                    _p(norms))
    return packed, norms


def codebook_dequant_rotated(packed, norms, d: int, bits: int) -> np.ndarray:
    packed = _c(packed, np.uint32)
    norms = _c(norms, np.uint16)
    y = np.empty(norms.shape + (d,), np.float64)
    lib().ora_codebook_dequant_rotated(_p(packed), _p(norms), norms.size, d, bits, _p(y))
    return y


def codebook_round_trip(packed, norms, d: int, bits: int, sgn) -> np.ndarray:
    packed = _c(packed, np.uint32)
    norms = _c(norms, np.uint16)
    out = np.empty(norms.shape + (d,), np.uint16)
    lib().ora_codebook_round_trip(_p(packed), _p(norms), norms.size, d, bits,
                                  _p(_c(sgn, np.float32)), _p(out))
    return out


def unpack_codes(packed, d: int, bits: int) -> np.ndarray:
    """LE bit stream -> integer codes [..., d] (pure numpy; used by tests)."""
    packed = _c(packed, np.uint32)
    flat = packed.reshape(-1, packed.shape[-1]).astype(np.uint64)
    out = np.empty((flat.shape[0], d), np.int64)
    for j in range(d):
        bit = j * bits
        w, off = bit // 32, bit % 32
        v = flat[:, w] >> np.uint64(off)
        if off + bits > 32:
            v |= flat[:, w + 1] << np.uint64(32 - off)
        out[:, j] = (v & np.uint64((1 << bits) - 1)).astype(np.int64)
    return out.reshape(packed.shape[:-1] + (d,))


# ------------------------------------------------------ cache semantics
def ring_slot(pos: int, window: int) -> int:
    return lib().ora_ring_slot(pos, window)


def slot_position(slot: int, offset: int, window: int) -> int:
    return lib().ora_slot_position(slot, offset, window)


def causal_mask(offset: int, seq_len: int) -> np.ndarray:
    m = np.empty((seq_len, offset + seq_len), np.float32)
    lib().ora_causal_mask(offset, seq_len, _p(m))
    return m


def sliding_mask(stored: int, seq_len: int, window: int) -> np.ndarray:
    m = np.empty((seq_len, stored + seq_len), np.float32)
    lib().ora_sliding_mask(stored, seq_len, window, _p(m))
    return m


def paged_address(block_table, pos: int, block_size: int = 16) -> int:
    bt = _c(block_table, np.int32)
    return lib().ora_paged_address(_p(bt), pos, block_size)


# ---------------------------------------------------------------- attention
def attention_f64(q, k, v, valid=None, scale: float = 1.0, tau: float = 0.0) -> np.ndarray:
    q = _c(q, np.float64)
    k = _c(k, np.float64)
    v = _c(v, np.float64)
    hq, d = q.shape
    t, hkv = k.shape[0], k.shape[1]
    out = np.empty((hq, d), np.float64)
    vm = None if valid is None else _c(valid, np.uint8)
    lib().ora_attention_f64(_p(q), _p(k), _p(v), None if vm is None else _p(vm), t, hq, hkv, d,
                            scale, tau, _p(out))
    return out


def lse_merge(m, l, o) -> np.ndarray:
    m = _c(m, np.float64)
    l = _c(l, np.float64)
    o = _c(o, np.float64)
    out = np.empty(o.shape[-1], np.float64)
    lib().ora_lse_merge(_p(m), _p(l), _p(o), m.size, o.shape[-1], _p(out))
    return out


def sdpa_bf16_decode(q, k, v, scale: float = 1.0, n_threads: int = 0) -> np.ndarray:
    q = _c(q, np.uint16)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    hq, d = q.shape
    t, hkv = k.shape[0], k.shape[1]
    out = np.empty((hq, d), np.uint16)
    lib().ora_sdpa_bf16_decode(_p(q), _p(k), _p(v), t, hq, hkv, d, scale, _p(out), n_threads)
    return out


# ------------------------------------------------------------- cache model
class OracleCache:
    """CPU model of one quantized cache: canonical codes per slot, the
    reference's offset / window semantics (src/cache.rs:166-310)."""

    def __init__(self, n_kv_heads: int, head_dim: int, bits: int, window: int = 0,
                 capacity: int = 0, mode: int = 0, seed: int = 42):
        self.H, self.D, self.bits, self.W, self.mode = n_kv_heads, head_dim, bits, window, mode
        # a ring stores position p at slot p mod Ws, Ws the window rounded up
        # to whole 16-token blocks (the device layout); the last W positions
        # are the visible ones
        self.Ws = (window + 15) // 16 * 16 if window > 0 else 0
        self.n_slots = self.Ws if window > 0 else capacity
        self.sgn = signs(head_dim, seed)
        self.words = (head_dim * bits + 31) // 32
        self.n_meta = 2 * (head_dim // 64) if mode == 0 else (1 if mode == 1 else 0)
        self.codes = np.zeros((self.n_slots, 2, self.H, self.words), np.uint32)
        self.meta = np.zeros((self.n_slots, 2, self.H, self.n_meta), np.uint16)
        self.offset = 0
        self.vis_begin = 0

    def quantize_rows(self, x_bf16):
        """[..., D] bf16 rows -> (packed, meta [..., n_meta]). Plain mode
        (mode 2, src/cache.rs:274-288) stores the rows as given: the bf16 bits,
        dim 2w in the low half of word w, and no meta."""
        if self.mode == 2:
            x = np.ascontiguousarray(np.asarray(x_bf16, np.uint16))
            return x.view(np.uint32).copy(), np.zeros(x.shape[:-1] + (0,), np.uint16)
        if self.mode == 0:
            y = rotate_rows(x_bf16, self.sgn)
            packed, sc, bi = affine_quantize(y, self.bits)
            meta = np.empty(sc.shape[:-1] + (2 * sc.shape[-1],), np.uint16)
            meta[..., 0::2] = sc
            meta[..., 1::2] = bi
            return packed, meta
        packed, norms = codebook_quantize(x_bf16, self.bits, self.sgn)
        return packed, norms[..., None]

    def quantize_rows_f32(self, x):
        """[..., D] f32 rows (a V row after v_norm) -> (packed, meta): affine
        and codebook modes quantize the f32 values; a plain cache stores them
        rounded to bf16 (RNE)."""
        if self.mode == 2:
            return self.quantize_rows(f32_to_bf16(x))
        if self.mode == 1:
            packed, norms = codebook_quantize_f32(x, self.bits, self.sgn)
            return packed, norms[..., None]
        y = rotate_rows_f32(x, self.sgn)
        packed, sc, bi = affine_quantize(y, self.bits)
        meta = np.empty(sc.shape[:-1] + (2 * sc.shape[-1],), np.uint16)
        meta[..., 0::2] = sc
        meta[..., 1::2] = bi
        return packed, meta

    def append(self, k_bf16, v_bf16) -> None:
        k_bf16 = np.asarray(k_bf16)
        kp, km = self.quantize_rows(k_bf16)
        vp, vm = self.quantize_rows(np.asarray(v_bf16))
        self._store(kp, km, vp, vm)

    def append_projected(self, k_bf16, v_bf16, w_bf16, eps: float, rope_dims: int,
                         theta: float) -> None:
        """append() of raw k_proj / v_proj rows through the layer's prologue
        (kv_prologue at the cache offset); v_bf16 None: a K==V layer. K
        leaves the prologue in bf16 and is stored as any K row; V leaves it in
        f32 (quantize_rows_f32)."""
        k, v = kv_prologue(k_bf16, v_bf16, self.offset, w_bf16, eps, rope_dims, theta)
        kp, km = self.quantize_rows(k)
        vp, vm = self.quantize_rows_f32(v)
        self._store(kp, km, vp, vm)

    def _store(self, kp, km, vp, vm) -> None:
        n = kp.shape[0]
        if self.W == 0 and self.offset + n > self.n_slots:
            raise ValueError("capacity exceeded")
        first = 0 if self.W == 0 else max(0, n - self.Ws)
        for i in range(first, n):
            s = ring_slot(self.offset + i, self.Ws)
            self.codes[s, 0], self.meta[s, 0] = kp[i], km[i]
            self.codes[s, 1], self.meta[s, 1] = vp[i], vm[i]
        self.offset += n

    def _plain_rows(self, packed) -> np.ndarray:
        """f64 values of stored plain rows (packed bf16 words)."""
        u = np.ascontiguousarray(packed).view(np.uint16)
        return bf16_to_f32(u).astype(np.float64)

    def _dequant_rows(self, packed, meta) -> np.ndarray:
        """Un-rotated f64 rows of quantized rows (packed, meta)."""
        if self.mode == 2:
            return self._plain_rows(packed)
        if self.mode == 0:
            y = affine_dequantize(packed, np.ascontiguousarray(meta[..., 0::2]),
                                  np.ascontiguousarray(meta[..., 1::2]), self.D, self.bits)
        else:
            y = codebook_dequant_rotated(packed, np.ascontiguousarray(meta[..., 0]), self.D, self.bits)
        return unrotate_rows_f64(y, self.sgn)

    def prefill(self, k_bf16, v_bf16, q_bf16, scale: float = 1.0, rows=None) -> np.ndarray:
        """update_and_fetch of an L-token chunk, then the chunk's attention
        (src/model/gemma4_attention.rs:84-104 with L > 1) under the mask of
        src/model/mod.rs:682-753: query position p = offset + i sees the
        visible keys j <= p, and on a ring of W slots only j > p - W. The keys
        are the positions visible before the chunk plus the chunk's own
        quantized rows (update_and_fetch returns both before trimming,
        src/cache.rs:266-310). Returns [L, Hq, D] f64, or with `rows` (chunk
        indices) only those queries' outputs, [len(rows), Hq, D]."""
        k_bf16, v_bf16 = np.asarray(k_bf16), np.asarray(v_bf16)
        n = k_bf16.shape[0]
        p0 = self.offset
        old_pos = self.visible_positions()
        ko, vo = self.dequant_kv(old_pos)
        kp, km = self.quantize_rows(k_bf16)
        vp, vm = self.quantize_rows(v_bf16)
        kn, vn = self._dequant_rows(kp, km), self._dequant_rows(vp, vm)
        self._store(kp, km, vp, vm)
        pos = np.concatenate([old_pos, np.arange(p0, p0 + n)])
        kk, vv = np.concatenate([ko, kn]), np.concatenate([vo, vn])
        q = bf16_to_f32(q_bf16).astype(np.float64)
        sel = list(range(n)) if rows is None else [int(i) for i in rows]
        out = np.empty((len(sel),) + q.shape[1:], np.float64)
        for o, i in enumerate(sel):
            p = p0 + i
            lo = self.vis_begin if self.W == 0 else max(self.vis_begin, p - self.W + 1)
            valid = ((pos >= lo) & (pos <= p)).astype(np.uint8)
            out[o] = attention_f64(q[i], kk, vv, valid, scale)
        return out

    def trim(self, keep_last: int) -> None:
        self.vis_begin = max(self.vis_begin, self.offset - keep_last)

    def visible_positions(self) -> np.ndarray:
        lo = self.vis_begin
        if self.W > 0:
            lo = max(lo, self.offset - self.W)
        return np.arange(max(lo, 0), self.offset)

    def stored_len(self) -> int:
        return len(self.visible_positions())

    def slots_of(self, pos: np.ndarray) -> np.ndarray:
        return pos % self.Ws if self.W > 0 else pos

    def rotated_kv(self, positions=None):
        """Dequantized rotated-domain K, V (f64) [n, H, D] for positions
        (quantized modes)."""
        if self.mode == 2:
            raise ValueError("a plain cache has no rotated domain")
        pos = self.visible_positions() if positions is None else np.asarray(positions)
        sl = self.slots_of(pos)
        out = []
        for kv in (0, 1):
            c = self.codes[sl, kv]
            m = self.meta[sl, kv]
            if self.mode == 0:
                y = affine_dequantize(c, np.ascontiguousarray(m[..., 0::2]),
                                      np.ascontiguousarray(m[..., 1::2]), self.D, self.bits)
            else:
                y = codebook_dequant_rotated(c, np.ascontiguousarray(m[..., 0]), self.D, self.bits)
            out.append(y)
        return out[0], out[1]

    def dequant_kv(self, positions=None):
        """Dequantized, un-rotated K, V (f64) [n, H, D] in chronological order
        (plain mode: the stored bf16 values)."""
        if self.mode == 2:
            pos = self.visible_positions() if positions is None else np.asarray(positions)
            sl = self.slots_of(pos)
            return self._plain_rows(self.codes[sl, 0]), self._plain_rows(self.codes[sl, 1])
        yk, yv = self.rotated_kv(positions)
        return unrotate_rows_f64(yk, self.sgn), unrotate_rows_f64(yv, self.sgn)

    def attention(self, q_bf16, scale: float = 1.0, tau: float = 0.0) -> np.ndarray:
        k, v = self.dequant_kv()
        q = bf16_to_f32(q_bf16).astype(np.float64)
        if k.shape[0] == 0:
            return np.zeros(q.shape)
        return attention_f64(q, k, v, None, scale, tau)

    def attention_weights(self, q_bf16, scale: float = 1.0) -> np.ndarray:
        """Exact softmax weights [Hq, T] over the visible positions (the
        `weights` of src/model/gemma4_attention.rs:224 before the tau gate)."""
        k, _ = self.dequant_kv()
        q = bf16_to_f32(q_bf16).astype(np.float64)
        hq, hkv = q.shape[0], k.shape[1]
        rep = hq // hkv
        s = np.empty((hq, k.shape[0]))
        for h in range(hkv):  # one GQA group at a time: [rep, D] x [D, T]
            s[h * rep:(h + 1) * rep] = q[h * rep:(h + 1) * rep] @ np.ascontiguousarray(k[:, h]).T
        s *= scale
        s -= s.max(axis=1, keepdims=True)
        w = np.exp(s)
        return w / w.sum(axis=1, keepdims=True)
