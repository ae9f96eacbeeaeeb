"""Python host binding of the fmkv C ABI (include/fmkv.h).

Mirrors the reference's Rust cache API (src/cache.rs:186-310) so callers and
tests read like the reference:

    cache = KVCache.new_quantized_with_window(head_dim=256, bits=4, window=1024,
                                              n_kv_heads=8)
    cache.update_and_fetch(k, v)          # append (store half); returns a view
    out = cache.attention(q, scale=1.0)   # decode read (SDPA replacement)
    cache.offset(), cache.stored_len(), cache.peek_kv()

Device memory and streams come from PyTorch (plumbing only): tensors are
passed to the library as raw device pointers. The HIP library is required;
nothing here computes on the CPU, and loading fails loudly when libfmkv.so is
missing.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

import torch  # imported before libfmkv.so so both share torch's HIP runtime

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libfmkv.so"

FMKV_OK = 0
FMKV_ERR_INVALID_ARG = 1
FMKV_ERR_UNSUPPORTED = 2
FMKV_ERR_OOM = 3
FMKV_ERR_HIP = 4
FMKV_ERR_CAPACITY = 5
MODE_AFFINE = 0
MODE_CODEBOOK = 1
MODE_PLAIN = 2  # unquantized bf16 rows (bits 16): KVCacheInner::Plain, src/cache.rs:174-178
PLAIN_BITS = 16
DTYPE_BF16 = 0
DTYPE_F32 = 1
BLOCK_TOKENS = 16

EXPORTED = (
    "fmkv_last_error", "fmkv_validate_desc", "fmkv_layout_bytes", "fmkv_cache_create",
    "fmkv_cache_destroy", "fmkv_cache_offset", "fmkv_cache_stored_len", "fmkv_cache_append",
    "fmkv_cache_trim", "fmkv_decode_attention", "fmkv_cache_fetch", "fmkv_cache_read_codes",
    "fmkv_pool_create", "fmkv_pool_destroy", "fmkv_paged_append", "fmkv_paged_decode_attention",
    "fmkv_cache_append_projected", "fmkv_paged_append_projected",
    "fmkv_pool_read_codes", "fmkv_set_blocks_per_split", "fmkv_set_sparse_v_gather",
    "fmkv_cache_decode_splits",
    "fmkv_profile_enable", "fmkv_profile_collect", "fmkv_profile_collect_each",
    "fmkv_decode_step", "fmkv_paged_decode_step",
    "fmkv_prefill_step", "fmkv_paged_prefill_step", "fmkv_decode_step_noalloc",
    "fmkv_decode_step_projected", "fmkv_paged_decode_step_projected",
)


class Exception_(RuntimeError):
    """Error raised for a non-zero fmkv status (mirrors mlx_rs::error::Exception)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"fmkv error {code}: {msg}")
        self.code = code


class CacheDesc(ctypes.Structure):
    _fields_ = [
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("capacity", ctypes.c_int64),
        ("sign_seed", ctypes.c_uint64),
    ]


class KvPrologue(ctypes.Structure):
    """fmkv_kv_prologue: the layer's k_norm / v_norm / RoPE fused into the
    append (src/model/gemma4_attention.rs:52-81)."""
    _fields_ = [
        ("k_norm_weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("rope_dims", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
        ("v_from_k", ctypes.c_int32),
    ]


def make_prologue(k_norm_weight: torch.Tensor, eps: float, rope_dims: int, rope_theta: float,
                  v_from_k: bool = False) -> KvPrologue:
    """k_norm_weight: bf16 [head_dim] on the device. The struct holds a
    reference to the tensor, so the weight lives as long as the prologue
    (the C struct itself carries only the device address)."""
    if k_norm_weight.dtype != torch.bfloat16 or k_norm_weight.dim() != 1:
        raise ValueError("k_norm_weight must be bf16 [head_dim]")
    if not k_norm_weight.is_contiguous():
        raise ValueError("k_norm_weight must be contiguous")
    pro = KvPrologue(k_norm_weight.data_ptr(), eps, rope_dims, rope_theta, 1 if v_from_k else 0)
    pro.weight = k_norm_weight
    return pro


def _check_prologue_weight(prologue: KvPrologue, head_dim: int) -> None:
    w = getattr(prologue, "weight", None)
    if w is not None and w.numel() != head_dim:
        raise ValueError(f"k_norm_weight has {w.numel()} elements; head_dim is {head_dim}")


_lib = None


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libfmkv.so (built by build.py); raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} not found: build the HIP library first (python {PKG_DIR / 'build.py'})")
    lib = ctypes.CDLL(str(p))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    P = ctypes.POINTER
    sig = {
        "fmkv_last_error": ([], ctypes.c_char_p),
        "fmkv_validate_desc": ([P(CacheDesc)], ctypes.c_int),
        "fmkv_layout_bytes": ([P(CacheDesc), P(i64), P(i64)], ctypes.c_int),
        "fmkv_cache_create": ([P(CacheDesc), P(vp)], ctypes.c_int),
        "fmkv_cache_destroy": ([vp], ctypes.c_int),
        "fmkv_cache_offset": ([vp, P(i64)], ctypes.c_int),
        "fmkv_cache_stored_len": ([vp, P(i64)], ctypes.c_int),
        "fmkv_cache_append": ([vp, vp, vp, i64, vp], ctypes.c_int),
        "fmkv_cache_trim": ([vp, i64], ctypes.c_int),
        "fmkv_decode_attention": ([vp, vp, i32, ctypes.c_float, ctypes.c_float, vp, i32, vp], ctypes.c_int),
        "fmkv_cache_fetch": ([vp, vp, vp, i32, vp], ctypes.c_int),
        "fmkv_cache_read_codes": ([vp, vp, vp, vp], ctypes.c_int),
        "fmkv_pool_create": ([P(CacheDesc), i64, P(vp)], ctypes.c_int),
        "fmkv_pool_destroy": ([vp], ctypes.c_int),
        "fmkv_paged_append": ([vp, vp, vp, vp, i32, vp, i32, i32, vp], ctypes.c_int),
        "fmkv_cache_append_projected": ([vp, vp, vp, i64, P(KvPrologue), vp], ctypes.c_int),
        "fmkv_paged_append_projected": ([vp, vp, vp, vp, i32, vp, i32, i32, P(KvPrologue), vp],
                                        ctypes.c_int),
        "fmkv_paged_decode_attention": ([vp, vp, vp, i32, vp, i32, i32, i32, ctypes.c_float,
                                         ctypes.c_float, vp, i32, vp], ctypes.c_int),
        "fmkv_pool_read_codes": ([vp, vp, vp, vp], ctypes.c_int),
        "fmkv_set_blocks_per_split": ([i32], ctypes.c_int),
        "fmkv_set_sparse_v_gather": ([i32], ctypes.c_int),
        "fmkv_cache_decode_splits": ([vp, P(i32)], ctypes.c_int),
        "fmkv_profile_enable": ([i32], ctypes.c_int),
        "fmkv_profile_collect": ([P(ctypes.c_double), P(i32)], ctypes.c_int),
        "fmkv_profile_collect_each": ([P(ctypes.c_float), i32, P(i32)], ctypes.c_int),
        "fmkv_decode_step": ([vp, vp, vp, i64, vp, i32, ctypes.c_float, ctypes.c_float, vp, i32,
                              vp], ctypes.c_int),
        "fmkv_decode_step_noalloc": ([vp, vp, vp, i64, vp, i32, ctypes.c_float, ctypes.c_float, vp,
                                      i32, vp], ctypes.c_int),
        "fmkv_prefill_step": ([vp, vp, vp, i64, vp, i32, ctypes.c_float, vp, i32, vp], ctypes.c_int),
        "fmkv_paged_prefill_step": ([vp, vp, vp, vp, i32, vp, i32, i32, vp, i32, ctypes.c_float, vp,
                                     i32, vp], ctypes.c_int),
        "fmkv_paged_decode_step": ([vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, vp, i32,
                                    ctypes.c_float, ctypes.c_float, vp, i32, vp], ctypes.c_int),
        "fmkv_decode_step_projected": ([vp, vp, vp, i64, P(KvPrologue), vp, i32, ctypes.c_float,
                                        ctypes.c_float, vp, i32, vp], ctypes.c_int),
        "fmkv_paged_decode_step_projected": ([vp, vp, vp, vp, i32, vp, vp, i32, i32, i32,
                                              P(KvPrologue), vp, i32, ctypes.c_float,
                                              ctypes.c_float, vp, i32, vp], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != FMKV_OK:
        raise Exception_(rc, load_library().fmkv_last_error().decode())


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("fmkv needs device tensors")
    if not t.is_contiguous():
        raise ValueError("fmkv needs contiguous tensors")
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def make_desc(n_kv_heads: int, head_dim: int, bits: int, window: int = 0, capacity: int = 0,
              mode: int = MODE_AFFINE, group_size: int = 64, sign_seed: int = 42) -> CacheDesc:
    return CacheDesc(n_kv_heads, head_dim, bits, group_size, mode, window, capacity, sign_seed)


def validate(desc: CacheDesc) -> None:
    _check(load_library().fmkv_validate_desc(ctypes.byref(desc)))


def layout_bytes(desc: CacheDesc) -> tuple[int, int]:
    b, a = ctypes.c_int64(), ctypes.c_int64()
    _check(load_library().fmkv_layout_bytes(ctypes.byref(desc), ctypes.byref(b), ctypes.byref(a)))
    return b.value, a.value


def set_blocks_per_split(bps: int) -> None:
    """Blocks per split-K work-group for decode attention (0: the plan's);
    a paged sequence's first split takes 4 x bps blocks when the grid holds
    at least four work-groups per CU."""
    _check(load_library().fmkv_set_blocks_per_split(bps))


def set_sparse_v_gather(on: bool) -> None:
    """Sparse-V after its statistics pass: the gather of the kept V rows
    (True, the default) or the gated pass and the split merge (False)."""
    _check(load_library().fmkv_set_sparse_v_gather(1 if on else 0))


def profile_enable(max_records: int) -> None:
    """Record HIP events around the next max_records split-K kernels."""
    _check(load_library().fmkv_profile_enable(max_records))


def profile_collect() -> tuple[float, int]:
    """(summed kernel milliseconds, launches timed) since the last collect."""
    ms, n = ctypes.c_double(), ctypes.c_int32()
    _check(load_library().fmkv_profile_collect(ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def profile_collect_each(capacity: int) -> list[float]:
    """Kernel milliseconds of each launch timed since the last collect."""
    buf, n = (ctypes.c_float * max(capacity, 1))(), ctypes.c_int32()
    _check(load_library().fmkv_profile_collect_each(buf, capacity, ctypes.byref(n)))
    return [buf[i] for i in range(n.value)]


class KVCache:
    """KV cache of one attention layer (src/cache.rs:166-172): quantized
    (affine or codebook) or plain bf16."""

    def __init__(self, desc: CacheDesc):
        self.desc = desc
        self._lib = load_library()
        h = ctypes.c_void_p()
        _check(self._lib.fmkv_cache_create(ctypes.byref(desc), ctypes.byref(h)))
        self._h = h

    # --- constructors mirroring src/cache.rs:202-227 --------------------------
    @classmethod
    def new_quantized_with_window(cls, head_dim: int, bits: int, window: int | None,
                                  n_kv_heads: int, capacity: int = 0,
                                  mode: int = MODE_AFFINE, sign_seed: int = 42) -> "KVCache":
        return cls(make_desc(n_kv_heads, head_dim, bits, window or 0, capacity, mode,
                             sign_seed=sign_seed))

    @classmethod
    def new_quantized(cls, head_dim: int, bits: int, n_kv_heads: int, capacity: int,
                      mode: int = MODE_AFFINE) -> "KVCache":
        return cls.new_quantized_with_window(head_dim, bits, None, n_kv_heads, capacity, mode)

    @classmethod
    def new_with_window(cls, head_dim: int, window: int | None, n_kv_heads: int,
                        capacity: int = 0) -> "KVCache":
        """The plain bf16 cache (KVCache::new_with_window, src/cache.rs:191-199)."""
        return cls(make_desc(n_kv_heads, head_dim, PLAIN_BITS, window or 0, capacity, MODE_PLAIN))

    @classmethod
    def new(cls, head_dim: int, n_kv_heads: int, capacity: int) -> "KVCache":
        """KVCache::new (src/cache.rs:187-189): plain, no window."""
        return cls.new_with_window(head_dim, None, n_kv_heads, capacity)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.fmkv_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- state (src/cache.rs:229-242) ------------------------------------------
    def offset(self) -> int:
        v = ctypes.c_int64()
        _check(self._lib.fmkv_cache_offset(self._h, ctypes.byref(v)))
        return v.value

    def stored_len(self) -> int:
        v = ctypes.c_int64()
        _check(self._lib.fmkv_cache_stored_len(self._h, ctypes.byref(v)))
        return v.value

    # --- append / fetch (src/cache.rs:247-310) ---------------------------------
    def append(self, keys: torch.Tensor, values: torch.Tensor, stream=None) -> None:
        """keys/values: bf16 [n_tokens, n_kv_heads, head_dim] on the device."""
        self._check_kv(keys, values)
        _check(self._lib.fmkv_cache_append(self._h, _ptr(keys), _ptr(values), keys.shape[0],
                                           _stream(stream)))

    def append_projected(self, keys: torch.Tensor, values: torch.Tensor | None,
                         prologue: KvPrologue, stream=None) -> None:
        """append() of raw k_proj / v_proj rows through the layer's prologue
        (k_norm + RoPE on K, v_norm on V; values None with prologue.v_from_k)."""
        if values is None:
            values = keys
        self._check_kv(keys, values)
        _check_prologue_weight(prologue, self.desc.head_dim)
        _check(self._lib.fmkv_cache_append_projected(self._h, _ptr(keys), _ptr(values),
                                                     keys.shape[0], ctypes.byref(prologue),
                                                     _stream(stream)))

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor, stream=None,
                         fetch: bool = False):
        """Store new positions; with fetch=True also return the visible
        dequantized K/V like the reference's return value."""
        self.append(keys, values, stream)
        return self.peek_kv(stream=stream) if fetch else None

    def peek_kv(self, dtype=torch.bfloat16, stream=None):
        n = self.stored_len()
        if n == 0:
            return None
        shape = (n, self.desc.n_kv_heads, self.desc.head_dim)
        k = torch.empty(shape, dtype=dtype, device="cuda")
        v = torch.empty(shape, dtype=dtype, device="cuda")
        _check(self._lib.fmkv_cache_fetch(self._h, _ptr(k), _ptr(v), _dtype_code(dtype),
                                          _stream(stream)))
        return k, v

    def trim(self, keep_last: int) -> None:
        _check(self._lib.fmkv_cache_trim(self._h, keep_last))

    # --- attention read (src/model/gemma4_attention.rs:94-103) -----------------
    def attention(self, q: torch.Tensor, scale: float = 1.0, sparse_v_tau: float = 0.0,
                  out: torch.Tensor | None = None, dtype=torch.bfloat16, stream=None) -> torch.Tensor:
        """q: bf16 [n_q_heads, head_dim] -> out [n_q_heads, head_dim]."""
        if q.dtype != torch.bfloat16 or q.dim() != 2 or q.shape[1] != self.desc.head_dim:
            raise ValueError("q must be bf16 [n_q_heads, head_dim]")
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_decode_attention(self._h, _ptr(q), q.shape[0], scale, sparse_v_tau,
                                               _ptr(out), _dtype_code(out.dtype), _stream(stream)))
        return out

    def decode_step(self, keys: torch.Tensor, values: torch.Tensor, q: torch.Tensor,
                    scale: float = 1.0, sparse_v_tau: float = 0.0, out: torch.Tensor | None = None,
                    dtype=torch.bfloat16, stream=None) -> torch.Tensor:
        """update_and_fetch(keys, values) then attention(q) in one call
        (src/model/gemma4_attention.rs:84-103); shapes as append / attention."""
        self._check_kv(keys, values)
        if q.dtype != torch.bfloat16 or q.dim() != 2 or q.shape[1] != self.desc.head_dim:
            raise ValueError("q must be bf16 [n_q_heads, head_dim]")
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_decode_step(self._h, _ptr(keys), _ptr(values), keys.shape[0],
                                          _ptr(q), q.shape[0], scale, sparse_v_tau, _ptr(out),
                                          _dtype_code(out.dtype), _stream(stream)))
        return out

    def decode_step_projected(self, keys: torch.Tensor, values: torch.Tensor | None,
                              prologue: KvPrologue, q: torch.Tensor, scale: float = 1.0,
                              sparse_v_tau: float = 0.0, out: torch.Tensor | None = None,
                              dtype=torch.bfloat16, stream=None) -> torch.Tensor:
        """decode_step() of raw k_proj / v_proj rows through the layer's
        prologue (src/model/gemma4_attention.rs:50-104 after the projections;
        values None with prologue.v_from_k)."""
        if values is None:
            values = keys
        self._check_kv(keys, values)
        _check_prologue_weight(prologue, self.desc.head_dim)
        if q.dtype != torch.bfloat16 or q.dim() != 2 or q.shape[1] != self.desc.head_dim:
            raise ValueError("q must be bf16 [n_q_heads, head_dim]")
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_decode_step_projected(
            self._h, _ptr(keys), _ptr(values), keys.shape[0], ctypes.byref(prologue), _ptr(q),
            q.shape[0], scale, sparse_v_tau, _ptr(out), _dtype_code(out.dtype), _stream(stream)))
        return out

    def prefill_step(self, keys: torch.Tensor, values: torch.Tensor, q: torch.Tensor,
                     scale: float = 1.0, out: torch.Tensor | None = None, dtype=torch.bfloat16,
                     stream=None) -> torch.Tensor:
        """update_and_fetch of an L-token chunk and the chunk's causal (sliding:
        banded) attention (src/model/gemma4_attention.rs:84-104 with L > 1,
        masks src/model/mod.rs:682-753). keys/values bf16 [L, n_kv_heads, D];
        q bf16 [L, n_q_heads, D]; returns [L, n_q_heads, D]."""
        self._check_kv(keys, values)
        if (q.dtype != torch.bfloat16 or q.dim() != 3 or q.shape[0] != keys.shape[0]
                or q.shape[2] != self.desc.head_dim):
            raise ValueError("q must be bf16 [n_tokens, n_q_heads, head_dim]")
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_prefill_step(self._h, _ptr(keys), _ptr(values), keys.shape[0],
                                           _ptr(q), q.shape[1], scale, _ptr(out),
                                           _dtype_code(out.dtype), _stream(stream)))
        return out

    def decode_splits(self) -> int:
        v = ctypes.c_int32()
        _check(self._lib.fmkv_cache_decode_splits(self._h, ctypes.byref(v)))
        return v.value

    # --- raw contents for bit-exact checks -------------------------------------
    def n_slots(self) -> int:
        """Stored slots: a ring's window rounded up to whole 16-token blocks,
        or a linear cache's capacity."""
        w = self.desc.window
        return (w + 15) // 16 * 16 if w > 0 else self.desc.capacity

    def read_codes(self, stream=None):
        """(codes uint32 [n_slots, 2, H, words], meta uint16 [n_slots, 2, H, n_meta])."""
        return _read_codes(self._lib.fmkv_cache_read_codes, self._h, self.desc, self.n_slots(), stream)

    def _check_kv(self, keys, values):
        d = self.desc
        for t in (keys, values):
            if t.dtype != torch.bfloat16 or t.dim() != 3 or t.shape[1:] != (d.n_kv_heads, d.head_dim):
                raise ValueError(f"K/V must be bf16 [n, {d.n_kv_heads}, {d.head_dim}], got "
                                 f"{tuple(t.shape)} {t.dtype}")
        if keys.shape != values.shape:
            raise ValueError("keys and values differ in shape")


@dataclass(frozen=True)
class LayerCacheSpec:
    """One layer's cache shape as Model::make_cache derives it
    (src/model/mod.rs:375-396 with the per-layer dims of :448-465)."""
    is_full: bool     # layer_types[i] == "full_attention"
    use_k_eq_v: bool  # attention_k_eq_v && is_full
    head_dim: int     # global_head_dim on full layers, else head_dim
    n_kv_heads: int   # num_global_key_value_heads on K==V layers
    window: int       # sliding_window on layers that are not K==V, else 0
    bits: int


def layer_cache_specs(layer_types, head_dim: int, n_kv_heads: int, *,
                      global_head_dim: int | None = None, n_global_kv_heads: int | None = None,
                      sliding_window: int | None = None, attention_k_eq_v: bool = False,
                      kv_quant_bits: int = 3, global_kv_quant_bits: int | None = None):
    """Per-layer cache shapes of a Gemma-4 stack, the choices of
    Model::make_cache (src/model/mod.rs:375-396) and the layer constructor
    (:448-465): a layer is full iff its type is "full_attention"; K==V
    layers are the full ones when attention_k_eq_v; only layers that are
    not K==V get the sliding window (so with attention_k_eq_v false every
    layer does, as in the reference); full layers use global_head_dim
    (default head_dim); K==V layers use n_global_kv_heads (default
    n_kv_heads). kv_quant_bits applies to every layer unless
    global_kv_quant_bits overrides it on full layers (a mixed 4/8-bit
    stack)."""
    specs = []
    for t in layer_types:
        is_full = t == "full_attention"
        k_eq_v = bool(attention_k_eq_v and is_full)
        specs.append(LayerCacheSpec(
            is_full, k_eq_v,
            (global_head_dim or head_dim) if is_full else head_dim,
            (n_global_kv_heads or n_kv_heads) if k_eq_v else n_kv_heads,
            0 if k_eq_v or not sliding_window else int(sliding_window),
            global_kv_quant_bits if (is_full and global_kv_quant_bits) else kv_quant_bits))
    return specs


def make_cache(layer_types, head_dim: int, n_kv_heads: int, *, capacity: int,
               global_head_dim: int | None = None, n_global_kv_heads: int | None = None,
               sliding_window: int | None = None, attention_k_eq_v: bool = False,
               kv_quant_bits: int | None = 3, global_kv_quant_bits: int | None = None,
               mode: int = MODE_CODEBOOK, sign_seed: int = 42) -> list:
    """One cache per layer, as Model::make_cache (src/model/mod.rs:375-396)
    builds them with KVCache::new_quantized_with_window(layer.kv_head_dim(),
    bits, window). The reference's quantized cache is the TurboQuant
    codebook (default 3 bits, src/main.rs:82-84), hence mode's default;
    MODE_AFFINE gives the 4/8-bit affine caches. `capacity` bounds the
    positions of the linear (window 0) caches, whose arenas are
    preallocated. kv_quant_bits None gives the reference's plain bf16
    caches (KVCache::new_with_window, --no-kv-quant) on every layer."""
    plain = kv_quant_bits is None
    specs = layer_cache_specs(layer_types, head_dim, n_kv_heads, global_head_dim=global_head_dim,
                              n_global_kv_heads=n_global_kv_heads, sliding_window=sliding_window,
                              attention_k_eq_v=attention_k_eq_v,
                              kv_quant_bits=PLAIN_BITS if plain else kv_quant_bits,
                              global_kv_quant_bits=None if plain else global_kv_quant_bits)
    caches = []
    for sp in specs:
        if plain:
            c = KVCache.new_with_window(sp.head_dim, sp.window or None, sp.n_kv_heads,
                                        capacity=0 if sp.window else capacity)
        else:
            c = KVCache.new_quantized_with_window(sp.head_dim, sp.bits, sp.window or None,
                                                  sp.n_kv_heads, capacity=0 if sp.window else capacity,
                                                  mode=mode, sign_seed=sign_seed)
        c.spec = sp
        caches.append(c)
    return caches


class PagedPool:
    """Pool of 16-token blocks shared by many sequences (batched decode)."""

    def __init__(self, desc: CacheDesc, n_blocks: int):
        self.desc = desc
        self.n_blocks = n_blocks
        self._lib = load_library()
        h = ctypes.c_void_p()
        _check(self._lib.fmkv_pool_create(ctypes.byref(desc), n_blocks, ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.fmkv_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def append(self, keys, values, block_tables, start_pos, stream=None) -> None:
        """keys/values bf16 [n_seqs, n_new, H, D]; block_tables int32 [n_seqs, max_blocks];
        start_pos int32 [n_seqs]."""
        n_seqs, n_new = keys.shape[0], keys.shape[1]
        _check(self._lib.fmkv_paged_append(self._h, _ptr(keys), _ptr(values), _ptr(block_tables),
                                           block_tables.shape[1], _ptr(start_pos), n_seqs, n_new,
                                           _stream(stream)))

    def append_projected(self, keys, values, block_tables, start_pos, prologue: KvPrologue,
                         stream=None) -> None:
        """append() of raw projections through the layer's prologue."""
        if values is None:
            values = keys
        n_seqs, n_new = keys.shape[0], keys.shape[1]
        _check_prologue_weight(prologue, self.desc.head_dim)
        _check(self._lib.fmkv_paged_append_projected(
            self._h, _ptr(keys), _ptr(values), _ptr(block_tables), block_tables.shape[1],
            _ptr(start_pos), n_seqs, n_new, ctypes.byref(prologue), _stream(stream)))

    def prefill_step(self, keys, values, block_tables, start_pos, q, scale: float = 1.0,
                     out=None, dtype=torch.bfloat16, stream=None):
        """append(keys, values, ...) at start_pos, then each sequence's causal
        attention of its n_new queries. keys/values bf16 [n_seqs, n_new,
        n_kv_heads, D]; q bf16 [n_seqs, n_new, n_q_heads, D]."""
        if q.dim() != 4 or q.shape[:2] != keys.shape[:2]:
            raise ValueError("q must be bf16 [n_seqs, n_new, n_q_heads, head_dim]")
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_paged_prefill_step(
            self._h, _ptr(keys), _ptr(values), _ptr(block_tables), block_tables.shape[1],
            _ptr(start_pos), keys.shape[0], keys.shape[1], _ptr(q), q.shape[2], scale, _ptr(out),
            _dtype_code(out.dtype), _stream(stream)))
        return out

    def attention(self, q, block_tables, seq_lens, max_seq_len: int, scale: float = 1.0,
                  sparse_v_tau: float = 0.0, out=None, dtype=torch.bfloat16, stream=None):
        """q bf16 [n_seqs, n_q_heads, D]; seq_lens int32 [n_seqs]."""
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_paged_decode_attention(
            self._h, _ptr(q), _ptr(block_tables), block_tables.shape[1], _ptr(seq_lens),
            q.shape[0], max_seq_len, q.shape[1], scale, sparse_v_tau, _ptr(out),
            _dtype_code(out.dtype), _stream(stream)))
        return out

    def decode_step(self, keys, values, block_tables, start_pos, seq_lens, max_seq_len: int, q,
                    scale: float = 1.0, sparse_v_tau: float = 0.0, out=None, dtype=torch.bfloat16,
                    stream=None):
        """append(keys, values, ...) at start_pos, then attention over seq_lens
        (= start_pos + n_new) in one call."""
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_paged_decode_step(
            self._h, _ptr(keys), _ptr(values), _ptr(block_tables), block_tables.shape[1],
            _ptr(start_pos), _ptr(seq_lens), keys.shape[0], keys.shape[1], max_seq_len, _ptr(q),
            q.shape[1], scale, sparse_v_tau, _ptr(out), _dtype_code(out.dtype), _stream(stream)))
        return out

    def decode_step_projected(self, keys, values, block_tables, start_pos, seq_lens,
                              max_seq_len: int, prologue: KvPrologue, q, scale: float = 1.0,
                              sparse_v_tau: float = 0.0, out=None, dtype=torch.bfloat16,
                              stream=None):
        """decode_step() of raw projections through the layer's prologue
        (RoPE positions from start_pos; values None with prologue.v_from_k)."""
        if values is None:
            values = keys
        _check_prologue_weight(prologue, self.desc.head_dim)
        if out is None:
            out = torch.empty(q.shape, dtype=dtype, device=q.device)
        _check(self._lib.fmkv_paged_decode_step_projected(
            self._h, _ptr(keys), _ptr(values), _ptr(block_tables), block_tables.shape[1],
            _ptr(start_pos), _ptr(seq_lens), keys.shape[0], keys.shape[1], max_seq_len,
            ctypes.byref(prologue), _ptr(q), q.shape[1], scale, sparse_v_tau, _ptr(out),
            _dtype_code(out.dtype), _stream(stream)))
        return out

    def read_codes(self, stream=None):
        return _read_codes(self._lib.fmkv_pool_read_codes, self._h, self.desc,
                           self.n_blocks * BLOCK_TOKENS, stream)


def _dtype_code(dtype) -> int:
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float32:
        return DTYPE_F32
    raise ValueError(f"unsupported output dtype {dtype}")


def words_per_row(desc: CacheDesc) -> int:
    return (desc.head_dim * desc.bits + 31) // 32


def meta_per_row(desc: CacheDesc) -> int:
    if desc.mode == MODE_PLAIN:
        return 0
    return 2 * (desc.head_dim // 64) if desc.mode == MODE_AFFINE else 1


def _read_codes(fn, handle, desc, n_slots, stream):
    H = desc.n_kv_heads
    codes = torch.zeros((n_slots, 2, H, words_per_row(desc)), dtype=torch.int32, device="cuda")
    meta = torch.zeros((n_slots, 2, H, meta_per_row(desc)), dtype=torch.int16, device="cuda")
    _check(fn(handle, _ptr(codes), _ptr(meta), _stream(stream)))
    return codes, meta
