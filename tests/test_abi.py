"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and validates descriptors before touching HIP."""
import re
from pathlib import Path

import pytest

import fmkv

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "fmkv.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(fmkv_\w+)\s*\(", text, re.M)))


def test_library_exports_header_symbols():
    lib = fmkv.load_library()
    syms = header_symbols()
    assert len(syms) >= 19
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(fmkv.EXPORTED)


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(n_kv_heads=0, head_dim=256, bits=4, capacity=16), fmkv.FMKV_ERR_INVALID_ARG),
        (dict(n_kv_heads=8, head_dim=100, bits=4, capacity=16), fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=1024, bits=4, capacity=16), fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=256, bits=3, capacity=16), fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=256, bits=5, capacity=16, mode=fmkv.MODE_CODEBOOK),
         fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=256, bits=4, window=-16), fmkv.FMKV_ERR_INVALID_ARG),
        (dict(n_kv_heads=8, head_dim=256, bits=4, window=(1 << 30) + 1), fmkv.FMKV_ERR_INVALID_ARG),
        (dict(n_kv_heads=8, head_dim=256, bits=4, capacity=0), fmkv.FMKV_ERR_INVALID_ARG),
        (dict(n_kv_heads=8, head_dim=256, bits=4, capacity=1 << 31), fmkv.FMKV_ERR_INVALID_ARG),
        (dict(n_kv_heads=8, head_dim=256, bits=4, group_size=32, capacity=16), fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=256, bits=4, mode=7, capacity=16), fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=256, bits=8, mode=fmkv.MODE_PLAIN, capacity=16),
         fmkv.FMKV_ERR_UNSUPPORTED),
        (dict(n_kv_heads=8, head_dim=96, bits=16, mode=fmkv.MODE_PLAIN, capacity=16),
         fmkv.FMKV_ERR_UNSUPPORTED),
    ],
)
def test_invalid_descriptors_rejected_before_hip(kw, code):
    with pytest.raises(fmkv.Exception_) as ei:
        fmkv.validate(fmkv.make_desc(**kw))
    assert ei.value.code == code
    assert fmkv.load_library().fmkv_last_error().decode()
    # cache creation reports the same error without a device
    with pytest.raises(fmkv.Exception_) as ei2:
        fmkv.KVCache(fmkv.make_desc(**kw))
    assert ei2.value.code == code


@pytest.mark.parametrize(
    "D,bits,mode,block",
    [(512, 8, 0, 16 * (2 * 512 + 8 * 4 * 2) // 2 * 1),  # 17408
     (256, 4, 0, 4608), (256, 8, 0, 8704), (512, 4, 0, 9216), (128, 4, 0, 2304),
     (256, 3, 1, 3328), (512, 2, 1, 4352),
     (128, 16, 2, 8192), (256, 16, 2, 16384), (512, 16, 2, 32768)],
)
def test_layout_bytes(D, bits, mode, block):
    if D == 512 and bits == 8:
        block = 17408
    b, a = fmkv.layout_bytes(fmkv.make_desc(2, D, bits, capacity=40, mode=mode))
    assert b == block
    assert a == block * 2 * 3  # 40 positions -> 3 blocks per head


def test_algorithmic_bytes_per_token_match_spec():
    """Per token per KV head, K+V codes plus f16 scale/bias: 288 B (D=256
    4-bit), 544 B (D=256 8-bit), 1088 B (D=512 8-bit)."""
    for D, bits, per_tok in ((256, 4, 288), (256, 8, 544), (512, 8, 1088)):
        b, _ = fmkv.layout_bytes(fmkv.make_desc(1, D, bits, capacity=16))
        assert b == 16 * per_tok


def test_ring_and_global_arena_sizes():
    b, a = fmkv.layout_bytes(fmkv.make_desc(8, 256, 4, window=1024))
    assert a == b * 8 * 64
    # any window: a ring of whole 16-token head-blocks (src/cache.rs:206 takes
    # sliding_window from the config as it is)
    for w, blocks in ((1000, 63), (5, 1), (17, 2), (1008, 63)):
        fmkv.validate(fmkv.make_desc(8, 256, 4, window=w))
        b, a = fmkv.layout_bytes(fmkv.make_desc(8, 256, 4, window=w))
        assert a == b * 8 * blocks
    b, a = fmkv.layout_bytes(fmkv.make_desc(2, 512, 8, capacity=32768))
    assert a == 17408 * 2 * 2048 == 2 * 32768 * 1088


def test_entry_points_reject_null_handles_before_hip():
    """Prefill, decode step and projected append validate their handle first
    (no device needed)."""
    lib = fmkv.load_library()
    assert lib.fmkv_prefill_step(None, None, None, 4, None, 8, 1.0, None,
                                 fmkv.DTYPE_BF16, None) == fmkv.FMKV_ERR_INVALID_ARG
    assert lib.fmkv_decode_step(None, None, None, 1, None, 8, 1.0, 0.0, None,
                                fmkv.DTYPE_BF16, None) == fmkv.FMKV_ERR_INVALID_ARG
    assert lib.fmkv_decode_step_noalloc(None, None, None, 1, None, 8, 1.0, 0.0, None,
                                        fmkv.DTYPE_BF16, None) == fmkv.FMKV_ERR_INVALID_ARG
    pro = fmkv.KvPrologue(None, 1e-6, 128, 1e4, 0)
    assert lib.fmkv_cache_append_projected(None, None, None, 1, pro, None) == fmkv.FMKV_ERR_INVALID_ARG
    assert lib.fmkv_decode_step_projected(None, None, None, 1, pro, None, 8, 1.0, 0.0, None,
                                          fmkv.DTYPE_BF16, None) == fmkv.FMKV_ERR_INVALID_ARG
    assert b"null" in lib.fmkv_last_error()


def test_plain_descriptor_and_layout():
    """Plain (bf16) caches: bits 16, no meta, K rows then V columns; a
    head-block is 16 tokens x head_dim x 2 bytes x 2 (KVCacheInner::Plain,
    src/cache.rs:174-178)."""
    d = fmkv.make_desc(2, 512, 16, capacity=32768, mode=fmkv.MODE_PLAIN)
    fmkv.validate(d)
    b, a = fmkv.layout_bytes(d)
    assert b == 16 * 512 * 2 * 2
    assert a == 2 * 32768 * 512 * 2 * 2
    assert fmkv.meta_per_row(d) == 0 and fmkv.words_per_row(d) == 256
