"""The oracle against its frozen fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): codes, scale/bias or norms bit for bit, the
f64 attention to 1e-12. A change of the oracle's arithmetic fails here
before it can move the contract the GPU tests check against."""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.npz"))


def test_fixtures_present():
    assert len(GOLDEN) >= 10


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_oracle_reproduces_fixture(ora, path):
    f = np.load(path)  # allow_pickle stays False: arrays only
    D, bits, mode, H, W, n = (int(x) for x in f["spec"])
    oc = ora.OracleCache(H, D, bits, W, 0 if W else n, mode)
    oc.append(f["k"][:n // 2], f["v"][:n // 2])
    oc.append(f["k"][n // 2:], f["v"][n // 2:])
    assert np.array_equal(oc.codes, f["codes"])
    assert np.array_equal(oc.meta, f["meta"])
    for scale in (1.0, 0.01):
        assert np.allclose(oc.attention(f["q"], scale), f[f"attn_{scale}"], rtol=0, atol=1e-12)
