"""The device argmax (ie_hip_argmax_rows) against the reference CPU argmax's scan
(src/sampler.cpp:26-31: start at element 0, move on a strictly greater value), restated
below as a plain loop and checked on rows built to hit its corner cases: ties (the lowest
index wins), NaNs (never chosen; a NaN in element 0 gives 0), rows of -inf (0), a maximum
in the last element, and widths that are not a multiple of 4 (the kernel's scalar path)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def cpu_scan(row) -> int:
    best = 0
    for i in range(1, len(row)):
        if row[i] > row[best]:
            best = i
    return best


def scan_fast(row) -> int:
    """The same scan for long rows, via numpy; pinned to cpu_scan in the test below."""
    if np.isnan(row[0]):
        return 0
    r = np.where(np.isnan(row), -np.inf, row)
    return int(np.argmax(r))


def corner_rows(n, rng):
    rows = [rng.standard_normal(n).astype(np.float32) for _ in range(12)]
    rows[1][[7, n // 2, n - 1]] = 50.0                    # a three-way tie
    rows[2][:] = -np.inf                                   # nothing above -inf
    rows[3][0] = np.nan                                    # NaN in element 0
    rows[4][[1, 5, n - 2]] = np.nan                        # NaNs elsewhere
    rows[4][9] = 77.0
    rows[5][n - 1] = 99.0                                  # the last element
    rows[6][:] = 3.0                                       # all equal
    rows[7][:] = np.nan                                    # all NaN
    rows[8][0] = -np.inf
    rows[8][1:] = np.nan                                   # -inf then NaNs
    rows[9][:] = -np.inf
    rows[9][n - 3] = -1e30                                 # one finite value
    rows[10][n // 3] = np.inf                              # +inf
    rows[10][2 * n // 3] = np.inf
    return np.stack(rows)


@pytest.mark.parametrize("n", [13, 64, 1000, 151936, 151937])
def test_argmax_rows_matches_the_cpu_scan(ie, dev, n):
    rng = np.random.default_rng(n)
    x = corner_rows(n, rng)
    out = torch.full((x.shape[0],), -5, dtype=torch.int32, device=dev)
    ie.argmax_rows(out, torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = [cpu_scan(r) if n <= 1000 else scan_fast(r) for r in x]
    if n <= 1000:
        assert want == [scan_fast(r) for r in x]  # the numpy form agrees with the loop
    assert list(got) == want


def test_argmax_rows_batch(ie, dev):
    """64 rows of the LM head's width, the decode step's shape."""
    rng = np.random.default_rng(64)
    x = rng.standard_normal((64, 151936)).astype(np.float32)
    out = torch.empty(64, dtype=torch.int32, device=dev)
    ie.argmax_rows(out, torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    assert list(out.cpu().numpy()) == [scan_fast(r) for r in x]
