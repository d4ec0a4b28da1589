"""The 32-row tile layout of an activation (IMQ_LD_TILED): tile_rows puts element (m, k) at
((((k/64) * 4 + (k%32)/8) * 2 + (k%64)/32) * 32 + m) * 8 + k%8, checked element by element
against that formula; untile_rows inverts it; rows past M are zero; each 1 KB piece
(64-column group g, k-step t) holds the 16 bytes lane (m, kb) of an MFMA kernel reads, at
16 (32 kb + m)."""

from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.mark.parametrize("m,k", [(32, 256), (5, 128), (1, 64)])
def test_tile_rows_formula_and_inverse(m, k):
    from ironmule_amd._native import tile_rows, untile_rows
    x = torch.arange(m * k, dtype=torch.float32).view(m, k).to(torch.bfloat16)
    t = tile_rows(x)
    assert t.shape == (32 * k,)
    xs = x.float().numpy()
    ts = t.float().numpy()
    for mm in range(32):
        for kk in range(k):
            off = ((((kk // 64) * 4 + (kk % 32) // 8) * 2 + (kk % 64) // 32) * 32 + mm) * 8 + kk % 8
            assert ts[off] == (xs[mm, kk] if mm < m else 0.0), (mm, kk)
    assert torch.equal(untile_rows(t, m, k), x)


def test_lane_pieces_are_contiguous():
    from ironmule_amd._native import tile_rows
    k = 128
    x = torch.arange(32 * k, dtype=torch.float32).view(32, k).to(torch.bfloat16)
    t = tile_rows(x).float().numpy()
    for g in range(k // 64):
        for step in range(4):
            piece = t[(g * 4 + step) * 512:(g * 4 + step + 1) * 512]  # 1 KB = 512 elements
            for lane in range(64):
                mm, kb = lane % 32, lane // 32
                want = x[mm, 64 * g + 32 * kb + 8 * step:64 * g + 32 * kb + 8 * step + 8].float().numpy()
                assert np.array_equal(piece[8 * lane:8 * lane + 8], want), (g, step, lane)
