"""GPU parity of the hand-written grouped projection GEMM (kvp_proj_gemm)
against the oracle's nn.Linear (oracle/backbone.py: float64 of the same
bf16-rounded operands).

bf16 outputs: within one bf16 ulp of the wide result; fp32 outputs (plain or
accumulated into the existing values, the residual add of out_proj):
max-abs <= 1e-4. Rows past `rows` are never written.
"""

import numpy as np
import pytest
import torch

from kvpersist import _lib
from kvpersist import backbone as kb
from oracle import backbone as ob

DEV = "cuda"


def _bf16_close(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > np.abs(want) * 2.0 ** -7 + 1e-5
    assert not bad.any(), (int(bad.sum()), got[bad][:4], want[bad][:4])


CASES = [
    # rows, K, N, groups, tile_n, out_dtype, accumulate, bias
    (1, 64, 256, 1, 256, 1, False, True),
    (300, 256, 256, 3, 128, 1, False, True),
    (1560, 1536, 1536, 3, 256, 1, False, True),
    (1560, 1536, 1536, 3, 128, 1, False, False),
    (257, 128, 384, 2, 128, 0, False, True),
    (1000, 1536, 1536, 1, 256, 0, True, True),
    # accumulate form, K of one chunk (residual loaded in the epilogue) and of
    # two (loaded during the first), ragged last row tile
    (130, 64, 128, 1, 128, 0, True, True),
    (257, 128, 256, 1, 128, 0, True, False),
    (1560, 1536, 1536, 1, 128, 0, True, True),
    (12480, 1536, 1536, 3, 256, 1, False, True),
    (12480, 1536, 1536, 3, 128, 1, False, True),
    (12480, 1536, 1536, 1, 128, 0, True, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,K,N,groups,tile_n,out_dt,acc,bias", CASES)
def test_proj_gemm_matches_oracle(rows, K, N, groups, tile_n, out_dt, acc, bias):
    print(f"proj_gemm rows={rows} K={K} N={N} groups={groups} tile={tile_n} out={out_dt} "
          f"acc={acc}", flush=True)
    rng = np.random.default_rng(rows + K + N + groups)
    x = ob.round_bf16(rng.standard_normal((rows, K)).astype(np.float32))
    w = ob.round_bf16((0.02 * rng.standard_normal((groups * N, K))).astype(np.float32))
    b = (0.1 * rng.standard_normal(groups * N)).astype(np.float32) if bias else None
    odt = torch.bfloat16 if out_dt == 1 else torch.float32
    guard = 3
    y0 = rng.standard_normal((groups, rows + guard, N)).astype(np.float32)
    if out_dt == 1:
        y0 = ob.round_bf16(y0)
    ys = [torch.from_numpy(y0[g]).to(DEV).to(odt) for g in range(groups)]
    xd = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    wd = torch.from_numpy(w).to(DEV).to(torch.bfloat16)
    bd = None if b is None else torch.from_numpy(b).to(DEV)
    kb.proj_gemm(xd, wd, bd, [y[:rows] for y in ys], accumulate=acc, tile_n=tile_n)
    torch.cuda.synchronize()
    # the oracle on a bounded sample of rows for the largest case
    sample = np.arange(rows) if rows <= 2000 else np.unique(
        np.concatenate([np.arange(300), rng.choice(rows, 700, replace=False), [rows - 1]]))
    for g in range(groups):
        got = ys[g].float().cpu().numpy()
        assert np.array_equal(got[rows:], y0[g][rows:]), "rows past the end were written"
        want = ob.linear(x[sample], w[g * N:(g + 1) * N], None if b is None else
                         b[g * N:(g + 1) * N])
        if acc:
            want = want + y0[g][sample]
        if out_dt == 1:
            _bf16_close(got[sample], want)
        else:
            assert np.abs(got[sample] - want).max() <= 1e-4, g


def test_proj_gemm_rejects_unsupported_shapes(lib):
    """Shape errors are reported before any device work (runs without a GPU)."""
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 1, 4, 96, 256, 1, 0, 256, None) != 0
    assert "not supported" in _lib.last_error()
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 1, 4, 64, 192, 1, 0, 256, None) != 0
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 1, 4, 64, 256, 1, 1, 256, None) != 0
    assert "fp32" in _lib.last_error()
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 4, 4, 64, 256, 1, 0, 256, None) != 0
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 2, 4, 64, 256, 1, 0, 256, None) != 0
    assert lib.kvp_proj_gemm(16, 16, None, 16, None, None, 1, 4, 64, 256, 1, 0, 64, None) != 0
