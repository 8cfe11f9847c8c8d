"""Pins of the motion producer oracle (oracle/farneback.py) on the CPU.

Each piece of the Farneback restatement is checked against an independent
library routine (scipy.ndimage) or a closed form chosen so that a plausible
mistake fails: a wrong border mode, a swapped channel or axis, a sign, a
missing inverse-Gram entry or a pyramid that does not carry the flow.
The trace post-processing is checked against the reference's own numpy form
(reference: traces/gen_motion_from_video.py:61-67,110-126).
"""

import numpy as np
import pytest
from scipy import ndimage

from kvpersist import workloads
from oracle import farneback as fb


def _texture(h, w, seed, sigma=2.0, pad=40):
    rng = np.random.default_rng(seed)
    t = ndimage.gaussian_filter(rng.standard_normal((h + 2 * pad, w + 2 * pad)), sigma,
                                mode="wrap")
    return (t - t.mean()) / t.std(), pad


def _shifted(tex, pad, h, w, dx, dy):
    """Texture sampled so that content moves by (+dx, +dy): I(x, y) = T(x - dx, y - dy)."""
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    return ndimage.map_coordinates(tex, [yy + pad - dy, xx + pad - dx], order=3, mode="wrap")


def _u8(img):
    return np.clip(np.rint(128 + 40 * img), 0, 255).astype(np.uint8)


# ---- filters and resize ---------------------------------------------------------------


@pytest.mark.parametrize("ksize,sigma", [(3, 0.0), (3, 0.5), (9, 1.5), (19, 3.5)])
def test_gaussian_blur_matches_scipy_mirror(ksize, sigma):
    rng = np.random.default_rng(ksize)
    img = rng.random((23, 31)) * 255
    k = fb.gaussian_kernel(ksize, sigma)
    assert abs(k.sum() - 1) < 1e-6 and np.allclose(k, k[::-1])
    if sigma > 0:
        x = np.arange(ksize) - ksize // 2
        assert np.abs(k - np.exp(-x * x / (2 * sigma * sigma)) / np.exp(
            -x * x / (2 * sigma * sigma)).sum()).max() < 1e-7
    want = ndimage.correlate1d(ndimage.correlate1d(img, k, axis=1, mode="mirror"), k, axis=0,
                               mode="mirror")
    assert np.abs(fb.gaussian_blur(img, ksize, sigma) - want).max() < 1e-9


def test_small_gaussian_is_the_fixed_three_tap():
    assert np.array_equal(fb.gaussian_kernel(3, 0), [0.25, 0.5, 0.25])


@pytest.mark.parametrize("src,dst", [((48, 64), (24, 32)), ((48, 64), (12, 16)),
                                     ((48, 64), (6, 8)), ((24, 32), (48, 64)),
                                     ((30, 52), (61, 103)), ((17, 9), (17, 9))])
def test_resize_linear_matches_scipy_zoom(src, dst):
    rng = np.random.default_rng(src[0] + dst[1])
    img = rng.random(src)
    got = fb.resize_linear(img, dst[1], dst[0])
    want = ndimage.zoom(img, (dst[0] / src[0], dst[1] / src[1]), order=1, grid_mode=True,
                        mode="nearest")
    assert got.shape == want.shape == dst
    assert np.abs(got - want).max() < 1e-9


def test_level_plan_follows_the_min_size_rule():
    plan = fb.level_plan(832, 480, 0.5, 3)
    assert [(p[0], p[3], p[4], p[5]) for p in plan] == [
        (3, 19, 104, 60), (2, 9, 208, 120), (1, 3, 416, 240), (0, 3, 832, 480)]
    assert plan[-1][2] == 0.0 and plan[0][2] == 3.5
    # 96 rows: 48 >= 32 but 24 < 32 -> one coarser level only
    assert [p[0] for p in fb.level_plan(160, 96, 0.5, 3)] == [1, 0]
    assert [p[0] for p in fb.level_plan(40, 40, 0.5, 5)] == [0]


# ---- polynomial expansion ----------------------------------------------------------------


@pytest.mark.parametrize("n,sigma", [(5, 1.2), (7, 1.5), (3, 0.0)])
def test_poly_exp_recovers_an_exact_quadratic(n, sigma):
    H, W = 40, 44
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float64)
    c, bx, by, axx, ayy, axy = 3.0, 0.7, -1.3, 0.05, -0.02, 0.03
    img = c + bx * xx + by * yy + axx * xx * xx + ayy * yy * yy + axy * xx * yy
    R = fb.poly_exp(img, n, sigma)
    inner = (slice(n, H - n), slice(n, W - n))
    yi, xi = yy[inner], xx[inner]
    # local expansion around each pixel (x0, y0): the gradient there and the fixed a's
    want = [by + 2 * ayy * yi + axy * xi, bx + 2 * axx * xi + axy * yi,
            np.full_like(xi, ayy), np.full_like(xi, axx), np.full_like(xi, axy)]
    for ch in range(5):
        assert np.abs(R[ch][inner] - want[ch]).max() < 1e-6, ch  # float32 taps


def test_poly_exp_constant_image_has_no_terms():
    R = fb.poly_exp(np.full((20, 24), 77.0), 5, 1.2)
    assert np.abs(R).max() < 1e-5  # float32 taps, |f| = 77


# ---- box filter and solve --------------------------------------------------------------


@pytest.mark.parametrize("winsize", [15, 5, 14])
def test_box_mean_matches_uniform_filter(winsize):
    rng = np.random.default_rng(winsize)
    a = rng.random((5, 26, 33))
    m = winsize // 2
    want = np.stack([ndimage.uniform_filter(a[c], size=2 * m + 1, mode="nearest")
                     for c in range(5)]) * ((2 * m + 1) ** 2 / winsize ** 2)
    assert np.abs(fb.box_mean(a, winsize) - want).max() < 1e-12


def test_solve_flow_is_the_regularised_2x2_solve():
    rng = np.random.default_rng(5)
    A = rng.random((2, 2))
    G = A @ A.T + np.eye(2)
    h = rng.standard_normal(2)
    # M holds G in (y, x) order and h = [h_y, h_x]; the flow is (x, y)
    Mb = np.array([G[0, 0], G[0, 1], G[1, 1], h[0], h[1]])[:, None, None]
    d = fb.solve_flow(Mb)[0, 0]
    det = G[0, 0] * G[1, 1] - G[0, 1] ** 2
    sol = np.linalg.solve(G, h) * det / (det + 1e-3)
    assert np.abs(d - sol[::-1]).max() < 1e-12


# ---- end to end ------------------------------------------------------------------------


def test_identical_frames_give_zero_flow_away_from_the_far_border():
    """Zero flow and R0 == R1 cancel delta-b everywhere except where the
    bilinear sample of R1 needs a pixel past the last row or column: there the
    outside branch keeps R0's linear terms. So with one level the flow is
    exactly zero outside a band of iterations * (winsize // 2) + 1 pixels along
    the right and bottom edges (the box filter widens the band once per
    iteration), and nonzero inside it; the pyramid keeps it small."""
    H, W = 96, 112
    tex, pad = _texture(H, W, 1)
    img = _u8(_shifted(tex, pad, H, W, 0, 0))
    flow = fb.calc_optical_flow_farneback(img, img, levels=0)
    assert flow.shape == (H, W, 2) and flow.dtype == np.float32
    band = 3 * 7 + 1
    assert not flow[:H - band, :W - band].any()
    assert flow[-1].any() and flow[:, -1].any()
    assert np.abs(flow[H - band - 1:, :]).any()
    pyr = fb.calc_optical_flow_farneback(img, img)
    mag = np.hypot(pyr[..., 0], pyr[..., 1])
    assert mag.max() < 0.2 and np.median(mag) < 1e-3


@pytest.mark.parametrize("dx,dy", [(0.6, -0.35), (-1.25, 0.8), (5.5, -3.0)])
def test_subpixel_translation_is_recovered(dx, dy):
    """Content moving by (dx, dy) gives flow (dx, dy) away from the borders,
    and the reverse pair gives its negation; 5.5 px needs the pyramid."""
    H, W = 96, 128
    tex, pad = _texture(H, W, 2, sigma=2.5)
    a = _u8(_shifted(tex, pad, H, W, 0, 0))
    b = _u8(_shifted(tex, pad, H, W, dx, dy))
    flow = fb.calc_optical_flow_farneback(a, b)
    inner = flow[20:-20, 20:-20]
    assert abs(np.median(inner[..., 0]) - dx) < 0.05
    assert abs(np.median(inner[..., 1]) - dy) < 0.05
    assert np.abs(inner[..., 0] - dx).mean() < 0.1 and np.abs(inner[..., 1] - dy).mean() < 0.1
    back = fb.calc_optical_flow_farneback(b, a)[20:-20, 20:-20]
    assert abs(np.median(back[..., 0]) + dx) < 0.05 and abs(np.median(back[..., 1]) + dy) < 0.05


def test_clip_pairs_equal_single_pairs():
    clip = workloads.synthetic_clip(3, 64, 96, seed=3)
    flows = fb.farneback_clip(clip)
    for p in range(2):
        assert np.array_equal(flows[p], fb.calc_optical_flow_farneback(clip[p], clip[p + 1]))


# ---- change rates and the trace --------------------------------------------------------


def _reference_form(flow, rows, cols, tt):
    """The reference's per-frame code path, written as it is (float32 flow)."""
    mag = np.linalg.norm(flow, axis=2)
    h, w = mag.shape
    ch, cw = h // rows, w // cols
    cm = mag[:rows * ch, :cols * cw].reshape(rows, ch, cols, cw).mean(axis=(1, 3))
    tokens = rows * cols
    num_tiles = tokens // tt + bool(tokens % tt)
    counts = np.full(num_tiles, tt)
    counts[-1] = tokens - (num_tiles - 1) * tt
    sums = np.add.reduceat(cm.reshape(-1), np.arange(0, num_tiles * tt, tt))
    return cm, sums / counts


def test_change_rates_match_the_reference_form():
    rng = np.random.default_rng(9)
    flows = rng.standard_normal((3, 480, 832, 2)).astype(np.float32)
    cm, change = fb.change_rates(flows, 30, 52, 16)
    assert change.shape == (3, 98)
    for p in range(3):
        rcm, rch = _reference_form(flows[p], 30, 52, 16)
        assert np.abs(cm[p] - rcm).max() < 1e-5
        assert np.abs(change[p] - rch).max() < 1e-5


def test_change_rates_closed_forms():
    flows = np.zeros((1, 32, 48, 2), dtype=np.float32)
    flows[..., 0], flows[..., 1] = 3.0, 4.0          # |flow| = 5 everywhere
    cm, change = fb.change_rates(flows, 2, 3, 4)     # 6 cells, tiles of 4 -> [4, 2]
    assert np.array_equal(cm, np.full((1, 2, 3), 5.0))
    assert np.array_equal(change, [[5.0, 5.0]])
    flows[0, :, 32:] = 0                              # last cell column static
    _, change = fb.change_rates(flows, 2, 3, 4)
    # cells row-major [5, 5, 0, 5, 5, 0]: tile 0 = (5+5+0+5)/4, tile 1 = (5+0)/2
    assert np.array_equal(change, [[3.75, 2.5]])
    with pytest.raises(ValueError):
        fb.change_rates(np.zeros((1, 30, 50, 2)), 4, 5, 4)


def test_trace_post_processing():
    rng = np.random.default_rng(11)
    pairs = rng.random((6, 98)) * 10
    change, tau, reuse = fb.trace_from_change(pairs, 50.0)
    assert np.array_equal(change[0], pairs[0]) and np.array_equal(change[1:], pairs)
    assert tau == np.percentile(pairs, 50)
    assert not reuse[0].any()
    assert reuse[1:].mean() == 0.5                   # distinct values, even count
    rows = fb.trace_rows(change, tau, reuse, 1560, 16)
    assert len(rows) == 7 * 98
    assert rows[97][4:6] == [97 * 16, 8]             # 1560 = 97 * 16 + 8
    assert rows[98 + 3] == [1, 3, f"{change[1, 3]:.6f}", int(change[1, 3] < tau), 48, 16,
                            int(reuse[1, 3])]
