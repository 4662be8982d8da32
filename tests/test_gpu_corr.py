"""GPU parity of the correlation path (volume, pyramid, lookup) through the C ABI
against the CPU oracle on the same seeded inputs.

Bars: indexing, shapes and the pyramid of a given level 0 are bitwise; with
integer-coded features (exact fp32 products and sums, alpha = 1/16) the whole
chain is bitwise; fp32 N(0,1) values are within helpers.TOL = 1e-4 of the
oracle's fp64-accumulated result, relative to max(|r|, rms(r)), and within
F16X3_TOL = 1e-5 under the batched path's default scaled fp16 split.
"""
import numpy as np
import pytest

from helpers import TOL, announce, assert_close_rel, gpu_or_fail, norm_rel
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu

# the batched path's scaled fp16 split (22 significant bits): its bar, a tenth
# of the north-star tolerance
F16X3_TOL = 1e-5


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


def run_single(slk, f, coords, alpha, levels=4, prec=0):
    C, h, w = f.shape[1:]
    dt = slk.SLK_F16 if f.dtype == np.float16 else slk.SLK_F32
    ctx = slk.Context(h, w, C=C, max_batch=1, levels=levels, corr_scale=alpha)
    ctx.set_corr_precision(prec)
    fi = slk.DeviceArray.from_host(f[0])
    fj = slk.DeviceArray.from_host(f[1])
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((levels * 49, h * w))
    ctx.build_correlation(fi, fj, dtype=dt)
    ctx.sample_correlation(cd, out)
    slk.hip().sync()
    pyr = [ctx.level_to_host(l) for l in range(levels)]
    res = out.to_host()
    ctx.close()
    return pyr, res


@pytest.mark.parametrize("h,w,levels,prec", [(48, 64, 4, 0), (48, 64, 4, 1), (54, 96, 4, 0),
                                             (54, 96, 4, 1), (12, 20, 3, 0), (7, 9, 1, 0)])
def test_single_edge_volume_pyramid_lookup(slk, h, w, levels, prec):
    """prec 0: bf16x3 split contraction (default), 1: fp32 MFMA."""
    announce(f"single edge h={h} w={w} levels={levels} prec={prec}")
    f = wl.frames(2, C=128, h=h, w=w, seed=100 + h)
    coords = wl.flow_coords(1, h, w, seed=7)[0]
    alpha = 1.0 / np.sqrt(128.0)
    pyr, out = run_single(slk, f, coords, alpha, levels, prec)
    vol = orc.corr_volume(f[0].reshape(128, -1), f[1].reshape(128, -1), alpha)
    # level shapes: floor halving
    for l, lev in enumerate(pyr):
        assert lev.shape == (h * w, h >> l, w >> l)
    assert_close_rel(pyr[0].reshape(h * w, -1), vol, what="level 0")
    # pyramid of the GPU's own level 0: bitwise
    for l in range(1, levels):
        np.testing.assert_array_equal(pyr[l], orc.avg_pool_2x2(pyr[l - 1]), err_msg=f"level {l}")
    # lookup of the GPU's own pyramid: fp32 vs fp64 weights only
    assert_close_rel(out, orc.lookup(pyr, coords), tol=1e-5, what="lookup(own pyramid)")
    # whole chain vs the oracle
    ref = orc.lookup(orc.pyramid(vol, h, w, levels), coords)
    assert_close_rel(out, ref, what="chain")


def test_integer_coded_chain_is_bitwise(slk):
    """Small-integer features: every product and partial sum is exact in fp32,
    so volume, pyramid and integer-coordinate lookups must match bitwise."""
    h, w = 48, 64
    rng = np.random.default_rng(3)
    f = rng.integers(-3, 4, size=(2, 128, h, w)).astype(np.float32)
    coords = (wl.grid_coords(h, w) + rng.integers(-6, 7, size=(2, h * w))).astype(np.float32)
    coords *= 1.0  # integer at level 0
    pyr, out = run_single(slk, f, coords, 1.0 / 16.0)
    vol = orc.corr_volume(f[0].reshape(128, -1), f[1].reshape(128, -1), 1.0 / 16.0)
    np.testing.assert_array_equal(pyr[0].reshape(h * w, -1), vol)
    ref_pyr = orc.pyramid(vol, h, w)
    for l in range(4):
        np.testing.assert_array_equal(pyr[l], ref_pyr[l])
    # level 0 channels with integer coords: pure window copy -> bitwise
    np.testing.assert_array_equal(out[:49], orc.lookup(ref_pyr, coords)[:49])
    # multiples of 8: integer at every level -> bitwise everywhere
    c8 = (wl.grid_coords(h, w) // 8 * 8 + 8 * rng.integers(-1, 2, size=(2, h * w))).astype(np.float32)
    _, out8 = run_single(slk, f, c8, 1.0 / 16.0)
    np.testing.assert_array_equal(out8, orc.lookup(ref_pyr, c8))


def test_fp16_features(slk):
    h, w = 48, 64
    f = wl.frames(2, C=128, h=h, w=w, seed=8).astype(np.float16)
    coords = wl.flow_coords(1, h, w, seed=9)[0]
    pyr, out = run_single(slk, f, coords, 1.0 / 16.0)
    vol = orc.corr_volume(f[0].reshape(128, -1), f[1].reshape(128, -1), 1.0 / 16.0)
    assert_close_rel(pyr[0].reshape(h * w, -1), vol, what="f16 level 0")
    assert_close_rel(out, orc.lookup(orc.pyramid(vol, h, w), coords), what="f16 chain")


def test_nonfinite_and_far_coords_give_zeros(slk):
    h, w = 12, 16
    f = wl.frames(2, C=128, h=h, w=w, seed=10)
    coords = wl.grid_coords(h, w)
    coords[0, 0] = np.nan
    coords[1, 1] = np.inf
    coords[0, 2] = -np.inf
    coords[0, 3] = 3e9
    coords[1, 4] = -3e9
    coords[0, 5] = 40.0
    pyr, out = run_single(slk, f, coords, 1.0 / 16.0)
    assert np.all(out[:, :6] == 0.0)
    assert np.all(np.isfinite(out))
    assert_close_rel(out, orc.lookup(pyr, coords), tol=1e-5)


def _window(slk, nframes, h, w, B, seed, max_batch=48, dev_idx=False, prec=None):
    f = wl.frames(nframes, C=128, h=h, w=w, seed=seed)
    ii, jj = wl.cyclic_edges(nframes)
    ii, jj = ii[:B], jj[:B]
    coords = wl.flow_coords(B, h, w, seed=seed + 1)
    alpha = 1.0 / 16.0
    ctx = slk.Context(h, w, C=128, max_batch=max_batch, corr_scale=alpha)
    if prec is not None:  # else the library's default, SLK_PREC_F16X3
        ctx.set_corr_precision(prec)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((B, 196, h * w))
    if dev_idx:
        iid = slk.DeviceArray.from_host(ii)
        jjd = slk.DeviceArray.from_host(jj)
        ctx.batch_build_and_sample_correlation_dev(fd, iid, jjd, B, cd, out)
    else:
        ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out)
    slk.hip().sync()
    res = out.to_host()
    ctx.close()
    return f, ii, jj, coords, res


@pytest.mark.parametrize("prec", [2, 0, 1])
def test_window_48_edges_matches_oracle(slk, prec):
    """Config corr_window: 12 frames, 48 edges; every edge checked on sampled
    pixels plus 6 edges in full (prec 2: the scaled fp16 split, held to
    F16X3_TOL; 0: the bf16 split; 1: fp32 MFMA)."""
    announce(f"corr window 48 edges prec={prec}")
    h, w = 48, 64
    tol = F16X3_TOL if prec == 2 else TOL
    f, ii, jj, coords, out = _window(slk, 12, h, w, 48, seed=20, prec=prec)
    assert np.all(np.isfinite(out))
    full = [0, 7, 18, 29, 40, 47]
    ref = orc.corr_batch(f, ii[full], jj[full], coords[full], 1.0 / 16.0)
    for k, e in enumerate(full):
        assert_close_rel(out[e], ref[k], tol=tol, what=f"edge {e}")
    # all 48 edges on 64 random pixels: direct fp64 evaluation of the windows
    rng = np.random.default_rng(0)
    pix = rng.choice(h * w, 64, replace=False)
    for e in range(48):
        fi = f[ii[e]].reshape(128, -1).astype(np.float64)
        fj = f[jj[e]].reshape(128, -1).astype(np.float64)
        vol = (fi[:, pix].T @ fj) / 16.0
        pyr = [vol.reshape(64, h, w).astype(np.float32)]
        for _ in range(3):
            pyr.append(orc.avg_pool_2x2(pyr[-1]))
        ref_sub = _lookup_rows(pyr, coords[e][:, pix])
        assert_close_rel(out[e][:, pix], ref_sub, tol=tol, what=f"edge {e} sampled")


@pytest.mark.parametrize("h,w", [(96, 128), (100, 128), (256, 24), (260, 80)])
def test_window_large_frames_sampled(slk, h, w):
    """Large feature maps, 12 edges in one launch. 96x128: 64 target tiles
    per source tile, the widest the tile marking handles with a 64-bit mask
    per lane (and the top bit set); 100x128: 67, which takes the per-tile
    marking path, and 6700 tiles per edge, several rounds of the tile
    compaction. 256x24 and 260x80: more than 247 rows, so the sources keep
    their pixel order (no sort by window row), with 32 target tiles (64-bit
    masks) and 108 (per-tile marking). Every edge is checked on 48 random
    pixels by direct fp64 evaluation of their windows."""
    announce(f"corr window {h}x{w}, 12 edges")
    f, ii, jj, coords, out = _window(slk, 6, h, w, 12, seed=50, max_batch=12)
    assert np.all(np.isfinite(out))
    rng = np.random.default_rng(1)
    pix = rng.choice(h * w, 48, replace=False)
    for e in range(12):
        fi = f[ii[e]].reshape(128, -1).astype(np.float64)
        fj = f[jj[e]].reshape(128, -1).astype(np.float64)
        vol = (fi[:, pix].T @ fj) / 16.0
        pyr = [vol.reshape(48, h, w).astype(np.float32)]
        for _ in range(3):
            pyr.append(orc.avg_pool_2x2(pyr[-1]))
        assert_close_rel(out[e][:, pix], _lookup_rows(pyr, coords[e][:, pix]),
                         what=f"edge {e} sampled")


def _lookup_rows(pyr, coords):
    """Lookup of selected source rows: pyr[l] is [n, h>>l, w>>l] for n chosen
    pixels whose coords are [2, n]; uses the oracle's level routine."""
    n = pyr[0].shape[0]
    out = np.zeros((len(pyr) * 49, n), np.float32)
    for l, lev in enumerate(pyr):
        H2, W2 = lev.shape[1:]
        orc.lib().orc_corr_lookup_level(np.ascontiguousarray(lev).reshape(-1),
                                        np.ascontiguousarray(coords, np.float32).reshape(-1), out,
                                        3, 1, n, H2, W2, float(np.float32(1.0 / (1 << l))), l)
    return out


def test_window_integer_coded_is_bitwise(slk):
    """Batched path with small-integer features: products, partial sums and the
    2x2 means of features and of the volume are all exact, so with coordinates
    that are multiples of 8 (integer at every level) all 196 channels match the
    oracle bitwise, and with integer coordinates the level-0 channels do."""
    announce("corr window integer-coded bitwise")
    h, w, n = 48, 64, 6
    rng = np.random.default_rng(11)
    f = rng.integers(-3, 4, size=(n, 128, h, w)).astype(np.float32)
    ii, jj = wl.cyclic_edges(n)
    B = len(ii)
    g = wl.grid_coords(h, w)[None]
    c1 = (g + rng.integers(-6, 7, size=(B, 2, h * w))).astype(np.float32)
    c8 = (g // 8 * 8 + 8 * rng.integers(-1, 2, size=(B, 2, h * w))).astype(np.float32)
    ctx = slk.Context(h, w, C=128, max_batch=B, corr_scale=1.0 / 16.0)
    fd = slk.DeviceArray.from_host(f)
    outs = []
    for c in (c1, c8):
        cd = slk.DeviceArray.from_host(c)
        out = slk.DeviceArray((B, 196, h * w))
        ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out)
        slk.hip().sync()
        outs.append(out.to_host())
    ctx.close()
    ref1 = orc.corr_batch(f, ii, jj, c1, 1.0 / 16.0)
    np.testing.assert_array_equal(outs[0][:, :49], ref1[:, :49])
    ref8 = orc.corr_batch(f, ii, jj, c8, 1.0 / 16.0)
    np.testing.assert_array_equal(outs[1], ref8)


def test_window_fp16_features(slk):
    """fp16 feature maps (the reference's fmap storage) through the batched path."""
    h, w, n = 24, 32, 5
    f = wl.frames(n, C=128, h=h, w=w, seed=12).astype(np.float16)
    ii, jj = wl.cyclic_edges(n)
    B = len(ii)
    coords = wl.flow_coords(B, h, w, seed=13)
    ctx = slk.Context(h, w, C=128, max_batch=B, corr_scale=1.0 / 16.0)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((B, 196, h * w))
    ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out, dtype=slk.SLK_F16)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    ref = orc.corr_batch(f.astype(np.float32), ii, jj, coords, 1.0 / 16.0)
    assert_close_rel(got, ref, tol=F16X3_TOL, what="fp16 window")


def test_window_fp16_features_config2(slk):
    """Config corr_window with the reference's fp16 fmaps (main.cu:677): 12
    frames of 128x48x64, 48 edges. Under the scaled fp16 split an fp16 fmap
    is its own hi (lo = 0): level-0 target tiles take the one pass hi.hi,
    whose products are the exact fp16 x fp16 products of the reference's
    cublasGemmEx (main.cu:1508-1515,1573-1581), pooled tiles hi.hi + hi.lo.
    Six edges in full against the fp64 oracle on the fp16 values: level 0
    (channels 0..48) is fp32 accumulation of exact products, the pooled
    levels carry the 22-bit split of their fp32 means; a dropped pooled lo
    pass would be ~2^-12 off and fail the bar."""
    announce("corr window 48 edges, fp16 fmaps")
    h, w, n, B = 48, 64, 12, 48
    f = wl.frames(n, C=128, h=h, w=w, seed=22).astype(np.float16)
    ii, jj = wl.cyclic_edges(n)
    coords = wl.flow_coords(B, h, w, seed=23)
    ctx = slk.Context(h, w, C=128, max_batch=B, corr_scale=1.0 / 16.0)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((B, 196, h * w))
    ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out, dtype=slk.SLK_F16)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    full = [0, 9, 21, 30, 38, 47]
    ref = orc.corr_batch(f.astype(np.float32), ii[full], jj[full], coords[full], 1.0 / 16.0)
    for k, e in enumerate(full):
        print(f"edge {e}: level 0 {_err_ratio(got[e][:49], ref[k][:49]):.3g}, "
              f"levels 1-3 {_err_ratio(got[e][49:], ref[k][49:]):.3g}")
        assert_close_rel(got[e][:49], ref[k][:49], tol=1e-6, what=f"edge {e} level 0")
        assert_close_rel(got[e], ref[k], tol=F16X3_TOL, what=f"edge {e}")


def _window_of(slk, f, coords, ii, jj, alpha=1.0 / 16.0, prec=None):
    n, C, h, w = f.shape
    ctx = slk.Context(h, w, C=C, max_batch=len(ii), corr_scale=alpha)
    if prec is not None:
        ctx.set_corr_precision(prec)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((len(ii), 196, h * w))
    ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    return got


def _err_ratio(got, ref):
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms)))


@pytest.mark.parametrize("prec", [2, 0])
def test_split_precision_wide_range_and_coherent_lo(slk, prec):
    """Margins of the hi/lo splits (hi.hi + hi.lo + lo.hi, lo.lo dropped)
    where they are smallest, for the scaled fp16 split (prec 2, the default,
    held to F16X3_TOL) and the bf16 split (prec 0, held to helpers.TOL):
    * wide dynamic range: every feature N(0,1) * 2^U(-8, 8), each channel
      also scaled by 2^U(-4, 4), so the result is dominated by a few large
      products and the small ones sit many binades below;
    * coherent lo: every feature is +-(1 + 2^-p) * 2^k, the split's half-way
      case (p = 11 for fp16, 8 for bf16: hi = 1, lo = 2^-p, the largest lo
      relative to hi), with signs that agree along the channels, so the
      dropped lo.lo terms (2^-2p of each product) add up instead of
      cancelling.
    The error ratios are printed."""
    h, w, n = 24, 32, 5
    bar, p = (F16X3_TOL, 11) if prec == 2 else (TOL, 8)
    ii, jj = wl.cyclic_edges(n)
    coords = wl.flow_coords(len(ii), h, w, seed=41)
    rng = np.random.default_rng(40)
    wide = (rng.standard_normal((n, 128, h, w)) * np.exp2(rng.uniform(-8, 8, (n, 128, h, w)))
            * np.exp2(rng.uniform(-4, 4, (1, 128, 1, 1)))).astype(np.float32)
    sign = np.where(rng.random((n, 1, h, w)) < 0.5, -1.0, 1.0)
    coh = (sign * (1.0 + 2.0 ** -p) * np.exp2(rng.integers(-2, 3, (n, 1, h, w)))
           * np.ones((1, 128, 1, 1))).astype(np.float32)
    for name, f in (("wide range", wide), ("coherent lo", coh)):
        got = _window_of(slk, f, coords, ii, jj, prec=prec)
        ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
        print(f"prec {prec} {name}: max |g - r| / max(|r|, rms) = {_err_ratio(got, ref):.3g}")
        assert_close_rel(got, ref, tol=bar, what=name)


def test_split_scale_per_pixel(slk):
    """Pixels many binades below their frame's largest: source frames 0, 1
    hold N(0,1) features times one factor 2^U(-24, 24) per pixel, target
    frames 2, 3 plain N(0,1). Under the scaled fp16 split every pixel takes
    its own scale, so each output is held to F16X3_TOL relative to the bound
    alpha |f_i| max_q |f_j(q)| of its own source pixel i (Cauchy-Schwarz over
    the channels; a pooled target's norm and a bilinear sample of cells never
    exceed the largest level-0 norm). One scale per frame would flush the
    small pixels' fp16 operands to zero (errors of order 1 against that
    bound). The worst ratio is printed."""
    h, w = 24, 32
    ii = np.array([0, 1, 0, 1], np.int32)
    jj = np.array([2, 3, 3, 2], np.int32)
    rng = np.random.default_rng(50)
    f = rng.standard_normal((4, 128, h, w))
    f[:2] *= np.exp2(rng.uniform(-24, 24, (2, 1, h, w)))
    f = f.astype(np.float32)
    coords = wl.flow_coords(len(ii), h, w, seed=51)
    got = _window_of(slk, f, coords, ii, jj, prec=2)
    ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
    norms = np.sqrt((f.astype(np.float64) ** 2).sum(axis=1)).reshape(4, h * w)
    bound = (1.0 / 16.0) * norms[ii][:, None, :] * norms[jj].max(axis=1)[:, None, None]
    ratio = float(np.max(np.abs(got.astype(np.float64) - ref) / bound))
    print(f"per-pixel scale: max |g - r| / (alpha |f_i| max|f_j|) = {ratio:.3g}")
    assert ratio <= F16X3_TOL


def test_device_indices_and_chunking(slk):
    """Device-resident ii/jj, and B above max_batch (processed in chunks)."""
    h, w = 24, 32
    f, ii, jj, coords, out_a = _window(slk, 6, h, w, 10, seed=30, max_batch=4)
    _, _, _, _, out_b = _window(slk, 6, h, w, 10, seed=30, max_batch=48, dev_idx=True)
    np.testing.assert_array_equal(out_a, out_b)
    ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
    assert_close_rel(out_a, ref)


def test_highres_shape(slk):
    """Config highres geometry: 54x96 (HW = 5184, not a multiple of the 128-pixel tile)."""
    announce("highres 54x96, 3 edges")
    h, w = 54, 96
    f, ii, jj, coords, out = _window(slk, 16, h, w, 3, seed=40)
    ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
    assert_close_rel(out, ref)


def test_standalone_pool_sample_and_layout_kernels(slk):
    rng = np.random.default_rng(5)
    h, w, M = 12, 16, 3
    HW = h * w
    vol = rng.standard_normal((M * HW, h, w)).astype(np.float32)
    vd = slk.DeviceArray.from_host(vol)
    pd = slk.DeviceArray((M * HW, h // 2, w // 2))
    slk.check(slk.lib().slk_avg_pool_2x2(vd.ptr, pd.ptr, M * HW, h, w, None))
    slk.hip().sync()
    np.testing.assert_array_equal(pd.to_host(), orc.avg_pool_2x2(vol))
    coords = wl.flow_coords(M, h, w, seed=6)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((M, 196, HW))
    out.zero()
    lvl1 = pd.to_host()
    slk.check(slk.lib().slk_corr_sample_level(pd.ptr, cd.ptr, out.ptr, M, 3, h, w, h // 2, w // 2,
                                              HW, 0.5, 1, None))
    slk.hip().sync()
    got = out.to_host()
    for e in range(M):
        ref = np.zeros((196, HW), np.float32)
        orc.lib().orc_corr_lookup_level(np.ascontiguousarray(lvl1[e * HW:(e + 1) * HW]).reshape(-1),
                                        np.ascontiguousarray(coords[e]).reshape(-1), ref, 3, h, w,
                                        h // 2, w // 2, 0.5, 1)
        assert_close_rel(got[e], ref, tol=1e-5)
        assert not got[e][:49].any() and not got[e][98:].any()
    hw2 = rng.standard_normal((M, HW, 2)).astype(np.float32)
    hd = slk.DeviceArray.from_host(hw2)
    chw = slk.DeviceArray((M, 2, HW))
    slk.check(slk.lib().slk_coords_hw2_to_2hw(hd.ptr, chw.ptr, M, HW, None))
    slk.hip().sync()
    np.testing.assert_array_equal(chw.to_host(), hw2.transpose(0, 2, 1))


def test_prepared_frames_match_per_call_preparation(slk):
    """slk_corr_prepare_frames + _prepared batches: bitwise the windows and
    lookups of slk_corr_batch_build_and_sample on the same fmaps, for a
    100-keyframe graph whose batches touch more frames than one launch
    prepares (B = 130 > max_batch = 48: several launches), with fp32 and
    fp16 fmaps; frame indices outside the prepared frames are rejected."""
    announce("prepared frames, 100 keyframes, 130 edges")
    h, w, n, B = 24, 32, 100, 130
    rng = np.random.default_rng(60)
    ii = rng.integers(0, n, B).astype(np.int32)
    jj = rng.integers(0, n, B).astype(np.int32)
    coords = wl.flow_coords(B, h, w, seed=61)
    cd = slk.DeviceArray.from_host(coords)
    for dtype, f in [(slk.SLK_F32, wl.frames(n, C=128, h=h, w=w, seed=62)),
                     (slk.SLK_F16, wl.frames(n, C=128, h=h, w=w, seed=63).astype(np.float16))]:
        ctx = slk.Context(h, w, C=128, max_batch=48, corr_scale=1.0 / 16.0)
        fd = slk.DeviceArray.from_host(f)
        a = slk.DeviceArray((B, 196, h * w))
        b = slk.DeviceArray((B, 196, h * w))
        ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, a, dtype=dtype)
        ctx.prepare_frames(fd, n, dtype=dtype)
        ctx.batch_build_and_sample_prepared(ii, jj, cd, b)
        slk.hip().sync()
        np.testing.assert_array_equal(b.to_host(), a.to_host())
        with pytest.raises(slk.SlkError):
            ctx.batch_build_and_sample_prepared(np.array([n], np.int32), np.array([0], np.int32),
                                                cd, b)
        ctx.close()
    # and against the oracle on a few edges
    full = [0, 57, 129]
    f = wl.frames(n, C=128, h=h, w=w, seed=62)
    ref = orc.corr_batch(f, ii[full], jj[full], coords[full], 1.0 / 16.0)
    ctx = slk.Context(h, w, C=128, max_batch=48, corr_scale=1.0 / 16.0)
    fd = slk.DeviceArray.from_host(f)
    out = slk.DeviceArray((B, 196, h * w))
    ctx.prepare_frames(fd, n)
    ctx.batch_build_and_sample_prepared(ii, jj, cd, out)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    for k, e in enumerate(full):
        assert_close_rel(got[e], ref[k], what=f"prepared edge {e}")
