"""numpy front-end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product library in
slam-hands_amd/ never imports this module.

Each wrapper names the reference function it restates (file:line in
vibekernels/slam-hands); the C side (oracle.c) carries statement-level
citations. Internals are fp64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile liboracle.so with gcc (make in oracle/)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        c_int, c_long, c_float, c_double = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double
        sig = {
            "orc_corr_volume": [_f32p, _f32p, c_int, c_int, c_double, _f32p],
            "orc_corr_volume_f16": [_u16p, _u16p, c_int, c_int, c_double, _f32p],
            "orc_avg_pool_2x2": [_f32p, _f32p, c_long, c_int, c_int],
            "orc_corr_lookup_level": [_f32p, _f32p, _f32p, c_int, c_int, c_int, c_int, c_int,
                                      c_float, c_int],
            "orc_corr_batch": [_f32p, c_int, c_int, c_int, _i32p, _i32p, c_int, _f32p, _f32p,
                               c_int, c_int, c_double],
            "orc_act_se3": [_f64p, _f64p, _f64p, _f64p],
            "orc_adj_se3": [_f64p, _f64p, _f64p, _f64p],
            "orc_rel_se3": [_f64p, _f64p, _f64p, _f64p, _f64p, _f64p],
            "orc_exp_se3": [_f64p, _f64p, _f64p],
            "orc_retr_se3": [_f64p, _f64p, _f64p, _f64p, _f64p],
            "orc_projmap": [_f32p, _f32p, _f32p, _i32p, _i32p, _f32p, _f32p, c_int, c_int, c_int],
            "orc_pose_retr": [_f32p, _f32p, c_int, c_int],
            "orc_disp_retr": [_f32p, _f32p, _i32p, c_int, c_int],
            "orc_frame_distance": [_f32p, _f32p, _f32p, _i32p, _i32p, _f32p, c_int, c_int, c_int,
                                   c_float],
            "orc_ba_linearize": [_f32p, _f32p, _f32p, _f32p, _f32p, _i32p, _i32p, _f64p, _f64p,
                                 _f64p, _f64p, _f64p, _f64p, c_int, c_int, c_int],
            "orc_cholesky_solve": [_f64p, _f64p, c_int],
        }
        for name, argtypes in sig.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = None
        L.orc_cholesky_solve.restype = c_int
        L.orc_num_threads.argtypes = []
        L.orc_num_threads.restype = c_int
        # orc_ba_iterate takes optional (NULL-able) debug outputs
        L.orc_ba_iterate.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i32p, _i32p,
                                     c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_float,
                                     c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p]
        L.orc_ba_iterate.restype = c_int
        vp = ctypes.c_void_p
        glue = {
            "orc_compute_motion": ([_f32p, _f32p, vp, _f32p, c_int, c_int, c_int], None),
            "orc_compute_target": ([_f32p, _f32p, _f32p, _f32p, _f32p, c_int, c_int], None),
            "orc_gather_rows": ([_f32p, _f32p, vp, c_int, c_long], None),
            "orc_scatter_rows": ([_f32p, _f32p, vp, c_int, c_long], None),
            "orc_scatter_mean": ([_f32p, _f32p, _i32p, c_int, c_long, _i32p], c_int),
            "orc_proximity_select": ([_f32p, c_int, c_int, c_int, c_int, c_int, c_float,
                                      _i32p, _i32p, c_int, _i32p, _i32p, c_int, c_int, _i32p,
                                      _i32p, c_int, ctypes.POINTER(c_int)], c_int),
            "orc_ba_edge_set": ([_i32p, _i32p, c_int, _i32p, _i32p, c_int, _f32p, _f32p,
                                 _f32p, _f32p, c_int, c_int, c_int, c_int, _i32p, _i32p,
                                 _f32p, _f32p, ctypes.POINTER(c_int)], c_int),
            "orc_oldest_mask": ([_i32p, c_int, c_int, _u8p], None),
            "orc_store_and_remove_edges": ([_u8p, c_int, _i32p, _i32p, _i32p, _i32p, _i32p,
                                            ctypes.POINTER(c_int), c_int, _f32p, c_long, _f32p,
                                            _f32p, _f32p, _f32p, c_long], c_int),
            "orc_init_new_edges": ([_f32p, _f32p, _f32p, _i32p, c_int, c_int, c_long, c_long],
                                   None),
            "orc_rm_keyframe": ([c_int, c_int, _f32p, _f32p, _f32p, c_long, _f32p, _f32p,
                                 c_long, c_long, _i32p, _i32p, _i32p, c_int,
                                 ctypes.POINTER(c_int), _i32p, _i32p, c_int,
                                 ctypes.POINTER(c_int), _f32p, _f32p, _f32p, _f32p, _f32p],
                                None),
        }
        for name, (argtypes, restype) in glue.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = L
    return _lib


def num_threads():
    return lib().orc_num_threads()


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ----------------------------------------------------------------- correlation
def corr_volume(fi, fj, alpha):
    """cuda_slam/main.cu:1500-1515: vol[p, q] = alpha * sum_c fi[c, p] fj[c, q]."""
    if fi.dtype == np.float16:
        C = fi.shape[0]
        HW = fi.size // C
        out = np.empty((HW, HW), np.float32)
        lib().orc_corr_volume_f16(_c(fi, np.float16).view(np.uint16).reshape(-1),
                                  _c(fj, np.float16).view(np.uint16).reshape(-1), C, HW,
                                  float(alpha), out)
        return out
    C = fi.shape[0]
    HW = fi.size // C
    out = np.empty((HW, HW), np.float32)
    lib().orc_corr_volume(_c(fi, np.float32), _c(fj, np.float32), C, HW, float(alpha), out)
    return out


def avg_pool_2x2(x):
    """cuda_slam/main.cu:1150-1170 over the last two axes, floor shapes."""
    x = _c(x, np.float32)
    H, W = x.shape[-2:]
    N = x.size // (H * W)
    out = np.empty(x.shape[:-2] + (H // 2, W // 2), np.float32)
    lib().orc_avg_pool_2x2(x, out, N, H, W)
    return out


def pyramid(vol, h, w, levels=4):
    """Levels of one edge: [HW, h>>l, w>>l] (main.cu:1519-1524, 1584-1597)."""
    HW = vol.shape[0]
    pyr = [vol.reshape(HW, h, w)]
    for _ in range(1, levels):
        pyr.append(avg_pool_2x2(pyr[-1]))
    return pyr


def lookup(pyr, coords, r=3):
    """main.cu:1529-1552 / 1599-1612: [levels*(2r+1)^2, HW] for one edge.
    coords: [2, h, w] or [2, HW] (x plane, y plane)."""
    levels = len(pyr)
    HW1, H1, W1 = pyr[0].shape[0], pyr[0].shape[1], pyr[0].shape[2]
    D = 2 * r + 1
    out = np.zeros((levels * D * D, HW1), np.float32)
    cc = _c(coords, np.float32).reshape(2, HW1)
    for l, lev in enumerate(pyr):
        H2, W2 = lev.shape[1], lev.shape[2]
        lib().orc_corr_lookup_level(_c(lev, np.float32).reshape(-1), cc.reshape(-1), out, r,
                                    H1, W1, H2, W2, float(np.float32(1.0 / (1 << l))), l)
    return out


def corr_batch(fmaps, ii, jj, coords, alpha, levels=4, r=3):
    """batch_build_and_sample_correlation (main.cu:1555-1613) on fp32 fmaps
    [nframes, C, h, w], coords [B, 2, h*w] -> [B, levels*(2r+1)^2, h*w]."""
    n, C, h, w = fmaps.shape
    B = len(ii)
    D = 2 * r + 1
    out = np.zeros((B, levels * D * D, h * w), np.float32)
    lib().orc_corr_batch(_c(fmaps, np.float32).reshape(-1), C, h, w, _c(ii, np.int32),
                         _c(jj, np.int32), B, _c(coords, np.float32).reshape(-1), out, levels, r,
                         float(alpha))
    return out


# ------------------------------------------------------------------------- SE3
def act_se3(t, q, X):
    Y = np.zeros(4)
    lib().orc_act_se3(_c(t, np.float64), _c(q, np.float64), _c(X, np.float64), Y)
    return Y


def adj_se3(t, q, X):
    Y = np.zeros(6)
    lib().orc_adj_se3(_c(t, np.float64), _c(q, np.float64), _c(X, np.float64), Y)
    return Y


def rel_se3(ti, qi, tj, qj):
    tij, qij = np.zeros(3), np.zeros(4)
    lib().orc_rel_se3(_c(ti, np.float64), _c(qi, np.float64), _c(tj, np.float64),
                      _c(qj, np.float64), tij, qij)
    return tij, qij


def exp_se3(xi):
    t, q = np.zeros(3), np.zeros(4)
    lib().orc_exp_se3(_c(xi, np.float64), t, q)
    return t, q


def retr_se3(xi, t, q):
    t1, q1 = np.zeros(3), np.zeros(4)
    lib().orc_retr_se3(_c(xi, np.float64), _c(t, np.float64), _c(q, np.float64), t1, q1)
    return t1, q1


def projmap(poses, disps, intr, ii, jj, H, W):
    """se3.cuh:118-177 -> coords [M, H, W, 2], valid [M, H, W]."""
    M = len(ii)
    coords = np.zeros((M, H, W, 2), np.float32)
    valid = np.zeros((M, H, W), np.float32)
    lib().orc_projmap(_c(poses, np.float32).reshape(-1), _c(disps, np.float32).reshape(-1),
                      _c(intr, np.float32), _c(ii, np.int32), _c(jj, np.int32), coords, valid,
                      M, H, W)
    return coords, valid


def pose_retr(poses, dx, t0, t1):
    """se3.cuh:179-193, returns the updated copy."""
    p = _c(poses, np.float32).copy()
    lib().orc_pose_retr(p.reshape(-1), _c(dx, np.float32).reshape(-1), t0, t1)
    return p


def disp_retr(disps, dz, inds):
    d = _c(disps, np.float32).copy()
    HW = d[0].size
    lib().orc_disp_retr(d.reshape(-1), _c(dz, np.float32).reshape(-1), _c(inds, np.int32),
                        len(inds), HW)
    return d


def frame_distance(poses, disps, intr, ii, jj, H, W, beta):
    dist = np.zeros(len(ii), np.float32)
    lib().orc_frame_distance(_c(poses, np.float32).reshape(-1),
                             _c(disps, np.float32).reshape(-1), _c(intr, np.float32),
                             _c(ii, np.int32), _c(jj, np.int32), dist, len(ii), H, W,
                             float(beta))
    return dist


# -------------------------------------------------------------------------- BA
def ba_linearize(target, weight, poses, disps, intr, ii, jj, H, W):
    """projective_transform_kernel (ba.cuh:39-221), fp64 outputs."""
    M = len(ii)
    HW = H * W
    Hs = np.zeros((4, M, 6, 6))
    vs = np.zeros((2, M, 6))
    Eii = np.zeros((M, 6, HW))
    Eij = np.zeros((M, 6, HW))
    Cii = np.zeros((M, HW))
    bz = np.zeros((M, HW))
    lib().orc_ba_linearize(_c(target, np.float32).reshape(-1),
                           _c(weight, np.float32).reshape(-1),
                           _c(poses, np.float32).reshape(-1), _c(disps, np.float32).reshape(-1),
                           _c(intr, np.float32), _c(ii, np.int32), _c(jj, np.int32),
                           Hs.reshape(-1), vs.reshape(-1), Eii.reshape(-1), Eij.reshape(-1),
                           Cii.reshape(-1), bz.reshape(-1), M, H, W)
    return Hs, vs, Eii, Eij, Cii, bz


def ba_iterate(poses, disps, intr, target, weight, eta, ii, jj, H, W, t0, t1, lm, ep,
               motion_only=False):
    """One BundleAdjustment::iterate (ba.cuh:476-803). Returns a dict with the
    updated poses/disps (copies) and the debug system S, b, dx, dz."""
    poses = _c(poses, np.float32).copy()
    disps = _c(disps, np.float32).copy()
    nframes = poses.shape[0]
    HW = H * W
    n = 6 * (t1 - t0)
    S = np.zeros((n, n))
    b = np.zeros(n)
    dx = np.zeros(n)
    dz = np.zeros((nframes, HW))
    st = lib().orc_ba_iterate(poses.reshape(-1), disps.reshape(-1), _c(intr, np.float32),
                              _c(target, np.float32).reshape(-1),
                              _c(weight, np.float32).reshape(-1),
                              _c(eta, np.float32).reshape(-1), _c(ii, np.int32),
                              _c(jj, np.int32), len(ii), nframes, H, W, t0, t1, float(lm),
                              float(ep), int(bool(motion_only)), S.ctypes.data, b.ctypes.data,
                              dx.ctypes.data, dz.ctypes.data)
    return {"status": st, "poses": poses, "disps": disps, "S": S, "b": b, "dx": dx, "dz": dz}


def cholesky_solve(S, b):
    S = _c(S, np.float64).copy()
    b = _c(b, np.float64).copy()
    st = lib().orc_cholesky_solve(S, b, len(b))
    return st, b


# ------------------------------------------------------------ update glue
def _ptr_or_null(a, dtype):
    return None if a is None else _c(a, dtype).ctypes.data


def compute_motion(coords1, target, h, w, coords0=None):
    """compute_motion_kernel (main.cu:1250-1273): [B][4][h*w]; coords0 None
    is the identity grid of alloc_coords0 (main.cu:2150-2163)."""
    c1 = _c(coords1, np.float32)
    B = c1.shape[0]
    c0 = None if coords0 is None else _c(coords0, np.float32)
    m = np.zeros((B, 4, h * w), np.float32)
    lib().orc_compute_motion(m.reshape(-1), c1.reshape(-1),
                             None if c0 is None else c0.ctypes.data,
                             _c(target, np.float32).reshape(-1), B, h, w)
    return m


def compute_target(coords, delta, wt_raw):
    """compute_target_kernel (main.cu:1282-1301): (target, weight) [n][2][hw]."""
    coords = _c(coords, np.float32)
    n, _, hw = coords.shape
    t = np.zeros((n, 2, hw), np.float32)
    wo = np.zeros((n, 2, hw), np.float32)
    lib().orc_compute_target(t.reshape(-1), wo.reshape(-1), coords.reshape(-1),
                             _c(delta, np.float32).reshape(-1),
                             _c(wt_raw, np.float32).reshape(-1), n, hw)
    return t, wo


def gather_rows(src, idx, n=None):
    """dst[e] = src[idx[e]] (the per-edge copy loops, main.cu:2216-2224)."""
    src = _c(src, np.float32)
    row = int(np.prod(src.shape[1:]))
    idx = None if idx is None else _c(idx, np.int32)
    n = len(idx) if idx is not None else n
    dst = np.zeros((n,) + src.shape[1:], np.float32)
    lib().orc_gather_rows(dst.reshape(-1), src.reshape(-1),
                          None if idx is None else idx.ctypes.data, n, row)
    return dst


def scatter_rows(dst, src, idx):
    """dst[idx[e]] = src[e] (main.cu:2245-2252, 2305-2309), on a copy of dst."""
    dst = _c(dst, np.float32).copy()
    src = _c(src, np.float32)
    row = int(np.prod(src.shape[1:]))
    idx = None if idx is None else _c(idx, np.int32)
    lib().orc_scatter_rows(dst.reshape(-1), src.reshape(-1),
                           None if idx is None else idx.ctypes.data, src.shape[0], row)
    return dst


def scatter_mean(src, ii):
    """GraphAgg scatter_mean (main.cu:2258-2296): (dst [na][...], active [na])."""
    src = _c(src, np.float32)
    ii = _c(ii, np.int32)
    n = len(ii)
    row = int(np.prod(src.shape[1:]))
    dst = np.zeros((max(n, 1),) + src.shape[1:], np.float32)
    active = np.zeros(max(n, 1), np.int32)
    na = lib().orc_scatter_mean(dst.reshape(-1), src.reshape(-1), ii, n, row, active)
    return dst[:na], active[:na]


def ba_edge_set(ii, jj, ii_inac, jj_inac, target, weight, target_inac, weight_inac,
                num_keyframes, forced_t0=-1, use_inactive=True):
    """BA edge set of run_update_pass (main.cu:2312-2390): dict with ii, jj,
    target, weight of the combined edges and t0."""
    ii, jj = _c(ii, np.int32), _c(jj, np.int32)
    ii_inac, jj_inac = _c(ii_inac, np.int32), _c(jj_inac, np.int32)
    target, weight = _c(target, np.float32), _c(weight, np.float32)
    hw = target.shape[2]
    target_inac = _c(target_inac, np.float32).reshape(-1, 2, hw)
    weight_inac = _c(weight_inac, np.float32).reshape(-1, 2, hw)
    cap = max(len(ii) + len(ii_inac), 1)
    bi = np.zeros(cap, np.int32)
    bj = np.zeros(cap, np.int32)
    bt = np.zeros((cap, 2, hw), np.float32)
    bw = np.zeros((cap, 2, hw), np.float32)
    t0 = ctypes.c_int(0)
    m = lib().orc_ba_edge_set(ii, jj, len(ii), ii_inac, jj_inac, len(ii_inac),
                              target.reshape(-1), weight.reshape(-1),
                              np.ascontiguousarray(target_inac).reshape(-1),
                              np.ascontiguousarray(weight_inac).reshape(-1), hw,
                              int(num_keyframes), int(forced_t0), int(bool(use_inactive)),
                              bi, bj, bt.reshape(-1), bw.reshape(-1), ctypes.byref(t0))
    return {"ii": bi[:m], "jj": bj[:m], "target": bt[:m], "weight": bw[:m], "t0": t0.value}


# ---------------------------------------------------------------- factor graph
def proximity_select(d, t, t0, t1, rad, nms, thresh, ii, jj, ii_inac=(), jj_inac=(),
                     max_factors=0):
    """add_proximity_factors (main.cu:1679-1779) from raw pair distances d
    [(t-t0)*(t-t1)]: (new edges [m][2], number of greedy-step edges)."""
    d = _c(d, np.float32).reshape(-1)
    ii, jj = _c(ii, np.int32), _c(jj, np.int32)
    ii_inac, jj_inac = _c(ii_inac, np.int32), _c(jj_inac, np.int32)
    cap = 2 * (max(t - t0, 0) * (rad + 1) + d.size) + 2
    ni = np.zeros(cap, np.int32)
    nj = np.zeros(cap, np.int32)
    m = ctypes.c_int(0)
    ne = lib().orc_proximity_select(d, int(t), int(t0), int(t1), int(rad), int(nms),
                                    float(thresh), ii, jj, len(ii), ii_inac, jj_inac,
                                    len(ii_inac), int(max_factors), ni, nj, cap,
                                    ctypes.byref(m))
    return np.stack([ni[:m.value], nj[:m.value]], 1), ne


def oldest_mask(age, to_remove):
    """Step 5 of add_proximity_factors (main.cu:1762-1769): uint8 mask of the
    to_remove oldest edges, equal ages in edge order."""
    age = _c(age, np.int32)
    mask = np.zeros(max(len(age), 1), np.uint8)
    lib().orc_oldest_mask(age, len(age), int(to_remove), mask)
    return mask[:len(age)]


def store_and_remove_edges(mask, ii, jj, age, ii_inac, jj_inac, max_inac, nets, target,
                           weight, target_inac, weight_inac):
    """store_and_remove_edges (main.cu:795-836) on copies: dict with the kept
    ii, jj, age, nets, target, weight (their first n_kept rows), the grown
    inactive ii, jj, target, weight, and n_kept / num_inac."""
    mask = np.ascontiguousarray(mask, np.uint8)
    ii, jj, age = (np.array(a, np.int32) for a in (ii, jj, age))
    n = len(ii)
    ni = ctypes.c_int(len(ii_inac))
    cap = max(max_inac, 1)
    iin = np.zeros(cap, np.int32)
    jin = np.zeros(cap, np.int32)
    iin[:len(ii_inac)] = ii_inac
    jin[:len(jj_inac)] = jj_inac
    nets, target, weight = (np.array(a, np.float32) for a in (nets, target, weight))
    net_row = nets[0].size if n else 0
    tw_row = target[0].size if n else 0
    tin = np.zeros((cap, tw_row), np.float32)
    win = np.zeros((cap, tw_row), np.float32)
    if len(target_inac):
        tin[:len(target_inac)] = np.asarray(target_inac, np.float32).reshape(len(target_inac),
                                                                             tw_row)
        win[:len(weight_inac)] = np.asarray(weight_inac, np.float32).reshape(len(weight_inac),
                                                                             tw_row)
    kept = lib().orc_store_and_remove_edges(mask, n, ii, jj, age, iin, jin, ctypes.byref(ni),
                                            int(max_inac), nets.reshape(-1), net_row,
                                            target.reshape(-1), weight.reshape(-1),
                                            tin.reshape(-1), win.reshape(-1), tw_row)
    m = ni.value
    return {"n_kept": kept, "ii": ii[:kept], "jj": jj[:kept], "age": age[:kept],
            "nets": nets[:kept], "target": target[:kept], "weight": weight[:kept],
            "num_inac": m, "ii_inac": iin[:m], "jj_inac": jin[:m],
            "target_inac": tin[:m].reshape((m,) + np.shape(target)[1:]),
            "weight_inac": win[:m].reshape((m,) + np.shape(weight)[1:])}


def init_new_edges(nets, edge_nets, weight, ii, first, count):
    """Hidden states of new edges (main.cu:1786-1796) on copies: (edge_nets,
    weight) with rows [first, first + count) set."""
    nets = _c(nets, np.float32)
    en, w = np.array(edge_nets, np.float32), np.array(weight, np.float32)
    lib().orc_init_new_edges(nets.reshape(-1), en.reshape(-1), w.reshape(-1), _c(ii, np.int32),
                             int(first), int(count), en[0].size, w[0].size)
    return en, w


def rm_keyframe(ix, st):
    """CudaDroid::rm_keyframe (main.cu:866-941) on copies of the state dict
    st (poses [t,7], disps [t,hw], fmaps [t,...] any dtype, nets/inps [t,...],
    ii/jj/age, ii_inac/jj_inac, edge_nets/target/weight, target_inac/
    weight_inac): the same dict after the removal (lists cut to their new
    lengths; arrays keep their row counts)."""
    o = {k: np.array(v) for k, v in st.items()}
    t = len(o["poses"])
    fm = np.ascontiguousarray(o["fmaps"]).view(np.float32).reshape(t, -1)
    hw = o["disps"][0].size
    net_row = o["nets"][0].size
    for k in ("poses", "disps", "nets", "inps", "edge_nets", "target", "weight", "target_inac",
              "weight_inac"):
        o[k] = np.ascontiguousarray(o[k], np.float32)
    for k in ("ii", "jj", "age", "ii_inac", "jj_inac"):
        o[k] = np.ascontiguousarray(o[k], np.int32)
    nk, nik = ctypes.c_int(0), ctypes.c_int(0)
    flat = lambda a: a.reshape(-1) if a.size else np.zeros(1, a.dtype)
    lib().orc_rm_keyframe(int(ix), t, flat(o["poses"]), flat(o["disps"]), flat(fm),
                          fm.shape[1], flat(o["nets"]), flat(o["inps"]), net_row, hw,
                          flat(o["ii"]), flat(o["jj"]), flat(o["age"]), len(o["ii"]),
                          ctypes.byref(nk), flat(o["ii_inac"]), flat(o["jj_inac"]),
                          len(o["ii_inac"]), ctypes.byref(nik), flat(o["edge_nets"]),
                          flat(o["target"]), flat(o["weight"]), flat(o["target_inac"]),
                          flat(o["weight_inac"]))
    o["fmaps"] = fm.view(np.asarray(st["fmaps"]).dtype).reshape(np.shape(st["fmaps"]))
    for k in ("ii", "jj", "age"):
        o[k] = o[k][:nk.value]
    for k in ("ii_inac", "jj_inac"):
        o[k] = o[k][:nik.value]
    return o
