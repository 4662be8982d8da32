"""ctypes binding of libslk (include/slk.h) plus the minimal HIP runtime calls
the tests and the benchmark need (device buffers, streams, events).

This is plumbing around the C ABI, not a second implementation: every compute
call goes to the gfx950 kernels in libslk.so, and a missing library or GPU is
an error, never a fallback.

Names mirror the reference's C++ members (cuda_slam/main.cu CudaDroid,
cuda_slam/ba.cuh BundleAdjustment, cuda_slam/corr.cuh CorrBlock).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libslk.so")
HIP_LIB = "libamdhip64.so"

SLK_OK, SLK_E_ARG, SLK_E_HIP, SLK_E_NOT_SPD, SLK_E_STATE = range(5)
SLK_F32, SLK_F16 = 0, 1
SLK_PREC_BF16X3, SLK_PREC_FP32, SLK_PREC_F16X3 = 0, 1, 2

# every entry point declared in include/slk.h
EXPORTS = [
    "slk_create", "slk_destroy", "slk_last_error", "slk_profile_enable", "slk_profile_kernel",
    "slk_set_corr_precision",
    "slk_corr_batch_build_and_sample", "slk_corr_batch_build_and_sample_dev",
    "slk_corr_batch_build_and_sample_dev_noalloc", "slk_corr_prepare_frames", "slk_corr_batch_build_and_sample_prepared",
    "slk_corr_build", "slk_corr_sample", "slk_corr_level", "slk_avg_pool_2x2",
    "slk_corr_sample_level", "slk_coords_hw2_to_2hw",
    "slk_projmap", "slk_pose_retr", "slk_disp_retr", "slk_frame_distance", "slk_clamp_disps",
    "slk_ba_iterate", "slk_ba_iterate_n", "slk_ba_status", "slk_ba_set_wait_limit", "slk_ba_last_system", "slk_ba_projective_transform",
    "slk_ba_accum", "slk_ba_damping_q", "slk_ba_eet6x6", "slk_ba_ev6x1", "slk_ba_evt6x1",
    "slk_ba_depth_update",
    "slk_compute_motion", "slk_fill_coords0", "slk_compute_target", "slk_gather_rows",
    "slk_scatter_rows", "slk_scatter_mean", "slk_ba_edge_set", "slk_proximity_factors",
    "slk_oldest_edges_mask", "slk_store_and_remove_edges", "slk_init_new_edges",
    "slk_rm_keyframe",
    "slk_update_create", "slk_update_destroy", "slk_update_num_layers", "slk_update_layer_name",
    "slk_update_layer_shape", "slk_update_set_conv", "slk_update_load_dir", "slk_update_forward",
    "slk_update_compute_eta", "slk_motion_filter",
    "slk_encoder_create", "slk_encoder_destroy", "slk_encoder_num_layers",
    "slk_encoder_layer_suffix", "slk_encoder_layer_shape", "slk_encoder_set_conv",
    "slk_encoder_load_dir", "slk_encoder_forward", "slk_encode_frame",
    "slk_nv12_to_bgr", "slk_p010_to_bgr", "slk_bgr8_to_bgrf", "slk_preprocess_image",
    "slk_write_poses_bin",
]


class SlkError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"slk error {code}: {msg}")
        self.code = code


def build():
    """Compile libslk.so for gfx950 (make in slam-hands_amd/)."""
    subprocess.run(["make", "-s", "-j8", "-C", HERE, "libslk.so"], check=True)
    return LIB_PATH


_lib = None
_hip = None

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_long
F = ctypes.c_float


def lib():
    """The loaded libslk.so. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                               "(there is no CPU fallback)")
        L_ = ctypes.CDLL(LIB_PATH)
        sig = {
            "slk_create": [ctypes.POINTER(P), I, I, I, I, I, I, F],
            "slk_destroy": [P],
            "slk_profile_enable": [P, I],
            "slk_profile_kernel": [P, I, ctypes.POINTER(ctypes.c_char_p),
                                   ctypes.POINTER(ctypes.c_double), ctypes.POINTER(I)],
            "slk_set_corr_precision": [P, I],
            "slk_corr_batch_build_and_sample": [P, P, I, L, P, P, I, P, P, P],
            "slk_corr_batch_build_and_sample_dev": [P, P, I, L, P, P, I, P, P, P],
            "slk_corr_batch_build_and_sample_dev_noalloc": [P, I, L, P, P, I, P, P, I, I, I,
                                                            F, P],
            "slk_corr_prepare_frames": [P, P, I, L, I, P],
            "slk_corr_batch_build_and_sample_prepared": [P, P, P, I, P, P, P],
            "slk_corr_build": [P, P, P, I, P],
            "slk_corr_sample": [P, P, P, P],
            "slk_corr_level": [P, I, ctypes.POINTER(P), ctypes.POINTER(I), ctypes.POINTER(I)],
            "slk_avg_pool_2x2": [P, P, L, I, I, P],
            "slk_corr_sample_level": [P, P, P, I, I, I, I, I, I, I, F, I, P],
            "slk_coords_hw2_to_2hw": [P, P, I, I, P],
            "slk_projmap": [P, P, P, P, P, P, P, I, I, I, P],
            "slk_pose_retr": [P, P, I, I, P],
            "slk_disp_retr": [P, P, P, I, I, P],
            "slk_frame_distance": [P, P, P, P, P, P, I, I, I, F, P],
            "slk_clamp_disps": [P, I, F, P],
            "slk_ba_iterate": [P, P, P, P, P, P, P, P, P, P, P, I, I, I, F, F, I, P],
            "slk_ba_iterate_n": [P, P, P, P, P, P, P, P, P, P, P, I, I, I, F, F, I, I, P],
            "slk_ba_status": [P, P],
            "slk_ba_set_wait_limit": [P, I],
            "slk_ba_last_system": [P, P, P, P, ctypes.POINTER(I), P],
            "slk_ba_projective_transform": [P] * 13 + [I, I, I, P],
            "slk_ba_accum": [P, P, P, P, I, I, I, P],
            "slk_ba_damping_q": [P, P, P, P, I, I, F, P],
            "slk_ba_eet6x6": [P, P, P, P, I, I, P],
            "slk_ba_ev6x1": [P, P, P, P, P, I, I, P],
            "slk_ba_evt6x1": [P, P, P, P, I, I, I, P],
            "slk_ba_depth_update": [P, P, P, P, P, I, I, P],
            "slk_compute_motion": [P, P, P, P, I, I, I, P],
            "slk_fill_coords0": [P, I, I, I, P],
            "slk_compute_target": [P, P, P, P, P, I, I, P],
            "slk_gather_rows": [P, P, P, I, L, P],
            "slk_scatter_rows": [P, P, P, I, L, P],
            "slk_scatter_mean": [P, P, P, P, I, L, P, P, ctypes.POINTER(I), P],
            "slk_ba_edge_set": [P, P, P, I, P, P, I, P, P, P, P, I, I, I, I, P, P, P, P, P,
                                P, ctypes.POINTER(I), ctypes.POINTER(I), P],
            "slk_proximity_factors": [P, P, P, P, I, I, I, I, I, F, F, P, P, I, P, P, I, I, P,
                                      P, I, ctypes.POINTER(I), ctypes.POINTER(I), P, P],
            "slk_store_and_remove_edges": [P, P, I, P, P, P, P, P, ctypes.POINTER(I), I, P, L,
                                           P, P, P, P, L, ctypes.POINTER(I), P],
            "slk_init_new_edges": [P, P, P, P, P, I, I, L, L, P],
            "slk_rm_keyframe": [P, I, I, P, P, P, I, P, P, L, P, P, P, I, ctypes.POINTER(I), P,
                                P, I, ctypes.POINTER(I), P, P, P, P, P, P],
        }
        sig.update({
            "slk_update_create": [ctypes.POINTER(P), I, I, I],
            "slk_update_destroy": [P],
            "slk_update_num_layers": [],
            "slk_update_layer_shape": [I, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I)],
            "slk_update_set_conv": [P, I, P, P],
            "slk_update_load_dir": [P, ctypes.c_char_p],
            "slk_update_forward": [P, P, P, P, P, P, P, P, I, P],
            "slk_update_compute_eta": [P, P, P, I, P],
            "slk_motion_filter": [P, P, P, P, I, P, P, ctypes.POINTER(F), P],
            "slk_encoder_create": [ctypes.POINTER(P), I, I, I, I, I],
            "slk_encoder_destroy": [P],
            "slk_encoder_num_layers": [],
            "slk_encoder_layer_shape": [P, I, ctypes.POINTER(I), ctypes.POINTER(I),
                                        ctypes.POINTER(I), ctypes.POINTER(I)],
            "slk_encoder_set_conv": [P, I, P, P],
            "slk_encoder_load_dir": [P, ctypes.c_char_p, ctypes.c_char_p],
            "slk_encoder_forward": [P, P, P, I, P],
            "slk_encode_frame": [P, P, P, P, P, P, P],
            "slk_nv12_to_bgr": [P, P, P, I, I, I, I, I, I, P],
            "slk_p010_to_bgr": [P, P, P, I, I, I, I, I, I, P],
            "slk_bgr8_to_bgrf": [P, P, I, I, I, I, I, P],
            "slk_preprocess_image": [P, P, I, I, P],
            "slk_write_poses_bin": [ctypes.c_char_p, I, P, P, I],
        })
        for name, args in sig.items():
            fn = getattr(L_, name)
            fn.argtypes = args
            fn.restype = I
        L_.slk_oldest_edges_mask.argtypes = [P, I, I, P]
        L_.slk_oldest_edges_mask.restype = None
        L_.slk_update_layer_name.argtypes = [I]
        L_.slk_update_layer_name.restype = ctypes.c_char_p
        L_.slk_encoder_layer_suffix.argtypes = [I]
        L_.slk_encoder_layer_suffix.restype = ctypes.c_char_p
        L_.slk_last_error.argtypes = []
        L_.slk_last_error.restype = ctypes.c_char_p
        _lib = L_
    return _lib


def check(code):
    if code != SLK_OK:
        raise SlkError(code, lib().slk_last_error().decode())
    return code


# ------------------------------------------------------------ HIP runtime --
class Hip:
    """The few libamdhip64 calls used by tests and bench."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        self.h = ctypes.CDLL(HIP_LIB)
        h = self.h
        h.hipMalloc.argtypes = [ctypes.POINTER(P), ctypes.c_size_t]
        h.hipFree.argtypes = [P]
        h.hipMemcpy.argtypes = [P, P, ctypes.c_size_t, I]
        h.hipMemcpyAsync.argtypes = [P, P, ctypes.c_size_t, I, P]
        h.hipMemset.argtypes = [P, I, ctypes.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
        h.hipStreamDestroy.argtypes = [P]
        h.hipStreamSynchronize.argtypes = [P]
        h.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        h.hipEventDestroy.argtypes = [P]
        h.hipEventRecord.argtypes = [P, P]
        h.hipEventSynchronize.argtypes = [P]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(F), P, P]
        h.hipGetDeviceCount.argtypes = [ctypes.POINTER(I)]
        h.hipGetErrorString.argtypes = [I]
        h.hipGetErrorString.restype = ctypes.c_char_p
        for fn in ("hipMalloc", "hipFree", "hipMemcpy", "hipMemcpyAsync", "hipMemset",
                   "hipDeviceSynchronize", "hipStreamCreate", "hipStreamDestroy",
                   "hipStreamSynchronize", "hipEventCreate", "hipEventDestroy", "hipEventRecord",
                   "hipEventSynchronize", "hipEventElapsedTime", "hipGetDeviceCount"):
            getattr(h, fn).restype = I

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.h.hipGetErrorString(rc).decode()} ({rc})")

    def device_count(self):
        n = I(0)
        rc = self.h.hipGetDeviceCount(ctypes.byref(n))
        return n.value if rc == 0 else 0

    def malloc(self, nbytes):
        p = P()
        self.ok(self.h.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)), "hipMalloc")
        return p.value

    def free(self, p):
        self.ok(self.h.hipFree(P(p)), "hipFree")

    def htod(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self.ok(self.h.hipMemcpy(P(dst), arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")

    def dtoh(self, arr, src):
        self.ok(self.h.hipMemcpy(arr.ctypes.data, P(src), arr.nbytes, self.D2H), "hipMemcpy D2H")
        return arr

    def memset(self, p, value, nbytes):
        self.ok(self.h.hipMemset(P(p), value, nbytes), "hipMemset")

    def dtod(self, dst, src, nbytes):
        self.ok(self.h.hipMemcpy(P(dst), P(src), int(nbytes), self.D2D), "hipMemcpy D2D")

    def dtod_async(self, dst, src, nbytes, stream=None):
        self.ok(self.h.hipMemcpyAsync(P(dst), P(src), int(nbytes), self.D2D, P(stream)),
                "hipMemcpyAsync D2D")

    def sync(self):
        self.ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self):
        s = P()
        self.ok(self.h.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s):
        self.ok(self.h.hipStreamSynchronize(P(s)), "hipStreamSynchronize")

    def event(self):
        e = P()
        self.ok(self.h.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream=None):
        self.ok(self.h.hipEventRecord(P(ev), P(stream)), "hipEventRecord")

    def elapsed_ms(self, e0, e1):
        self.ok(self.h.hipEventSynchronize(P(e1)), "hipEventSynchronize")
        ms = F(0)
        self.ok(self.h.hipEventElapsedTime(ctypes.byref(ms), P(e0), P(e1)), "hipEventElapsedTime")
        return ms.value


def hip():
    global _hip
    if _hip is None:
        _hip = Hip()
    return _hip


class DeviceArray:
    """A device buffer with a numpy shape/dtype."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = hip().malloc(self.nbytes)

    @classmethod
    def from_host(cls, arr, dtype=None):
        arr = np.ascontiguousarray(arr, dtype=dtype)
        d = cls(arr.shape, arr.dtype)
        hip().htod(d.ptr, arr)
        return d

    def upload(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes == self.nbytes
        hip().htod(self.ptr, arr)

    def to_host(self):
        return hip().dtoh(np.empty(self.shape, self.dtype), self.ptr)

    def zero(self):
        hip().memset(self.ptr, 0, self.nbytes)

    def free(self):
        if self.ptr:
            hip().free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(x):
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    return x


def _host_i32(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data


class Context:
    """slk_ctx: correlation scratch + BA state for h x w feature maps."""

    def __init__(self, h, w, C=128, max_batch=48, levels=4, radius=3, corr_scale=1.0 / 16.0):
        self.h, self.w, self.C, self.levels = h, w, C, levels
        self.corr_precision = SLK_PREC_F16X3  # the library's default
        self.ptr = P()
        check(lib().slk_create(ctypes.byref(self.ptr), h, w, C, max_batch, levels, radius,
                               float(corr_scale)))

    def close(self):
        if self.ptr:
            lib().slk_destroy(self.ptr)
            self.ptr = P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_corr_precision(self, precision):
        check(lib().slk_set_corr_precision(self.ptr, int(precision)))
        self.corr_precision = int(precision)

    # main.cu:1555 batch_build_and_sample_correlation
    def batch_build_and_sample_correlation(self, fmaps, ii, jj, coords, out, dtype=SLK_F32,
                                           fmap_stride=None, stream=None):
        ii_h, ii_p = _host_i32(ii)
        jj_h, jj_p = _host_i32(jj)
        stride = fmap_stride if fmap_stride is not None else self.C * self.h * self.w
        check(lib().slk_corr_batch_build_and_sample(self.ptr, _p(fmaps), dtype, stride, ii_p,
                                                    jj_p, len(ii_h), _p(coords), _p(out), stream))

    def batch_build_and_sample_correlation_dev(self, fmaps, ii_dev, jj_dev, B, coords, out,
                                               dtype=SLK_F32, fmap_stride=None, stream=None):
        stride = fmap_stride if fmap_stride is not None else self.C * self.h * self.w
        check(lib().slk_corr_batch_build_and_sample_dev(self.ptr, _p(fmaps), dtype, stride,
                                                        _p(ii_dev), _p(jj_dev), B, _p(coords),
                                                        _p(out), stream))

    # frames split once per pass, then batches over them (slk_corr_prepare_frames)
    def prepare_frames(self, fmaps, nframes, dtype=SLK_F32, fmap_stride=None, stream=None):
        stride = fmap_stride if fmap_stride is not None else self.C * self.h * self.w
        check(lib().slk_corr_prepare_frames(self.ptr, _p(fmaps), dtype, stride, nframes, stream))

    def batch_build_and_sample_prepared(self, ii, jj, coords, out, stream=None):
        (ii, iip), (_jj, jjp) = _host_i32(ii), _host_i32(jj)
        check(lib().slk_corr_batch_build_and_sample_prepared(
            self.ptr, iip, jjp, len(ii), _p(coords), _p(out), stream))

    # main.cu:1500 build_correlation / :1529 sample_correlation
    def build_correlation(self, f_i, f_j, dtype=SLK_F32, stream=None):
        check(lib().slk_corr_build(self.ptr, _p(f_i), _p(f_j), dtype, stream))

    def sample_correlation(self, coords, out, stream=None):
        check(lib().slk_corr_sample(self.ptr, _p(coords), _p(out), stream))

    def level(self, l):
        ptr, h2, w2 = P(), I(), I()
        check(lib().slk_corr_level(self.ptr, l, ctypes.byref(ptr), ctypes.byref(h2),
                                   ctypes.byref(w2)))
        return ptr.value, h2.value, w2.value

    def level_to_host(self, l):
        ptr, h2, w2 = self.level(l)
        HW = self.h * self.w
        return hip().dtoh(np.empty((HW, h2, w2), np.float32), ptr)

    # ba.cuh:476 BundleAdjustment::iterate
    def ba_iterate(self, poses, disps, intr, target, weight, eta, ii_dev, jj_dev, ii, jj, t0,
                   t1, lm, ep, motion_only=False, stream=None):
        ii_h, ii_p = _host_i32(ii)
        jj_h, jj_p = _host_i32(jj)
        check(lib().slk_ba_iterate(self.ptr, _p(poses), _p(disps), _p(intr), _p(target),
                                   _p(weight), _p(eta), _p(ii_dev), _p(jj_dev), ii_p, jj_p,
                                   len(ii_h), t0, t1, float(lm), float(ep), int(bool(motion_only)),
                                   stream))

    def ba_iterate_n(self, poses, disps, intr, target, weight, eta, ii_dev, jj_dev, ii, jj, t0,
                     t1, lm, ep, iters, motion_only=False, stream=None):
        """`iters` BA iterations on one edge set (slk_ba_iterate_n)."""
        ii_h, ii_p = _host_i32(ii)
        jj_h, jj_p = _host_i32(jj)
        check(lib().slk_ba_iterate_n(self.ptr, _p(poses), _p(disps), _p(intr), _p(target),
                                     _p(weight), _p(eta), _p(ii_dev), _p(jj_dev), ii_p, jj_p,
                                     len(ii_h), t0, t1, float(lm), float(ep),
                                     int(bool(motion_only)), int(iters), stream))

    def profile_enable(self, on=True):
        check(lib().slk_profile_enable(self.ptr, int(bool(on))))

    def profile(self):
        """{kernel name: (total ms, launches)} since profile_enable."""
        out = {}
        k = 0
        while True:
            name, ms, n = ctypes.c_char_p(), ctypes.c_double(), I()
            rc = lib().slk_profile_kernel(self.ptr, k, ctypes.byref(name), ctypes.byref(ms),
                                          ctypes.byref(n))
            if rc == SLK_E_ARG:
                return out
            check(rc)
            out[name.value.decode()] = (ms.value, n.value)
            k += 1

    def ba_status(self, stream=None):
        return lib().slk_ba_status(self.ptr, stream)

    def ba_set_wait_limit(self, polls):
        """Polls before a workgroup of an overlapped BA step stops waiting for
        its solve (negative: the default); see include/slk.h."""
        check(lib().slk_ba_set_wait_limit(self.ptr, polls))

    def ba_last_system(self, stream=None):
        n = I()
        check(lib().slk_ba_last_system(self.ptr, None, None, None, ctypes.byref(n), stream))
        S = np.zeros((n.value, n.value))
        b = np.zeros(n.value)
        dx = np.zeros(n.value)
        check(lib().slk_ba_last_system(self.ptr, S.ctypes.data, b.ctypes.data, dx.ctypes.data,
                                       ctypes.byref(n), stream))
        return S, b, dx


class UpdateModule:
    """slk_update_*: the update operator (UpdateModule / ConvGRU of
    cuda_slam/main.cu:385-667) on device arrays."""

    def __init__(self, max_batch, h, w):
        self.h, self.w, self.max_batch = h, w, max_batch
        p = P()
        check(lib().slk_update_create(ctypes.byref(p), max_batch, h, w))
        self.ptr = p

    @staticmethod
    def layers():
        """[(name, co, ci, k)] in the ABI's layer order."""
        L = lib()
        out = []
        for i in range(L.slk_update_num_layers()):
            co, ci, k = I(), I(), I()
            check(L.slk_update_layer_shape(i, ctypes.byref(co), ctypes.byref(ci), ctypes.byref(k)))
            out.append((L.slk_update_layer_name(i).decode(), co.value, ci.value, k.value))
        return out

    def set_weights(self, weights):
        """weights: {name: (w [co, ci, k, k], b [co]) float32 host arrays}."""
        for i, (name, co, ci, k) in enumerate(self.layers()):
            w, b = weights[name]
            w = np.ascontiguousarray(w, np.float32)
            b = np.ascontiguousarray(b, np.float32)
            assert w.shape == (co, ci, k, k) and b.shape == (co,), name
            check(lib().slk_update_set_conv(self.ptr, i, w.ctypes.data, b.ctypes.data))

    def load_dir(self, path):
        check(lib().slk_update_load_dir(self.ptr, os.fsencode(path)))

    def forward(self, corr, motion, net, inp, delta, weight, agg, batch, stream=None):
        check(lib().slk_update_forward(self.ptr, _p(corr), _p(motion), _p(net), _p(inp),
                                       _p(delta), _p(weight), _p(agg), batch, stream))

    def compute_eta(self, agg, eta, num_kf, stream=None):
        check(lib().slk_update_compute_eta(self.ptr, _p(agg), _p(eta), num_kf, stream))

    def motion_filter(self, ctx, f_last, f_cur, net_kf, inp_kf, dtype=SLK_F32, stream=None):
        """compute_motion_gru: mean flow magnitude of one update step between
        the last keyframe and the current frame."""
        out = F()
        check(lib().slk_motion_filter(ctx.ptr, self.ptr, _p(f_last), _p(f_cur), dtype,
                                      _p(net_kf), _p(inp_kf), ctypes.byref(out), stream))
        return out.value

    def close(self):
        if self.ptr:
            lib().slk_update_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Encoder:
    """slk_encoder_*: HalfBasicEncoder (cuda_slam/main.cu:306-381), the fp16
    feature (fnet: out_dim 128, instance norm) or context (cnet: 256, no
    norm) network, on device arrays."""

    def __init__(self, in_h, in_w, out_dim, use_norm, max_batch=1):
        self.in_h, self.in_w, self.out_dim = in_h, in_w, out_dim
        p = P()
        check(lib().slk_encoder_create(ctypes.byref(p), in_h, in_w, out_dim, int(use_norm),
                                       max_batch))
        self.ptr = p

    def layers(self):
        """[(suffix, co, ci, k, stride)] in the ABI's layer order."""
        L_ = lib()
        out = []
        for i in range(L_.slk_encoder_num_layers()):
            co, ci, k, s = I(), I(), I(), I()
            check(L_.slk_encoder_layer_shape(self.ptr, i, ctypes.byref(co), ctypes.byref(ci),
                                             ctypes.byref(k), ctypes.byref(s)))
            out.append((L_.slk_encoder_layer_suffix(i).decode(), co.value, ci.value, k.value,
                        s.value))
        return out

    def set_weights(self, weights, prefix):
        """weights: {prefix_suffix: (w [co, ci, k, k], b [co]) float32}."""
        for i, (suffix, co, ci, k, _) in enumerate(self.layers()):
            w, b = weights[f"{prefix}_{suffix}"]
            w = np.ascontiguousarray(w, np.float32)
            b = np.ascontiguousarray(b, np.float32)
            assert w.shape == (co, ci, k, k) and b.shape == (co,), suffix
            check(lib().slk_encoder_set_conv(self.ptr, i, w.ctypes.data, b.ctypes.data))

    def load_dir(self, path, prefix):
        check(lib().slk_encoder_load_dir(self.ptr, os.fsencode(path), prefix.encode()))

    def forward(self, image, out, batch=1, stream=None):
        """image [B][3][H][W] fp32 -> out [B][out_dim][H/8][W/8] fp16."""
        check(lib().slk_encoder_forward(self.ptr, _p(image), _p(out), batch, stream))

    def close(self):
        if self.ptr:
            lib().slk_encoder_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def encode_frame(fnet, cnet, bgr, fmap, net, inp, stream=None):
    """CudaDroid::encode_frame: BGR [H][W][3] -> fmap fp16, net / inp fp32."""
    check(lib().slk_encode_frame(fnet.ptr, cnet.ptr, _p(bgr), _p(fmap), _p(net), _p(inp), stream))


def nv12_to_bgr(y, uv, out, src_w, src_h, y_stride, uv_stride, dst_w, dst_h, stream=None):
    check(lib().slk_nv12_to_bgr(_p(y), _p(uv), _p(out), src_w, src_h, y_stride, uv_stride,
                                dst_w, dst_h, stream))


def p010_to_bgr(y, uv, out, src_w, src_h, y_stride_bytes, uv_stride_bytes, dst_w, dst_h,
                stream=None):
    check(lib().slk_p010_to_bgr(_p(y), _p(uv), _p(out), src_w, src_h, y_stride_bytes,
                                uv_stride_bytes, dst_w, dst_h, stream))


def bgr8_to_bgrf(src, out, src_w, src_h, stride, dst_w, dst_h, stream=None):
    check(lib().slk_bgr8_to_bgrf(_p(src), _p(out), src_w, src_h, stride, dst_w, dst_h, stream))


def preprocess_image(bgr, rgb, H, W, stream=None):
    check(lib().slk_preprocess_image(_p(bgr), _p(rgb), H, W, stream))


def write_poses_bin(path, timestamps, poses, cam_to_world=False):
    """The reference's pose file: [nk: i32][timestamps: i32 x nk][poses: f32 x nk x 7]."""
    ts = np.ascontiguousarray(timestamps, np.int32)
    ps = np.ascontiguousarray(poses, np.float32).reshape(-1, 7)
    assert ts.shape[0] == ps.shape[0]
    check(lib().slk_write_poses_bin(os.fsencode(path), ts.shape[0], ts.ctypes.data,
                                    ps.ctypes.data, int(cam_to_world)))
