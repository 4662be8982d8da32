// SE3 Lie-group device functions (quaternion form), templated on the scalar
// type: float for the reprojection feeding the correlation lookup, double for
// bundle adjustment. Same formulas and small-angle branches as
// cuda_slam/se3.cuh:8-114 (pose = [t, q(xyzw)], tangent xi = [tau, phi],
// retraction T <- exp(xi) * T).
#pragma once

#include <hip/hip_runtime.h>

namespace slk {

template <typename T>
__device__ __forceinline__ void act_so3(const T* q, const T* X, T* Y) {
    T uv[3];
    uv[0] = T(2) * (q[1] * X[2] - q[2] * X[1]);
    uv[1] = T(2) * (q[2] * X[0] - q[0] * X[2]);
    uv[2] = T(2) * (q[0] * X[1] - q[1] * X[0]);
    Y[0] = X[0] + q[3] * uv[0] + (q[1] * uv[2] - q[2] * uv[1]);
    Y[1] = X[1] + q[3] * uv[1] + (q[2] * uv[0] - q[0] * uv[2]);
    Y[2] = X[2] + q[3] * uv[2] + (q[0] * uv[1] - q[1] * uv[0]);
}

// Homogeneous point [X, Y, Z, W] -> [R X + W t, W]  (se3.cuh:19-26)
template <typename T>
__device__ __forceinline__ void act_se3(const T* t, const T* q, const T* X, T* Y) {
    act_so3(q, X, Y);
    Y[3] = X[3];
    Y[0] += X[3] * t[0];
    Y[1] += X[3] * t[1];
    Y[2] += X[3] * t[2];
}

// Adjoint-transpose action on a 6-vector (se3.cuh:28-41)
template <typename T>
__device__ __forceinline__ void adj_se3(const T* t, const T* q, const T* X, T* Y) {
    const T qinv[4] = {-q[0], -q[1], -q[2], q[3]};
    act_so3(qinv, &X[0], &Y[0]);
    act_so3(qinv, &X[3], &Y[3]);
    T u[3], v[3];
    u[0] = t[2] * X[1] - t[1] * X[2];
    u[1] = t[0] * X[2] - t[2] * X[0];
    u[2] = t[1] * X[0] - t[0] * X[1];
    act_so3(qinv, u, v);
    Y[3] += v[0];
    Y[4] += v[1];
    Y[5] += v[2];
}

// Tij = Tj * Ti^-1  (se3.cuh:43-54)
template <typename T>
__device__ __forceinline__ void rel_se3(const T* ti, const T* qi, const T* tj,
                                        const T* qj, T* tij, T* qij) {
    qij[0] = -qj[3] * qi[0] + qj[0] * qi[3] - qj[1] * qi[2] + qj[2] * qi[1];
    qij[1] = -qj[3] * qi[1] + qj[1] * qi[3] - qj[2] * qi[0] + qj[0] * qi[2];
    qij[2] = -qj[3] * qi[2] + qj[2] * qi[3] - qj[0] * qi[1] + qj[1] * qi[0];
    qij[3] = qj[3] * qi[3] + qj[0] * qi[0] + qj[1] * qi[1] + qj[2] * qi[2];
    act_so3(qij, ti, tij);
    tij[0] = tj[0] - tij[0];
    tij[1] = tj[1] - tij[1];
    tij[2] = tj[2] - tij[2];
}

template <typename T>
__device__ __forceinline__ void exp_so3(const T* phi, T* q) {
    const T theta_sq = phi[0] * phi[0] + phi[1] * phi[1] + phi[2] * phi[2];
    const T theta_p4 = theta_sq * theta_sq;
    const T theta = sqrt(theta_sq);
    T imag, real;
    if (theta_sq < T(1e-8)) {
        imag = T(0.5) - (T(1) / T(48)) * theta_sq + (T(1) / T(3840)) * theta_p4;
        real = T(1) - (T(1) / T(8)) * theta_sq + (T(1) / T(384)) * theta_p4;
    } else {
        imag = sin(T(0.5) * theta) / theta;
        real = cos(T(0.5) * theta);
    }
    q[0] = imag * phi[0];
    q[1] = imag * phi[1];
    q[2] = imag * phi[2];
    q[3] = real;
}

template <typename T>
__device__ __forceinline__ void cross_inplace(const T* a, T* b) {
    const T x0 = a[1] * b[2] - a[2] * b[1];
    const T x1 = a[2] * b[0] - a[0] * b[2];
    const T x2 = a[0] * b[1] - a[1] * b[0];
    b[0] = x0;
    b[1] = x1;
    b[2] = x2;
}

template <typename T>
__device__ __forceinline__ void exp_se3(const T* xi, T* t, T* q) {
    exp_so3(xi + 3, q);
    T tau[3] = {xi[0], xi[1], xi[2]};
    const T phi[3] = {xi[3], xi[4], xi[5]};
    const T theta_sq = phi[0] * phi[0] + phi[1] * phi[1] + phi[2] * phi[2];
    const T theta = sqrt(theta_sq);
    t[0] = tau[0];
    t[1] = tau[1];
    t[2] = tau[2];
    if (theta > T(1e-4)) {
        const T a = (T(1) - cos(theta)) / theta_sq;
        cross_inplace(phi, tau);
        t[0] += a * tau[0];
        t[1] += a * tau[1];
        t[2] += a * tau[2];
        const T b = (theta - sin(theta)) / (theta * theta_sq);
        cross_inplace(phi, tau);
        t[0] += b * tau[0];
        t[1] += b * tau[1];
        t[2] += b * tau[2];
    }
}

template <typename T>
__device__ __forceinline__ void retr_se3(const T* xi, const T* t, const T* q, T* t1, T* q1) {
    T dt[3] = {0, 0, 0};
    T dq[4] = {0, 0, 0, 1};
    exp_se3(xi, dt, dq);
    q1[0] = dq[3] * q[0] + dq[0] * q[3] + dq[1] * q[2] - dq[2] * q[1];
    q1[1] = dq[3] * q[1] + dq[1] * q[3] + dq[2] * q[0] - dq[0] * q[2];
    q1[2] = dq[3] * q[2] + dq[2] * q[3] + dq[0] * q[1] - dq[1] * q[0];
    q1[3] = dq[3] * q[3] - dq[0] * q[0] - dq[1] * q[1] - dq[2] * q[2];
    act_so3(dq, t, t1);
    t1[0] += dt[0];
    t1[1] += dt[1];
    t1[2] += dt[2];
}

template <typename T>
__device__ __forceinline__ void load_pose(const float* poses, int k, T* t, T* q) {
    t[0] = T(poses[k * 7 + 0]);
    t[1] = T(poses[k * 7 + 1]);
    t[2] = T(poses[k * 7 + 2]);
    q[0] = T(poses[k * 7 + 3]);
    q[1] = T(poses[k * 7 + 4]);
    q[2] = T(poses[k * 7 + 5]);
    q[3] = T(poses[k * 7 + 6]);
}

}  // namespace slk
