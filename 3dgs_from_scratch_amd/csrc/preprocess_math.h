// Per-Gaussian preprocess math shared by the projection / SH kernels.
//
// The forward projection below is the exact sequence of fp32 operations the
// CPU oracle (oracle/preprocess.py) restates: every product and sum is rounded
// separately (this file is compiled with -ffp-contract=off), divisions and
// square roots are IEEE correctly rounded.  That makes u, v, the 2D covariance
// and the conic bit-identical between oracle and GPU for identical inputs, so
// the integer tile rectangles and the chi-square cut in the blend agree exactly.
#pragma once

#include "gs_common.h"

namespace gs {

struct Camera {
    float w[12];  // rows 0..2 of world_to_camera, row-major (3x4)
    float fx, fy, cx, cy;
    float lim_x, lim_y;  // frustum clamp of x/z and y/z for the Jacobian
};

__device__ __forceinline__ Camera load_camera(const float *__restrict__ w2c,
                                              const float *__restrict__ K, int width,
                                              int height) {
    Camera c;
#pragma unroll
    for (int i = 0; i < 12; ++i) c.w[i] = w2c[i];
    c.fx = K[0];
    c.cx = K[2];
    c.fy = K[4];
    c.cy = K[5];
    // src/torch_rasterizer.py:87-88
    c.lim_x = (kFrustumClampFactor * fmaxf(c.cx, (float)width - c.cx)) / c.fx;
    c.lim_y = (kFrustumClampFactor * fmaxf(c.cy, (float)height - c.cy)) / c.fy;
    return c;
}

// IEEE correctly rounded fp32 square root.  The device sqrtf is accurate to
// about 1 ulp but not correctly rounded (and the compiler folds
// (float)sqrt((double)x) back into sqrtf), so the candidate is corrected with an
// exact midpoint test: the midpoint m of two adjacent floats has 25 significant
// bits, so m*m is exact in double, and sqrt(x) < m <=> x < m*m.
__device__ __forceinline__ float sqrt_rn(float x) {
    float s = sqrtf(x);
    if (!(x > 0.0f) || !isfinite(x)) return s;  // 0, negatives, NaN, inf
    const double xd = (double)x;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const float lo = __uint_as_float(__float_as_uint(s) - 1u);
        const float hi = __uint_as_float(__float_as_uint(s) + 1u);
        const double mlo = 0.5 * ((double)s + (double)lo);
        const double mhi = 0.5 * ((double)s + (double)hi);
        if (xd < mlo * mlo)
            s = lo;
        else if (xd > mhi * mhi)
            s = hi;
        else
            break;
    }
    return s;
}

// min(max(x, lo), hi) propagating NaN like torch.clamp (fminf/fmaxf drop NaN).
__device__ __forceinline__ float clamp_nan(float x, float lo, float hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

// Rotation matrix of an (x, y, z, w) unit quaternion (src/gaussian.py:64-79).
__device__ __forceinline__ void quat_to_rot(float qx, float qy, float qz, float qw, float R[9]) {
    R[0] = 1.0f - 2.0f * (qy * qy + qz * qz);
    R[1] = 2.0f * (qx * qy - qz * qw);
    R[2] = 2.0f * (qx * qz + qy * qw);
    R[3] = 2.0f * (qx * qy + qz * qw);
    R[4] = 1.0f - 2.0f * (qx * qx + qz * qz);
    R[5] = 2.0f * (qy * qz - qx * qw);
    R[6] = 2.0f * (qx * qz - qy * qw);
    R[7] = 2.0f * (qy * qz + qx * qw);
    R[8] = 1.0f - 2.0f * (qx * qx + qy * qy);
}

struct Projection {
    float xc, yc, zc;  // camera-space centre
    float u, v;        // image-space centre
    float a, b, c;     // 2D covariance incl. low-pass filter (b = off-diagonal)
    float A, B, C;     // conic (inverse covariance)
    float ru, rv;      // 3-sigma radii along u and v
    bool cov_done;     // covariance computed (passed opacity and depth culls)
    bool keep;         // passes every cull
};

// Forward projection of one Gaussian (src/torch_rasterizer.py:41-144 semantics,
// src/cuda/kernel.cu:46-155,411-500 data flow).
__device__ __forceinline__ Projection project_gaussian(const Camera &cam, float px, float py,
                                                       float pz, float sx, float sy, float sz,
                                                       float qx, float qy, float qz, float qw,
                                                       float opacity, float near_plane,
                                                       float far_plane, float min_opacity,
                                                       float min_radius, float max_radius,
                                                       int width, int height) {
    Projection p;
    const float *w = cam.w;
    p.xc = w[0] * px + w[1] * py + w[2] * pz + w[3];
    p.yc = w[4] * px + w[5] * py + w[6] * pz + w[7];
    p.zc = w[8] * px + w[9] * py + w[10] * pz + w[11];
    p.u = p.v = 0.0f;
    p.a = p.b = p.c = 0.0f;
    p.A = p.B = p.C = 0.0f;
    p.ru = p.rv = 0.0f;
    p.cov_done = false;
    p.keep = false;
    if (!(opacity >= min_opacity) || !(p.zc > near_plane) || !(p.zc < far_plane)) return p;

    p.u = (cam.fx * p.xc) / p.zc + cam.cx;
    p.v = (cam.fy * p.yc) / p.zc + cam.cy;

    float R[9];
    quat_to_rot(qx, qy, qz, qw, R);
    // M = R * diag(s); Sigma_world = M M^T
    const float m00 = R[0] * sx, m01 = R[1] * sy, m02 = R[2] * sz;
    const float m10 = R[3] * sx, m11 = R[4] * sy, m12 = R[5] * sz;
    const float m20 = R[6] * sx, m21 = R[7] * sy, m22 = R[8] * sz;
    const float s00 = m00 * m00 + m01 * m01 + m02 * m02;
    const float s01 = m00 * m10 + m01 * m11 + m02 * m12;
    const float s02 = m00 * m20 + m01 * m21 + m02 * m22;
    const float s11 = m10 * m10 + m11 * m11 + m12 * m12;
    const float s12 = m10 * m20 + m11 * m21 + m12 * m22;
    const float s22 = m20 * m20 + m21 * m21 + m22 * m22;

    // Jacobian of the pinhole projection at the clamped x/z, y/z (src/torch_rasterizer.py:82-98)
    const float invz = 1.0f / p.zc;
    const float xn = p.xc * invz;
    const float yn = p.yc * invz;
    const float xcl = clamp_nan(xn, -cam.lim_x, cam.lim_x);
    const float ycl = clamp_nan(yn, -cam.lim_y, cam.lim_y);
    const float j00 = cam.fx * invz;
    const float j02 = (-cam.fx * xcl) * invz;
    const float j11 = cam.fy * invz;
    const float j12 = (-cam.fy * ycl) * invz;

    // T = J * W[:3,:3] (2x3); Sigma_2D = T Sigma_world T^T
    const float t00 = j00 * w[0] + j02 * w[8];
    const float t01 = j00 * w[1] + j02 * w[9];
    const float t02 = j00 * w[2] + j02 * w[10];
    const float t10 = j11 * w[4] + j12 * w[8];
    const float t11 = j11 * w[5] + j12 * w[9];
    const float t12 = j11 * w[6] + j12 * w[10];
    const float q00 = t00 * s00 + t01 * s01 + t02 * s02;
    const float q01 = t00 * s01 + t01 * s11 + t02 * s12;
    const float q02 = t00 * s02 + t01 * s12 + t02 * s22;
    const float q10 = t10 * s00 + t11 * s01 + t12 * s02;
    const float q11 = t10 * s01 + t11 * s11 + t12 * s12;
    const float q12 = t10 * s02 + t11 * s12 + t12 * s22;
    p.a = (q00 * t00 + q01 * t01 + q02 * t02) + kLowPassFilter;
    p.b = q00 * t10 + q01 * t11 + q02 * t12;
    p.c = (q10 * t10 + q11 * t11 + q12 * t12) + kLowPassFilter;
    p.cov_done = true;

    const bool finite_cov = isfinite(p.a) && isfinite(p.b) && isfinite(p.c);
    const float det = p.a * p.c - p.b * p.b;
    const float inv_det = 1.0f / fmaxf(det, 1e-12f);
    const float A = p.c * inv_det;
    const float B = -p.b * inv_det;
    const float C = p.a * inv_det;
    const float ru = sqrt_rn(fmaxf(p.a, 1e-12f)) * kSigmaExtent;
    const float rv = sqrt_rn(fmaxf(p.c, 1e-12f)) * kSigmaExtent;
    const float r = fmaxf(ru, rv);
    const bool keep = finite_cov && isfinite(ru) && isfinite(rv) && r >= min_radius &&
                      r <= max_radius && p.u > -ru && p.u < (float)width + ru && p.v > -rv &&
                      p.v < (float)height + rv;
    if (keep) {
        p.A = A;
        p.B = B;
        p.C = C;
        p.ru = ru;
        p.rv = rv;
        p.keep = true;
    } else {
        p.u = p.v = 0.0f;
    }
    return p;
}

// Pixel AABB -> tile rectangle (src/cuda/kernel.cu:784-818, src/torch_rasterizer.py:159-173).
// Returns false when the rectangle is empty.
struct TileRect {
    int tx0, tx1, ty0, ty1;  // inclusive tile bounds
};

__device__ __forceinline__ bool tile_rect(float u, float v, float ru, float rv, int width,
                                          int height, int tile_size, TileRect &r) {
    const float wmax = (float)(width - 1), hmax = (float)(height - 1);
    const int u0 = (int)fminf(fmaxf(floorf(u - ru), 0.0f), wmax);
    const int u1 = (int)fminf(fmaxf(floorf(u + ru), 0.0f), wmax);
    const int v0 = (int)fminf(fmaxf(floorf(v - rv), 0.0f), hmax);
    const int v1 = (int)fminf(fmaxf(floorf(v + rv), 0.0f), hmax);
    if (u0 > u1 || v0 > v1) return false;
    r.tx0 = u0 / tile_size;
    r.tx1 = u1 / tile_size;
    r.ty0 = v0 / tile_size;
    r.ty1 = v1 / tile_size;
    return true;
}

// Spherical-harmonic basis for degrees 1..3 at unit direction (x, y, z)
// (src/gaussian.py:29-52; sign convention of that file).
__device__ __forceinline__ void sh_basis_rest(float x, float y, float z, float b[15]) {
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    b[0] = -kShC1 * y;
    b[1] = kShC1 * z;
    b[2] = -kShC1 * x;
    b[3] = kShC2xy * xy;
    b[4] = kShC2xy * yz;
    b[5] = kShC2zz * (3.0f * zz - 1.0f);
    b[6] = kShC2xy * xz;
    b[7] = kShC2xxyy * (xx - yy);
    b[8] = kShC3yxx * y * (xx - yy);
    b[9] = kShC3xyz * (x * y * z);
    b[10] = kShC3yzz * y * (4.0f * zz - xx - yy);
    b[11] = kShC3zzz * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    b[12] = kShC3xzz * x * (4.0f * zz - xx - yy);
    b[13] = kShC3zxx * z * (xx - yy);
    b[14] = kShC3xxx * x * (xx - 3.0f * yy);
}

// d basis_k / d(x, y, z) for the 15 higher-order basis functions.
__device__ __forceinline__ void sh_basis_rest_grad(float x, float y, float z, float dx[15],
                                                   float dy[15], float dz[15]) {
    const float xx = x * x, yy = y * y, zz = z * z;
    dx[0] = 0.0f;                  dy[0] = -kShC1;                 dz[0] = 0.0f;
    dx[1] = 0.0f;                  dy[1] = 0.0f;                   dz[1] = kShC1;
    dx[2] = -kShC1;                dy[2] = 0.0f;                   dz[2] = 0.0f;
    dx[3] = kShC2xy * y;           dy[3] = kShC2xy * x;            dz[3] = 0.0f;
    dx[4] = 0.0f;                  dy[4] = kShC2xy * z;            dz[4] = kShC2xy * y;
    dx[5] = 0.0f;                  dy[5] = 0.0f;                   dz[5] = 6.0f * kShC2zz * z;
    dx[6] = kShC2xy * z;           dy[6] = 0.0f;                   dz[6] = kShC2xy * x;
    dx[7] = 2.0f * kShC2xxyy * x;  dy[7] = -2.0f * kShC2xxyy * y;  dz[7] = 0.0f;
    dx[8] = 2.0f * kShC3yxx * x * y;
    dy[8] = kShC3yxx * (xx - 3.0f * yy);
    dz[8] = 0.0f;
    dx[9] = kShC3xyz * y * z;
    dy[9] = kShC3xyz * x * z;
    dz[9] = kShC3xyz * x * y;
    dx[10] = -2.0f * kShC3yzz * x * y;
    dy[10] = kShC3yzz * (4.0f * zz - xx - 3.0f * yy);
    dz[10] = 8.0f * kShC3yzz * y * z;
    dx[11] = -6.0f * kShC3zzz * x * z;
    dy[11] = -6.0f * kShC3zzz * y * z;
    dz[11] = kShC3zzz * (6.0f * zz - 3.0f * xx - 3.0f * yy);
    dx[12] = kShC3xzz * (4.0f * zz - 3.0f * xx - yy);
    dy[12] = -2.0f * kShC3xzz * x * y;
    dz[12] = 8.0f * kShC3xzz * x * z;
    dx[13] = 2.0f * kShC3zxx * x * z;
    dy[13] = -2.0f * kShC3zxx * y * z;
    dz[13] = kShC3zxx * (xx - yy);
    dx[14] = 3.0f * kShC3xxx * (xx - yy);
    dy[14] = -6.0f * kShC3xxx * x * y;
    dz[14] = 0.0f;
}

// Backward of project_gaussian for a kept Gaussian: gradients of (u, v) and of
// the conic (A, B, C) flowing back to the world mean, scale and quaternion.
// Exact derivative of the forward above, with the clamped x/z (y/z) treated as
// a constant when the clamp is active (src/torch_rasterizer.py:93-94).
__device__ __forceinline__ void project_gaussian_backward(
    const Camera &cam, float px, float py, float pz, float sx, float sy, float sz, float qx,
    float qy, float qz, float qw, float ca, float cb, float cc, float g_u, float g_v, float g_A,
    float g_B, float g_C, float &g_px, float &g_py, float &g_pz, float &g_sx, float &g_sy,
    float &g_sz, float &g_qx, float &g_qy, float &g_qz, float &g_qw) {
    const float *w = cam.w;
    const float xc = w[0] * px + w[1] * py + w[2] * pz + w[3];
    const float yc = w[4] * px + w[5] * py + w[6] * pz + w[7];
    const float zc = w[8] * px + w[9] * py + w[10] * pz + w[11];
    const float invz = 1.0f / zc;
    const float invz2 = invz * invz;

    // conic -> covariance: d(Sigma^-1) = -Sigma^-1 dSigma Sigma^-1
    float g_a, g_b, g_c;
    const float det = ca * cc - cb * cb;
    if (det >= 1e-12f) {
        const float inv = 1.0f / det;
        const float A = cc * inv, B = -cb * inv, C = ca * inv;
        g_a = -(g_A * A * A + g_B * A * B + g_C * B * B);
        g_b = -(2.0f * g_A * A * B + g_B * (A * C + B * B) + 2.0f * g_C * B * C);
        g_c = -(g_A * B * B + g_B * B * C + g_C * C * C);
    } else {  // determinant clamped at 1e-12: inverse scale is constant
        const float inv = 1e12f;
        g_a = g_C * inv;
        g_b = -g_B * inv;
        g_c = g_A * inv;
    }

    // recompute the forward intermediates
    float R[9];
    quat_to_rot(qx, qy, qz, qw, R);
    const float s[3] = {sx, sy, sz};
    float M[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) M[i * 3 + j] = R[i * 3 + j] * s[j];
    float S[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            S[i * 3 + j] = M[i * 3] * M[j * 3] + M[i * 3 + 1] * M[j * 3 + 1] +
                           M[i * 3 + 2] * M[j * 3 + 2];

    const float xn = xc * invz, yn = yc * invz;
    const bool x_free = fabsf(xn) <= cam.lim_x;
    const bool y_free = fabsf(yn) <= cam.lim_y;
    const float xcl = clamp_nan(xn, -cam.lim_x, cam.lim_x);
    const float ycl = clamp_nan(yn, -cam.lim_y, cam.lim_y);
    const float j00 = cam.fx * invz;
    const float j02 = (-cam.fx * xcl) * invz;
    const float j11 = cam.fy * invz;
    const float j12 = (-cam.fy * ycl) * invz;
    float T[6];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        T[j] = j00 * w[j] + j02 * w[8 + j];
        T[3 + j] = j11 * w[4 + j] + j12 * w[8 + j];
    }
    float P[6];  // T * Sigma_world
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            P[i * 3 + j] = T[i * 3] * S[j] + T[i * 3 + 1] * S[3 + j] + T[i * 3 + 2] * S[6 + j];

    // Sigma_2D = T Sw T^T, symmetric gradient G2 = [[g_a, g_b/2], [g_b/2, g_c]]
    const float hb = 0.5f * g_b;
    float GT[6];  // dL/dT = 2 G2 T Sw
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        GT[j] = 2.0f * (g_a * P[j] + hb * P[3 + j]);
        GT[3 + j] = 2.0f * (hb * P[j] + g_c * P[3 + j]);
    }
    float GS[9];  // dL/dSw = T^T G2 T
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int k = 0; k < 3; ++k)
            GS[j * 3 + k] = g_a * T[j] * T[k] + hb * (T[j] * T[3 + k] + T[3 + j] * T[k]) +
                            g_c * T[3 + j] * T[3 + k];
    // Sw = M M^T -> dL/dM = 2 GS M (GS symmetric)
    float GM[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            GM[i * 3 + j] = 2.0f * (GS[i * 3] * M[j] + GS[i * 3 + 1] * M[3 + j] +
                                    GS[i * 3 + 2] * M[6 + j]);
    // M = R diag(s)
    g_sx = GM[0] * R[0] + GM[3] * R[3] + GM[6] * R[6];
    g_sy = GM[1] * R[1] + GM[4] * R[4] + GM[7] * R[7];
    g_sz = GM[2] * R[2] + GM[5] * R[5] + GM[8] * R[8];
    float GR[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) GR[i * 3 + j] = GM[i * 3 + j] * s[j];
    g_qx = 2.0f * (qy * (GR[1] + GR[3]) + qz * (GR[2] + GR[6]) + qw * (GR[7] - GR[5])) -
           4.0f * qx * (GR[4] + GR[8]);
    g_qy = 2.0f * (qx * (GR[1] + GR[3]) + qw * (GR[2] - GR[6]) + qz * (GR[5] + GR[7])) -
           4.0f * qy * (GR[0] + GR[8]);
    g_qz = 2.0f * (qw * (GR[3] - GR[1]) + qx * (GR[2] + GR[6]) + qy * (GR[5] + GR[7])) -
           4.0f * qz * (GR[0] + GR[4]);
    g_qw = 2.0f * (qz * (GR[3] - GR[1]) + qy * (GR[2] - GR[6]) + qx * (GR[7] - GR[5]));

    // T = J W -> dL/dJ
    const float gj00 = GT[0] * w[0] + GT[1] * w[1] + GT[2] * w[2];
    const float gj02 = GT[0] * w[8] + GT[1] * w[9] + GT[2] * w[10];
    const float gj11 = GT[3] * w[4] + GT[4] * w[5] + GT[5] * w[6];
    const float gj12 = GT[3] * w[8] + GT[4] * w[9] + GT[5] * w[10];

    // J and (u, v) -> camera-space centre
    float gx = g_u * cam.fx * invz;
    float gy = g_v * cam.fy * invz;
    float gz = -(g_u * cam.fx * xc + g_v * cam.fy * yc) * invz2;
    gz += -cam.fx * invz2 * gj00 - cam.fy * invz2 * gj11;
    if (x_free) {  // j02 = -fx x / z^2
        gx += -cam.fx * invz2 * gj02;
        gz += 2.0f * cam.fx * xc * invz2 * invz * gj02;
    } else {  // j02 = -fx xcl / z
        gz += cam.fx * xcl * invz2 * gj02;
    }
    if (y_free) {
        gy += -cam.fy * invz2 * gj12;
        gz += 2.0f * cam.fy * yc * invz2 * invz * gj12;
    } else {
        gz += cam.fy * ycl * invz2 * gj12;
    }
    // p_cam = W p + t -> world
    g_px = w[0] * gx + w[4] * gy + w[8] * gz;
    g_py = w[1] * gx + w[5] * gy + w[9] * gz;
    g_pz = w[2] * gx + w[6] * gy + w[10] * gz;
}

}  // namespace gs
