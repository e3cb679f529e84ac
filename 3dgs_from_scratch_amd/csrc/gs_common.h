// Shared device constants and helpers for the gfx950 rasterizer kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gs_rasterizer.h"

namespace gs {

// Constants of the rendering model (src/torch_rasterizer.py:5-6, src/cuda/kernel.cu:23-25).
constexpr float kLowPassFilter = 0.3f;       // added to the 2D covariance diagonal
constexpr float kFrustumClampFactor = 1.3f;  // Jacobian evaluated at most 1.3x past the image edge
constexpr float kTransmittanceEps = 1e-10f;  // 1 - alpha + eps keeps the product positive
constexpr float kSigmaExtent = 3.0f;         // radius = 3 standard deviations

// Real spherical-harmonic basis constants, degrees 0..3 (src/gaussian.py:6-21).
constexpr float kShC0 = 0.28209479177387814f;
constexpr float kShC1 = 0.4886025119029199f;
constexpr float kShC2xy = 1.0925484305920792f;
constexpr float kShC2zz = 0.31539156525252005f;
constexpr float kShC2xxyy = 0.5462742152960396f;
constexpr float kShC3yxx = 0.5900435899266435f;
constexpr float kShC3xyz = 2.890611442640554f;
constexpr float kShC3yzz = 0.4570457994644658f;
constexpr float kShC3zzz = 0.3731763325901154f;
constexpr float kShC3xzz = 0.4570457994644658f;
constexpr float kShC3zxx = 1.445305721320277f;
constexpr float kShC3xxx = 0.5900435899266435f;

constexpr int kShRestCoeffs = 15;  // degrees 1..3

constexpr int kWave = 64;

inline int ceil_div(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

// Status helper: last launch error as an int status.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? GS_OK : static_cast<int>(e);
}

// Zero `bytes` of device memory on `stream` with a fill kernel (capi.hip).
int zero_bytes(void *ptr, size_t bytes, hipStream_t stream);

}  // namespace gs
