// Training-loop kernels around the rasterizer: a fused Adam step over several
// parameter tensors, the densification statistics of src/strategy.py:47-68,
// and a row gather that rebuilds parameter / optimizer-state tensors after
// pruning, cloning or splitting (src/strategy.py:71-229).
//
// All three are HBM-streaming kernels with coalesced accesses: one launch
// covers every tensor (blockIdx.y selects the tensor).

#include "gs_common.h"
#include "../../include/gs_rasterizer.h"

namespace gs {

constexpr int kTrainBlock = 256;
constexpr int kMaxBatch = 32;  // tensors per launch (passed by value as a kernel argument)

struct AdamBatch {
    GsAdamTensor t[kMaxBatch];
};

struct GatherBatch {
    GsGatherTensor t[kMaxBatch];
};

// ----------------------------------------------------------------- Adam
// torch.optim.Adam (no weight decay, no amsgrad) for tensor y of the batch, in
// PyTorch's operation order:
//   m += (1 - b1) (g - m)   (lerp);   v = v b2 + (1 - b2) g g
//   p -= (lr / (1 - b1^t)) * (m / (sqrt(v) / sqrt(1 - b2^t) + eps))
// with the bias corrections precomputed on the host per tensor and 1 - b
// rounded from double on the host (PyTorch's float(1 - beta)).
__global__ __launch_bounds__(kTrainBlock) void adam_kernel(AdamBatch batch, float beta2,
                                                           float one_m_b1, float one_m_b2,
                                                           float eps) {
    const GsAdamTensor &t = batch.t[blockIdx.y];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < t.count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float g = t.grad ? t.grad[i] : 0.0f;
        const float m0 = t.exp_avg[i];
        const float m = m0 + one_m_b1 * (g - m0);
        const float v = t.exp_avg_sq[i] * beta2 + one_m_b2 * (g * g);
        t.exp_avg[i] = m;
        t.exp_avg_sq[i] = v;
        const float denom = sqrtf(v) / t.bias_correction2_sqrt + eps;
        t.param[i] = t.param[i] - t.step_size * (m / denom);
    }
}

// ------------------------------------------------------ densification state
// src/strategy.py:47-68: for Gaussians with both radii > 0,
//   grads += |(du * W/2, dv * H/2)|, count += 1.
__global__ __launch_bounds__(kTrainBlock) void accumulate_grad2d_kernel(
    int64_t n, const float *__restrict__ grad_points, const float *__restrict__ radii,
    float half_w, float half_h, float *__restrict__ grads, float *__restrict__ count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (!(radii[2 * i] > 0.0f && radii[2 * i + 1] > 0.0f)) return;
    const float gx = grad_points[2 * i] * half_w, gy = grad_points[2 * i + 1] * half_h;
    grads[i] += sqrtf(gx * gx + gy * gy);
    count[i] += 1.0f;
}

// ------------------------------------------------------------- row gather
// dst row r of tensor y = src row src_rows[r] (+ delta row r), or zeros when
// fresh_rows[r] and the tensor zeroes fresh rows (optimizer state of new
// Gaussians).  Element-parallel: consecutive threads copy consecutive floats.
__global__ __launch_bounds__(kTrainBlock) void gather_rows_kernel(
    int64_t n_out, const int32_t *__restrict__ src_rows, const uint8_t *__restrict__ fresh_rows,
    GatherBatch batch) {
    const GsGatherTensor &t = batch.t[blockIdx.y];
    const int64_t total = n_out * t.width;
    const bool narrow = total <= 0x7fffffffLL;  // 32-bit index arithmetic
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = narrow ? (int64_t)((uint32_t)e / (uint32_t)t.width) : e / t.width;
        const int c = (int)(e - r * t.width);
        float v;
        if (t.zero_fresh && fresh_rows && fresh_rows[r]) {
            v = 0.0f;
        } else {
            v = t.src[(int64_t)src_rows[r] * t.width + c];
            if (t.delta) v += t.delta[e];
        }
        t.dst[e] = v;
    }
}

}  // namespace gs

using namespace gs;

static int grid_for(int64_t elems) {
    const int64_t blocks = (elems + kTrainBlock - 1) / kTrainBlock;
    return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);  // grid-stride beyond
}

extern "C" int gs_adam_step(const GsAdamTensor *tensors, int32_t n_tensors, double beta1,
                            double beta2, double eps, hipStream_t stream) {
    if (n_tensors < 0 || (n_tensors > 0 && !tensors)) return GS_ERR_INVALID_ARGUMENT;
    if (!(beta1 >= 0.0 && beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0 && eps >= 0.0))
        return GS_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < n_tensors; ++i) {
        const GsAdamTensor &t = tensors[i];
        if (t.count < 0 || (t.count > 0 && (!t.param || !t.exp_avg || !t.exp_avg_sq)) ||
            !(t.bias_correction2_sqrt > 0.0f))
            return GS_ERR_INVALID_ARGUMENT;
    }
    for (int first = 0; first < n_tensors; first += kMaxBatch) {
        const int nb = n_tensors - first < kMaxBatch ? n_tensors - first : kMaxBatch;
        AdamBatch batch{};
        int64_t max_count = 0;
        for (int i = 0; i < nb; ++i) {
            batch.t[i] = tensors[first + i];
            if (batch.t[i].count > max_count) max_count = batch.t[i].count;
        }
        if (max_count == 0) continue;
        hipLaunchKernelGGL(adam_kernel, dim3(grid_for(max_count), nb), dim3(kTrainBlock), 0,
                           stream, batch, (float)beta2, (float)(1.0 - beta1), (float)(1.0 - beta2),
                           (float)eps);
        const int st = launch_status();
        if (st) return st;
    }
    return GS_OK;
}

extern "C" int gs_accumulate_grad2d(const float *grad_points_image, const float *radii, int64_t n,
                                    int32_t width, int32_t height, float *grads, float *count,
                                    hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_points_image || !radii || !grads || !count) return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(accumulate_grad2d_kernel, dim3(ceil_div(n, kTrainBlock)), dim3(kTrainBlock),
                       0, stream, n, grad_points_image, radii, (float)width / 2.0f,
                       (float)height / 2.0f, grads, count);
    return launch_status();
}

extern "C" int gs_gather_rows(int64_t n_out, const int32_t *src_rows, const uint8_t *fresh_rows,
                              const GsGatherTensor *tensors, int32_t n_tensors,
                              hipStream_t stream) {
    if (n_out < 0 || n_tensors < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n_out == 0 || n_tensors == 0) return GS_OK;
    if (!src_rows || !tensors) return GS_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < n_tensors; ++i) {
        const GsGatherTensor &t = tensors[i];
        if (t.width <= 0 || !t.dst || !t.src) return GS_ERR_INVALID_ARGUMENT;
    }
    for (int first = 0; first < n_tensors; first += kMaxBatch) {
        const int nb = n_tensors - first < kMaxBatch ? n_tensors - first : kMaxBatch;
        GatherBatch batch{};
        int64_t max_elems = 0;
        for (int i = 0; i < nb; ++i) {
            batch.t[i] = tensors[first + i];
            if (n_out * batch.t[i].width > max_elems) max_elems = n_out * batch.t[i].width;
        }
        hipLaunchKernelGGL(gather_rows_kernel, dim3(grid_for(max_elems), nb), dim3(kTrainBlock), 0,
                           stream, n_out, src_rows, fresh_rows, batch);
        const int st = launch_status();
        if (st) return st;
    }
    return GS_OK;
}
