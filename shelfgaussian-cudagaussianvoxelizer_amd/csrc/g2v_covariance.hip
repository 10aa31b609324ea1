// Covariances from per-Gaussian scales and rotation quaternions, and the chain rule back to them:
// the covariance construction ShelfGaussian runs before the voxelizer
// (reference test/gaussian_voxelizer.py:14-37 quat_to_rotmat / get_covariance, used at :168-169).
//
//   q^ = q / |q|  (q = (r, x, y, z), real part first)
//   R  = rotation matrix of q^                                 (gaussian_voxelizer.py:14-28)
//   M  = R diag(s),  Sigma = M M^T, written row-major (N, 9)   (gaussian_voxelizer.py:30-37)
//
// Backward, from G = dL/dSigma (the voxelizer's grad_cov):
//   dL/dM = (G + G^T) M,  dL/dR_ij = (dL/dM)_ij s_j,  dL/ds_j = sum_i (dL/dM)_ij R_ij,
//   dL/dq^_k = sum_ij dL/dR_ij dR_ij/dq^_k,  dL/dq = (dL/dq^ - q^ (q^ . dL/dq^)) / |q|.
// One thread per Gaussian; both directions are a few hundred flops per Gaussian and memory-light.
#include "../../include/g2v.h"
#include "g2v_internal.h"

namespace g2v {
namespace {

constexpr int kCovThreads = 256;

struct Rot {
    float r, x, y, z;   // the normalised quaternion
    float inv_norm;     // 1 / |q|
    float R[9];
};

__device__ __forceinline__ Rot rot_of(const float* __restrict__ q4) {
    Rot o;
    const float r = q4[0], x = q4[1], y = q4[2], z = q4[3];
    const float norm = sqrtf(r * r + x * x + y * y + z * z);
    o.inv_norm = 1.0f / norm;
    o.r = r / norm;
    o.x = x / norm;
    o.y = y / norm;
    o.z = z / norm;
    const float rr = o.r, xx = o.x, yy = o.y, zz = o.z;
    o.R[0] = 1.0f - 2.0f * (yy * yy + zz * zz);
    o.R[1] = 2.0f * (xx * yy - rr * zz);
    o.R[2] = 2.0f * (xx * zz + rr * yy);
    o.R[3] = 2.0f * (xx * yy + rr * zz);
    o.R[4] = 1.0f - 2.0f * (xx * xx + zz * zz);
    o.R[5] = 2.0f * (yy * zz - rr * xx);
    o.R[6] = 2.0f * (xx * zz - rr * yy);
    o.R[7] = 2.0f * (yy * zz + rr * xx);
    o.R[8] = 1.0f - 2.0f * (xx * xx + yy * yy);
    return o;
}

__global__ void __launch_bounds__(kCovThreads) k_cov_from_scale_rot(int n, const float* __restrict__ scales,
                                                                    const float* __restrict__ rotations,
                                                                    float* __restrict__ cov) {
    const int g = blockIdx.x * kCovThreads + threadIdx.x;
    if (g >= n) return;
    const Rot o = rot_of(rotations + 4 * (int64_t)g);
    const float s[3] = {scales[3 * (int64_t)g], scales[3 * (int64_t)g + 1], scales[3 * (int64_t)g + 2]};
    float Mm[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) Mm[3 * i + j] = o.R[3 * i + j] * s[j];
    float* out = cov + 9 * (int64_t)g;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            out[3 * i + j] = Mm[3 * i] * Mm[3 * j] + Mm[3 * i + 1] * Mm[3 * j + 1] + Mm[3 * i + 2] * Mm[3 * j + 2];
}

__global__ void __launch_bounds__(kCovThreads) k_cov_from_scale_rot_bwd(int n, const float* __restrict__ scales,
                                                                        const float* __restrict__ rotations,
                                                                        const float* __restrict__ grad_cov,
                                                                        float* __restrict__ grad_scales,
                                                                        float* __restrict__ grad_rotations) {
    const int g = blockIdx.x * kCovThreads + threadIdx.x;
    if (g >= n) return;
    const Rot o = rot_of(rotations + 4 * (int64_t)g);
    const float s[3] = {scales[3 * (int64_t)g], scales[3 * (int64_t)g + 1], scales[3 * (int64_t)g + 2]};
    const float* G = grad_cov + 9 * (int64_t)g;
    float Gs[9];   // G + G^T
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) Gs[3 * i + j] = G[3 * i + j] + G[3 * j + i];
    float Mm[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) Mm[3 * i + j] = o.R[3 * i + j] * s[j];
    float dM[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            dM[3 * i + j] = Gs[3 * i] * Mm[j] + Gs[3 * i + 1] * Mm[3 + j] + Gs[3 * i + 2] * Mm[6 + j];
    float ds[3] = {0.0f, 0.0f, 0.0f}, dR[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            dR[3 * i + j] = dM[3 * i + j] * s[j];
            ds[j] += dM[3 * i + j] * o.R[3 * i + j];
        }
    // dR/dq^ of the rotation formula, contracted with dR
    const float r = o.r, x = o.x, y = o.y, z = o.z;
    const float dr = 2.0f * (-z * dR[1] + y * dR[2] + z * dR[3] - x * dR[5] - y * dR[6] + x * dR[7]);
    const float dx = 2.0f * (y * dR[1] + z * dR[2] + y * dR[3] - 2.0f * x * dR[4] - r * dR[5] + z * dR[6] +
                             r * dR[7] - 2.0f * x * dR[8]);
    const float dy = 2.0f * (-2.0f * y * dR[0] + x * dR[1] + r * dR[2] + x * dR[3] + z * dR[5] - r * dR[6] +
                             z * dR[7] - 2.0f * y * dR[8]);
    const float dz = 2.0f * (-2.0f * z * dR[0] - r * dR[1] + x * dR[2] + r * dR[3] - 2.0f * z * dR[4] +
                             y * dR[5] + x * dR[6] + y * dR[7]);
    // through the normalisation q^ = q / |q|
    const float dot = r * dr + x * dx + y * dy + z * dz;
    float* gq = grad_rotations + 4 * (int64_t)g;
    gq[0] = (dr - r * dot) * o.inv_norm;
    gq[1] = (dx - x * dot) * o.inv_norm;
    gq[2] = (dy - y * dot) * o.inv_norm;
    gq[3] = (dz - z * dot) * o.inv_norm;
    float* gs = grad_scales + 3 * (int64_t)g;
    gs[0] = ds[0];
    gs[1] = ds[1];
    gs[2] = ds[2];
}

}  // namespace

hipError_t launch_cov_from_scale_rot(int n, const float* scales, const float* rotations, float* cov, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    G2V_LAUNCH(k_cov_from_scale_rot, dim3((unsigned)ceil_div(n, kCovThreads)), dim3(kCovThreads), 0, s, n, scales,
               rotations, cov);
    return hipGetLastError();
}

hipError_t launch_cov_from_scale_rot_bwd(int n, const float* scales, const float* rotations, const float* grad_cov,
                                         float* grad_scales, float* grad_rotations, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    G2V_LAUNCH(k_cov_from_scale_rot_bwd, dim3((unsigned)ceil_div(n, kCovThreads)), dim3(kCovThreads), 0, s, n,
               scales, rotations, grad_cov, grad_scales, grad_rotations);
    return hipGetLastError();
}

}  // namespace g2v
