// Backward of the G2V splat for gfx950, atomic-free
// (reference src/cuda_gaussian_voxelizer.cu:1226-1482, :1920-2057).
//
// Per (Gaussian g, voxel v in its box): e = exp(-0.5 dx^T A dx), w = o e, q = A dx,
// inv = 1 / max(D_v, eps), t_v = (D_v >= eps) ? sum_c gF_vc F_vc : 0, u_gv = sum_c gF_vc f_gc,
//     gw = gD_v + (u_gv - t_v) inv        (gw = gD_v without features)
//     d mu += gw w q,  d Sigma += 0.5 gw w q q^T (symmetric),  d o += gw e,  d f_g += gF_v w inv
//
// Kernels:
//   k_bwd_density   features=None: one wave per Gaussian over its box voxels, wave reduction.
//   k_voxel_dot     t_v for every voxel (the reference's bmm, .cu:1995-1996).
//   k_bwd_tile      tile-major: U^T = G_tile (64 x C) . F_list^T on the matrix cores (3-term bf16
//                   split), then gw and the ten geometric partial sums of every (tile, Gaussian)
//                   pair, stored at the pair's Gaussian->Tile CSR slot.
//   k_bwd_gauss     Gaussian-major: sums the pair partials of its CSR row (fixed order) and
//                   gathers d f_g over its box voxels.  Every output row has one owner.
#include "g2v_internal.h"

namespace g2v {

constexpr int kNumGrads = 10;  // mu xyz, cov xx yy zz xy xz yz, opacity

__device__ __forceinline__ void accumulate_grads(float (&gr)[kNumGrads], float gw, float e, float o,
                                                 float qx, float qy, float qz) {
    const float gwd = gw * o * e;
    gr[0] += gwd * qx;
    gr[1] += gwd * qy;
    gr[2] += gwd * qz;
    const float h = 0.5f * gwd;
    gr[3] += h * qx * qx;
    gr[4] += h * qy * qy;
    gr[5] += h * qz * qz;
    gr[6] += h * qx * qy;
    gr[7] += h * qx * qz;
    gr[8] += h * qy * qz;
    gr[9] += gw * e;
}

__device__ __forceinline__ void write_grads(const float (&gr)[kNumGrads], int g, float* grad_means,
                                            float* grad_cov, float* grad_opacity) {
    grad_means[g * 3 + 0] = gr[0];
    grad_means[g * 3 + 1] = gr[1];
    grad_means[g * 3 + 2] = gr[2];
    float* c = grad_cov + g * 9;
    c[0] = gr[3]; c[1] = gr[6]; c[2] = gr[7];
    c[3] = gr[6]; c[4] = gr[4]; c[5] = gr[8];
    c[6] = gr[7]; c[7] = gr[8]; c[8] = gr[5];
    grad_opacity[g] = gr[9];
}

// ------------------------------------------------------------------------------------------
// Density only: one wave per Gaussian walks the voxels of its box (z fastest).
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_bwd_density(Grid G, int n, const float* __restrict__ gD,
                                                     const float* __restrict__ means,
                                                     const float* __restrict__ opacity,
                                                     const float* __restrict__ cov_inv,
                                                     const int* __restrict__ lb,
                                                     const int* __restrict__ ub,
                                                     float* __restrict__ grad_means,
                                                     float* __restrict__ grad_cov,
                                                     float* __restrict__ grad_opacity) {
    const int lane = threadIdx.x & 63;
    const int g = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (g >= n) return;
    GaussParams p;
    load_params(p, g, means, cov_inv, opacity, lb, ub);
    const int ex = p.ub[0] - p.lb[0] + 1, ey = p.ub[1] - p.lb[1] + 1, ez = p.ub[2] - p.lb[2] + 1;
    const int nv = (ex > 0 && ey > 0 && ez > 0) ? ex * ey * ez : 0;
    const int eyz = ey * ez;
    float gr[kNumGrads] = {};
    for (int i = lane; i < nv; i += 64) {
        const int ix = i / eyz, r = i - ix * eyz;
        const int iy = r / ez, iz = r - iy * ez;
        const int x = p.lb[0] + ix, y = p.lb[1] + iy, z = p.lb[2] + iz;
        float qx, qy, qz;
        const float e = eval_gauss(p, centre(G, 0, x), centre(G, 1, y), centre(G, 2, z), qx, qy, qz);
        accumulate_grads(gr, gD[voxel_index(G, x, y, z)], e, p.o, qx, qy, qz);
    }
#pragma unroll
    for (int k = 0; k < kNumGrads; ++k) gr[k] = wave_sum(gr[k]);
    if (lane == 0) write_grads(gr, g, grad_means, grad_cov, grad_opacity);
}

hipError_t launch_backward_density(const Grid& G, int n, const float* grad_density,
                                   const float* means, const float* opacity, const float* cov_inv,
                                   const int* lb, const int* ub, float* grad_means, float* grad_cov,
                                   float* grad_opacity, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    G2V_LAUNCH(k_bwd_density, dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, s, G, n,
                       grad_density, means, opacity, cov_inv, lb, ub, grad_means, grad_cov,
                       grad_opacity);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// t_v = (D_v >= eps) ? sum_c gF_vc F_vc : 0, one wave per voxel.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_voxel_dot(int64_t V, int C, const float* __restrict__ gF,
                                                   const float* __restrict__ F,
                                                   const float* __restrict__ D,
                                                   float* __restrict__ t) {
    const int lane = threadIdx.x & 63;
    const int64_t v = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (v >= V) return;
    const float* a = gF + v * C;
    const float* b = F + v * C;
    float s = 0.0f;
    if ((C & 3) == 0) {
        for (int c = lane * 4; c < C; c += 256) {
            const float4 x = *reinterpret_cast<const float4*>(a + c);
            const float4 y = *reinterpret_cast<const float4*>(b + c);
            s += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
        }
    } else {
        for (int c = lane; c < C; c += 64) s += a[c] * b[c];
    }
    s = wave_sum(s);
    if (lane == 0) t[v] = (D[v] >= kEps) ? s : 0.0f;
}

// ------------------------------------------------------------------------------------------
// Tile-major geometric partials (MFMA for U).
// ------------------------------------------------------------------------------------------
constexpr int kBtThreads = 256;      // 4 waves: (voxel block mb = wave & 1) x (Gaussian group wave >> 1)
constexpr int kBtNbw = 4;            // 32-Gaussian N blocks per wave per pass
constexpr int kBtPass = 2 * kBtNbw * 32;  // Gaussians per pass (256)

struct BtSmem {
    int vlin[64];
    float gD[64], inv[64], tv[64];
    int gid[kBtPass];
    float xch[2][kBtPass][kNumGrads + 1];
};

__global__ void __launch_bounds__(kBtThreads, 2) k_bwd_tile(
    Grid G, int C, const float* __restrict__ gD, const float* __restrict__ gF,
    const float* __restrict__ means, const float* __restrict__ opacity,
    const float* __restrict__ cov_inv, const int* __restrict__ lb, const int* __restrict__ ub,
    const int* __restrict__ g2t_offsets, const int* __restrict__ toff,
    const int* __restrict__ sorted_gauss, int M, const float* __restrict__ density,
    const float* __restrict__ tvox, const float* __restrict__ features,
    float* __restrict__ pair_partials) {
    __shared__ BtSmem sm;
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    const int tile = uniform(xcd_remap(blockIdx.x, gridDim.x));
    if (tile >= T) return;
    const int j0 = uniform(min(max(toff[tile], 0), M));
    const int Ng = uniform(min(max(toff[tile + 1], j0), M)) - j0;
    if (Ng <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int mb = wave & 1, ngrp = wave >> 1;
    const int tyz = G.tiles[1] * G.tiles[2];
    const int tx = tile / tyz, ty = (tile - tx * tyz) / G.tiles[2], tz = tile % G.tiles[2];

    if (threadIdx.x < 64) {
        int x, y, z;
        tile_voxel(G, tile, threadIdx.x, x, y, z);
        const bool ok = in_grid(G, x, y, z);
        const int64_t v = ok ? voxel_index(G, x, y, z) : 0;
        sm.vlin[threadIdx.x] = ok ? (int)v : -1;
        sm.gD[threadIdx.x] = ok ? gD[v] : 0.0f;
        sm.inv[threadIdx.x] = ok ? 1.0f / fmaxf(density[v], kEps) : 0.0f;
        sm.tv[threadIdx.x] = ok ? tvox[v] : 0.0f;
    }
    const bool vec_ok = (C & 3) == 0;

    for (int pbase = 0; pbase < Ng; pbase += kBtPass) {
        const int pcount = min(kBtPass, Ng - pbase);
        __syncthreads();
        for (int k = threadIdx.x; k < kBtPass; k += kBtThreads)
            sm.gid[k] = k < pcount ? sorted_gauss[j0 + pbase + k] : -1;
        __syncthreads();

        f32x16 acc[kBtNbw];
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) acc[j] = f32x16{};
        int nact = 0;  // active N blocks of this wave (uniform)
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) nact += ((ngrp + 2 * j) * 32 < pcount) ? 1 : 0;

        const int arow = sm.vlin[mb * 32 + (lane & 31)];
        const int koff = (lane >> 5) * 8;
        for (int c0 = 0; c0 < C; c0 += 16) {
            const int c = c0 + koff;
            const int valid = max(0, min(8, C - c));
            float av[8];
            if (arow >= 0) load8(gF + (int64_t)arow * C + c, valid, vec_ok, av);
            else {
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i] = 0.0f;
            }
            bf16x8 ah, al;
            split8(av, ah, al);
#pragma unroll
            for (int j = 0; j < kBtNbw; ++j) {
                if (j < nact) {
                    const int g = sm.gid[(ngrp + 2 * j) * 32 + (lane & 31)];
                    float bv[8];
                    if (g >= 0) load8(features + (int64_t)g * C + c, valid, vec_ok, bv);
                    else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) bv[i] = 0.0f;
                    }
                    bf16x8 bh, bl;
                    split8(bv, bh, bl);
                    acc[j] = mfma3_32x32x16(ah, al, bh, bl, acc[j]);
                }
            }
        }

        // gw and geometric partials of each (tile, Gaussian) pair held by this lane's column
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) {
            const int slot = (ngrp + 2 * j) * 32 + (lane & 31);
            float gr[kNumGrads] = {};
            const int g = sm.gid[slot];
            if (j < nact && g >= 0) {
                GaussParams p;
                load_params(p, g, means, cov_inv, opacity, lb, ub);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r = mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                    if (sm.vlin[r] < 0) continue;
                    const int x = tx * kTile + (r >> 4), y = ty * kTile + ((r >> 2) & 3), z = tz * kTile + (r & 3);
                    if (!in_box(p, x, y, z)) continue;
                    float qx, qy, qz;
                    const float e = eval_gauss(p, centre(G, 0, x), centre(G, 1, y), centre(G, 2, z), qx, qy, qz);
                    const float gw = sm.gD[r] + (acc[j][i] - sm.tv[r]) * sm.inv[r];
                    accumulate_grads(gr, gw, e, p.o, qx, qy, qz);
                }
            }
#pragma unroll
            for (int k = 0; k < kNumGrads; ++k) gr[k] += __shfl_xor(gr[k], 32, 64);
            if (lane < 32) {
#pragma unroll
                for (int k = 0; k < kNumGrads; ++k) sm.xch[mb][slot][k] = gr[k];
            }
        }
        __syncthreads();
        for (int slot = threadIdx.x; slot < pcount; slot += kBtThreads) {
            const int g = sm.gid[slot];
            const int tx0 = lb[g * 3] / kTile, ty0 = lb[g * 3 + 1] / kTile, tz0 = lb[g * 3 + 2] / kTile;
            const int dy = ub[g * 3 + 1] / kTile - ty0 + 1, dz = ub[g * 3 + 2] / kTile - tz0 + 1;
            const int64_t pair = (int64_t)g2t_offsets[g] + ((tx - tx0) * dy + (ty - ty0)) * dz + (tz - tz0);
            if (pair < 0 || pair >= M) continue;   // malformed CSR: never write outside the buffer
            float* out = pair_partials + pair * kNumGrads;
#pragma unroll
            for (int k = 0; k < kNumGrads; ++k) out[k] = sm.xch[0][slot][k] + sm.xch[1][slot][k];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Gaussian-major: reduce the pair partials of a CSR row; gather d f_g over the box voxels.
// ------------------------------------------------------------------------------------------
constexpr int kBgThreads = 256;

__global__ void __launch_bounds__(kBgThreads) k_bwd_gauss(
    Grid G, int n, int C, int M, const float* __restrict__ gF, const float* __restrict__ means,
    const float* __restrict__ opacity, const float* __restrict__ cov_inv,
    const int* __restrict__ lb, const int* __restrict__ ub, const int* __restrict__ g2t_offsets,
    const float* __restrict__ density, const float* __restrict__ pair_partials,
    float* __restrict__ grad_means, float* __restrict__ grad_cov, float* __restrict__ grad_opacity,
    float* __restrict__ grad_features) {
    __shared__ float red[4][kNumGrads];
    __shared__ float coef[kBgThreads];
    __shared__ int vrow[kBgThreads];
    const int g = blockIdx.x;
    if (g >= n) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    // 1. geometric gradients: fixed-order sum of this Gaussian's pair partials
    const int p0 = min(max(g2t_offsets[g], 0), M), p1 = min(max(g2t_offsets[g + 1], p0), M);
    float gr[kNumGrads] = {};
    for (int p = p0 + threadIdx.x; p < p1; p += kBgThreads) {
#pragma unroll
        for (int k = 0; k < kNumGrads; ++k) gr[k] += pair_partials[(int64_t)p * kNumGrads + k];
    }
#pragma unroll
    for (int k = 0; k < kNumGrads; ++k) gr[k] = wave_sum(gr[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kNumGrads; ++k) red[wave][k] = gr[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float tot[kNumGrads];
#pragma unroll
        for (int k = 0; k < kNumGrads; ++k) tot[k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
        write_grads(tot, g, grad_means, grad_cov, grad_opacity);
    }

    // 2. d f_g = sum_v gF_v w_gv / max(D_v, eps) over the voxels of the box
    GaussParams p;
    load_params(p, g, means, cov_inv, opacity, lb, ub);
    const int ex = p.ub[0] - p.lb[0] + 1, ey = p.ub[1] - p.lb[1] + 1, ez = p.ub[2] - p.lb[2] + 1;
    const int nv = (ex > 0 && ey > 0 && ez > 0) ? ex * ey * ez : 0;
    const int eyz = ey * ez;
    const bool vec = (C & 3) == 0;
    for (int cb = 0; cb < C; cb += 4 * kBgThreads) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        const int c = cb + threadIdx.x * 4;
        for (int vb = 0; vb < nv; vb += kBgThreads) {
            __syncthreads();
            const int i = vb + threadIdx.x;
            if (i < nv) {
                const int ix = i / eyz, r = i - ix * eyz;
                const int iy = r / ez, iz = r - iy * ez;
                const int x = p.lb[0] + ix, y = p.lb[1] + iy, z = p.lb[2] + iz;
                float qx, qy, qz;
                const float e = eval_gauss(p, centre(G, 0, x), centre(G, 1, y), centre(G, 2, z), qx, qy, qz);
                const int64_t v = voxel_index(G, x, y, z);
                coef[threadIdx.x] = p.o * e / fmaxf(density[v], kEps);
                vrow[threadIdx.x] = (int)v;
            }
            __syncthreads();
            const int cnt = min(kBgThreads, nv - vb);
            if (c < C) {
                if (vec) {
                    for (int k = 0; k < cnt; ++k) {
                        const float4 x = *reinterpret_cast<const float4*>(gF + (int64_t)vrow[k] * C + c);
                        const float cf = coef[k];
                        acc.x += cf * x.x; acc.y += cf * x.y; acc.z += cf * x.z; acc.w += cf * x.w;
                    }
                } else {
                    for (int k = 0; k < cnt; ++k) {
                        const float* row = gF + (int64_t)vrow[k] * C + c;
                        const float cf = coef[k];
                        acc.x += cf * row[0];
                        if (c + 1 < C) acc.y += cf * row[1];
                        if (c + 2 < C) acc.z += cf * row[2];
                        if (c + 3 < C) acc.w += cf * row[3];
                    }
                }
            }
        }
        if (c < C) {
            float* o = grad_features + (int64_t)g * C + c;
            o[0] = acc.x;
            if (c + 1 < C) o[1] = acc.y;
            if (c + 2 < C) o[2] = acc.z;
            if (c + 3 < C) o[3] = acc.w;
        }
    }
}

size_t backward_feats_workspace(const Grid& G, int n, int C, int64_t M) {
    (void)n; (void)C;
    const int64_t V = (int64_t)G.dims[0] * G.dims[1] * G.dims[2];
    Carver c(nullptr, (size_t)-1);
    c.take<float>(V > 0 ? V : 1);                       // t_v
    c.take<float>((M > 0 ? M : 1) * kNumGrads);         // pair partials
    return c.off + 256;
}

hipError_t launch_backward_feats(const Grid& G, int n, int C, const float* grad_density,
                                 const float* grad_feats, const float* means, const float* opacity,
                                 const float* cov_inv, const int* lb, const int* ub,
                                 const int* g2t_offsets, int64_t M, const int* tile_offsets,
                                 const int* sorted_gauss, const float* density,
                                 const float* grid_feats, const float* features,
                                 float* grad_means, float* grad_cov, float* grad_opacity,
                                 float* grad_features, void* ws, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t V = (int64_t)G.dims[0] * G.dims[1] * G.dims[2];
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    Carver cv(ws, (size_t)-1);
    float* tv = cv.take<float>(V > 0 ? V : 1);
    float* partials = cv.take<float>((M > 0 ? M : 1) * kNumGrads);
    if (V > 0)
        G2V_LAUNCH(k_voxel_dot, dim3((unsigned)ceil_div(V, 4)), dim3(256), 0, s, V, C,
                           grad_feats, grid_feats, density, tv);
    if (M > 0 && T > 0) {
        const int blocks = (int)ceil_div(T, 8) * 8;
        G2V_LAUNCH(k_bwd_tile, dim3(blocks), dim3(kBtThreads), 0, s, G, C, grad_density,
                           grad_feats, means, opacity, cov_inv, lb, ub, g2t_offsets, tile_offsets,
                           sorted_gauss, (int)M, density, (const float*)tv, features, partials);
    }
    G2V_LAUNCH(k_bwd_gauss, dim3(n), dim3(kBgThreads), 0, s, G, n, C, (int)M, grad_feats, means,
                       opacity, cov_inv, lb, ub, g2t_offsets, density, (const float*)partials,
                       grad_means, grad_cov, grad_opacity, grad_features);
    return hipGetLastError();
}

}  // namespace g2v
