// Per-tile forward splat for gfx950 (reference src/cuda_gaussian_voxelizer.cu:7-136, :767-966,
// :1793, :1848-1849).
//
// One workgroup owns one 4x4x4 tile: every voxel of the grid is written by exactly one
// workgroup, so there are no atomics, no zero-fill of the output and no second normalisation
// pass.  Empty tiles write zeros.
//
// Feature splat, per tile with Ng Gaussians in its list:
//     W (64 voxels x Ng)    w_gv = o_g exp(-0.5 dx^T A dx) inside the Gaussian's box, else 0
//     D_v = sum_g w_gv,  S (64 x C) = W' F_list (Ng x C),  grid_feats = S / max(D, eps)
// where W' keeps only w > 0 (reference .cu:936).  S is computed on the matrix cores as three
// bf16 MFMAs per K step (hi*hi + hi*lo + lo*hi of a two-term bf16 split, fp32 accumulation),
// which keeps about 16 significant bits per product.  W is built once per tile in LDS, already
// split and in the MFMA A-operand layout; feature rows are gathered straight from global
// memory into the B-operand layout.
#include "g2v_internal.h"

namespace g2v {

// ------------------------------------------------------------------------------------------
// Density only: one wave per tile, one voxel per lane, Gaussian parameters wave-uniform.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_fwd_density(Grid G, const float* __restrict__ means,
                                                     const float* __restrict__ opacity,
                                                     const float* __restrict__ cov_inv,
                                                     const int* __restrict__ lb,
                                                     const int* __restrict__ ub,
                                                     const int* __restrict__ toff,
                                                     const int* __restrict__ sorted_gauss,
                                                     int M, float* __restrict__ density) {
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    const int nblocks = gridDim.x;
    const int tile = uniform(xcd_remap(blockIdx.x, nblocks) * 4 + (threadIdx.x >> 6));
    if (tile >= T) return;
    const int lane = threadIdx.x & 63;
    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);
    const float cx = centre(G, 0, x), cy = centre(G, 1, y), cz = centre(G, 2, z);
    const int j0 = uniform(min(max(toff[tile], 0), M));
    const int j1 = uniform(min(max(toff[tile + 1], j0), M));
    float acc = 0.0f;
    for (int j = j0; j < j1; ++j) {
        const int g = uniform(sorted_gauss[j]);
        GaussParams p;
        load_params(p, g, means, cov_inv, opacity, lb, ub);
        if (!in_box(p, x, y, z)) continue;
        float qx, qy, qz;
        acc += p.o * eval_gauss(p, cx, cy, cz, qx, qy, qz);
    }
    if (in_grid(G, x, y, z)) density[voxel_index(G, x, y, z)] = acc;
}

hipError_t launch_forward_density(const Grid& G, const float* means, const float* opacity,
                                  const float* cov_inv, const int* lb, const int* ub,
                                  const int* tile_offsets, const int* sorted_gauss, int M,
                                  float* density, hipStream_t s) {
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    if (T <= 0) return hipSuccess;
    const int groups = (int)ceil_div(T, 4);
    const int blocks = (int)ceil_div(groups, 8) * 8;
    G2V_LAUNCH(k_fwd_density, dim3(blocks), dim3(256), 0, s, G, means, opacity, cov_inv, lb,
                       ub, tile_offsets, sorted_gauss, M, density);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Feature splat (MFMA 32x32x16 bf16, 3-term split).
// ------------------------------------------------------------------------------------------
constexpr int kFwdThreads = 256;               // 4 waves
constexpr int kFwdKMax = 256;                  // Gaussians held in LDS per K chunk (multiple of 16)
constexpr int kFwdKSteps = kFwdKMax / 16;
constexpr int kFwdChanPerWave = 64;            // two 32-wide N blocks per wave
constexpr int kFwdChanPerPass = kFwdChanPerWave * 4;

struct FwdSmem {
    bf16x8 whi[kFwdKSteps][2][64];   // A operand, hi part: [k step][voxel block][lane]
    bf16x8 wlo[kFwdKSteps][2][64];   // A operand, lo part
    int gid[kFwdKMax];               // Gaussian id of each K slot, -1 for padding
    float dpart[4][64];              // per-wave partial densities
    float inv_den[64];               // 1 / max(D, eps)
    int vlin[64];                    // linear voxel index, -1 outside the grid
};

// Builds the split W for K slots [kbeg, kbeg + klen) of the tile list into LDS; accumulates
// the raw density of this wave's Gaussians into dacc (one voxel per lane).
__device__ __forceinline__ void fwd_build_w(FwdSmem& sm, const Grid& G, int j0, int kbeg, int klen,
                                            int ksteps, bool add_density, float& dacc,
                                            const float* __restrict__ means,
                                            const float* __restrict__ opacity,
                                            const float* __restrict__ cov_inv,
                                            const int* __restrict__ lb, const int* __restrict__ ub,
                                            const int* __restrict__ sorted_gauss, int x, int y,
                                            int z, float cx, float cy, float cz) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int noct = ksteps * 2;
    for (int o = wave; o < noct; o += 4) {
        float wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kk = o * 8 + i;  // slot within this chunk
            float w = 0.0f;
            int g = -1;
            if (kk < klen) {
                g = uniform(sorted_gauss[j0 + kbeg + kk]);
                GaussParams p;
                load_params(p, g, means, cov_inv, opacity, lb, ub);
                if (in_box(p, x, y, z)) {
                    float qx, qy, qz;
                    w = p.o * eval_gauss(p, cx, cy, cz, qx, qy, qz);
                }
                if (add_density) dacc += w;
            }
            wv[i] = (w > 0.0f) ? w : 0.0f;   // feature gate of the reference (.cu:936)
            if (lane == 0) sm.gid[kk] = g;
        }
        bf16x8 h, l;
        split8(wv, h, l);
        const int s = o >> 1, mb = lane >> 5;
        const int slot = (o & 1) * 32 + (lane & 31);
        sm.whi[s][mb][slot] = h;
        sm.wlo[s][mb][slot] = l;
    }
}

__global__ void __launch_bounds__(kFwdThreads, 2) k_fwd_feats(
    Grid G, int C, const float* __restrict__ means, const float* __restrict__ opacity,
    const float* __restrict__ cov_inv, const int* __restrict__ lb, const int* __restrict__ ub,
    const int* __restrict__ toff, const int* __restrict__ sorted_gauss, int M,
    const float* __restrict__ features, float* __restrict__ density,
    float* __restrict__ grid_feats) {
    __shared__ FwdSmem sm;
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    const int tile = uniform(xcd_remap(blockIdx.x, gridDim.x));
    if (tile >= T) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);
    const float cx = centre(G, 0, x), cy = centre(G, 1, y), cz = centre(G, 2, z);
    if (wave == 0) sm.vlin[lane] = in_grid(G, x, y, z) ? (int)voxel_index(G, x, y, z) : -1;

    const int j0 = uniform(min(max(toff[tile], 0), M));
    const int Ng = uniform(min(max(toff[tile + 1], j0), M)) - j0;
    const int nkc = (Ng + kFwdKMax - 1) / kFwdKMax;
    const bool vec_ok = (C % 4) == 0;
    float dacc = 0.0f;

    for (int cbase = 0; cbase < C; cbase += kFwdChanPerPass) {
        f32x16 acc[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};

        for (int kc = 0; kc < nkc; ++kc) {
            const int kbeg = kc * kFwdKMax;
            const int klen = min(kFwdKMax, Ng - kbeg);
            const int ksteps = (klen + 15) >> 4;
            if (nkc > 1 || cbase == 0) {
                __syncthreads();  // previous readers of W are done
                fwd_build_w(sm, G, j0, kbeg, klen, ksteps, cbase == 0, dacc, means, opacity,
                            cov_inv, lb, ub, sorted_gauss, x, y, z, cx, cy, cz);
                __syncthreads();
            }
            const int cw = cbase + wave * kFwdChanPerWave + (lane & 31);
            for (int s = 0; s < ksteps; ++s) {
                bf16x8 bh[2], bl[2];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const int c = cw + nb * 32;
                    float f[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int g = sm.gid[s * 16 + (lane >> 5) * 8 + i];
                        f[i] = (g >= 0 && c < C) ? features[(int64_t)g * C + c] : 0.0f;
                    }
                    split8(f, bh[nb], bl[nb]);
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const bf16x8 ah = sm.whi[s][mb][lane];
                    const bf16x8 al = sm.wlo[s][mb][lane];
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma3_32x32x16(ah, al, bh[nb], bl[nb], acc[mb][nb]);
                }
            }
        }
        (void)vec_ok;

        if (cbase == 0) {
            sm.dpart[wave][lane] = dacc;
            __syncthreads();
            if (wave == 0) {
                const float D = ((sm.dpart[0][lane] + sm.dpart[1][lane]) + sm.dpart[2][lane]) + sm.dpart[3][lane];
                sm.inv_den[lane] = 1.0f / fmaxf(D, kEps);
                if (sm.vlin[lane] >= 0) density[sm.vlin[lane]] = D;
            }
            __syncthreads();
        }

        // epilogue: D layout of 32x32 MFMA -> row = 8*(i/4) + 4*(lane/32) + i%4, col = lane%32
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                const int v = sm.vlin[r];
                if (v < 0) continue;
                const float inv = sm.inv_den[r];
                float* row = grid_feats + (int64_t)v * C;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const int c = cbase + wave * kFwdChanPerWave + nb * 32 + (lane & 31);
                    if (c < C) row[c] = acc[mb][nb][i] * inv;
                }
            }
        }
    }
}

hipError_t launch_forward_feats(const Grid& G, int C, const float* means, const float* opacity,
                                const float* cov_inv, const int* lb, const int* ub,
                                const int* tile_offsets, const int* sorted_gauss, int M,
                                const float* features, float* density, float* grid_feats,
                                hipStream_t s) {
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    if (T <= 0) return hipSuccess;
    if (C <= 0)
        return launch_forward_density(G, means, opacity, cov_inv, lb, ub, tile_offsets, sorted_gauss,
                                      M, density, s);
    const int blocks = (int)ceil_div(T, 8) * 8;
    G2V_LAUNCH(k_fwd_feats, dim3(blocks), dim3(kFwdThreads), 0, s, G, C, means, opacity,
                       cov_inv, lb, ub, tile_offsets, sorted_gauss, M, features, density, grid_feats);
    return hipGetLastError();
}

}  // namespace g2v
