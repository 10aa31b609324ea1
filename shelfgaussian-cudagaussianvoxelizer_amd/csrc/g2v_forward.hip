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
// split and in the MFMA A-operand layout.  The features are split once per call into packed
// (hi, lo) bf16 pairs, so a B fragment (8 Gaussians x 1 channel per lane) is 8 dword gathers
// and 8 byte permutes; the gathers of the next K step are issued before the current MFMAs.
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
// Features as packed bf16 pairs: low half = hi part, high half = lo part of the 2-term split.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_split_pack(const float* __restrict__ src, int n, int C, int Cp,
                                                    uint32_t* __restrict__ dst) {
    // (n + 1) x Cp packed pairs: row n and columns >= C are zero, so padded K slots and channels
    // can be gathered without bounds checks
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)(n + 1) * Cp) return;
    const int64_t r = i / Cp;
    const int c = (int)(i - r * Cp);
    const float v = (r < n && c < C) ? src[r * C + c] : 0.0f;
    __bf16 h, l;
    split_bf16(v, h, l);
    dst[i] = (uint32_t)__builtin_bit_cast(unsigned short, h) |
             ((uint32_t)__builtin_bit_cast(unsigned short, l) << 16);
}

// B fragment (hi and lo) from 8 packed pairs: element i of the fragment is pair u[i].
__device__ __forceinline__ void unpack8(const uint32_t (&u)[8], bf16x8& hi, bf16x8& lo) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 h, l;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = __builtin_amdgcn_perm(u[2 * j + 1], u[2 * j], 0x05040100u);
        l[j] = __builtin_amdgcn_perm(u[2 * j + 1], u[2 * j], 0x07060302u);
    }
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, l);
}

// ------------------------------------------------------------------------------------------
// Feature splat (MFMA 32x32x16 bf16, 3-term split).
// ------------------------------------------------------------------------------------------
constexpr int kFwdThreads = 512;               // 8 waves
constexpr int kFwdKMax = 256;                  // Gaussians held in LDS per K chunk (multiple of 16)
constexpr int kFwdKSteps = kFwdKMax / 16;
constexpr int kFwdWaves = kFwdThreads / 64;
constexpr int kFwdChanPerWave = 32;            // one 32-wide N block per wave
constexpr int kFwdChanPerPass = kFwdChanPerWave * kFwdWaves;

constexpr int kFwdPB = 8 * kFwdWaves;          // list entries staged at a time: one octet per wave

struct FwdSmem {
    bf16x8 whi[kFwdKSteps][2][64];   // A operand, hi part: [k step][voxel block][lane]
    bf16x8 wlo[kFwdKSteps][2][64];   // A operand, lo part
    alignas(16) int gid[kFwdKMax];   // Gaussian id of each K slot (the zero row n for padding)
    ParamTile<kFwdPB> pt;            // parameters of the entries being turned into weights
    float dpart[kFwdWaves][64];      // per-wave partial densities
    alignas(16) float inv_den[64];   // 1 / max(D, eps)
    alignas(16) int vlin[64];        // linear voxel index, -1 outside the grid
};

// Builds the split W for K slots [kbeg, kbeg + klen) of the tile list into LDS, 32 entries at a
// time (their parameters staged cooperatively in LDS, one octet of 8 entries per wave); adds the
// raw density of this wave's entries to dacc (one voxel per lane).
__device__ __forceinline__ void fwd_build_w(FwdSmem& sm, const Grid& G, int j0, int kbeg, int klen,
                                            int ksteps, bool add_density, float& dacc,
                                            const float* __restrict__ means,
                                            const float* __restrict__ opacity,
                                            const float* __restrict__ cov_inv,
                                            const int* __restrict__ lb, const int* __restrict__ ub,
                                            const int* __restrict__ sorted_gauss, int zero_row,
                                            int x, int y, int z, float cx, float cy, float cz) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nslots = ksteps * 16;
    for (int b0 = 0; b0 < nslots; b0 += kFwdPB) {
        __syncthreads();   // the previous batch of parameters is consumed
        stage_params(sm.pt, sorted_gauss + j0 + kbeg + b0, max(0, min(kFwdPB, klen - b0)), means, cov_inv,
                     opacity, lb, ub);
        __syncthreads();
        const int o = (b0 >> 3) + wave;   // octet of K slots handled by this wave
        if (o * 8 < nslots) {
            float wv[8];
#pragma unroll 2
            for (int i = 0; i < 8; ++i) {
                const int k = wave * 8 + i;
                const int g = sm.pt.gid[k];
                float w = 0.0f;
                if (g >= 0) {
                    GaussParams p;
                    read_params(sm.pt, k, p);
                    if (in_box(p, x, y, z)) {
                        float qx, qy, qz;
                        w = p.o * eval_gauss(p, cx, cy, cz, qx, qy, qz);
                    }
                    if (add_density) dacc += w;
                }
                wv[i] = (w > 0.0f) ? w : 0.0f;   // feature gate of the reference (.cu:936)
                if (lane == 0) sm.gid[o * 8 + i] = g >= 0 ? g : zero_row;
            }
            bf16x8 h, l;
            split8(wv, h, l);
            const int s = o >> 1, mb = lane >> 5;
            const int slot = (o & 1) * 32 + (lane & 31);
            sm.whi[s][mb][slot] = h;
            sm.wlo[s][mb][slot] = l;
        }
    }
}

__global__ void __launch_bounds__(kFwdThreads, 2) k_fwd_feats(
    Grid G, int C, const float* __restrict__ means, const float* __restrict__ opacity,
    const float* __restrict__ cov_inv, const int* __restrict__ lb, const int* __restrict__ ub,
    const int* __restrict__ toff, const int* __restrict__ sorted_gauss, int M, int n, int Cp,
    const uint32_t* __restrict__ fpk, float* __restrict__ density,
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
    float dacc = 0.0f;

    for (int cbase = 0; cbase < C; cbase += kFwdChanPerPass) {
        f32x16 acc[2];
        acc[0] = f32x16{};
        acc[1] = f32x16{};

        for (int kc = 0; kc < nkc; ++kc) {
            const int kbeg = kc * kFwdKMax;
            const int klen = min(kFwdKMax, Ng - kbeg);
            const int ksteps = ((klen + 31) >> 5) * 2;   // even: the MFMA loop takes steps in pairs
            if (nkc > 1 || cbase == 0) {
                __syncthreads();  // previous readers of W are done
                fwd_build_w(sm, G, j0, kbeg, klen, ksteps, cbase == 0, dacc, means, opacity,
                            cov_inv, lb, ub, sorted_gauss, n, x, y, z, cx, cy, cz);
                __syncthreads();
            }
            const int c = cbase + wave * kFwdChanPerWave + (lane & 31);
            if (cbase + wave * kFwdChanPerWave < Cp) {   // wave-uniform: this wave has channels
                // packed pairs of K step ks for this lane's channel; padding reads the zero row
                auto gather = [&](int ks, uint32_t (&u)[8]) {
                    const int* gp = &sm.gid[ks * 16 + (lane >> 5) * 8];
                    const int4 ga = *reinterpret_cast<const int4*>(gp);
                    const int4 gb = *reinterpret_cast<const int4*>(gp + 4);
                    const int gs[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) u[i] = fpk[(int64_t)gs[i] * Cp + c];
                };
                auto step = [&](int ks, const uint32_t (&u)[8]) {
                    bf16x8 bh, bl;
                    unpack8(u, bh, bl);
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
                        acc[mb] = mfma3_32x32x16(sm.whi[ks][mb][lane], sm.wlo[ks][mb][lane], bh, bl, acc[mb]);
                };
                // loads and steps are unconditional (ksteps is even, the prefetch index is
                // clamped) so the next step's gather stays in flight across this step's MFMAs
                uint32_t ua[8], ub[8];
                const int klast = ksteps - 1;
                if (ksteps > 0) {
                    gather(0, ua);
                    for (int ks = 0; ks < ksteps; ks += 2) {
                        gather(ks + 1, ub);
                        step(ks, ua);
                        gather(min(ks + 2, klast), ua);
                        step(ks + 1, ub);
                    }
                }
            }
        }

        if (cbase == 0) {
            sm.dpart[wave][lane] = dacc;
            __syncthreads();
            if (wave == 0) {
                float D = 0.0f;
#pragma unroll
                for (int w = 0; w < kFwdWaves; ++w) D += sm.dpart[w][lane];
                sm.inv_den[lane] = 1.0f / fmaxf(D, kEps);
                if (sm.vlin[lane] >= 0) density[sm.vlin[lane]] = D;
            }
            __syncthreads();
        }

        // epilogue: D layout of 32x32 MFMA -> row = 8*(i/4) + 4*(lane/32) + i%4, col = lane%32
        const int c = cbase + wave * kFwdChanPerWave + (lane & 31);
        if (c < C) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r0 = mb * 32 + 8 * q + 4 * (lane >> 5);
                    const int4 vl = *reinterpret_cast<const int4*>(&sm.vlin[r0]);
                    const float4 iv = *reinterpret_cast<const float4*>(&sm.inv_den[r0]);
                    const int vs[4] = {vl.x, vl.y, vl.z, vl.w};
                    const float is[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii)
                        if (vs[ii] >= 0) grid_feats[(int64_t)vs[ii] * C + c] = acc[mb][q * 4 + ii] * is[ii];
                }
            }
        }
    }
}

hipError_t launch_forward_feats(const Grid& G, int C, const float* means, const float* opacity,
                                const float* cov_inv, const int* lb, const int* ub,
                                const int* tile_offsets, const int* sorted_gauss, int M, int n,
                                const float* features, uint32_t* fpk, float* density,
                                float* grid_feats, hipStream_t s) {
    const int T = G.tiles[0] * G.tiles[1] * G.tiles[2];
    if (T <= 0) return hipSuccess;
    if (C <= 0)
        return launch_forward_density(G, means, opacity, cov_inv, lb, ub, tile_offsets, sorted_gauss,
                                      M, density, s);
    const int Cp = packed_channels(C);
    const int64_t count = (int64_t)(n + 1) * Cp;
    G2V_LAUNCH(k_split_pack, dim3((unsigned)ceil_div(count, 256)), dim3(256), 0, s, features, n, C, Cp, fpk);
    const int blocks = (int)ceil_div(T, 8) * 8;
    G2V_LAUNCH(k_fwd_feats, dim3(blocks), dim3(kFwdThreads), 0, s, G, C, means, opacity,
                       cov_inv, lb, ub, tile_offsets, sorted_gauss, M, n, Cp, (const uint32_t*)fpk, density,
                       grid_feats);
    return hipGetLastError();
}

}  // namespace g2v
