// Device-side helpers shared by the G2V kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace g2v {

constexpr int kTile = 4;                 // 4x4x4 voxel tiles (reference include/utils.cuh:50-52)
constexpr int kVoxPerTile = 64;          // one voxel per lane of a wave64
constexpr float kEps = 1e-6f;            // density clamp (reference include/utils.cuh:80)
constexpr int kWave = 64;

// Element type of the feature tensors (features, grid_feats, grad_features): the G2V_DTYPE_*
// codes of the C ABI.
constexpr int kDtF32 = 0;
constexpr int kDtBF16 = 1;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Grid geometry passed by value to every kernel.
//
// A batch of B scenes on the same grid is one problem with B x N Gaussians: Gaussian g belongs to
// scene g / N, tile t of scene b is tile b T + t of the batch (T tiles per scene) and region r of
// scene b is region b R + r, and the voxel rows of scene b start at row b X Y Z of the outputs.
// dims and tiles stay those of one scene; every box, tile and voxel coordinate is scene-local.
struct Grid {
    float r0[3];      // range lower corner
    float r1[3];      // range upper corner
    float s[3];       // voxel size
    int dims[3];      // X, Y, Z
    int tiles[3];     // Tx, Ty, Tz
    int scenes;       // B (1: a single scene)
    int scene_n;      // N, Gaussians per scene (used when scenes > 1)
};

__host__ __device__ __forceinline__ int scene_tiles(const Grid& G) { return G.tiles[0] * G.tiles[1] * G.tiles[2]; }
__host__ __device__ __forceinline__ int64_t scene_voxels(const Grid& G) {
    return (int64_t)G.dims[0] * G.dims[1] * G.dims[2];
}
// Scene of the batch's Gaussian g.
__host__ __device__ __forceinline__ int scene_of(const Grid& G, int g) {
    return G.scenes > 1 && G.scene_n > 0 ? g / G.scene_n : 0;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations and meets the
// other waves, without the release fence of __syncthreads.  That fence also waits for every
// outstanding global load and store of the wave (one in-order counter): direct-to-LDS loads kept in
// flight on purpose, and stores that no thread of the kernel reads back.  A caller that needs loaded
// data in LDS waits for it (vmcnt) before the barrier.
__device__ __forceinline__ void lds_barrier() {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15 << 0) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
}

// Voxel (x, y, z) of in-tile voxel index lv (x slowest, z fastest; reference .cu:43-55).
__device__ __forceinline__ void tile_voxel(const Grid& G, int tile, int lv, int& x, int& y, int& z) {
    const int tyz = G.tiles[1] * G.tiles[2];
    const int tx = tile / tyz;
    const int rem = tile - tx * tyz;
    const int ty = rem / G.tiles[2];
    const int tz = rem - ty * G.tiles[2];
    x = tx * kTile + (lv >> 4);
    y = ty * kTile + ((lv >> 2) & 3);
    z = tz * kTile + (lv & 3);
}

__device__ __forceinline__ bool in_grid(const Grid& G, int x, int y, int z) {
    return x < G.dims[0] && y < G.dims[1] && z < G.dims[2];
}

__device__ __forceinline__ int64_t voxel_index(const Grid& G, int x, int y, int z) {
    return ((int64_t)x * G.dims[1] + y) * G.dims[2] + z;
}

// Gaussian parameters used by the splat: mean, inverse covariance (row-major), opacity, box.
struct GaussParams {
    float mu[3];
    float A[9];
    float o;
    int lb[3], ub[3];
};

__device__ __forceinline__ void load_params(GaussParams& p, int g, const float* __restrict__ means,
                                            const float* __restrict__ cov_inv,
                                            const float* __restrict__ opacity,
                                            const int* __restrict__ lb, const int* __restrict__ ub) {
#pragma unroll
    for (int k = 0; k < 3; ++k) p.mu[k] = means[g * 3 + k];
#pragma unroll
    for (int k = 0; k < 9; ++k) p.A[k] = cov_inv[g * 9 + k];
    p.o = opacity[g];
#pragma unroll
    for (int k = 0; k < 3; ++k) { p.lb[k] = lb[g * 3 + k]; p.ub[k] = ub[g * 3 + k]; }
}

// Parameters of K consecutive entries of a Gaussian list, staged in LDS as structure of
// arrays (consecutive entries in consecutive banks; a wave-uniform entry is a broadcast read).
template <int K>
struct ParamTile {
    float mu[3][K];
    float A[9][K];
    float o[K];
    int lb[3][K];
    int ub[3][K];
    int gid[K];   // Gaussian id, -1 past the end of the list
};

// Cooperative load of list entries [0, count) (Gaussian ids list[0..count)) into pt.
template <int K>
__device__ __forceinline__ void stage_params(ParamTile<K>& pt, const int* __restrict__ list, int count,
                                             const float* __restrict__ means,
                                             const float* __restrict__ cov_inv,
                                             const float* __restrict__ opacity,
                                             const int* __restrict__ lb, const int* __restrict__ ub) {
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        if (k < count) {
            const int g = list[k];
            pt.gid[k] = g;
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                pt.mu[a][k] = means[g * 3 + a];
                pt.lb[a][k] = lb[g * 3 + a];
                pt.ub[a][k] = ub[g * 3 + a];
            }
#pragma unroll
            for (int a = 0; a < 9; ++a) pt.A[a][k] = cov_inv[g * 9 + a];
            pt.o[k] = opacity[g];
        } else {
            pt.gid[k] = -1;
        }
    }
}

template <int K>
__device__ __forceinline__ void read_params(const ParamTile<K>& pt, int k, GaussParams& p) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        p.mu[a] = pt.mu[a][k];
        p.lb[a] = pt.lb[a][k];
        p.ub[a] = pt.ub[a][k];
    }
#pragma unroll
    for (int a = 0; a < 9; ++a) p.A[a] = pt.A[a][k];
    p.o = pt.o[k];
}

__device__ __forceinline__ bool in_box(const GaussParams& p, int x, int y, int z) {
    return !(x < p.lb[0] || x > p.ub[0] || y < p.lb[1] || y > p.ub[1] || z < p.lb[2] || z > p.ub[2]);
}

// e = exp(-0.5 dx^T A dx), q = A dx, dx = centre - mu  (reference .cu:1239-1245)
__device__ __forceinline__ float eval_gauss(const GaussParams& p, float cx, float cy, float cz,
                                            float& qx, float& qy, float& qz) {
    const float d0 = cx - p.mu[0], d1 = cy - p.mu[1], d2 = cz - p.mu[2];
    qx = p.A[0] * d0 + p.A[1] * d1 + p.A[2] * d2;
    qy = p.A[3] * d0 + p.A[4] * d1 + p.A[5] * d2;
    qz = p.A[6] * d0 + p.A[7] * d1 + p.A[8] * d2;
    const float m = d0 * qx + d1 * qy + d2 * qz;
    return __expf(-0.5f * m);
}

// q = A dx alone, with the same operations as eval_gauss (so the same values).
__device__ __forceinline__ void gauss_q(const GaussParams& p, float cx, float cy, float cz, float& qx,
                                        float& qy, float& qz) {
    const float d0 = cx - p.mu[0], d1 = cy - p.mu[1], d2 = cz - p.mu[2];
    qx = p.A[0] * d0 + p.A[1] * d1 + p.A[2] * d2;
    qy = p.A[3] * d0 + p.A[4] * d1 + p.A[5] * d2;
    qz = p.A[6] * d0 + p.A[7] * d1 + p.A[8] * d2;
}

constexpr float kq = -0.72134752044448170f;   // -log2(e)/2: exp(-m/2) = exp2(kq m)

// One Gaussian's values as the forward's tile kernels read them, packed into one aligned 64-byte
// record (written beside its G->T rows): mean, opacity, the exponent coefficients kq A00,
// kq (A01 + A10), kq A11, kq (A02 + A20), kq (A12 + A21), kq A22, and the box.  A list entry then
// costs one 64-byte gather instead of one from each of five arrays.
struct alignas(16) DenParams {
    float mux, muy, muz, o;
    float a00, a01, a11, a02;
    float a12, a22;
    int lbx, lby;
    int lbz, ubx, uby, ubz;
};
static_assert(sizeof(DenParams) == 64, "DenParams is four 16-byte words");

__device__ __forceinline__ float centre(const Grid& G, int a, int i) {
    return fmaf((float)i + 0.5f, G.s[a], G.r0[a]);
}

// Split x into bf16 hi + bf16 lo with x ~= hi + lo (relative residual about 2^-17).
__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
    hi = (__bf16)x;
    lo = (__bf16)(x - (float)hi);
}

// Eight values at once, converted in pairs (one packed conversion per pair for hi and for lo).
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const f32x2 x = {v[2 * p], v[2 * p + 1]};
        const bf16x2 h = __builtin_convertvector(x, bf16x2);
        const bf16x2 l = __builtin_convertvector(x - __builtin_convertvector(h, f32x2), bf16x2);
        hi[2 * p] = h[0];
        hi[2 * p + 1] = h[1];
        lo[2 * p] = l[0];
        lo[2 * p + 1] = l[1];
    }
}

// acc += (a_hi + a_lo) (b_hi + b_lo) without the lo*lo term: three bf16 MFMAs, fp32 accumulate.
__device__ __forceinline__ f32x16 mfma3_32x32x16(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                                 const bf16x8& bl, f32x16 acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
    return acc;
}

// The product with terms known to be zero left out: BEX, B's low part is zero (B holds
// bfloat16 values exactly); AEX, A's low part is zero.  The remaining terms are added in the same
// order, so the result equals the three-term product's (an exact zero term changes nothing but
// the sign of a zero sum).
template <bool AEX, bool BEX>
__device__ __forceinline__ f32x16 mfma_split_32x32x16(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                                      const bf16x8& bl, f32x16 acc) {
    if constexpr (!AEX) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    if constexpr (!BEX) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
}

// Same three-term product on the 16 x 16 x 32 shape.  Operand lanes: A row l%16, k 8(l/16)+i;
// B column l%16, k 8(l/16)+i; D element i at row 4(l/16)+i, column l%16.
__device__ __forceinline__ f32x4 mfma3_16x16x32(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                               const bf16x8& bl, f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    return acc;
}

template <bool AEX, bool BEX>
__device__ __forceinline__ f32x4 mfma_split_16x16x32(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                                    const bf16x8& bl, f32x4 acc) {
    if constexpr (!AEX) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    if constexpr (!BEX) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}

// v of lane l ^ m within each 32-lane half, for m in {1, 2, 4, 8, 16}: DPP quad permutes for 1
// and 2, ds_swizzle (bit mode) for 4, 8 and 16; no LDS address is needed.
template <int M>
__device__ __forceinline__ float xor_shfl(float v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16, "xor mask");
    const int iv = __float_as_int(v);
    if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
    else if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(iv, 0x1F | (M << 10)));
}

// Sums of 16 values per lane over the 32 lanes of each half-wave, transposed: afterwards lanes
// 2k and 2k+1 (of each half) hold the sum of value k.  Each butterfly step hands half of the
// remaining values to the partner lane: 8 + 4 + 2 + 1 + 1 exchanges instead of 16 x 5.
__device__ __forceinline__ float transpose_sum16(const float (&v)[16], int l /* lane % 32 */) {
    float w[8];
    const bool b16 = l & 16, b8 = l & 8, b4 = l & 4, b2 = l & 2;
#pragma unroll
    for (int k = 0; k < 8; ++k)
        w[k] = (b16 ? v[k + 8] : v[k]) + xor_shfl<16>(b16 ? v[k] : v[k + 8]);
    float u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        u[k] = (b8 ? w[k + 4] : w[k]) + xor_shfl<8>(b8 ? w[k] : w[k + 4]);
    float t[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        t[k] = (b4 ? u[k + 2] : u[k]) + xor_shfl<4>(b4 ? u[k] : u[k + 2]);
    const float q = (b2 ? t[1] : t[0]) + xor_shfl<2>(b2 ? t[0] : t[1]);
    return q + xor_shfl<1>(q);
}

// Wave64 sum (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Load 8 consecutive floats p[0..7] where only the first `valid` (0..8) are in bounds; the
// rest read as 0.  `vec_ok` says p is 16-byte aligned so two dwordx4 loads can be used.
__device__ __forceinline__ void load8(const float* __restrict__ p, int valid, bool vec_ok, float (&v)[8]) {
    if (valid >= 8 && vec_ok) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (i < valid) ? p[i] : 0.0f;
    }
}


// Feature element e of a row of type T, as float.
template <typename T>
__device__ __forceinline__ float feat_at(const T* __restrict__ p, int64_t e) {
    if constexpr (sizeof(T) == 2) return (float)p[e];
    else return p[e];
}

}  // namespace g2v
