// Backward of the G2V splat for gfx950, atomic-free and deterministic
// (reference src/cuda_gaussian_voxelizer.cu:1226-1482, :1920-2057).
//
// Per (Gaussian g, voxel v in its box): e = exp(-0.5 dx^T A dx), w = o e, q = A dx,
// inv = 1 / max(D_v, eps), t_v = (D_v >= eps) ? sum_c gF_vc F_vc : 0, u_gv = sum_c gF_vc f_gc,
//     gw = gD_v + (u_gv - t_v) inv        (gw = gD_v without features)
//     d mu += gw w q,  d Sigma += 0.5 gw w q q^T (symmetric),  d o += gw e,  d f_g += gF_v w inv
//
// With features the work is split in three phases so that every gF row is read from HBM
// twice instead of once per overlapping Gaussian (the reference re-reads it per pair):
//   A  k_bwd_tile    one workgroup per 4x4x4 tile: U^T = G_tile (64 x C) . F_list^T on the matrix
//                    cores (3-term bf16 split, fp32 accumulate); t_v from U (sum_g [w>0] w u / D is
//                    sum_c gF F); gw; ten moments of r = gw e over the pair's voxels (sum r d,
//                    sum r d d^T, sum r with d = centre - mu), stored at the pair's G->T CSR
//                    slot; the split weights w/max(D,eps) of the pair.
//   B  k_bwd_region  one workgroup per (region of 2x2xRZ tiles, 128-channel chunk): for every
//                    tile of the region, (region rows x 64 voxels) . (64 voxels x 128 channels) on
//                    the matrix cores, accumulated in registers (a wave owns 32 region rows);
//                    writes one partial d f row per (region, Gaussian) pair at its G->R CSR slot.
//   C  k_bwd_gauss   one workgroup per Gaussian: fixed-order sums of its pair moments, turned
//                    into d mu, d Sigma and d o by its inverse covariance, and of its region
//                    partial rows.
// Without features, k_bwd_density walks each Gaussian's box with one wave.
#include "g2v_internal.h"
#include <type_traits>

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

// Regions of the feature-gradient phase: 2 x 2 tiles in x, y and up to 4 tiles in z.
struct Regions {
    int cell[3];   // voxels per region along each axis
    int n[3];      // region grid
    int total;
};

static Regions make_regions(const Grid& G) {
    Regions R;
    const int rz = min(G.tiles[2], 4);
    R.cell[0] = 2 * kTile;
    R.cell[1] = 2 * kTile;
    R.cell[2] = rz * kTile;
    for (int a = 0; a < 3; ++a) R.n[a] = (G.dims[a] + R.cell[a] - 1) / R.cell[a];
    R.total = R.n[0] * R.n[1] * R.n[2];
    return R;
}

// ------------------------------------------------------------------------------------------
// Density only: one wave per Gaussian walks the voxels of its box.  Per voxel, with d = centre - mu,
// q = A d and r = gD e, e = exp(-d^T q / 2): the Gaussian's gradients are d mu = o sum r q,
// d Sigma = o/2 sum r q q^T (symmetric), d o = sum r (reference .cu:1304-1362 with gw = gD:
// sum gw w q, sum gw w q q^T / 2, sum gw e, w = o e), with o and 1/2 applied once per Gaussian.
// The lanes take the box's (y, z) cells (z fastest, 64 at a time) and walk x.  Along a lane's
// line only dx changes: with q' = kq q = q0 + b dx (b = kq A e_x, q0 = kq A (0, dy, dz)), the exponent
// of exp2 is d^T q' = alpha + beta dx + gamma dx^2, and the line's sums of r, r q' and r q' q'^T
// follow from R0 = sum r, R1 = sum r dx, R2 = sum r dx^2 (q0 R0 + b R1, q0 q0^T R0 +
// (q0 b^T + b q0^T) R1 + b b^T R2), turned into them once per line.  A voxel then costs an exp2 and
// about ten other operations.  dx = x s_x + (r0_x + s_x/2 - mu_x), x an exact float integer.  The
// lane's gD loads run one chunk of four voxels ahead.  The factors kq and kq^2 come off with o and
// 1/2.  kNarrow: the scene's voxel byte offsets fit in 32 bits (loads from a scalar base and a
// 32-bit offset).
// ------------------------------------------------------------------------------------------

// floor(a / b) for 0 <= a < 2^23, b > 0: the correctly rounded float quotient never reaches the
// next integer for such a (its distance to it, at least 1/b, exceeds half an ulp of a/b).
__device__ __forceinline__ int small_quot(int a, int b) { return (int)((float)a / (float)b); }

template <bool kNarrow>
__global__ void __launch_bounds__(256) k_bwd_density(Grid G, int n, const float* __restrict__ gD,
                                                     const float* __restrict__ means,
                                                     const float* __restrict__ opacity,
                                                     const float* __restrict__ cov_inv,
                                                     const int* __restrict__ lb,
                                                     const int* __restrict__ ub,
                                                     float* __restrict__ grad_means,
                                                     float* __restrict__ grad_cov,
                                                     float* __restrict__ grad_opacity) {
    constexpr int kChunk = 4;
    const int lane = threadIdx.x & 63;
    const int g = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (g >= n) return;
    gD += scene_of(G, g) * scene_voxels(G);   // the scene's voxels
    GaussParams p;
    load_params(p, g, means, cov_inv, opacity, lb, ub);
    const int ex = p.ub[0] - p.lb[0] + 1, ey = p.ub[1] - p.lb[1] + 1, ez = p.ub[2] - p.lb[2] + 1;
    const bool live = ex > 0 && ey > 0 && ez > 0;
    float off[3], B[9];
#pragma unroll
    for (int a = 0; a < 3; ++a) off[a] = fmaf(0.5f, G.s[a], G.r0[a]) - p.mu[a];
#pragma unroll
    for (int k = 0; k < 9; ++k) B[k] = kq * p.A[k];
    const float bq[3] = {B[0], B[3], B[6]};   // q' per unit dx
    float sr = 0.f, sq[3] = {0.f, 0.f, 0.f}, sqq[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int eyz = live ? ey * ez : 0;
    const unsigned Y = (unsigned)G.dims[1], Z = (unsigned)G.dims[2], YZ = Y * Z;
    const int nchunks = (ex + kChunk - 1) / kChunk;
    auto gload = [&](unsigned v) {
        return kNarrow ? *reinterpret_cast<const float*>(reinterpret_cast<const char*>(gD) + (v << 2)) : gD[v];
    };
    for (int s0 = 0; s0 < eyz; s0 += 64) {
        const int sl = s0 + lane;
        const bool act = sl < eyz;
        const int iy = eyz < (1 << 22) ? small_quot(sl, ez) : sl / ez;   // sl < eyz + 64 < 2^23
        const int iz = sl - iy * ez;
        const float dy = fmaf((float)(p.lb[1] + iy), G.s[1], off[1]);
        const float dz = fmaf((float)(p.lb[2] + iz), G.s[2], off[2]);
        const float q0[3] = {fmaf(B[1], dy, B[2] * dz), fmaf(B[4], dy, B[5] * dz), fmaf(B[7], dy, B[8] * dz)};
        const float alpha = fmaf(dy, q0[1], dz * q0[2]);
        const float beta = fmaf(B[3], dy, fmaf(B[6], dz, q0[0]));
        const float gamma = B[0];
        float R0 = 0.f, R1 = 0.f, R2 = 0.f;
        if (act) {
            // every load is issued (a chunk past the line's end reloads its last voxel), so that the
            // counter of loads stays exact across the uniform branches below
            const unsigned vb = ((unsigned)p.lb[0] * Y + (unsigned)(p.lb[1] + iy)) * Z + (unsigned)(p.lb[2] + iz);
            auto ld = [&](int xo) { return gload(vb + (unsigned)min(xo, ex - 1) * YZ); };
            float fx = (float)p.lb[0];
            float cur[kChunk];
#pragma unroll
            for (int k = 0; k < kChunk; ++k) cur[k] = ld(k);
            for (int c = 0; c < nchunks; ++c) {
                float nxt[kChunk];
#pragma unroll
                for (int k = 0; k < kChunk; ++k) nxt[k] = ld((c + 1) * kChunk + k);
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    if (c * kChunk + k < ex) {
                        const float dx = fmaf(fx, G.s[0], off[0]);
                        const float r = cur[k] * __builtin_amdgcn_exp2f(fmaf(fmaf(gamma, dx, beta), dx, alpha));
                        R0 += r;
                        const float rdx = r * dx;
                        R1 += rdx;
                        R2 = fmaf(rdx, dx, R2);
                        fx += 1.0f;
                    }
                }
#pragma unroll
                for (int k = 0; k < kChunk; ++k) cur[k] = nxt[k];
            }
        }
        // the line's sums in q': q' = q0 + b dx
        sr += R0;
#pragma unroll
        for (int a = 0; a < 3; ++a) sq[a] += fmaf(q0[a], R0, bq[a] * R1);
        const int pi[6] = {0, 1, 2, 0, 0, 1}, pj[6] = {0, 1, 2, 1, 2, 2};   // xx yy zz xy xz yz
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const int a = pi[k], b = pj[k];
            sqq[k] += fmaf(q0[a] * q0[b], R0, fmaf(fmaf(q0[a], bq[b], bq[a] * q0[b]), R1, bq[a] * bq[b] * R2));
        }
    }
    // the wave's sums: lanes 2k, 2k + 1 of each half hold value k after the transposed butterfly
    float vs[16] = {sq[0], sq[1], sq[2], sqq[0], sqq[1], sqq[2], sqq[3], sqq[4], sqq[5], sr, 0.f, 0.f, 0.f, 0.f,
                    0.f, 0.f};
    float t = transpose_sum16(vs, lane & 31);
    t += __shfl_xor(t, 32, 64);
    // value k of lane 2k: mu xyz, cov xx yy zz xy xz yz, opacity (the order of write_grads)
    const float fq = p.o / kq, fqq = 0.5f * p.o / (kq * kq);
    const int k = (lane & 31) >> 1;
    const float gv = k < 3 ? fq * t : (k < 9 ? fqq * t : t);
    if (lane < 20 && (lane & 1) == 0) {
        if (k < 3) grad_means[g * 3 + k] = gv;
        else if (k == 9) grad_opacity[g] = gv;
        else {
            // symmetric 3x3: xx yy zz on the diagonal, xy xz yz on both sides
            const int j = k - 3;
            const int i0 = j < 3 ? 4 * j : (j == 3 ? 1 : (j == 4 ? 2 : 5));
            const int i1 = j < 3 ? 4 * j : (j == 3 ? 3 : (j == 4 ? 6 : 7));
            grad_cov[g * 9 + i0] = gv;
            grad_cov[g * 9 + i1] = gv;
        }
    }
}

hipError_t launch_backward_density(const Grid& G, int n, const float* grad_density,
                                   const float* means, const float* opacity, const float* cov_inv,
                                   const int* lb, const int* ub, float* grad_means, float* grad_cov,
                                   float* grad_opacity, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)ceil_div(n, 4)), block(256);
    if (scene_voxels(G) < (int64_t(1) << 30))
        G2V_LAUNCH(k_bwd_density<true>, grid, block, 0, s, G, n, grad_density, means, opacity, cov_inv, lb, ub,
                   grad_means, grad_cov, grad_opacity);
    else
        G2V_LAUNCH(k_bwd_density<false>, grid, block, 0, s, G, n, grad_density, means, opacity, cov_inv, lb, ub,
                   grad_means, grad_cov, grad_opacity);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Features split once into 32-channel chunks of bf16 hi/lo: chunk k of row g is 128 contiguous
// bytes, hi[32] then lo[32].  Row n and the channels >= C are zero.
// ------------------------------------------------------------------------------------------
constexpr int kBtKc = 32;                  // channels per chunk
constexpr int kBtRowBytes = kBtKc * 4;     // bytes of one row's chunk (hi and lo)

// bfloat16 features need no split: their chunks are kBtKcBf = 64 channels of the row itself, 128
// bytes (the same bytes per chunk row as a float chunk's hi and lo).
constexpr int kBtKcBf = 2 * kBtKc;

template <typename T>
__global__ void __launch_bounds__(256) k_split_chunks(const T* __restrict__ src, int n, int C, int nchk,
                                                      __bf16* __restrict__ dst) {
    // one thread per 8 channels of a row (an octet of a chunk): 16-byte hi and lo stores
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    constexpr bool kBf = sizeof(T) == 2;
    const int noct = nchk * ((kBf ? kBtKcBf : kBtKc) / 8);
    if (i >= (int64_t)(n + 1) * noct) return;
    const int64_t r = i / noct;
    const int oc = (int)(i - r * noct);
    const int c = oc * 8;
    float v[8];
    if (sizeof(T) == 4 && r < n && c + 8 <= C && ((uintptr_t)(src + r * C + c) & 15) == 0) {
        const float4 a = *reinterpret_cast<const float4*>(src + r * C + c);
        const float4 b = *reinterpret_cast<const float4*>(src + r * C + c + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (r < n && c + e < C) ? feat_at(src, r * C + c + e) : 0.0f;
    }
    bf16x8 h, l;
    split8(v, h, l);
    if constexpr (kBf) {   // the row padded to nchk * 64 channels (l is zero)
        *reinterpret_cast<bf16x8*>(dst + r * nchk * kBtKcBf + c) = h;
        return;
    }
    __bf16* row = dst + (r * nchk + c / kBtKc) * (2 * kBtKc);
    *reinterpret_cast<bf16x8*>(row + c % kBtKc) = h;
    *reinterpret_cast<bf16x8*>(row + kBtKc + c % kBtKc) = l;
}

// ------------------------------------------------------------------------------------------
// Phase A: tile-major U, t_v, gw, geometric partials, split weights.
// ------------------------------------------------------------------------------------------
constexpr int kBtThreads = 512;                        // 8 waves
constexpr int kBtWaves = kBtThreads / 64;
constexpr int kBtGroups = 4;                           // Gaussian groups (wave >> 1)
constexpr int kBtNbw = 2;                              // 32-Gaussian N blocks per wave per pass
constexpr int kBtPass = kBtGroups * kBtNbw * 32;       // 256 Gaussians per pass
constexpr int kBtStages = 3;                           // F chunks resident in LDS (loaded 2 ahead)
constexpr int kBtDma = kBtPass / 8 / kBtWaves;         // 1 KB direct-to-LDS loads per wave per chunk
constexpr int kWtRow = 128;                            // bf16 per pair: 64 hi then 64 lo

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Slot swizzle of 128-byte LDS rows of 16-byte pieces: piece q of row r sits at slot q ^ swz(r).
// Any 8 consecutive rows get distinct swz values, and any 16 consecutive rows give distinct
// (row parity, swz) pairs, so reading one piece from each of 8 (32 banks) or 16 (64 banks)
// consecutive rows per LDS cycle is free of bank conflicts.
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// Direct-to-LDS loads: lane l writes its 16 (or 4) bytes from gptr at LDS address lds + 16*l
// (4*l).  Issued as inline assembly so that the compiler does not attach conservative waits to
// later LDS reads; every consumer waits explicitly (wait_vm) and meets the other waves at a
// barrier.  M0 carries the wave-uniform LDS base and needs one wait state before the load.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gptr), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :: "v"(gptr), "s"(lds) : "memory", "m0");
}
// Scalar-base forms: the wave-uniform base in SGPRs and a 32-bit per-lane byte offset, so that a
// chunk's advance is scalar work and the per-lane offsets stay fixed across the chunk loop.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma16s_nt(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
// Streaming variants (non-temporal): for data read once, so that it does not evict the feature
// rows that many tiles re-read.
__device__ __forceinline__ void dma16_nt(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(gptr), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4_nt(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
                 :: "v"(gptr), "s"(lds) : "memory", "m0");
}

// FU: the upstream feature gradient is the cosine loss's, G = k1 target + k2 grid_feats per voxel,
// formed on chip from two raw chunks (target and grid_feats) per stage; the F rows then use two
// buffers (loaded one chunk ahead) so that the second raw chunk fits.
template <bool FU>
struct BtSmem {
    static constexpr int kFStages = FU ? 2 : kBtStages;   // F chunk buffers
    static constexpr int kSrc = FU ? 2 : 1;               // raw G sources per stage
    union {
        // F chunk rows of the pass's Gaussians; the 16-byte piece q of row r sits at slot
        // q ^ swz(r), so that the lanes of one LDS cycle (8 or 16 consecutive rows) hit distinct
        // 16-byte bank groups
        unsigned char frow[kFStages][kBtPass * kBtRowBytes];
        float xch[2][kBtPass][kNumGrads];   // epilogue exchange, used after the K loop has drained
        struct {
            float xch_room[2][kBtPass][kNumGrads];
            // the exponentials of epilogue 1, read again by epilogue 2: [wave][N block][q4][lane]
            // (FU: no room beside the two F buffers; epilogue 2 evaluates them again)
            float4 e[FU ? 1 : kBtWaves][kBtNbw][4][64];
        } ep;
    } u;
    // G chunks as loaded (fp32, voxel-major, pieces at q ^ swz(v)); FU: [0] target, [1] grid_feats
    float graw[kBtStages][kSrc][64][kBtKc];
    bf16x8 ahi[2][2][2][64];   // A operand (G chunk), hi: [buffer][k half][voxel block][lane]
    bf16x8 alo[2][2][2][64];
    int vlin[64];
    float gD[64], inv[64], tv[64], D[64];
    float kc[2][FU ? 64 : 1];  // FU: the voxel's k1, k2 (scaled by the loss's upstream gradient)
    ParamTile<kBtPass> pt;     // parameters of this pass's list entries
    int pidx[kBtPass];         // G->T pair of each entry with this tile (-1: none)
    float tpart[kBtGroups][64];
};
static_assert(sizeof(float) * 2 * kBtNbw * 16 * 64 * kBtGroups <= BtSmem<true>::kFStages * kBtPass * kBtRowBytes,
              "the k-half exchange fits in the F buffers");
static_assert(sizeof(BtSmem<false>::u) == sizeof(BtSmem<false>::u.frow) && sizeof(BtSmem<true>::u) == sizeof(BtSmem<true>::u.frow),
              "the epilogue's exponentials fit in the F buffers");


// s_waitcnt immediate that waits for vmcnt <= n and leaves the other counters alone.
__device__ constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// Waits until at most n vector-memory loads of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(N));
    __builtin_amdgcn_sched_barrier(0);
}



// Geometry of one lane's 16 epilogue elements against its Gaussian.  The elements of a lane are
// the 2 x 2 x 4 voxel block x = x0 + a, y = y0 + 2b, z = z0 + c of the tile (a, b < 2, c < 4), so
// dx = centre - mu and the box test (bit masks) split by axis.
struct LaneGeom {
    float dx[2], dy[2], dz[4];
    unsigned inx, iny, inz;               // bit a / b / c: the offset lies in the Gaussian's box
};

__device__ __forceinline__ void lane_geom(const Grid& G, const GaussParams& p, int x0, int y0, int z0,
                                          LaneGeom& L) {
#pragma clang fp contract(off)
    L.inx = L.iny = L.inz = 0;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int x = x0 + a, y = y0 + 2 * a;
        L.dx[a] = centre(G, 0, x) - p.mu[0];
        L.dy[a] = centre(G, 1, y) - p.mu[1];
        L.inx |= (x >= p.lb[0] && x <= p.ub[0]) ? (1u << a) : 0u;
        L.iny |= (y >= p.lb[1] && y <= p.ub[1]) ? (1u << a) : 0u;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int z = z0 + c;
        L.dz[c] = centre(G, 2, z) - p.mu[2];
        L.inz |= (z >= p.lb[2] && z <= p.ub[2]) ? (1u << c) : 0u;
    }
}

// The exponent -m/2 of a lane's element (a, b, c), split by axis and scaled by kq so that
// e = exp2(Fxy[a][b] + Fz[c] + Gxy[a][b] dz[c]) (m = d^T A d summed in this order).
struct LaneExp {
    float Fxy[2][2], Gxy[2][2], Fz[4];
};

// Contraction is off in these helpers, so that every phase A instantiation that inlines them
// computes the same e (and so the same split weights) for the same pair, whatever the code around.
__device__ __forceinline__ void lane_exp(const GaussParams& p, const LaneGeom& L, LaneExp& E) {
#pragma clang fp contract(off)
    const float sxy = p.A[1] + p.A[3], sxz = p.A[2] + p.A[6], syz = p.A[5] + p.A[7];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float dx = L.dx[a], dy = L.dy[b];
            E.Fxy[a][b] = kq * fmaf(fmaf(p.A[0], dx, sxy * dy), dx, p.A[4] * dy * dy);
            E.Gxy[a][b] = kq * fmaf(sxz, dx, syz * dy);
        }
#pragma unroll
    for (int c = 0; c < 4; ++c) E.Fz[c] = kq * (p.A[8] * L.dz[c] * L.dz[c]);
}

__device__ __forceinline__ float lane_e(const LaneExp& E, const LaneGeom& L, int a, int b, int c) {
#pragma clang fp contract(off)
    return __builtin_amdgcn_exp2f(fmaf(E.Gxy[a][b], L.dz[c], E.Fxy[a][b] + E.Fz[c]));
}

// BF: features and grad_feats are bfloat16.  A chunk is then 64 channels (the split rows hold the
// values themselves, 128 bytes per chunk row, as k_split_chunks<__bf16> writes them; the grad_feats
// chunk rows are 128 bytes of bfloat16), and each k half of 32 channels is two 16-channel slices:
// the A and B "hi" operands carry slice 0 and the "lo" operands slice 1, with one MFMA each.
// FU (with VEC, float32): the upstream feature gradient is the cosine loss's (cg), gF_ is unused.
template <bool VEC, bool BF, bool FU>
__global__ void __launch_bounds__(kBtThreads, 1) k_bwd_tile(
    Grid G, int n, int C, int nchk, const float* __restrict__ gD, const void* __restrict__ gF_,
    const float* __restrict__ means, const float* __restrict__ opacity,
    const float* __restrict__ cov_inv, const int* __restrict__ lb, const int* __restrict__ ub,
    const int* __restrict__ g2t_offsets, const int* __restrict__ toff,
    const int* __restrict__ sorted_gauss, int M, const float* __restrict__ density,
    const void* __restrict__ grid_feats, int gdt, const __bf16* __restrict__ fsp,
    float* __restrict__ pair_partials, __bf16* __restrict__ wt, CosG cg, int skip_le,
    const int* __restrict__ tlist, const int* __restrict__ tcount) {
    static_assert(!FU || (VEC && !BF), "the fused cosine gradient takes 16-byte float32 rows");
    __shared__ BtSmem<FU> sm;
    const int T = scene_tiles(G);
    // tb: the batch's tile (its list), tile: the scene's; with tlist, workgroup i takes the i-th
    // long tile of the compacted list
    int tb;
    if (tlist) {
        const int i = uniform(xcd_remap(blockIdx.x, gridDim.x));
        if (i >= uniform(*tcount)) return;
        tb = uniform(tlist[i]);
    } else {
        tb = uniform(xcd_remap(blockIdx.x, gridDim.x));
        if (tb >= T * G.scenes) return;
    }
    const int scene = uniform(tb / T), tile = tb - scene * T;
    if (scene > 0) {   // the scene's voxel rows
        const int64_t vb = scene * scene_voxels(G);
        gD += vb;
        density += vb;
        gF_ = static_cast<const char*>(gF_) + vb * C * (BF ? 2 : 4);
        grid_feats = static_cast<const char*>(grid_feats) + vb * C * (gdt == kDtBF16 ? 2 : 4);
        if constexpr (FU) {
            cg.tgt += vb * C;
            cg.coef += 2 * vb;
        }
    }
    const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
    const int mb = wave >> 2, ngrp = wave & 3;   // voxel block (epilogues) / k half (K loop), N group
    const int tyz = G.tiles[1] * G.tiles[2];
    const int tx = tile / tyz, ty = (tile - tx * tyz) / G.tiles[2], tz = tile % G.tiles[2];
    // every voxel of the tile inside the grid (no row of the A operand is cleared)
    const bool tile_in = (tx + 1) * kTile <= G.dims[0] && (ty + 1) * kTile <= G.dims[1] &&
                         (tz + 1) * kTile <= G.dims[2];

    // the tile's voxel values are requested with its list bounds (they do not depend on them)
    int vx = 0;
    bool vok = false;
    float vgd = 0.0f, vd = 0.0f;
    if (threadIdx.x < 64) {
        int x, y, z;
        tile_voxel(G, tile, threadIdx.x, x, y, z);
        vok = in_grid(G, x, y, z);
        vx = vok ? (int)voxel_index(G, x, y, z) : 0;
        vgd = gD[vx];
        vd = density[vx];
    }
    const int j0 = uniform(min(max(toff[tb], 0), M));
    const int Ng = uniform(min(max(toff[tb + 1], j0), M)) - j0;
    if (Ng <= skip_le) return;   // empty, or a short list that k_bwd_tile_short takes
    // the first pass's list entries, requested before the voxel values are staged (raw values at
    // clamped positions; the entries past the pass are selected away where they are used)
    const int lwave = uniform(threadIdx.x >> 6), llane = threadIdx.x & 63;
    const int pc0 = min(kBtPass, Ng);
    const int l0 = sorted_gauss[j0 + min((int)threadIdx.x, pc0 - 1)];
    int lrow0[kBtDma];
#pragma unroll
    for (int i = 0; i < kBtDma; ++i) lrow0[i] = sorted_gauss[j0 + min((lwave + kBtWaves * i) * 8 + (llane >> 3), pc0 - 1)];
    if (threadIdx.x < 64) {
        const bool ok = vok;
        const int64_t v = vx;
        sm.vlin[threadIdx.x] = ok ? (int)v : -1;
        sm.gD[threadIdx.x] = ok ? vgd : 0.0f;
        sm.D[threadIdx.x] = ok ? vd : 0.0f;
        sm.inv[threadIdx.x] = ok ? 1.0f / fmaxf(vd, kEps) : 0.0f;
        sm.tv[threadIdx.x] = 0.0f;
        if constexpr (FU) {
            const float scale = cg.grad_loss[0] * cg.inv_count;   // as the loss's own backward forms it
            sm.kc[0][threadIdx.x] = ok ? cg.coef[2 * v] * scale : 0.0f;
            sm.kc[1][threadIdx.x] = ok ? cg.coef[2 * v + 1] * scale : 0.0f;
        }
    }
    __syncthreads();

    typedef typename std::conditional<BF, __bf16, float>::type GT;   // element of grad_feats
    const GT* gF = static_cast<const GT*>(gF_);
    constexpr int kKc = BF ? kBtKcBf : kBtKc;   // channels per chunk
    // Lists longer than one pass: t_v = sum_c gF_vc F_vc straight from grid_feats.
    const bool multi = Ng > kBtPass;
    if (multi && VEC && !BF && (FU || gdt != kDtBF16) && ((uintptr_t)grid_feats & 15) == 0) {
        // float rows of 16-byte multiples: the wave's 8 voxels at once, 8 lanes per row reading
        // 16-byte pieces (many loads in flight), then a sum over the row's 8 lanes.  FU: G = k1
        // target + k2 grid_feats formed per value, as the loss's own backward forms it.
        const int r = wave * 8 + (lane >> 3), q = lane & 7;
        const int v = sm.vlin[r];
        float s = 0.0f;
        if (v >= 0) {
            const float* arow = FU ? cg.tgt + (int64_t)v * C : reinterpret_cast<const float*>(gF) + (int64_t)v * C;
            const float4* a4 = reinterpret_cast<const float4*>(arow);
            const float4* b4 = reinterpret_cast<const float4*>(static_cast<const float*>(grid_feats) + (int64_t)v * C);
            const int n4 = C / 4;
            float k1 = 1.0f, k2 = 0.0f;
            if constexpr (FU) {
                k1 = sm.kc[0][r];
                k2 = sm.kc[1][r];
            }
#pragma unroll 4
            for (int c4 = q; c4 < n4; c4 += 8) {
                float4 x = a4[c4];
                const float4 y = b4[c4];
                if constexpr (FU) {
                    x.x = k1 * x.x + k2 * y.x;
                    x.y = k1 * x.y + k2 * y.y;
                    x.z = k1 * x.z + k2 * y.z;
                    x.w = k1 * x.w + k2 * y.w;
                }
                s = fmaf(x.x, y.x, s);
                s = fmaf(x.y, y.y, s);
                s = fmaf(x.z, y.z, s);
                s = fmaf(x.w, y.w, s);
            }
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if (q == 0 && v >= 0) sm.tv[r] = sm.D[r] >= kEps ? s : 0.0f;
    } else if (multi) {
        for (int k = 0; k < 8; ++k) {
            const int r = wave * 8 + k;
            const int v = sm.vlin[r];
            if (v < 0) continue;
            const GT* a = gF + (int64_t)v * C;
            float s = 0.0f;
            if constexpr (FU) {
                // G = k1 target + k2 grid_feats, as the loss's backward rounds it to float
                const float k1 = sm.kc[0][r], k2 = sm.kc[1][r];
                const float* tg = cg.tgt + (int64_t)v * C;
                const float* b = static_cast<const float*>(grid_feats) + (int64_t)v * C;
                for (int c = lane; c < C; c += 64) {
                    const float gv = k1 * tg[c] + k2 * b[c];
                    s += gv * b[c];
                }
            } else if (gdt == kDtBF16) {
                const __bf16* b = static_cast<const __bf16*>(grid_feats) + (int64_t)v * C;
                for (int c = lane; c < C; c += 64) s += (float)a[c] * (float)b[c];
            } else {
                const float* b = static_cast<const float*>(grid_feats) + (int64_t)v * C;
                for (int c = lane; c < C; c += 64) s += (float)a[c] * b[c];
            }
            s = wave_sum(s);
            if (lane == 0) sm.tv[r] = sm.D[r] >= kEps ? s : 0.0f;
        }
    }

    // G staging: direct-to-LDS loads of the raw chunk (voxel rows clamped to a valid row, channels
    // clamped into the row).  Row v of a stage keeps its 16-byte piece p (channels 4p..4p+3) at
    // slot p ^ swz(v), so that the A-operand reads (8 or 16 consecutive rows per LDS cycle) are
    // free of bank conflicts.  VEC: one 16-byte load per lane, lane = (row, slot); otherwise four 4-byte
    // loads per lane, each covering two rows.
    // BF: a chunk row is 128 bytes of bfloat16; with VEC (C % 8 == 0, 16-byte aligned rows) lane l
    // loads 16-byte piece l % 8 of row l / 8 of the wave's 8 rows (stage rows of 128 bytes, pieces
    // in order, read whole by write_a); without VEC write_a loads the A operand itself.
    // FU: the target and grid_feats chunks of the same rows, into sources 0 and 1 of the stage.
    constexpr int kNG = BF ? (VEC ? 1 : 0) : (VEC ? 1 : 4);   // G loads per wave per chunk and source
    constexpr int kNGs = kNG > 0 ? kNG : 1;
    constexpr int kSrc = FU ? 2 : 1;
    const GT* gsrc[kSrc][kNGs];
    int gcoff[kNGs];   // channel of this lane's load within a chunk
    // VEC float: chunks wholly inside the rows are loaded from a wave-uniform base (the source's
    // start plus the chunk) and the lane's fixed 32-bit byte offset, when every row offset fits
    const GT* gbase[kSrc];
    uint32_t goff[kNGs];
    gbase[0] = FU ? reinterpret_cast<const GT*>(cg.tgt) : gF;
    gbase[kSrc - 1] = FU ? static_cast<const GT*>(grid_feats) : gF;
    const bool g32 = (int64_t)G.dims[0] * G.dims[1] * G.dims[2] * C * (int64_t)sizeof(GT) <= 0xffffffffLL;
#pragma unroll
    for (int k = 0; k < kNG; ++k) {
        const int v = (BF || VEC) ? wave * 8 + (lane >> 3) : wave * 8 + 2 * k + (lane >> 5);
        const int64_t row = (int64_t)max(sm.vlin[v], 0) * C;
        if constexpr (FU) {
            gsrc[0][k] = reinterpret_cast<const GT*>(cg.tgt) + row;
            gsrc[kSrc - 1][k] = static_cast<const GT*>(grid_feats) + row;
        } else {
            gsrc[0][k] = gF + row;
        }
        gcoff[k] = BF ? 8 * (lane & 7)
                      : (VEC ? 4 * ((lane & 7) ^ swz(v)) : 4 * (((lane & 31) >> 2) ^ swz(v)) + (lane & 3));
        goff[k] = (uint32_t)((row + gcoff[k]) * (int64_t)sizeof(GT));
    }
    auto dma_g = [&](int chunk, int stage) {
#pragma unroll
        for (int sr = 0; sr < kSrc; ++sr)
#pragma unroll
            for (int k = 0; k < kNG; ++k) {
                if constexpr (BF) {
                    dma16_nt(gsrc[sr][k] + min(chunk * kKc + gcoff[k], C - 8),
                             uniform(lds_addr(reinterpret_cast<char*>(&sm.graw[stage][sr][0][0]) + wave * 8 * 128)));
                } else if (VEC) {
                    const uint32_t lds = uniform(lds_addr(&sm.graw[stage][sr][wave * 8][0]));
                    if (g32 && chunk * kBtKc + kBtKc <= C)   // wave-uniform
                        dma16s_nt(gbase[sr] + chunk * kBtKc, goff[k], lds);
                    else
                        dma16_nt(gsrc[sr][k] + min(chunk * kBtKc + gcoff[k], C - 4), lds);
                } else {
                    dma4_nt(gsrc[sr][k] + min(chunk * kBtKc + gcoff[k], C - 1),
                            uniform(lds_addr(&sm.graw[stage][sr][wave * 8 + 2 * k][0])));
                }
            }
    };

    const uint32_t fstride = (uint32_t)nchk * kBtRowBytes;   // bytes of one Gaussian's split row
    const char* fbase = reinterpret_cast<const char*>(fsp);
    const int ks = mb;                // k half of every chunk this wave multiplies (channels 16ks..16ks+15)
    const int h = lane >> 5;

    for (int pbase = 0; pbase < Ng; pbase += kBtPass) {
        const int pcount = min(kBtPass, Ng - pbase);
        // LDS-only barriers here and in the epilogues: the weight and partial stores (read by later
        // kernels only) stay in flight while the next steps run
        lds_barrier();

        // F rows by direct-to-LDS loads: row group rg = wave + kBtWaves*i (8 rows, 1 KB) is
        // loaded by this wave; lane = (row rg*8 + lane/8, slot lane%8) and slot p carries the
        // 16-byte piece p ^ swz(row) of the row's chunk.  Rows past the list read the zero row;
        // groups wholly past it are not loaded (no wave reads them).  A wave issues exactly
        // nld = (its groups within the list) + kNG loads per chunk, so the wait counts below are
        // exact.  The rows' Gaussians come straight from the list, so that the first chunks' loads
        // are issued before the parameters are staged and both are in flight together.
        const int* list = sorted_gauss + j0 + pbase;
        const int kent = threadIdx.x;                        // this thread's list entry (staging)
        int gk, grow[kBtDma];
        if (pbase == 0) {   // requested at the tile start
            gk = kent < pcount ? l0 : -1;
#pragma unroll
            for (int i = 0; i < kBtDma; ++i) grow[i] = (wave + kBtWaves * i) * 8 + (lane >> 3) < pcount ? lrow0[i] : n;
        } else {
            gk = kent < pcount ? list[kent] : -1;
#pragma unroll
            for (int i = 0; i < kBtDma; ++i) {
                const int r = (wave + kBtWaves * i) * 8 + (lane >> 3);
                grow[i] = r < pcount ? list[r] : n;
            }
        }
        uint32_t doff[kBtDma];
#pragma unroll
        for (int i = 0; i < kBtDma; ++i) {
            const int rg = wave + kBtWaves * i;
            const int r = rg * 8 + (lane >> 3);
            const int piece = (lane & 7) ^ swz(r);
            doff[i] = (rg * 8 < pcount) ? (uint32_t)grow[i] * fstride + (uint32_t)piece * 16u : (uint32_t)n * fstride;
        }
        // the wave's groups within the list are its first nf (rg grows with i)
        int nf = 0;
#pragma unroll
        for (int i = 0; i < kBtDma; ++i) nf += ((wave + kBtWaves * i) * 8 < pcount) ? 1 : 0;
        nf = uniform(nf);
        auto dma_f = [&](int chunk, int buf, int i0, int i1) {
#pragma unroll
            for (int i = 0; i < kBtDma; ++i) {
                if (i < i0 || i >= i1) continue;
                const int rg = wave + kBtWaves * i;
                dma16s(fbase + (size_t)chunk * kBtRowBytes, doff[i],
                       uniform(lds_addr(&sm.u.frow[buf][rg * 8 * kBtRowBytes])));
            }
        };
        const int clast = nchk - 1;
        // Odd passes walk the chunks backwards: a long list's next pass then starts on the G chunks
        // the previous pass read last, which are still in L2 (forward order re-read the tile's G
        // from HBM at every pass).  Chunk nchk (past the end) stays past the end.
        const bool rev = ((pbase / kBtPass) & 1) != 0;
        auto cm = [&](int c) { return (rev && c <= clast) ? clast - c : c; };

        // this thread's entry: parameters and its G->T pair with this tile, requested first
        float emu[3] = {0.f, 0.f, 0.f}, eA[9] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, eo = 0.f;
        int elb[3] = {0, 0, 0}, eub[3] = {0, 0, 0}, eoff = 0;
        if (gk >= 0) {
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                emu[q] = means[gk * 3 + q];
                elb[q] = lb[gk * 3 + q];
                eub[q] = ub[gk * 3 + q];
            }
#pragma unroll
            for (int q = 0; q < 9; ++q) eA[q] = cov_inv[gk * 9 + q];
            eo = opacity[gk];
            eoff = g2t_offsets[gk];
        }
        // the first chunks' loads (G three chunks ahead, F two, or one with FU), in flight with them
        dma_g(cm(0), 0);
        dma_f(cm(0), 0, 0, nf);
        dma_g(cm(min(1, clast)), 1);
        if constexpr (!FU) dma_f(cm(min(1, clast)), 1, 0, nf);
        dma_g(cm(min(2, clast)), 2);
        if (kent < kBtPass) {
            sm.pt.gid[kent] = gk;
            int pair = -1;
            if (gk >= 0) {
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    sm.pt.mu[q][kent] = emu[q];
                    sm.pt.lb[q][kent] = elb[q];
                    sm.pt.ub[q][kent] = eub[q];
                }
#pragma unroll
                for (int q = 0; q < 9; ++q) sm.pt.A[q][kent] = eA[q];
                sm.pt.o[kent] = eo;
                const int tx0 = elb[0] / kTile, ty0 = elb[1] / kTile, tz0 = elb[2] / kTile;
                const int dy = eub[1] / kTile - ty0 + 1, dz = eub[2] / kTile - tz0 + 1;
                const int64_t pr = (int64_t)eoff + ((tx - tx0) * dy + (ty - ty0)) * dz + (tz - tz0);
                pair = (pr >= 0 && pr < M) ? (int)pr : -1;   // malformed CSR: never write outside the buffer
            }
            sm.pidx[kent] = pair;
        }
        // Every load of the pass start complete (the first chunks' too: the parameter stores above
        // already waited for most of them).  A thread that staged no entry would otherwise reach the
        // K loop with the parameter loads still pending for the compiler's wait counts, which
        // then wait for all loads inside the K loop wherever their registers are reused there.
        wait_vm<0>();
        lds_barrier();

        // wave (ks, ngrp) accumulates k half ks of every chunk for both voxel blocks m and its N
        // blocks ngrp + 4j; the halves are added after the K loop
        f32x16 acc2[2][kBtNbw];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int j = 0; j < kBtNbw; ++j) acc2[m][j] = f32x16{};
        int nact = 0;
        int gcol[kBtNbw];
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) {
            nact += ((ngrp + kBtGroups * j) * 32 < pcount) ? 1 : 0;
            gcol[j] = sm.pt.gid[(ngrp + kBtGroups * j) * 32 + (lane & 31)];
        }
        nact = uniform(nact);
        // A operand of chunk ch, split once per value: thread (voxel sv, channel quad sq) reads its
        // four raw G values (stage gs), masks them (row outside the grid, channels past C),
        // splits them and writes hi and lo into A buffer ab: channels 4sq.. of the chunk are k
        // half sq/4, lane group (sq/2)&1, half sq&1 of the lane's 16-byte fragment.
        // float: wave w writes the fragments of voxel block w&1, lane group (w/2)&1, k half w/4,
        // lane (sv&31, sq&1): 32 whole 16-byte fragments, one contiguous 512-byte run per array, so
        // the 8-byte writes are free of bank conflicts (a wave of 8 voxels x 8 quads would put four
        // writes on every bank); its reads, 16 bytes of 32 consecutive rows at pieces sq and sq^1,
        // stay conflict-free through the row swizzle.  bfloat16 rows are not swizzled, so there the
        // wave keeps 8 voxels x 8 octets (each read covers whole rows).
        const int sv = BF ? threadIdx.x >> 3 : (((threadIdx.x >> 6) & 1) << 5) | ((threadIdx.x & 63) >> 1);
        const int sq = BF ? threadIdx.x & 7 : ((threadIdx.x >> 8) << 2) | (((threadIdx.x >> 7) & 1) << 1) | (threadIdx.x & 1);
        const bool svok = sm.vlin[sv] >= 0;
        auto write_a = [&](int ch, int gs, int ab) {
            const int lim = svok ? min(max(C - (ch * kKc + 4 * sq), 0), 4) : 0;
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            const int L = ((sq >> 1) & 1) * 32 + (sv & 31);
            if constexpr (BF) {
                // bfloat16: thread (sv, sq) takes channels 8sq..8sq+7 of the 64-channel chunk, i.e.
                // k half sq/4, slice (sq/2)&1 (A buffer ahi for slice 0, alo for slice 1), lane
                // group sq&1 of the voxel's fragment; values past the row or the grid are cleared
                const int lim8 = svok ? min(max(C - (ch * kKc + 8 * sq), 0), 8) : 0;
                uint4 xr;
                if constexpr (VEC) {
                    xr = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(&sm.graw[gs][0][0][0]) +
                                                         sv * 128 + sq * 16);
                } else {
                    const unsigned short* row =
                        reinterpret_cast<const unsigned short*>(gF + (int64_t)max(sm.vlin[sv], 0) * C);
                    unsigned e[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) e[i] = row[min(ch * kKc + 8 * sq + i, C - 1)];
                    xr = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
                }
                auto keep = [&](int w) {   // mask of word w (elements 2w and 2w + 1)
                    return (2 * w < lim8 ? 0x0000ffffu : 0u) | (2 * w + 1 < lim8 ? 0xffff0000u : 0u);
                };
                xr.x &= keep(0);
                xr.y &= keep(1);
                xr.z &= keep(2);
                xr.w &= keep(3);
                const int Lb = (sq & 1) * 32 + (sv & 31);
                bf16x8* dst = ((sq >> 1) & 1) ? &sm.alo[ab][sq >> 2][sv >> 5][Lb] : &sm.ahi[ab][sq >> 2][sv >> 5][Lb];
                *reinterpret_cast<uint4*>(dst) = xr;
                return;
            }
            // one 16-byte LDS read, then the values past the row or the grid are cleared with bit
            // masks (a select per value would let the compiler split the read into guarded parts)
            uint4 xr = *reinterpret_cast<const uint4*>(&sm.graw[gs][0][sv][4 * (sq ^ swz(sv))]);
            if constexpr (FU) {
                // G = k1 target + k2 grid_feats (the expression of the loss's own backward)
                const uint4 xf = *reinterpret_cast<const uint4*>(&sm.graw[gs][kSrc - 1][sv][4 * (sq ^ swz(sv))]);
                const float k1 = sm.kc[0][sv], k2 = sm.kc[1][sv];
                xr.x = __float_as_uint(k1 * __uint_as_float(xr.x) + k2 * __uint_as_float(xf.x));
                xr.y = __float_as_uint(k1 * __uint_as_float(xr.y) + k2 * __uint_as_float(xf.y));
                xr.z = __float_as_uint(k1 * __uint_as_float(xr.z) + k2 * __uint_as_float(xf.z));
                xr.w = __float_as_uint(k1 * __uint_as_float(xr.w) + k2 * __uint_as_float(xf.w));
            }
            if (!(tile_in && ch * kKc + kKc <= C)) {   // wave-uniform: rows or channels to clear
                xr.x &= 0u - (unsigned)(0 < lim);
                xr.y &= 0u - (unsigned)(1 < lim);
                xr.z &= 0u - (unsigned)(2 < lim);
                xr.w &= 0u - (unsigned)(3 < lim);
            }
            const f32x2 x01 = {__uint_as_float(xr.x), __uint_as_float(xr.y)};
            const f32x2 x23 = {__uint_as_float(xr.z), __uint_as_float(xr.w)};
            const bf16x2 h01 = __builtin_convertvector(x01, bf16x2), h23 = __builtin_convertvector(x23, bf16x2);
            const bf16x2 l01 = __builtin_convertvector(x01 - __builtin_convertvector(h01, f32x2), bf16x2);
            const bf16x2 l23 = __builtin_convertvector(x23 - __builtin_convertvector(h23, f32x2), bf16x2);
            const bf16x4 hv = {h01[0], h01[1], h23[0], h23[1]}, lv = {l01[0], l01[1], l23[0], l23[1]};
            *reinterpret_cast<bf16x4*>(reinterpret_cast<char*>(&sm.ahi[ab][sq >> 2][sv >> 5][L]) + (sq & 1) * 8) = hv;
            *reinterpret_cast<bf16x4*>(reinterpret_cast<char*>(&sm.alo[ab][sq >> 2][sv >> 5][L]) + (sq & 1) * 8) = lv;
        };
        // N block j of chunk ch (F stage st, A buffer ab) against both voxel blocks
        // Operands of one chunk step, A (both voxel blocks) and B (both N blocks), read from LDS
        // together at the step's start, so that one LDS latency precedes the step's MFMAs (the B
        // rows of an N block past the list hold stale values and are not multiplied).
        struct StepOps {
            bf16x8 ah[2], al[2], bh[kBtNbw], bl[kBtNbw];
        };
        auto load_ops = [&](int st, int ab, StepOps& o) {
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                o.ah[m] = sm.ahi[ab][ks][m][lane];
                o.al[m] = sm.alo[ab][ks][m][lane];
            }
#pragma unroll
            for (int j = 0; j < kBtNbw; ++j) {
                // float: pieces 2ks+h (hi) and 4+2ks+h (lo); bfloat16: pieces 4ks+h (slice 0) and
                // 4ks+2+h (slice 1)
                const int r = (ngrp + kBtGroups * j) * 32 + (lane & 31), sr = swz(r);
                const int qh = BF ? 4 * ks + h : 2 * ks + h, ql = BF ? 4 * ks + 2 + h : 4 + 2 * ks + h;
                const unsigned char* rowp = &sm.u.frow[st][r * kBtRowBytes];
                o.bh[j] = *reinterpret_cast<const bf16x8*>(rowp + ((qh ^ sr) << 4));
                o.bl[j] = *reinterpret_cast<const bf16x8*>(rowp + ((ql ^ sr) << 4));
            }
        };
        // N block j of the step against both voxel blocks
        auto mult = [&](int j, const StepOps& o) {
            if (j < nact) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    if constexpr (BF) {   // slices 0 and 1
                        acc2[m][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o.ah[m], o.bh[j], acc2[m][j], 0, 0, 0);
                        acc2[m][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o.al[m], o.bl[j], acc2[m][j], 0, 0, 0);
                    } else {
                        acc2[m][j] = mfma_split_32x32x16<false, false>(o.ah[m], o.al[m], o.bh[j], o.bl[j], acc2[m][j]);
                    }
                }
            }
        };

        // Pipeline over chunks (every load is direct-to-LDS; F two chunks ahead, G three).  Step
        // ch starts with the A operand of chunk ch (A buffer ch&1), the F rows of chunk ch and the
        // G values of chunk ch+1 in LDS.  Between its MFMAs (which run on in the matrix unit) it
        // writes the A operand of chunk ch+1 and issues the loads of F(ch+2) and G(ch+3); then it
        // waits until only those loads are outstanding.  G(ch+3) goes to the stage of G(ch), whose
        // A operand was written in the previous step.
        // The chunk loop, instantiated for the wave's group count NF (exact wait immediates;
        // waves of one workgroup may run different instantiations, with the same barriers).
        auto chunk_loop = [&](auto nfc) {
            constexpr int NF = decltype(nfc)::value;
            constexpr int kLd = NF + kNG;   // loads per wave per chunk
            // G(0), F(0), G(1), F(1), G(2) were issued at the pass start
            wait_vm<kLd>();               // G(0), F(0), G(1) complete
            lds_barrier();
            write_a(cm(0), 0, 0);
            lds_barrier();
            for (int ch = 0; ch < nchk; ++ch) {
                const int st = ch % kBtStages, ab = ch & 1;
                StepOps ops;
                load_ops(st, ab, ops);
                asm volatile("" ::: "memory");   // every operand read issued before the first MFMA
                mult(0, ops);
                __builtin_amdgcn_sched_barrier(0);
                write_a(cm(ch + 1), (ch + 1) % kBtStages, ab ^ 1);
                dma_f(cm(min(ch + 2, clast)), (ch + 2) % kBtStages, 0, min(NF, kBtDma / 2));
                __builtin_amdgcn_sched_barrier(0);
                mult(1, ops);
                __builtin_amdgcn_sched_barrier(0);
                dma_f(cm(min(ch + 2, clast)), (ch + 2) % kBtStages, kBtDma / 2, NF);
                dma_g(cm(min(ch + 3, clast)), st);
                wait_vm<kLd>();           // F(ch+1) and G(ch+2) complete
                lds_barrier();
            }
        };
        // FU: two F buffers, so F(ch+1) is loaded at the start of step ch into the buffer that step
        // ch-1 read, and waited for at its end; G (two sources) is still three chunks ahead.
        auto chunk_loop_fu = [&](auto nfc) {
            constexpr int NF = decltype(nfc)::value;
            constexpr int kLg = kSrc * kNG;   // G loads per wave per chunk
            // G(0), F(0), G(1), G(2) were issued at the pass start
            wait_vm<kLg>();               // G(0), F(0), G(1) complete
            lds_barrier();
            write_a(cm(0), 0, 0);
            lds_barrier();
            for (int ch = 0; ch < nchk; ++ch) {
                const int st = ch % kBtStages, fb = ch & 1, ab = ch & 1;
                dma_f(cm(min(ch + 1, clast)), fb ^ 1, 0, NF);
                StepOps ops;
                load_ops(fb, ab, ops);
                asm volatile("" ::: "memory");   // every operand read issued before the first MFMA
                mult(0, ops);
                __builtin_amdgcn_sched_barrier(0);
                write_a(cm(ch + 1), (ch + 1) % kBtStages, ab ^ 1);
                __builtin_amdgcn_sched_barrier(0);
                mult(1, ops);
                __builtin_amdgcn_sched_barrier(0);
                dma_g(cm(min(ch + 3, clast)), st);
                wait_vm<kLg>();           // F(ch+1) and G(ch+2) complete
                lds_barrier();
            }
        };
        static_assert(kBtDma == 4, "group-count dispatch");
        auto run = [&](auto nfc) {
            if constexpr (FU) chunk_loop_fu(nfc);
            else chunk_loop(nfc);
        };
        switch (nf) {
            case 4: run(std::integral_constant<int, 4>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 1: run(std::integral_constant<int, 1>{}); break;
            default: run(std::integral_constant<int, 0>{}); break;
        }
        // drain the surplus loads of the last steps before the F buffers are reused
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();

        // Sum the two k halves: wave (ks, ngrp) keeps voxel block mb = ks and hands the other
        // block to its partner through LDS.  Both partners add (half 0) + (half 1).
        f32x16 acc[kBtNbw];
        {
            // [ngrp][m][j][i][lane]: block m of N group ngrp, written by the wave that does not keep it
            float* xb = reinterpret_cast<float*>(&sm.u.frow[0][0]) + ngrp * (2 * kBtNbw * 16 * 64) + lane;
            constexpr int kXm = kBtNbw * 16 * 64;
            if (ks == 0) {
#pragma unroll
                for (int j = 0; j < kBtNbw; ++j)
#pragma unroll
                    for (int i = 0; i < 16; ++i) xb[kXm + (j * 16 + i) * 64] = acc2[1][j][i];
            } else {
#pragma unroll
                for (int j = 0; j < kBtNbw; ++j)
#pragma unroll
                    for (int i = 0; i < 16; ++i) xb[(j * 16 + i) * 64] = acc2[0][j][i];
            }
            __syncthreads();
            if (ks == 0) {
#pragma unroll
                for (int j = 0; j < kBtNbw; ++j)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[j][i] = acc2[0][j][i] + xb[(j * 16 + i) * 64];
            } else {
#pragma unroll
                for (int j = 0; j < kBtNbw; ++j)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[j][i] = xb[kXm + (j * 16 + i) * 64] + acc2[1][j][i];
            }
            __syncthreads();   // the exchange area is reused by the epilogues
        }

        // ---- epilogue 1: split weights w / max(D, eps) of every pair; t_v from U (single pass).
        // Lane = Gaussian column lane%32 of N block j; element i is the tile's voxel row
        // r = 32 mb + 8 (i/4) + 4 (lane/32) + i%4.  Branch-free: an element outside the grid, the
        // Gaussian's box or the list gets e = 0 (and so w = 0).  The validity bits are kept in
        // registers and the exponentials in LDS (the F buffers are free after the K loop), where
        // epilogue 2 reads them back instead of evaluating them again (FU: the two F buffers leave no
        // room, and epilogue 2 evaluates them again).
        unsigned rowok = 0;   // bit i: row r of element i lies in the grid
#pragma unroll
        for (int i = 0; i < 16; ++i)
            rowok |= (sm.vlin[mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3)] >= 0) ? (1u << i) : 0u;
        float rowt[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) rowt[i] = 0.0f;
        unsigned okm[kBtNbw];
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) {
            okm[j] = 0;
            if (j >= nact) continue;   // wave-uniform
            const int slot = (ngrp + kBtGroups * j) * 32 + (lane & 31);
            const bool gok = gcol[j] >= 0;
            GaussParams p;
            read_params(sm.pt, slot, p);
            LaneGeom L;
            lane_geom(G, p, tx * kTile + 2 * mb, ty * kTile + h, tz * kTile, L);
            LaneExp E;
            lane_exp(p, L, E);
            __bf16* wrow = wt + (int64_t)(j0 + pbase + slot) * kWtRow;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                __bf16 hs[4], ls[4];
                float ev[4];
                const int a = q4 >> 1, b = q4 & 1;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    // element i: voxel row r = mb*32 + 8 q4 + 4h + ii, at x = x0 + a, y = y0 + 2b,
                    // z = z0 + ii; the exponential is always evaluated, then selected
                    const int i = q4 * 4 + ii;
                    const int r = mb * 32 + 8 * q4 + 4 * h + ii;
                    const bool ok = gok & (((rowok >> i) & (L.inx >> a) & (L.iny >> b) & (L.inz >> ii) & 1u) != 0u);
                    const float e = ok ? lane_e(E, L, a, b, ii) : 0.0f;
                    ev[ii] = e;
                    okm[j] |= ok ? (1u << i) : 0u;
                    const float w = p.o * e;
                    const float wtil = w * sm.inv[r];
                    split_bf16(wtil, hs[ii], ls[ii]);
                    // a select, not a product with 0: columns past the list hold whatever
                    // the unloaded F rows left in LDS
                    rowt[i] += (w > 0.0f) ? wtil * acc[j][i] : 0.0f;
                }
                if constexpr (!FU) sm.u.ep.e[wave][j][q4][lane] = make_float4(ev[0], ev[1], ev[2], ev[3]);
                if (gok) {
                    const int r0 = mb * 32 + 8 * q4 + 4 * h;
                    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                    bf16x4 hv = {hs[0], hs[1], hs[2], hs[3]};
                    bf16x4 lv = {ls[0], ls[1], ls[2], ls[3]};
                    *reinterpret_cast<bf16x4*>(wrow + r0) = hv;
                    *reinterpret_cast<bf16x4*>(wrow + 64 + r0) = lv;
                }
            }
        }
        if (!multi) {
            // rows are shared by the 32 lanes of each half-wave: reduce over them (lanes 2i and
            // 2i+1 of a half end up with the sum of element i)
            const float rs = transpose_sum16(rowt, lane & 31);
            if ((lane & 1) == 0) {
                const int i = (lane >> 1) & 15;
                sm.tpart[ngrp][mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3)] = rs;
            }
            lds_barrier();
            if (threadIdx.x < 64) {
                const int r = threadIdx.x;
                const float s = ((sm.tpart[0][r] + sm.tpart[1][r]) + sm.tpart[2][r]) + sm.tpart[3][r];
                // sum_g [w>0] w u / max(D, eps) = sum_c gF F; zero where D < eps (reference .cu:1450)
                sm.tv[r] = (sm.vlin[r] >= 0 && sm.D[r] >= kEps) ? s : 0.0f;
            }
            lds_barrier();
        }

        // ---- epilogue 2: r = gw e of every element (e from epilogue 1; an invalid element
        // adds exact zeros) and its moments over the lane's 2 x 2 x 4 voxels relative to the
        // mean (d = centre - mu): sum r d, sum r d d^T (times o) and sum r.  Phase C turns them
        // into d mu = A (o sum r d), d Sigma = A (o sum r d d^T) A^T / 2 and d o = sum r, since
        // q = A d, sum gw w q = o A sum r d and sum gw w q q^T = o A (sum r d d^T) A^T.
#pragma unroll
        for (int j = 0; j < kBtNbw; ++j) {
            const int slot = (ngrp + kBtGroups * j) * 32 + (lane & 31);
            float gr[kNumGrads] = {};
            if (j < nact) {   // wave-uniform
                GaussParams p;
                read_params(sm.pt, slot, p);
                LaneGeom L;
                lane_geom(G, p, tx * kTile + 2 * mb, ty * kTile + h, tz * kTile, L);
                // e from epilogue 1 (FU: evaluated again; no LDS is free to keep it)
                LaneExp E;
                if constexpr (FU) lane_exp(p, L, E);
                float m0 = 0.f, mx = 0.f, my = 0.f, mz = 0.f, mxx = 0.f, myy = 0.f, mzz = 0.f, mxy = 0.f,
                      mxz = 0.f, myz = 0.f;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int a = q4 >> 1, b = q4 & 1;
                    float ev[4] = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (!FU) {
                        const float4 e4 = sm.u.ep.e[wave][j][q4][lane];
                        ev[0] = e4.x;
                        ev[1] = e4.y;
                        ev[2] = e4.z;
                        ev[3] = e4.w;
                    }
                    float s0 = 0.f, sz = 0.f, szz = 0.f;
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int i = q4 * 4 + ii;
                        const int r = mb * 32 + 8 * q4 + 4 * h + ii;
                        const float gw = sm.gD[r] + (acc[j][i] - sm.tv[r]) * sm.inv[r];
                        const float e = FU ? lane_e(E, L, a, b, ii) : ev[ii];
                        const float rr = ((okm[j] >> i) & 1u) ? gw * e : 0.0f;
                        s0 += rr;
                        const float rz = rr * L.dz[ii];
                        sz += rz;
                        szz = fmaf(rz, L.dz[ii], szz);
                    }
                    const float dx = L.dx[a], dy = L.dy[b];
                    m0 += s0;
                    mx = fmaf(dx, s0, mx);
                    my = fmaf(dy, s0, my);
                    mz += sz;
                    mxx = fmaf(dx * dx, s0, mxx);
                    myy = fmaf(dy * dy, s0, myy);
                    mzz += szz;
                    mxy = fmaf(dx * dy, s0, mxy);
                    mxz = fmaf(dx, sz, mxz);
                    myz = fmaf(dy, sz, myz);
                }
                gr[0] = p.o * mx;
                gr[1] = p.o * my;
                gr[2] = p.o * mz;
                gr[3] = p.o * mxx;
                gr[4] = p.o * myy;
                gr[5] = p.o * mzz;
                gr[6] = p.o * mxy;
                gr[7] = p.o * mxz;
                gr[8] = p.o * myz;
                gr[9] = m0;
            }
#pragma unroll
            for (int k = 0; k < kNumGrads; ++k) gr[k] += __shfl_xor(gr[k], 32, 64);
            if (lane < 32) {
#pragma unroll
                for (int k = 0; k < kNumGrads; ++k) sm.u.xch[mb][slot][k] = gr[k];
            }
        }
        lds_barrier();
        for (int slot = threadIdx.x; slot < pcount; slot += kBtThreads) {
            const int pair = sm.pidx[slot];
            if (pair < 0) continue;
            float* out = pair_partials + (int64_t)pair * kNumGrads;
#pragma unroll
            for (int k = 0; k < kNumGrads; ++k) out[k] = sm.u.xch[0][slot][k] + sm.u.xch[1][slot][k];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Phase A for short lists (1 .. smax <= kBsMax Gaussians).  k_bwd_tile holds one tile per CU (its LDS is
// sized for 256-Gaussian passes), so a short list leaves that tile's chain of loads and barriers
// bare; here a 4-wave workgroup with about 17 KB of LDS takes the tile and many run per CU.  The
// per-pair results are those of k_bwd_tile up to float32 rounding: U = G F^T from float32 products
// of gF and the split features' hi + lo (the matrix-core path leaves out lo x lo), t_v from U,
// the same e (the same helper operations) and so the same split weights, and the moments summed
// over the voxels in another order.  Which kernel takes a tile depends on its list length alone.
// Thread = (voxel row lane, Gaussian slots wave + 4 i): the slots are dealt round robin over the waves.
// ------------------------------------------------------------------------------------------
constexpr int kBsThreads = 256;
constexpr int kBsMax = 64;     // longest list the kernel can take
constexpr int kBsKc = 32;      // channels per staged chunk

struct BsSmem {
    float g[64][kBsKc + 1];    // gF chunk, voxel-major; rows padded so that lanes (voxels) hit distinct banks
    float f[kBsKc][4][kBsMax / 4];   // feature chunk: [channel][wave][i] of slot wave + 4 i (a wave reads its slots at once)
    ParamTile<kBsMax> pt;
    int vlin[64];
    float gD[64], inv[64], D[64], tv[64];
    float tpart[kBsThreads / 64][64];
};

// e of Gaussian p at voxel (x, y, z) with the operations of lane_geom / lane_exp / lane_e (so the
// same value); in: the voxel lies in the Gaussian's box.
__device__ __forceinline__ float voxel_e(const Grid& G, const GaussParams& p, int x, int y, int z, float& dx,
                                         float& dy, float& dz, bool& in) {
#pragma clang fp contract(off)
    dx = centre(G, 0, x) - p.mu[0];
    dy = centre(G, 1, y) - p.mu[1];
    dz = centre(G, 2, z) - p.mu[2];
    in = x >= p.lb[0] && x <= p.ub[0] && y >= p.lb[1] && y <= p.ub[1] && z >= p.lb[2] && z <= p.ub[2];
    const float sxy = p.A[1] + p.A[3], sxz = p.A[2] + p.A[6], syz = p.A[5] + p.A[7];
    const float fxy = kq * fmaf(fmaf(p.A[0], dx, sxy * dy), dx, p.A[4] * dy * dy);
    const float gxy = kq * fmaf(sxz, dx, syz * dy);
    const float fz = kq * (p.A[8] * dz * dz);
    return __builtin_amdgcn_exp2f(fmaf(gxy, dz, fxy + fz));
}

// BF: grad_feats and the features are bfloat16 (the split rows then hold 64-channel chunks of the
// values).
template <bool BF>
__global__ void __launch_bounds__(kBsThreads) k_bwd_tile_short(
    Grid G, int n, int C, int nchk, const float* __restrict__ gD, const void* __restrict__ gF_,
    const float* __restrict__ means, const float* __restrict__ opacity, const float* __restrict__ cov_inv,
    const int* __restrict__ lb, const int* __restrict__ ub, const int* __restrict__ g2t_offsets,
    const int* __restrict__ toff, const int* __restrict__ sorted_gauss, int M, const float* __restrict__ density,
    const __bf16* __restrict__ fsp, float* __restrict__ pair_partials, __bf16* __restrict__ wt, int smax) {
    __shared__ BsSmem sm;
    const int T = scene_tiles(G);
    const int tb = uniform(xcd_remap(blockIdx.x, gridDim.x));   // the batch's tile (its list)
    if (tb >= T * G.scenes) return;
    const int j0 = uniform(min(max(toff[tb], 0), M));
    const int Ng = uniform(min(max(toff[tb + 1], j0), M)) - j0;
    if (Ng <= 0 || Ng > smax) return;
    const int scene = uniform(tb / T), tile = tb - scene * T;
    typedef typename std::conditional<BF, __bf16, float>::type GT;   // element of grad_feats
    const GT* gF = static_cast<const GT*>(gF_);
    if (scene > 0) {   // the scene's voxel rows
        const int64_t vb = scene * scene_voxels(G);
        gD += vb;
        density += vb;
        gF += vb * C;
    }
    const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);   // voxel row lane of the tile

    // Staging roles.  gF: voxel row sr, channels 8 sq .. 8 sq + 7 of a chunk.  Features: slots fs
    // and fs + 32 (the zero row past the list), channels 4 fo .. 4 fo + 3.  A chunk's values are loaded into
    // registers one chunk ahead (the first chunk's loads go out with the tile's own), stored to
    // LDS at the chunk's start.
    const int sr = threadIdx.x >> 2, sq = threadIdx.x & 3;
    const int fs = threadIdx.x >> 3, fo = threadIdx.x & 7;
    int rx, ry, rz;
    tile_voxel(G, tile, sr, rx, ry, rz);
    const bool srok = in_grid(G, rx, ry, rz);
    const GT* gsrc = gF + (srok ? voxel_index(G, rx, ry, rz) : 0) * C;
    const bool gvec = (C & 7) == 0 && ((uintptr_t)gF & 15) == 0;   // 16-byte row pieces
    const int rowlen = nchk * 2 * kBtKc;                              // bf16 per split feature row
    const __bf16* frow[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        frow[h] = fsp + (int64_t)(fs + 32 * h < Ng ? sorted_gauss[j0 + fs + 32 * h] : n) * rowlen;
    float gv[8], fv[2][4];
    auto load_g = [&](int c0) {
        const int c = c0 + 8 * sq;
        if (gvec) {   // whole octets: C % 8 == 0
            if (c < C) {
                if constexpr (BF) {
                    const uint4 h = *reinterpret_cast<const uint4*>(gsrc + c);
                    const unsigned w[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        gv[2 * i] = __uint_as_float(w[i] << 16);
                        gv[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                    }
                } else {
                    const float4 q0 = *reinterpret_cast<const float4*>(gsrc + c);
                    const float4 q1 = *reinterpret_cast<const float4*>(gsrc + c + 4);
                    gv[0] = q0.x; gv[1] = q0.y; gv[2] = q0.z; gv[3] = q0.w;
                    gv[4] = q1.x; gv[5] = q1.y; gv[6] = q1.z; gv[7] = q1.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) gv[i] = 0.0f;
            }
        } else {      // every element loaded (clamped into the row) before any is masked
#pragma unroll
            for (int i = 0; i < 8; ++i) gv[i] = (float)gsrc[min(c + i, C - 1)];
#pragma unroll
            for (int i = 0; i < 8; ++i) gv[i] = c + i < C ? gv[i] : 0.0f;
        }
    };
    auto load_f = [&](int c0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if constexpr (BF) {   // the values themselves, 64-channel chunks: element c at offset c
                const uint2 hv = *reinterpret_cast<const uint2*>(frow[h] + c0 + 4 * fo);
                fv[h][0] = __uint_as_float(hv.x << 16);
                fv[h][1] = __uint_as_float(hv.x & 0xffff0000u);
                fv[h][2] = __uint_as_float(hv.y << 16);
                fv[h][3] = __uint_as_float(hv.y & 0xffff0000u);
            } else {              // chunk c0 / 32: hi[32] then lo[32]
                const __bf16* ck = frow[h] + (c0 / kBtKc) * (2 * kBtKc);
                const uint2 hv = *reinterpret_cast<const uint2*>(ck + 4 * fo);
                const uint2 lv = *reinterpret_cast<const uint2*>(ck + kBtKc + 4 * fo);
                fv[h][0] = __uint_as_float(hv.x << 16) + __uint_as_float(lv.x << 16);
                fv[h][1] = __uint_as_float(hv.x & 0xffff0000u) + __uint_as_float(lv.x & 0xffff0000u);
                fv[h][2] = __uint_as_float(hv.y << 16) + __uint_as_float(lv.y << 16);
                fv[h][3] = __uint_as_float(hv.y & 0xffff0000u) + __uint_as_float(lv.y & 0xffff0000u);
            }
        }
    };
    load_g(0);
    load_f(0);
    if (threadIdx.x < 64) {
        const bool ok = in_grid(G, x, y, z);
        const int64_t v = ok ? voxel_index(G, x, y, z) : 0;
        sm.vlin[lane] = ok ? (int)v : -1;
        sm.gD[lane] = ok ? gD[v] : 0.0f;
        sm.D[lane] = ok ? density[v] : 0.0f;
        sm.inv[lane] = ok ? 1.0f / fmaxf(density[v], kEps) : 0.0f;
    }
    stage_params(sm.pt, sorted_gauss + j0, Ng, means, cov_inv, opacity, lb, ub);

    // U: thread (voxel lane, slots wave + 4 i) over 32-channel chunks staged in LDS; a wave
    // multiplies only its slots' quads that hold list entries
    const int nq = uniform((max(Ng - wave, 0) + 15) / 16);   // quads of 4 slots with an entry
    float u[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) u[i] = 0.0f;
    for (int c0 = 0; c0 < C; c0 += kBsKc) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sm.g[sr][8 * sq + i] = srok ? gv[i] : 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int sl = fs + 32 * h;
#pragma unroll
            for (int i = 0; i < 4; ++i) sm.f[4 * fo + i][sl & 3][sl >> 2] = fv[h][i];
        }
        __syncthreads();   // also orders the tile's own values and parameters before their reads
        if (c0 + kBsKc < C) {   // the next chunk's loads run under this chunk's products
            load_g(c0 + kBsKc);
            load_f(c0 + kBsKc);
        }
#pragma unroll 4
        for (int c = 0; c < kBsKc; ++c) {
            const float a = sm.g[lane][c];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (q < nq) {   // wave-uniform
                    const float4 f4 = *reinterpret_cast<const float4*>(&sm.f[c][wave][4 * q]);
                    u[4 * q] = fmaf(a, f4.x, u[4 * q]);
                    u[4 * q + 1] = fmaf(a, f4.y, u[4 * q + 1]);
                    u[4 * q + 2] = fmaf(a, f4.z, u[4 * q + 2]);
                    u[4 * q + 3] = fmaf(a, f4.w, u[4 * q + 3]);
                }
            }
        }
        __syncthreads();
    }

    // split weights of every pair (row lane of the pair's weight row) and t_v from U
    const bool rowok = sm.vlin[lane] >= 0;
    const float inv = sm.inv[lane];
    float tsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int slot = wave + 4 * i;
        if (slot >= Ng) break;   // wave-uniform
        GaussParams p;
        read_params(sm.pt, slot, p);
        float dx, dy, dz;
        bool in;
        const float e0 = voxel_e(G, p, x, y, z, dx, dy, dz, in);
        const float e = (rowok && in) ? e0 : 0.0f;
        const float w = p.o * e;
        const float wtil = w * inv;
        __bf16 hs, ls;
        split_bf16(wtil, hs, ls);
        __bf16* wrow = wt + (int64_t)(j0 + slot) * kWtRow;
        wrow[lane] = hs;
        wrow[64 + lane] = ls;
        tsum += (w > 0.0f) ? wtil * u[i] : 0.0f;
    }
    sm.tpart[wave][lane] = tsum;
    lds_barrier();   // the weight stores stay in flight (later kernels read them)
    if (threadIdx.x < 64) {
        const float s = ((sm.tpart[0][lane] + sm.tpart[1][lane]) + sm.tpart[2][lane]) + sm.tpart[3][lane];
        // sum_g [w>0] w u / max(D, eps) = sum_c gF F; zero where D < eps (reference .cu:1450)
        sm.tv[lane] = (rowok && sm.D[lane] >= kEps) ? s : 0.0f;
    }
    lds_barrier();

    // r = gw e and its moments over the tile's voxels (d = centre - mu), as k_bwd_tile stores them
    const float tv = sm.tv[lane], gd = sm.gD[lane];
    const int tyz = G.tiles[1] * G.tiles[2];
    const int tx = tile / tyz, ty = (tile - tx * tyz) / G.tiles[2], tz = tile % G.tiles[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int slot = wave + 4 * i;
        if (slot >= Ng) break;   // wave-uniform
        GaussParams p;
        read_params(sm.pt, slot, p);
        float dx, dy, dz;
        bool in;
        const float e0 = voxel_e(G, p, x, y, z, dx, dy, dz, in);
        const float gw = gd + (u[i] - tv) * inv;
        const float r = (rowok && in) ? gw * e0 : 0.0f;
        const float m[16] = {r * dx, r * dy, r * dz, r * dx * dx, r * dy * dy, r * dz * dz,
                             r * dx * dy, r * dx * dz, r * dy * dz, r, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        // lanes 2k and 2k + 1 of each half-wave get the half's sum of m[k]; lane 2k adds the other
        // half's and stores value k of the pair
        float t = transpose_sum16(m, lane & 31);
        t += __shfl_down(t, 32, 64);
        const int k = lane >> 1;
        if ((lane & 1) == 0 && k < kNumGrads) {
            const int g = sm.pt.gid[slot];
            const int tx0 = p.lb[0] / kTile, ty0 = p.lb[1] / kTile, tz0 = p.lb[2] / kTile;
            const int ey = p.ub[1] / kTile - ty0 + 1, ez = p.ub[2] / kTile - tz0 + 1;
            const int64_t pair = (int64_t)g2t_offsets[g] + ((tx - tx0) * ey + (ty - ty0)) * ez + (tz - tz0);
            if (pair >= 0 && pair < M)   // malformed CSR: never write outside the buffer
                pair_partials[pair * kNumGrads + k] = k < kNumGrads - 1 ? p.o * t : t;
        }
    }
}

// ------------------------------------------------------------------------------------------
// Phase B's row table: for every region row (a Gaussian of the region's ascending list) and
// every tile slot of the region, the Tile->Gaussian entry of that (tile, Gaussian) pair.
// ------------------------------------------------------------------------------------------
constexpr int kBrSlots = 16;   // tiles per region (2 x 2 x up to 4), slot ((tx&1)*2 + (ty&1))*RZ + tz%RZ

// Fills n ints with v (also used where a stream may be captured: no memset nodes).
__global__ void __launch_bounds__(256) k_fill_i32(int64_t n, int v, int* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = v;
}

hipError_t launch_fill_i32(int64_t n, int v, int* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    G2V_LAUNCH(k_fill_i32, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, n, v, dst);
    return hipGetLastError();
}

// Per region row k (the k-th pair of the region-sorted G->R CSR): the row's Gaussian r_gids[k],
// the row's table entries set to M (absent pair: the zero row of the split weights), and, by
// workgroup 0, that zero row itself (kWtRow bfloat16 zeros at wt_zero).
__global__ void __launch_bounds__(256) k_region_rows(int MR, int M, const int* __restrict__ r_pairs_sorted,
                                                     const int* __restrict__ r_gauss, int* __restrict__ r_gids,
                                                     int* __restrict__ table, int* __restrict__ wt_zero) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.x == 0 && threadIdx.x < kWtRow / 2) wt_zero[threadIdx.x] = 0;
    if (k >= MR) return;
    r_gids[k] = r_gauss[min(max(r_pairs_sorted[k], 0), MR - 1)];
    int4* row = reinterpret_cast<int4*>(table + (int64_t)k * kBrSlots);
    const int4 m = make_int4(M, M, M, M);
#pragma unroll
    for (int q = 0; q < kBrSlots / 4; ++q) row[q] = m;
}

// Row table of phase B: for region row r (its position in the region's ascending Gaussian list,
// at G->R slot roff[R] + r) and tile slot s, table[(roff[R] + r) * kBrSlots + s] is the
// Tile->Gaussian index of the pair (tile, Gaussian), or M (the zero row of the split weights)
// when the Gaussian does not touch that tile.  The table is filled with M beforehand.
__global__ void __launch_bounds__(256) k_region_table(Grid G, Regions RG, int M, int MR,
                                                      const int* __restrict__ sorted_tiles,
                                                      const int* __restrict__ sorted_gauss,
                                                      const int* __restrict__ roff,
                                                      const int* __restrict__ r_gids,
                                                      int* __restrict__ table) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= M) return;
    const int tb = sorted_tiles[j], g = sorted_gauss[j];   // the batch's tile
    const int T = scene_tiles(G);
    const int scene = tb / T, t = tb - scene * T;
    const int tyz = G.tiles[1] * G.tiles[2];
    const int tx = t / tyz, ty = (t - tx * tyz) / G.tiles[2], tz = t % G.tiles[2];
    const int tpz = RG.cell[2] / kTile;
    const int R = scene * RG.total + ((tx >> 1) * RG.n[1] + (ty >> 1)) * RG.n[2] + tz / tpz;   // the batch's region
    const int slot = ((tx & 1) * 2 + (ty & 1)) * tpz + tz % tpz;
    const int a = min(max(roff[R], 0), MR);
    const int b = min(max(roff[R + 1], a), MR);
    int lo = a, hi = b;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (r_gids[mid] < g) lo = mid + 1;
        else hi = mid;
    }
    if (lo < b && r_gids[lo] == g) table[(int64_t)lo * kBrSlots + slot] = j;
}

// ------------------------------------------------------------------------------------------
// Phase B: per-region partial feature gradients, accumulated in registers.
//
// Work item = (region, 128-channel chunk); 8 waves.  A pass covers up to 384 rows of the region's
// Gaussian list in 16-row blocks; block b of the pass belongs to wave b % 8, so a wave owns
// RB = ceil(blocks / 8) or one fewer blocks (RB <= 3) and every wave's work follows the row
// count, not a fixed 256-row step.  For every tile of the region the tile's gF chunk (64 voxels x
// 128 channels) is staged in LDS, split hi/lo in the MFMA B layout, and each wave adds
//     (its rows x 64 voxels of split pair weights) . (64 voxels x 128 channels)
// with 16 x 16 x 32 MFMAs, where a row whose Gaussian does not touch the tile reads the zero row
// of the weights.  Every row is owned by one lane set and summed over the tiles in a fixed order:
// no atomics, no LDS accumulators.  Software pipeline one tile ahead: while tile k is
// multiplied, the weights of tile k+1 are loaded into the other register set, the gF values of
// tile k+1 are written to the other LDS buffer, and the gF values of tile k+2 are loaded into
// registers.
// ------------------------------------------------------------------------------------------
constexpr int kBrThreads = 512;   // 8 waves
constexpr int kBrWaves = kBrThreads / 64;
constexpr int kBrCc = 128;        // channels per work item
constexpr int kBrCb = kBrCc / 16; // 16-channel MFMA column blocks
constexpr int kBrRbMax = 3;       // 16-row blocks per wave and pass
constexpr int kBrPass = kBrWaves * kBrRbMax * 16;   // region rows per pass
static_assert(kBrPass * kBrSlots % kBrThreads == 0 && kBrPass <= 2 * kBrThreads, "row-table staging shape");

// FU: the upstream feature gradient is the cosine loss's (k1 target + k2 grid_feats per voxel);
// kc holds (k1, k2) of the voxels of the region's tiles, in the order of tl_org.
template <bool FU>
struct BrSmem {
    bf16x8 bhi[2][2][kBrCb][64];   // B operand (gF chunk): [buffer][k step of 32 voxels][channel block][lane]
    bf16x8 blo[2][2][kBrCb][64];
    int tab[kBrPass][kBrSlots + 1];       // row table of this pass's rows (M: absent pair); padded row
    int rslot[kBrPass];                   // G->R slot of each row of the pass
    int tl_org[kBrSlots][3], tl_s[kBrSlots];   // tiles of the region (inside the grid): first voxel, slot
    int ntl;
    float2 kc[FU ? kBrSlots : 1][FU ? 64 : 1];
};

// gF chunk of the tile whose first voxel is (x0, y0, z0), for the staging thread: channel sc of the chunk, voxel octets so and
// so + 4 (tile-local x = 2k + so/2, y = 2(so&1) + i/4, z = i%4 for value v[k][i]).  Buffer loads
// from the tile origin: a per-thread offset for each (x, y) pair and a uniform offset for each z.
// Coordinates are clamped into the grid, so every load stays inside gF (the descriptor's range
// ends at gF's end as well); bit i + 8k of the returned mask marks the values that are real.
// Offsets need 16 * Y * Z * C < 2^32 (checked on the host).
// GB: gF holds bfloat16 values (2-byte loads, widened exactly).  IN: the tile lies inside the grid
// and the chunk inside the row (no clamps; every value is real).
template <bool GB, bool IN>
__device__ __forceinline__ unsigned br_load_tile(const Grid& G, int C, int c0, int x0, int y0, int z0, int sc, int so,
                                                 const void* __restrict__ gF, float (&v)[2][8]) {
    constexpr int kEs = GB ? 2 : 4;   // bytes per element
    const int X = G.dims[0], Y = G.dims[1], Z = G.dims[2];
    const int64_t origin = ((int64_t)(x0 * Y + y0) * Z + z0) * C + c0;
    const int64_t left = ((int64_t)X * Y * Z * C - origin) * kEs;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(gF) + origin * kEs), (short)0, (int)min(left, (int64_t)0x7fffffff),
        0x00020000);
    const bool cok = IN || c0 + sc < C;
    const unsigned cc = IN ? (unsigned)sc : (unsigned)(min(c0 + sc, C - 1) - c0);
    unsigned voff[2][2];
    bool xok[2], yok[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int x = x0 + 2 * k + (so >> 1);
        xok[k] = IN || x < X;
        const unsigned xl = IN ? (unsigned)(2 * k + (so >> 1)) : (unsigned)(min(x, X - 1) - x0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int y = y0 + 2 * (so & 1) + h;
            if (k == 0) yok[h] = IN || y < Y;
            const unsigned yl = IN ? (unsigned)(2 * (so & 1) + h) : (unsigned)(min(y, Y - 1) - y0);
            voff[k][h] = ((xl * Y + yl) * Z * C + cc) * (unsigned)kEs;
        }
    }
    int soff[4];
    bool zok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        zok[i] = IN || z0 + i < Z;
        soff[i] = (IN ? i : min(z0 + i, Z - 1) - z0) * C * kEs;
    }
    unsigned mask = 0;
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // aux 2: non-temporal (grad_feats is streamed once per region)
            if constexpr (GB)
                v[k][i] = __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b16(rsrc, voff[k][i >> 2], soff[i & 3], 2)
                                          << 16);
            else
                v[k][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff[k][i >> 2], soff[i & 3], 2));
            mask |= (cok && xok[k] && yok[i >> 2] && zok[i & 3]) ? (1u << (i + 8 * k)) : 0u;
        }
    return IN ? 0xffffu : mask;
}

// Paired form of br_load_tile for even C (rows aligned to two channels): the staging thread takes
// channels cp2 and cp2 + 1 of the chunk (cp2 = 2 cp) for the 8 voxels of octet o (tile-local
// x = o/2, y = 2(o&1) + i/4, z = i%4 for value v[h][i] of channel cp2 + h), with one 2-channel load
// per voxel: half the load instructions of the one-channel form.  Bit i + 8h of the mask marks the
// values that are real.  IN as for br_load_tile.
template <bool GB, bool IN>
__device__ __forceinline__ unsigned br_load_tile2(const Grid& G, int C, int c0, int x0, int y0, int z0, int cp2, int o,
                                                  const void* __restrict__ gF, float (&v)[2][8]) {
    constexpr int kEs = GB ? 2 : 4;   // bytes per element
    const int X = G.dims[0], Y = G.dims[1], Z = G.dims[2];
    const int64_t origin = ((int64_t)(x0 * Y + y0) * Z + z0) * C + c0;
    const int64_t left = ((int64_t)X * Y * Z * C - origin) * kEs;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(gF) + origin * kEs), (short)0, (int)min(left, (int64_t)0x7fffffff),
        0x00020000);
    const bool cok = IN || c0 + cp2 < C;   // C even: both channels of the pair or neither
    const unsigned cc = IN ? (unsigned)cp2 : (unsigned)(min(c0 + cp2, C - 2) - c0);
    const int x = x0 + (o >> 1);
    const bool xok = IN || x < X;
    const unsigned xl = IN ? (unsigned)(o >> 1) : (unsigned)(min(x, X - 1) - x0);
    unsigned voff[2];
    bool yok[2];
#pragma unroll
    for (int hy = 0; hy < 2; ++hy) {
        const int y = y0 + 2 * (o & 1) + hy;
        yok[hy] = IN || y < Y;
        const unsigned yl = IN ? (unsigned)(2 * (o & 1) + hy) : (unsigned)(min(y, Y - 1) - y0);
        voff[hy] = ((xl * Y + yl) * Z * C + cc) * (unsigned)kEs;
    }
    int soff[4];
    bool zok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        zok[i] = IN || z0 + i < Z;
        soff[i] = (IN ? i : min(z0 + i, Z - 1) - z0) * C * kEs;
    }
    unsigned mask = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // aux 2: non-temporal (grad_feats is streamed once per region)
        if constexpr (GB) {
            const unsigned w = (unsigned)__builtin_amdgcn_raw_buffer_load_b32(rsrc, voff[i >> 2], soff[i & 3], 2);
            v[0][i] = __uint_as_float(w << 16);
            v[1][i] = __uint_as_float(w & 0xffff0000u);
        } else {
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff[i >> 2], soff[i & 3], 2));
            v[0][i] = __uint_as_float(w[0]);
            v[1][i] = __uint_as_float(w[1]);
        }
        const unsigned ok = (cok && xok && yok[i >> 2] && zok[i & 3]) ? 1u : 0u;
        mask |= (ok << i) | (ok << (i + 8));
    }
    return IN ? 0xffffu : mask;
}

// Tile loop of one phase-B pass for a wave that owns NB row blocks (pass blocks wave + 8b,
// b < NB; NB may be 0).  Every wave runs the same staging work and the same sequence of
// barriers, whatever its NB, so waves of one workgroup may run different instantiations.  The
// weights of a tile (A operand) are held once per wave: those of k step s for tile k+1 are
// loaded as soon as the MFMAs of k step s of tile k are issued.  LDS hand-offs use lds_barrier,
// so loads stay in flight across the barrier and the compiler waits for each where its registers
// are used.
// FU: gF is the target and gF2 grid_feats; a staged value is k1 target + k2 grid_feats.
template <int NB, bool GB, bool P2, bool FU, bool IN>
__device__ __forceinline__ void br_tiles(BrSmem<FU>& sm, const Grid& G, int C, int c0, int ntl, int prow,
                                         const void* __restrict__ gF, const void* __restrict__ gF2,
                                         const __bf16* __restrict__ wt, float* __restrict__ gpart) {
    constexpr int NR = NB > 0 ? NB : 1;   // register arrays (unused when NB == 0)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // staging: channel sc, octets so and so + 4; or (P2) channels 2 cp and 2 cp + 1, octet ot
    const int sc = threadIdx.x & (kBrCc - 1), so = threadIdx.x >> 7;
    const int cp2 = 2 * (threadIdx.x & (kBrCc / 2 - 1)), ot = threadIdx.x / (kBrCc / 2);
    const int q = lane >> 4, cl = lane & 15;

    float pre[2][8];
    float pre2[FU ? 2 : 1][FU ? 8 : 1];   // FU: grid_feats values of the same voxels and channels
    unsigned pmask = 0;
    // tpos: the tile's position in tl_org (FU: its row of kc)
    auto stage = [&](int buf, int tpos) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            float u[8];
            if constexpr (FU) {
                // tile-local voxel of value i: 8 ot + i (P2) or 32 k + 8 so + i
                const float2* kr = &sm.kc[tpos][P2 ? 8 * ot : 32 * k + 8 * so];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float2 kk = kr[i];
                    const float gv = kk.x * pre[k][i] + kk.y * pre2[k][i];
                    u[i] = (pmask >> (i + 8 * k)) & 1u ? gv : 0.0f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) u[i] = (pmask >> (i + 8 * k)) & 1u ? pre[k][i] : 0.0f;
            }
            bf16x8 hh, ll;
            split8(u, hh, ll);
            // P2: channel cp2 + k of octet ot (k step ot / 4, lane group ot % 4); else voxel octet
            // so + 4k (k step k, lane group so) of channel sc
            const int ch = P2 ? cp2 + k : sc, ks = P2 ? (ot >> 2) : k, lg = P2 ? (ot & 3) : so;
            sm.bhi[buf][ks][ch >> 4][lg * 16 + (ch & 15)] = hh;
            if constexpr (!GB) sm.blo[buf][ks][ch >> 4][lg * 16 + (ch & 15)] = ll;   // zero for bfloat16
        }
    };
    // A operand of row block b for k step s of a tile: row 16 (wave + 8b) + l%16, voxels
    // 32s + 8(l/16) + i; wj[b] is the pair's weight row (M: absent pair, the zero row).
    bf16x8 wh[NR][2], wl[NR][2];
    int wj[NR];
    auto rows_of = [&](int k) {
        const int slot = sm.tl_s[k];
#pragma unroll
        for (int b = 0; b < NB; ++b) wj[b] = sm.tab[16 * (wave + kBrWaves * b) + cl][slot];
    };
    auto load_w = [&](int s) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const __bf16* wrow = wt + (int64_t)wj[b] * kWtRow + 8 * q + 32 * s;
            wh[b][s] = *reinterpret_cast<const bf16x8*>(wrow);
            wl[b][s] = *reinterpret_cast<const bf16x8*>(wrow + 64);
        }
    };
    f32x4 acc[NR][kBrCb];
#pragma unroll
    for (int b = 0; b < NR; ++b)
#pragma unroll
        for (int cb = 0; cb < kBrCb; ++cb) acc[b][cb] = f32x4{};
    // k step s of the tile in LDS buffer buf.  B fragments are read one channel block ahead of
    // their MFMAs; the scheduling barriers keep the compiler from hoisting every LDS read of the
    // step into registers.
    auto half = [&](int buf, int s) {
        if constexpr (NB > 0) {
            bf16x8 bh[2], bl[2];
            bh[0] = sm.bhi[buf][s][0][lane];
            bl[0] = sm.blo[buf][s][0][lane];
#pragma unroll
            for (int cb = 0; cb < kBrCb; ++cb) {
                if (cb + 1 < kBrCb) {
                    bh[(cb + 1) & 1] = sm.bhi[buf][s][cb + 1][lane];
                    bl[(cb + 1) & 1] = sm.blo[buf][s][cb + 1][lane];
                }
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[b][cb] = mfma_split_16x16x32<false, GB>(wh[b][s], wl[b][s], bh[cb & 1], bl[cb & 1], acc[b][cb]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    const int klast = ntl - 1;
    // prologue: tile 0 staged, gF of tile 1 and the weights of tile 0 in flight (in the order
    // the loop issues them, so that the compiler's waits at the loop head stay exact)
    // the tile at position k of the region's list, from its first voxel (no tile-id divisions here)
    auto load_tile = [&](int k) {
        const int x0 = uniform(sm.tl_org[k][0]), y0 = uniform(sm.tl_org[k][1]), z0 = uniform(sm.tl_org[k][2]);
        if constexpr (FU) {   // same voxels and channels, so the same mask
            if constexpr (P2) br_load_tile2<GB, IN>(G, C, c0, x0, y0, z0, cp2, ot, gF2, pre2);
            else br_load_tile<GB, IN>(G, C, c0, x0, y0, z0, sc, so, gF2, pre2);
        }
        if constexpr (P2) return br_load_tile2<GB, IN>(G, C, c0, x0, y0, z0, cp2, ot, gF, pre);
        else return br_load_tile<GB, IN>(G, C, c0, x0, y0, z0, sc, so, gF, pre);
    };
    pmask = load_tile(0);
    stage(0, 0);
    pmask = load_tile(min(1, klast));
    rows_of(0);
    load_w(0);
    load_w(1);
    lds_barrier();
    for (int k = 0; k < ntl; ++k) {
        const int kn = min(k + 1, klast);
        stage((k + 1) & 1, kn);
        pmask = load_tile(min(k + 2, klast));
        rows_of(kn);
        __builtin_amdgcn_sched_barrier(0);
        half(k & 1, 0);
        load_w(0);
        __builtin_amdgcn_sched_barrier(0);
        half(k & 1, 1);
        load_w(1);
        lds_barrier();
    }

    // D element i of (b, cb): pass row 16 (wave + 8b) + 4 (l/16) + i, channel c0 + 16 cb + l%16
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lr = 16 * (wave + kBrWaves * b) + 4 * q + i;
            if (lr >= prow) continue;
            float* dst = gpart + (int64_t)sm.rslot[lr] * C + c0 + cl;
#pragma unroll
            for (int cb = 0; cb < kBrCb; ++cb)
                if (c0 + 16 * cb + cl < C) dst[16 * cb] = acc[b][cb][i];
        }
    }
}

// A pass's row table (this thread's entries) and G->R slots, as loaded (rows past the pass read the
// region's last row).
constexpr int kBrPer = kBrPass * kBrSlots / kBrThreads;
struct BrRows {
    int tv[kBrPer];
    int rs[2];
};

__device__ __forceinline__ void br_load_rows(BrRows& L, int rp, int KR, int M, int MR, int jr0,
                                             const int* __restrict__ r_pairs, const int* __restrict__ table) {
#pragma unroll
    for (int e0 = 0; e0 < kBrPer; ++e0) {
        const int e = threadIdx.x + e0 * kBrThreads;
        const int r = min(rp + e / kBrSlots, KR - 1);
        // clamped: a row table or slot list from a workspace that was not prepared for these
        // Gaussians cannot send a load or a store outside the weights or the partial rows
        L.tv[e0] = min(max(table[(int64_t)(jr0 + r) * kBrSlots + e % kBrSlots], 0), M);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = threadIdx.x + h * kBrThreads;
        L.rs[h] = r < kBrPass ? min(max(r_pairs[jr0 + min(rp + r, KR - 1)], 0), MR - 1) : 0;
    }
}

// One pass of phase B over rows rp .. rp + prow - 1 of the region (prow <= 384): stages the
// pass's row table and G->R slots (L, from br_load_rows; the first pass's are requested together with
// the region's tile list), then runs the tile loop with this wave's block count.
template <bool GB, bool P2, bool FU>
__device__ __forceinline__ void br_pass(BrSmem<FU>& sm, const Grid& G, int C, int c0, int ntl, int rp,
                                        int KR, int M, int MR, int jr0, const void* __restrict__ gF,
                                        const void* __restrict__ gF2, const int* __restrict__ r_pairs,
                                        const int* __restrict__ table, const __bf16* __restrict__ wt,
                                        float* __restrict__ gpart, bool interior, const BrRows& L) {
    const int wave = threadIdx.x >> 6;
    const int prow = min(KR - rp, kBrPass);
    const int nblk = (prow + 15) >> 4;
    const int nb = uniform((nblk - wave + kBrWaves - 1) / kBrWaves);   // row blocks of this wave
    __syncthreads();   // the previous pass is done with both buffers and the row tables
    {
        constexpr int kPer = kBrPer;
        const int (&tv)[kPer] = L.tv;
        const int (&rs)[2] = L.rs;
#pragma unroll
        for (int e0 = 0; e0 < kPer; ++e0) {
            const int e = threadIdx.x + e0 * kBrThreads;
            sm.tab[e / kBrSlots][e % kBrSlots] = e / kBrSlots < prow ? tv[e0] : M;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = threadIdx.x + h * kBrThreads;
            if (r < kBrPass) sm.rslot[r] = rs[h];
        }
    }
    __syncthreads();
    static_assert(kBrRbMax == 3, "block-count dispatch");
    auto run = [&](auto inc) {
        constexpr bool IN = decltype(inc)::value;
        if (nb >= 3) br_tiles<3, GB, P2, FU, IN>(sm, G, C, c0, ntl, prow, gF, gF2, wt, gpart);
        else if (nb == 2) br_tiles<2, GB, P2, FU, IN>(sm, G, C, c0, ntl, prow, gF, gF2, wt, gpart);
        else if (nb == 1) br_tiles<1, GB, P2, FU, IN>(sm, G, C, c0, ntl, prow, gF, gF2, wt, gpart);
        else br_tiles<0, GB, P2, FU, IN>(sm, G, C, c0, ntl, prow, gF, gF2, wt, gpart);
    };
    if (interior) run(std::true_type{});
    else run(std::false_type{});
}

// P2: even C with rows aligned to two channels, so the gF staging loads take two channels at once.
// FU (float32): the upstream feature gradient is the cosine loss's (cg; gF unused), formed per
// value from the target and grid_feats.
template <bool GB, bool P2, bool FU>
__global__ void __launch_bounds__(kBrThreads, 1) k_bwd_region(
    Grid G, Regions RG, int C, int nchunk, const void* __restrict__ gF,
    const int* __restrict__ toff, int M, const int* __restrict__ roff,
    const int* __restrict__ r_pairs, const int* __restrict__ table, int MR,
    const __bf16* __restrict__ wt, float* __restrict__ gpart, const void* __restrict__ grid_feats, CosG cg) {
    static_assert(!FU || !GB, "the fused cosine gradient takes float32 rows");
    __shared__ BrSmem<FU> sm;
    const int idx = xcd_remap(blockIdx.x, gridDim.x);
    const int Rb = uniform(idx / nchunk);   // the batch's region (its list)
    const int chunk = uniform(idx - Rb * nchunk);
    if (Rb >= RG.total * G.scenes) return;
    const int c0 = chunk * kBrCc;
    const int jr0 = uniform(min(max(roff[Rb], 0), MR));
    const int KR = uniform(min(max(roff[Rb + 1], jr0), MR)) - jr0;
    if (KR <= 0) return;
    // the first pass's row table, requested together with the region's tile list below
    BrRows rows;
    br_load_rows(rows, 0, KR, M, MR, jr0, r_pairs, table);
    const int scene = uniform(Rb / RG.total), R = Rb - scene * RG.total;   // R: the scene's region
    const int tbase = scene * scene_tiles(G);                               // its first tile in the batch
    if (scene > 0) {   // the scene's voxel rows
        const int64_t vb = scene * scene_voxels(G);
        gF = static_cast<const char*>(gF) + vb * C * (GB ? 2 : 4);
        if constexpr (FU) {
            grid_feats = static_cast<const float*>(grid_feats) + vb * C;
            cg.tgt += vb * C;
            cg.coef += 2 * vb;
        }
    }

    if (threadIdx.x < 64) {
        // the region's tiles with a non-empty list, in slot order ((a, b) then z): lane s checks
        // slot s (its list bounds loaded by all slots at once) and takes its place among the kept
        // slots below it
        const int rnyz = RG.n[1] * RG.n[2];
        const int rx = R / rnyz, ry = (R - rx * rnyz) / RG.n[2], rz = R % RG.n[2];
        const int tpz = RG.cell[2] / kTile;
        const int s = threadIdx.x;
        const int ab = s / max(tpz, 1), cz = s - ab * tpz;
        const int tx = rx * 2 + (ab >> 1), ty = ry * 2 + (ab & 1), tz = rz * tpz + cz;
        bool keep = s < 4 * tpz && tx < G.tiles[0] && ty < G.tiles[1] && tz < G.tiles[2];
        if (keep) {
            const int t = (tx * G.tiles[1] + ty) * G.tiles[2] + tz;
            keep = min(max(toff[tbase + t + 1], 0), M) > min(max(toff[tbase + t], 0), M);   // non-empty list
        }
        const unsigned long long kept = __ballot(keep);
        if (keep) {
            const int k = __popcll(kept & ((1ull << s) - 1ull));
            sm.tl_s[k] = s;
            sm.tl_org[k][0] = tx * kTile;
            sm.tl_org[k][1] = ty * kTile;
            sm.tl_org[k][2] = tz * kTile;
        }
        if (s == 0) sm.ntl = __popcll(kept);
    }
    __syncthreads();
    const int ntl = uniform(sm.ntl);
    if (ntl == 0) return;   // every row stays zero: phase C reads no partial row of this region
    if constexpr (FU) {
        // (k1, k2) of every voxel of the region's tiles (0 outside the grid; those values are
        // masked anyway); the first pass's barrier orders these stores before their reads.  Two
        // guarded entries per thread (ntl * 64 <= 2 * kBrThreads) and the tile origins from
        // tl_org: a loop with a per-thread trip count here would leave values that the tile loop
        // shares with it divergent, and its buffer descriptors with them.
        static_assert(kBrSlots * 64 <= 2 * kBrThreads, "two coefficient entries per thread");
        const float scale = cg.grad_loss[0] * cg.inv_count;   // as the loss's own backward forms it
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = threadIdx.x + h * kBrThreads;
            if (e < ntl * 64) {
                const int* org = sm.tl_org[e >> 6];
                const int lv = e & 63;
                const int x = org[0] + (lv >> 4), y = org[1] + ((lv >> 2) & 3), z = org[2] + (lv & 3);
                float2 kk = make_float2(0.0f, 0.0f);
                if (in_grid(G, x, y, z)) {
                    const float2 c = *reinterpret_cast<const float2*>(cg.coef + 2 * voxel_index(G, x, y, z));
                    kk = make_float2(c.x * scale, c.y * scale);
                }
                sm.kc[e >> 6][lv] = kk;
            }
        }
        gF = cg.tgt;
    }

    // every voxel of the region's tiles inside the grid and the whole chunk inside the rows: the
    // staging loads need no clamps and every staged value is real
    bool interior;
    {
        const int rnyz = RG.n[1] * RG.n[2];
        const int rx = R / rnyz, ry = (R - rx * rnyz) / RG.n[2], rz = R % RG.n[2];
        interior = uniform((rx + 1) * RG.cell[0] <= G.dims[0] && (ry + 1) * RG.cell[1] <= G.dims[1] &&
                           (rz + 1) * RG.cell[2] <= G.dims[2] && c0 + kBrCc <= C) != 0;
    }
    br_pass<GB, P2, FU>(sm, G, C, c0, ntl, 0, KR, M, MR, jr0, gF, grid_feats, r_pairs, table, wt, gpart,
                        interior, rows);
    for (int rp = kBrPass; rp < KR; rp += kBrPass) {
        BrRows more;
        br_load_rows(more, rp, KR, M, MR, jr0, r_pairs, table);
        br_pass<GB, P2, FU>(sm, G, C, c0, ntl, rp, KR, M, MR, jr0, gF, grid_feats, r_pairs, table, wt, gpart,
                            interior, more);
    }
}

// ------------------------------------------------------------------------------------------
// Phase C: per Gaussian, fixed-order sums of the geometric partials and the region rows.
// ------------------------------------------------------------------------------------------
constexpr int kBgThreads = 256;

// OBF16: grad_features is stored as bfloat16 (rounded to nearest even), else float.
template <bool OBF16>
__global__ void __launch_bounds__(kBgThreads) k_bwd_gauss(
    int n, int C, int M, int MR, const int* __restrict__ g2t_offsets, const float* __restrict__ cov_inv,
    const float* __restrict__ pair_partials, const int* __restrict__ g2r_offsets,
    const float* __restrict__ gpart, float* __restrict__ grad_means, float* __restrict__ grad_cov,
    float* __restrict__ grad_opacity, void* __restrict__ grad_features_out) {
    __shared__ float red[4][kNumGrads];
    const int g = blockIdx.x;
    if (g >= n) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
        // the pair values are o sum r d (3), o sum r d d^T (xx yy zz xy xz yz) and sum r, with
        // r = gw e and d = centre - mu: d mu = A (o sum r d), d Sigma = A (o sum r d d^T) A^T / 2,
        // d o = sum r (A = cov_inv, row-major)
        float t[kNumGrads];
#pragma unroll
        for (int k = 0; k < kNumGrads; ++k) t[k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
        float A[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) A[k] = cov_inv[g * 9 + k];
        const float P[9] = {t[3], t[6], t[7], t[6], t[4], t[8], t[7], t[8], t[5]};
        float B[9];   // A P
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int k = 0; k < 3; ++k)
                B[i * 3 + k] = fmaf(A[i * 3], P[k], fmaf(A[i * 3 + 1], P[3 + k], A[i * 3 + 2] * P[6 + k]));
        auto bat = [&](int i, int l) {   // (A P A^T)_il / 2
            return 0.5f * fmaf(B[i * 3], A[l * 3], fmaf(B[i * 3 + 1], A[l * 3 + 1], B[i * 3 + 2] * A[l * 3 + 2]));
        };
        float gr[kNumGrads];
#pragma unroll
        for (int i = 0; i < 3; ++i) gr[i] = fmaf(A[i * 3], t[0], fmaf(A[i * 3 + 1], t[1], A[i * 3 + 2] * t[2]));
        gr[3] = bat(0, 0);
        gr[4] = bat(1, 1);
        gr[5] = bat(2, 2);
        gr[6] = bat(0, 1);
        gr[7] = bat(0, 2);
        gr[8] = bat(1, 2);
        gr[9] = t[9];
        write_grads(gr, g, grad_means, grad_cov, grad_opacity);
    }
    const int r0 = min(max(g2r_offsets[g], 0), MR), r1 = min(max(g2r_offsets[g + 1], r0), MR);
    // region rows summed in ascending order per channel; a bfloat16 output is the float sum rounded
    // to nearest even.  The rows are read once: nontemporal loads keep them from displacing cached
    // data (0.18 -> 0.15 ms at config 3)
    typedef typename std::conditional<OBF16, __bf16, float>::type OT;
    OT* out = static_cast<OT*>(grad_features_out) + (int64_t)g * C;
    if ((C & 3) == 0) {
        for (int c = threadIdx.x * 4; c < C; c += kBgThreads * 4) {
            float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int r = r0; r < r1; ++r) {
                const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(gpart + (int64_t)r * C + c));
                s.x += v[0]; s.y += v[1]; s.z += v[2]; s.w += v[3];
            }
            const f32x4 nv = {s.x, s.y, s.z, s.w};
            if constexpr (OBF16) {
                typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                *reinterpret_cast<bf16x4*>(out + c) = __builtin_convertvector(nv, bf16x4);
            } else {
                __builtin_nontemporal_store(nv, reinterpret_cast<f32x4*>(out + c));
            }
        }
    } else {
        for (int c = threadIdx.x; c < C; c += kBgThreads) {
            float s = 0.0f;
            for (int r = r0; r < r1; ++r) s += gpart[(int64_t)r * C + c];
            out[c] = (OT)s;
        }
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
static int feature_chunks(int C) { return (C + kBtKc - 1) / kBtKc; }
// Chunks of phase A for the feature type: 32 channels (float, split hi/lo) or 64 (bfloat16).
static int feature_chunks(int C, int fdt) { return fdt == kDtBF16 ? (C + kBtKcBf - 1) / kBtKcBf : feature_chunks(C); }

struct PlanBufs {
    int* g2r_offsets;
    long long* total;
    void* scan_ws;
    size_t bytes;
};

static PlanBufs carve_plan(void* ws, int n) {
    Carver c(ws, (size_t)-1);
    PlanBufs b;
    b.g2r_offsets = c.take<int>(n + 1);
    b.total = c.take<long long>(1);
    b.scan_ws = c.take<char>(scan_workspace(n > 0 ? n : 1));
    b.bytes = c.off + 256;
    return b;
}

size_t backward_plan_workspace(int n) { return carve_plan(nullptr, n).bytes; }

hipError_t backward_plan_async(const Grid& G, int n, const int* lb, const int* ub, void* plan_ws,
                               long long* mr_host, hipStream_t s) {
    const Regions RG = make_regions(G);
    const PlanBufs b = carve_plan(plan_ws, n);
    *mr_host = 0;
    hipError_t e = launch_cell_count(n, lb, ub, RG.cell, b.g2r_offsets, s);
    if (e != hipSuccess || n <= 0) return e;
    e = scan_i32(b.g2r_offsets + 1, b.g2r_offsets + 1, n, true, b.total, b.scan_ws, s);
    if (e != hipSuccess) return e;
    return hipMemcpyAsync(mr_host, b.total, sizeof(long long), hipMemcpyDeviceToHost, s);
}

int* backward_plan_cells(const Grid& G, void* plan_ws, int n, int cell[3], void** scan_ws) {
    const Regions RG = make_regions(G);
    const PlanBufs b = carve_plan(plan_ws, n);
    for (int a = 0; a < 3; ++a) cell[a] = RG.cell[a];
    *scan_ws = b.scan_ws;
    return b.g2r_offsets;
}

hipError_t backward_plan(const Grid& G, int n, const int* lb, const int* ub, void* plan_ws,
                         long long* num_region_pairs, hipStream_t s) {
    long long MR = 0;
    hipError_t e = backward_plan_async(G, n, lb, ub, plan_ws, &MR, s);
    if (e != hipSuccess) return e;
    e = hipStreamSynchronize(s);
    *num_region_pairs = MR;
    return e;
}

struct FeatBufs {
    __bf16* fsp;
    float* partials;
    __bf16* wt;
    int* r_cells;
    int* r_pairs;
    int* r_gauss;
    int* r_cells_sorted;
    int* r_pairs_sorted;
    int* r_gids;
    int* table;
    int* roff;
    void* sort_ws;
    float* gpart;
    int* tl;
    size_t bytes;
};

static FeatBufs carve_feats(void* ws, const Grid& G, int n, int C, int64_t M, int64_t MR) {
    const Regions RG = make_regions(G);
    const int64_t m = M > 0 ? M : 1, mr = MR > 0 ? MR : 1;
    Carver c(ws, (size_t)-1);
    FeatBufs b;
    b.fsp = c.take<__bf16>((int64_t)(n + 1) * feature_chunks(C) * 2 * kBtKc);
    b.partials = c.take<float>(m * kNumGrads);
    b.wt = c.take<__bf16>((m + 1) * kWtRow);   // row M is zero (rows of absent pairs read it)
    b.r_cells = c.take<int>(mr);
    b.r_pairs = c.take<int>(mr);
    b.r_gauss = c.take<int>(mr);
    b.r_cells_sorted = c.take<int>(mr);
    b.r_pairs_sorted = c.take<int>(mr);
    b.r_gids = c.take<int>(mr);
    b.table = c.take<int>(mr * kBrSlots);
    const int nreg = RG.total * G.scenes;   // regions of the batch
    b.roff = c.take<int>(nreg + 1);
    b.sort_ws = c.take<char>(sort_workspace(MR, nreg));
    b.gpart = c.take<float>(mr * (C > 0 ? C : 1));
    {   // long-tile list of phase A: a count, then at most min(T, M) tiles
        const int64_t T = (int64_t)scene_tiles(G) * G.scenes;
        b.tl = c.take<int>(1 + (M < T ? M : T));
    }
    b.bytes = c.off + 256;
    return b;
}

size_t backward_feats_workspace(const Grid& G, int n, int C, int64_t M, int64_t MR) {
    return carve_feats(nullptr, G, n, C, M, MR).bytes;
}

hipError_t launch_backward_prepare(const Grid& G, int n, int C, const void* features, int fdt, const int* lb,
                                   const int* ub, int64_t M, const int* sorted_tiles, const int* sorted_gauss,
                                   const void* plan_ws, int64_t MR, void* ws, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const Regions RG = make_regions(G);
    const int nchk = feature_chunks(C, fdt);
    if (!split_rows_fit(n, C)) return hipErrorInvalidValue;   // byte offsets of the split rows are 32-bit
    const FeatBufs b = carve_feats(ws, G, n, C, M, MR);
    const PlanBufs pb = carve_plan(const_cast<void*>(plan_ws), n);
    hipError_t e;

    // features as 32-channel chunks of bf16 hi/lo (64-channel chunks of the values for bfloat16
    // features): the B operand of phase A, plus a zero row
    const int64_t fcount = (int64_t)(n + 1) * nchk * ((fdt == kDtBF16 ? kBtKcBf : kBtKc) / 8);   // one thread per 8 channels
    if (fdt == kDtBF16)
        G2V_LAUNCH(k_split_chunks<__bf16>, dim3((unsigned)ceil_div(fcount, 256)), dim3(256), 0, s,
                   static_cast<const __bf16*>(features), n, C, nchk, b.fsp);
    else
        G2V_LAUNCH(k_split_chunks<float>, dim3((unsigned)ceil_div(fcount, 256)), dim3(256), 0, s,
                   static_cast<const float*>(features), n, C, nchk, b.fsp);
    // Region -> Gaussian CSR (pairs carry their G->R slot so partial rows land Gaussian-major) and
    // the row table of phase B
    const int nreg = RG.total * G.scenes;   // regions of the batch: scene b's region r is b R + r
    if (MR > 0) {
        e = launch_fill_cells(n, lb, ub, pb.g2r_offsets, RG.cell, RG.n, b.r_cells, b.r_pairs, b.r_gauss, s,
                              G.scenes > 1 ? G.scene_n : 0, RG.total);
        if (e != hipSuccess) return e;
        e = radix_sort_pairs(b.r_cells, b.r_pairs, b.r_cells_sorted, b.r_pairs_sorted, MR, nreg, b.sort_ws, s);
        if (e != hipSuccess) return e;
    }
    e = launch_tile_offsets(b.r_cells_sorted, MR, nreg, b.roff, s);
    if (e != hipSuccess) return e;
    if (MR > 0 && M > 0) {
        G2V_LAUNCH(k_region_rows, dim3((unsigned)ceil_div(MR, 256)), dim3(256), 0, s, (int)MR, (int)M,
                   (const int*)b.r_pairs_sorted, (const int*)b.r_gauss, b.r_gids, b.table,
                   reinterpret_cast<int*>(b.wt + M * kWtRow));
        G2V_LAUNCH(k_region_table, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, s, G, RG, (int)M, (int)MR,
                   sorted_tiles, sorted_gauss, (const int*)b.roff, (const int*)b.r_gids, b.table);
    }
    return hipGetLastError();
}

hipError_t launch_backward_feats(const Grid& G, int n, int C, const float* grad_density,
                                 const void* grad_feats, const float* means, const float* opacity,
                                 const float* cov_inv, const int* lb, const int* ub,
                                 const int* g2t_offsets, int64_t M, const int* tile_offsets,
                                 const int* sorted_tiles, const int* sorted_gauss, const float* density,
                                 const void* grid_feats, const void* features, int fdt,
                                 const void* plan_ws, int64_t MR, float* grad_means, float* grad_cov,
                                 float* grad_opacity, void* grad_features, void* ws, bool prepared,
                                 hipStream_t s, const CosG* cos) {
    if (n <= 0) return hipSuccess;
    // the fused cosine gradient: float32 rows of 16-byte multiples, 16-byte aligned
    if (cos && (fdt != kDtF32 || (C & 3) != 0 || ((uintptr_t)cos->tgt & 15) != 0 || ((uintptr_t)grid_feats & 15) != 0 ||
                !cos->tgt || !cos->coef || !cos->grad_loss))
        return hipErrorInvalidValue;
    const CosG cg = cos ? *cos : CosG{nullptr, nullptr, nullptr, 0.0f};
    const Regions RG = make_regions(G);
    const int T = scene_tiles(G) * G.scenes;   // tiles of the batch
    const int nchk = feature_chunks(C, fdt);
    if (!split_rows_fit(n, C)) return hipErrorInvalidValue;   // byte offsets of the split rows are 32-bit
    const FeatBufs b = carve_feats(ws, G, n, C, M, MR);
    const PlanBufs pb = carve_plan(const_cast<void*>(plan_ws), n);
    if (!prepared) {
        const hipError_t e = launch_backward_prepare(G, n, C, features, fdt, lb, ub, M, sorted_tiles,
                                                     sorted_gauss, plan_ws, MR, ws, s);
        if (e != hipSuccess) return e;
    }
    if (M > 0 && T > 0) {
        const int blocks = (int)ceil_div(T, 8) * 8;
        // 16-byte G loads: 4 float or 8 bfloat16 channels per load, rows 16-byte aligned
        const bool vec = (C & (fdt == kDtBF16 ? 7 : 3)) == 0 && ((uintptr_t)grad_feats & 15) == 0;
        // lists of at most short_list_max(C) Gaussians go to k_bwd_tile_short (not with the fused
        // cosine gradient, whose tiles all take k_bwd_tile).  When fewer tiles can be long than
        // there are tiles (a sparse problem), k_bwd_tile walks a compacted list of the long ones.
        const int skip_le = cos ? 0 : min(short_list_max(C), kBsMax);
        const int nlong = long_tiles_bound(M, T, skip_le);
        const int* tlist = nullptr;
        const int* tcount = nullptr;
        if (nlong < T && nlong > 0) {
            const hipError_t e = launch_long_tiles(tile_offsets, T, (int)M, skip_le, b.tl, b.tl + 1, nlong, s);
            if (e != hipSuccess) return e;
            tcount = b.tl;
            tlist = b.tl + 1;
        }
        const int lblocks = (int)ceil_div(nlong, 8) * 8;
        if (!cos) {
            if (fdt == kDtBF16)
                G2V_LAUNCH(k_bwd_tile_short<true>, dim3(blocks), dim3(kBsThreads), 0, s, G, n, C, nchk, grad_density,
                           grad_feats, means, opacity, cov_inv, lb, ub, g2t_offsets, tile_offsets, sorted_gauss, (int)M,
                           density, (const __bf16*)b.fsp, b.partials, b.wt, skip_le);
            else
                G2V_LAUNCH(k_bwd_tile_short<false>, dim3(blocks), dim3(kBsThreads), 0, s, G, n, C, nchk, grad_density,
                           grad_feats, means, opacity, cov_inv, lb, ub, g2t_offsets, tile_offsets, sorted_gauss, (int)M,
                           density, (const __bf16*)b.fsp, b.partials, b.wt, skip_le);
        }
#define G2V_BT(V, F, FU)                                                                                      \
    G2V_LAUNCH((k_bwd_tile<V, F, FU>), dim3(lblocks), dim3(kBtThreads), 0, s, G, n, C, nchk, grad_density,         \
               grad_feats, means, opacity, cov_inv, lb, ub, g2t_offsets, tile_offsets, sorted_gauss, (int)M, density,        \
               grid_feats, fdt, (const __bf16*)b.fsp, b.partials, b.wt, cg, skip_le, tlist, tcount)
        if (nlong == 0) {
            // every list is short: k_bwd_tile_short took them all
        } else if (cos) {
            G2V_BT(true, false, true);
        } else if (fdt == kDtBF16) {
            if (vec) G2V_BT(true, true, false);
            else G2V_BT(false, true, false);
        } else {
            if (vec) G2V_BT(true, false, false);
            else G2V_BT(false, false, false);
        }
#undef G2V_BT
    }
    if (MR > 0 && M > 0) {
        const int nchunk = (C + kBrCc - 1) / kBrCc;
        const int64_t items = (int64_t)RG.total * G.scenes * nchunk;
        const int blocks = (int)ceil_div(items, 8) * 8;
        // two-channel staging loads: even C and a grad_feats base aligned to two elements
        const bool pair = (C & 1) == 0 && ((uintptr_t)grad_feats & (fdt == kDtBF16 ? 3 : 7)) == 0;
#define G2V_BR(GBV, P2V, FU)                                                                                  \
    G2V_LAUNCH((k_bwd_region<GBV, P2V, FU>), dim3(blocks), dim3(kBrThreads), 0, s, G, RG, C, nchunk, grad_feats,   \
               tile_offsets, (int)M, (const int*)b.roff, (const int*)b.r_pairs_sorted, (const int*)b.table, (int)MR, \
               (const __bf16*)b.wt, b.gpart, grid_feats, cg)
        if (cos) {   // C % 4 == 0 and 16-byte aligned rows: the paired loads apply
            G2V_BR(false, true, true);
        } else if (fdt == kDtBF16) {
            if (pair) G2V_BR(true, true, false);
            else G2V_BR(true, false, false);
        } else {
            if (pair) G2V_BR(false, true, false);
            else G2V_BR(false, false, false);
        }
#undef G2V_BR
    }
    if (fdt == kDtBF16)
        G2V_LAUNCH(k_bwd_gauss<true>, dim3(n), dim3(kBgThreads), 0, s, n, C, (int)M, (int)MR, g2t_offsets,
                   cov_inv, (const float*)b.partials, (const int*)pb.g2r_offsets, (const float*)b.gpart, grad_means,
                   grad_cov, grad_opacity, grad_features);
    else
        G2V_LAUNCH(k_bwd_gauss<false>, dim3(n), dim3(kBgThreads), 0, s, n, C, (int)M, (int)MR, g2t_offsets,
                   cov_inv, (const float*)b.partials, (const int*)pb.g2r_offsets, (const float*)b.gpart, grad_means,
                   grad_cov, grad_opacity, grad_features);
    return hipGetLastError();
}

}  // namespace g2v
