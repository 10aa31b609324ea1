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
// Features as packed bf16 pairs: low half = hi part, high half = lo part of the 2-term split.
// ------------------------------------------------------------------------------------------
// T: float features, packed as (hi, lo) bf16 pairs, 4 bytes per channel; or __bf16 features,
// packed as they are, 2 bytes per channel.
template <typename T>
__global__ void __launch_bounds__(256) k_split_pack(const T* __restrict__ src, int n, int C, int Cp,
                                                    uint32_t* __restrict__ dst) {
    // (n + 1) x Cp packed pairs: row n and columns >= C are zero, so padded K slots and channels
    // can be gathered without bounds checks.  One thread per 4 channels (16-byte store).
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nq = Cp / 4;
    if (i >= (int64_t)(n + 1) * nq) return;
    const int64_t r = i / nq;
    const int c = (int)(i - r * nq) * 4;
    float v[4];
    if constexpr (sizeof(T) == 4) {
        if (r < n && c + 4 <= C && ((uintptr_t)(src + r * C + c) & 15) == 0) {
            const float4 a = *reinterpret_cast<const float4*>(src + r * C + c);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (r < n && c + e < C) ? (float)src[r * C + c + e] : 0.0f;
        }
    } else {
        // bfloat16 features are packed as they are: 2 bytes per channel (rows of Cp values)
        unsigned short h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            h[e] = (r < n && c + e < C) ? __builtin_bit_cast(unsigned short, src[r * C + c + e]) : (unsigned short)0;
        *reinterpret_cast<uint2*>(reinterpret_cast<unsigned short*>(dst) + r * Cp + c) =
            make_uint2(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16));
        return;
    }
    uint4 o;
    uint32_t* op = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        __bf16 h, l;
        split_bf16(v[e], h, l);
        op[e] = (uint32_t)__builtin_bit_cast(unsigned short, h) | ((uint32_t)__builtin_bit_cast(unsigned short, l) << 16);
    }
    *reinterpret_cast<uint4*>(dst + r * Cp + c) = o;
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
// Feature splat (MFMA 32x32x16 bf16, 3-term split), channel-quad layout.
//
// A wave owns 64 voxels x 128 channels: 2 voxel blocks x 4 channel blocks of 32x32.  Column j of
// channel block c is channel 4j + c (of the wave's 128), so the B fragment of lane (j, h) for
// all four channel blocks comes from one 16-byte load per Gaussian row (4 packed channels), and
// the four results of one output row sit in one lane as 4 consecutive channels (float4 store).
// Per K step (16 Gaussians) a wave issues 8 dwordx4 gathers, 32 byte permutes and 24 MFMAs.
// ------------------------------------------------------------------------------------------
constexpr int kFwdThreads = 256;               // 4 waves
constexpr int kFwdWaves = kFwdThreads / 64;
constexpr int kFwdChanPerWave = 128;
constexpr int kFwdChanPerPass = kFwdChanPerWave * kFwdWaves;
constexpr int kFwdKMax = 256;                  // Gaussians held in LDS per K chunk (multiple of 32)
constexpr int kFwdKSteps = kFwdKMax / 16;

static_assert(kFwdChanPerWave == kPackedChannelAlign, "packed rows are padded to one wave's channels");

// One list entry as the W build reads it, relative to the tile's first voxel (x0, y0, z0): the
// exponent of exp2 at voxel (x0+a, y0+b, z0+c) is
//     F(a,b) + Gxy(a,b) dz_c + fz_c,
//     F = a00 dx^2 + a01 dx dy + a11 dy^2,  Gxy = a02 dx + a12 dy,  fz_c = kq A22 dz_c^2,
// with dx, dy the offsets of the voxel centre from the mean, a00 = kq A00, a01 = kq (A01 + A10),
// a11 = kq A11, a02 = kq (A02 + A20), a12 = kq (A12 + A21), kq = -log2(e)/2, so that
// exp2(...) = exp(-dx^T A dx / 2) (reference .cu:911-921), dz_c = (z centre of layer c) - mu2 and
// a22 = kq A22 formed by the thread that reads the record.  A voxel outside the box in z (bit c of
// zmask clear) has fz_c = -inf; one outside it in x or y (bit 4a+b of xymask clear) gets F = -inf;
// either way the weight is exactly 0, as the reference's box test makes it.  48 bytes, so that
// the records of a whole 256-entry chunk fit beside its W at two workgroups per CU.
struct alignas(16) FwdRec {
    float mux, muy, o, a12;
    float a00, a01, a11, a02;
    float mu2, a22;
    uint32_t xymask, zmask;
};
static_assert(sizeof(FwdRec) == 48, "FwdRec is three 16-byte words");

// The box masks of a record for the tile whose first voxel is (x0, y0, z0) (box l..u).
__device__ __forceinline__ void fwd_record_masks(FwdRec& r, const int (&l)[3], const int (&u)[3], int x0, int y0,
                                                 int z0) {
    uint32_t xm = 0, ym = 0, zm = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        zm |= (z0 + c >= l[2] && z0 + c <= u[2]) ? (1u << c) : 0u;
        xm |= (x0 + c >= l[0] && x0 + c <= u[0]) ? (1u << c) : 0u;
        ym |= (y0 + c >= l[1] && y0 + c <= u[1]) ? (1u << c) : 0u;
    }
    r.zmask = zm;
    uint32_t m = 0;
#pragma unroll
    for (int a = 0; a < 4; ++a) m |= (xm >> a) & 1u ? ym << (4 * a) : 0u;
    r.xymask = m;
}

// The record of a Gaussian from its packed DenParams (the coefficients kq A00, kq (A01 + A10), ...
// formed by the G->T fill) for the tile whose first voxel is (x0, y0, z0).
__device__ __forceinline__ FwdRec fwd_record_packed(const DenParams& w, int x0, int y0, int z0) {
    FwdRec r;
    r.mux = w.mux;
    r.muy = w.muy;
    r.o = w.o;
    r.a00 = w.a00;
    r.a01 = w.a01;
    r.a11 = w.a11;
    r.a02 = w.a02;
    r.a12 = w.a12;
    r.mu2 = w.muz;
    r.a22 = w.a22;
    const int l[3] = {w.lbx, w.lby, w.lbz}, u[3] = {w.ubx, w.uby, w.ubz};
    fwd_record_masks(r, l, u, x0, y0, z0);
    return r;
}

// A record past the list: every weight is exactly 0 (o = 0, empty masks).
__device__ __forceinline__ FwdRec fwd_record_empty() {
    FwdRec r;
    r.mux = r.muy = r.o = r.a12 = 0.0f;
    r.a00 = r.a01 = r.a11 = r.a02 = 0.0f;
    r.mu2 = r.a22 = 0.0f;
    r.xymask = r.zmask = 0;
    return r;
}

// Weights o e of the four voxels (x0 + col / 4, y0 + col % 4, z0 + c) of column col against the
// LDS record rec (three 16-byte reads): F and Gxy once per column, one fma, one add and one exp2
// per voxel.  cxl, cyl: centre of the column; cz: centres of the tile's z layers.
__device__ __forceinline__ void fwd_column_weights(const FwdRec* rec, int col, float cxl, float cyl,
                                                   const float (&cz)[4], float (&w)[4]) {
    const uint4* rp = reinterpret_cast<const uint4*>(rec);
    const uint4 q0 = rp[0], q1 = rp[1], q2 = rp[2];
    const uint32_t m = q2.z, zm = q2.w;
    const float dx = cxl - __uint_as_float(q0.x), dy = cyl - __uint_as_float(q0.y);
    const float ro = __uint_as_float(q0.z), a12 = __uint_as_float(q0.w);
    const float a00 = __uint_as_float(q1.x), a01 = __uint_as_float(q1.y);
    const float a11 = __uint_as_float(q1.z), a02 = __uint_as_float(q1.w);
    const float mu2 = __uint_as_float(q2.x), a22 = __uint_as_float(q2.y);
    float dz[4], fz[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        dz[c] = cz[c] - mu2;
        fz[c] = ((zm >> c) & 1u) ? a22 * dz[c] * dz[c] : -__builtin_inff();
    }
    float F = fmaf(fmaf(a00, dx, a01 * dy), dx, a11 * dy * dy);
    F = ((m >> col) & 1u) ? F : -__builtin_inff();
    const float Gxy = fmaf(a02, dx, a12 * dy);
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = ro * __builtin_amdgcn_exp2f(fmaf(Gxy, dz[c], F) + fz[c]);
}

// ------------------------------------------------------------------------------------------
// Density only: two waves per tile, each walking every other batch of 64 entries of the tile's
// list in ascending order: lane k gathers entry k's packed 64-byte DenParams (written by the G->T
// fill; one gather instead of one from each of five arrays, whose L2 misses bounded the kernel),
// turns it into its tile-relative record and writes that into the wave's LDS slab (the packed
// records of the wave's next batch are gathered while the current ones are evaluated).  Lane
// (col = lane % 16, ph = lane / 16) then takes the voxel column col and the entries ph, ph + 4, ...
// of the slab, forming each entry's four weights of the column with the
// operations of fwd_column_weights (so the weights of the feature splat); the z terms dz_c and
// fz_c, the same for every column, are formed once per entry by the lane that builds its record.
// The four lane groups' sums are added at the end, then the two waves' sums (first wave + second).
// The sum is the reference's (.cu:7-136) in another order.
// ------------------------------------------------------------------------------------------
constexpr int kDenWaves = 4;

// A FwdRec with its four z terms: dz_c = (centre of layer c) - mu2 and fz_c as fwd_column_weights
// forms them (80 bytes).
struct alignas(16) DenRec {
    float mux, muy, o, a12;
    float a00, a01, a11, a02;
    float dz[4];
    float fz[4];
    uint32_t xymask, pad[3];
};
static_assert(sizeof(DenRec) == 80, "DenRec is five 16-byte words");

__device__ __forceinline__ DenRec den_record(const FwdRec& r, const float (&cz)[4]) {
    DenRec d;
    d.mux = r.mux;
    d.muy = r.muy;
    d.o = r.o;
    d.a12 = r.a12;
    d.a00 = r.a00;
    d.a01 = r.a01;
    d.a11 = r.a11;
    d.a02 = r.a02;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        d.dz[c] = cz[c] - r.mu2;
        d.fz[c] = ((r.zmask >> c) & 1u) ? r.a22 * d.dz[c] * d.dz[c] : -__builtin_inff();
    }
    d.xymask = r.xymask;
    d.pad[0] = d.pad[1] = d.pad[2] = 0;
    return d;
}

// LDS hand-off between the lanes of one wave: waits for the wave's LDS operations; the compiler
// barriers keep the slab's reads and writes on their side of it.
__device__ __forceinline__ void wave_lds_sync() {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15 << 0) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __asm__ __volatile__("" ::: "memory");
}

__global__ void __launch_bounds__(kDenWaves * 64) k_fwd_density(Grid G, const DenParams* __restrict__ drec,
                                                               const int* __restrict__ toff,
                                                               const int* __restrict__ sorted_gauss,
                                                               int M, float* __restrict__ density) {
    __shared__ DenRec slab[kDenWaves][64];
    __shared__ float half1[kDenWaves / 2][4][16];   // the second wave's column sums of each tile
    const int T = scene_tiles(G);
    // Two waves per tile: wave half h takes the list's 64-entry batches h, h + 2, ... (twice the
    // waves in flight for a kernel that mostly waits on its record loads); the tile's density is
    // (half 0) + (half 1), added in that order.  tb: the batch's tile (its list), tile: the scene's.
    const int wv = threadIdx.x >> 6, half = wv & 1;
    const int tb = uniform(xcd_remap(blockIdx.x, gridDim.x) * (kDenWaves / 2) + (wv >> 1));
    const bool live = tb < T * G.scenes;   // uniform per wave; every wave meets the barrier below
    const int scene = uniform(live ? tb / T : 0), tile = live ? tb - scene * T : 0;
    density += scene * scene_voxels(G);
    const int lane = threadIdx.x & 63, col = lane & 15, ph = lane >> 4;
    DenRec* sl = slab[wv];
    int x0, y0, z0;
    tile_voxel(G, tile, 0, x0, y0, z0);
    const float cxl = centre(G, 0, x0 + (col >> 2)), cyl = centre(G, 1, y0 + (col & 3));
    float cz[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) cz[c] = centre(G, 2, z0 + c);
    const int j0 = live ? uniform(min(max(toff[tb], 0), M)) : 0;
    const int j1 = live ? uniform(min(max(toff[tb + 1], j0), M)) : 0;
    // A batch's packed records (one 64-byte gather per entry) are held across the previous batch's
    // evaluation and turned into tile records after it, so the gathers' latency passes under that
    // evaluation; the list entries run one batch further ahead.  graw < 0: past the list (an empty
    // record).
    auto load_raw = [&](int g, DenParams& w) {
        if (g >= 0) w = drec[g];
    };
    auto record = [&](int g, const DenParams& w) {
        return den_record(g >= 0 ? fwd_record_packed(w, x0, y0, z0) : fwd_record_empty(), cz);
    };
    float dacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int jh = j0 + 64 * half;   // this wave's first batch
    DenParams raw = {};
    int graw = jh + lane < j1 ? sorted_gauss[jh + lane] : -1;
    load_raw(graw, raw);
    int gnext = jh + 128 + lane < j1 ? sorted_gauss[jh + 128 + lane] : -1;
    for (int jb = jh; jb < j1; jb += 128) {
        const DenRec cur = record(graw, raw);
        wave_lds_sync();   // the previous records are read
        sl[lane] = cur;
        wave_lds_sync();
        graw = gnext;
        load_raw(graw, raw);   // before the next entry load: the counter of loads is in order
        gnext = jb + 256 + lane < j1 ? sorted_gauss[jb + 256 + lane] : -1;
        // slots past the list hold empty records (weight 0), so every lane group runs the same count
        const int n4 = uniform((min(64, j1 - jb) + 3) >> 2);
        for (int k4 = 0; k4 < n4; ++k4) {
            // fwd_column_weights with the z terms read from the record
            const uint4* rp = reinterpret_cast<const uint4*>(&sl[4 * k4 + ph]);
            const uint4 q0 = rp[0], q1 = rp[1], q2 = rp[2], q3 = rp[3], q4 = rp[4];
            const float dx = cxl - __uint_as_float(q0.x), dy = cyl - __uint_as_float(q0.y);
            const float ro = __uint_as_float(q0.z), a12 = __uint_as_float(q0.w);
            const float a00 = __uint_as_float(q1.x), a01 = __uint_as_float(q1.y);
            const float a11 = __uint_as_float(q1.z), a02 = __uint_as_float(q1.w);
            const float dz[4] = {__uint_as_float(q2.x), __uint_as_float(q2.y), __uint_as_float(q2.z),
                                 __uint_as_float(q2.w)};
            const float fz[4] = {__uint_as_float(q3.x), __uint_as_float(q3.y), __uint_as_float(q3.z),
                                 __uint_as_float(q3.w)};
            float F = fmaf(fmaf(a00, dx, a01 * dy), dx, a11 * dy * dy);
            F = ((q4.x >> col) & 1u) ? F : -__builtin_inff();
            const float Gxy = fmaf(a02, dx, a12 * dy);
#pragma unroll
            for (int c = 0; c < 4; ++c) dacc[c] += ro * __builtin_amdgcn_exp2f(fmaf(Gxy, dz[c], F) + fz[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {   // the four lane groups: (ph 0 + ph 1) + (ph 2 + ph 3)
        dacc[c] += xor_shfl<16>(dacc[c]);
        dacc[c] += __shfl_xor(dacc[c], 32, 64);
    }
    if (half == 1 && ph == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) half1[wv >> 1][c][col] = dacc[c];
    }
    lds_barrier();
    const int x = x0 + (col >> 2), y = y0 + (col & 3);
    if (live && half == 0 && ph == 0 && x < G.dims[0] && y < G.dims[1]) {
        float* out = density + voxel_index(G, x, y, z0);
        const int nz = min(kTile, G.dims[2] - z0);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (c < nz) out[c] = dacc[c] + half1[wv >> 1][c][col];
    }
}

hipError_t launch_forward_density(const Grid& G, const DenParams* drec, const int* tile_offsets,
                                  const int* sorted_gauss, int M, float* density, hipStream_t s) {
    const int T = scene_tiles(G) * G.scenes;
    if (T <= 0) return hipSuccess;
    if (M > 0 && !drec) return hipErrorInvalidValue;
    const int groups = (int)ceil_div(T, kDenWaves / 2);   // two waves per tile
    const int blocks = (int)ceil_div(groups, 8) * 8;
    G2V_LAUNCH(k_fwd_density, dim3(blocks), dim3(kDenWaves * 64), 0, s, G, drec, tile_offsets, sorted_gauss, M,
               density);
    return hipGetLastError();
}

struct FwdSmem {
    bf16x8 whi[kFwdKSteps][2][64];   // A operand, hi part: [k step][voxel block][lane]
    bf16x8 wlo[kFwdKSteps][2][64];   // A operand, lo part
    alignas(16) uint32_t roff[kFwdKMax];   // byte offset of each K slot's packed row (zero row for padding)
    FwdRec rec[kFwdKMax];            // the K chunk's entries
    alignas(16) float dpart[kFwdWaves][64];   // per-wave partial densities
    alignas(16) float inv_den[64];   // 1 / max(D, eps)
    alignas(16) int vlin[64];        // linear voxel index, -1 outside the grid
};

// Builds the split W for K slots [kbeg, kbeg + 16*ksteps) of the tile list into LDS (slots past
// klen get weight 0 and the zero row).  First each thread turns one entry into its tile-relative
// record.  Then thread t owns the voxel column (x0 + a, y0 + b), col = 4a + b = t % 16, and the
// octets t/16, t/16 + 16, ...: for each of the octet's eight entries it forms F and Gxy once and
// the four weights of its column from them, and writes the column's four voxels as finished A
// fragments (8 entries x 1 voxel each).  Adds the raw weights of the column's voxels to dacc
// (a build repeated for a later channel pass adds them again; only the first pass reads dacc).
__device__ __forceinline__ void fwd_build_w(FwdSmem& sm, int j0, int kbeg, int klen, int ksteps,
                                            float (&dacc)[4], const DenParams* __restrict__ drec,
                                            const int* __restrict__ sorted_gauss, uint32_t row_bytes,
                                            uint32_t zero_off, int x0, int y0, int z0,
                                            const float (&cz)[4], float cxl, float cyl) {
    const int nslots = ksteps * 16;
    for (int k = threadIdx.x; k < nslots; k += kFwdThreads) {
        if (k < klen) {
            const int g = sorted_gauss[j0 + kbeg + k];
            sm.rec[k] = fwd_record_packed(drec[g], x0, y0, z0);   // one 64-byte gather
            sm.roff[k] = (uint32_t)g * row_bytes;
        } else {
            sm.rec[k] = fwd_record_empty();
            sm.roff[k] = zero_off;
        }
    }
    __syncthreads();
    const int col = threadIdx.x & 15;
    const int noct = ksteps * 2;
    for (int o = threadIdx.x >> 4; o < noct; o += kFwdThreads / 16) {
        float wv[4][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float w[4];
            fwd_column_weights(&sm.rec[o * 8 + i], col, cxl, cyl, cz, w);   // 16 lanes each
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dacc[c] += w[c];
                wv[c][i] = fmaxf(w[c], 0.0f);   // feature gate of the reference (.cu:936)
            }
        }
        // voxel (a, b, c) of the tile is row 16a + 4b + c of W: block a/2, row 16(a%2) + 4b + c
        const int s = o >> 1, mb = col >> 3;
        const int slot = (o & 1) * 32 + (col & 7) * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            bf16x8 h, l;
            split8(wv[c], h, l);
            sm.whi[s][mb][slot + c] = h;
            sm.wlo[s][mb][slot + c] = l;
        }
    }
}

// Density and features of a tile that no Gaussian touches: zero (the general path forms the same
// zeros and stores them from one wave per 128 channels).  Every wave of the workgroup stores whole
// columns (x, y): a column's voxel rows z0 .. z0 + nz - 1 are one contiguous run.
template <bool OBF16>
__device__ __forceinline__ void fwd_zero_tile(const Grid& G, int tile, int C, float* __restrict__ density,
                                                        void* __restrict__ grid_feats_out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);
    if (threadIdx.x < 64 && in_grid(G, x, y, z)) density[voxel_index(G, x, y, z)] = 0.0f;
    const int x0 = x & ~(kTile - 1), y0 = y & ~(kTile - 1), z0 = z & ~(kTile - 1);
    constexpr int kEs = OBF16 ? 2 : 4;
    const int64_t run = (int64_t)min(kTile, G.dims[2] - z0) * C * kEs;   // bytes of a column
    for (int c = wave; c < kTile * kTile; c += kFwdWaves) {
        const int xc = x0 + (c >> 2), yc = y0 + (c & 3);
        if (xc >= G.dims[0] || yc >= G.dims[1]) continue;   // wave-uniform
        char* dst = static_cast<char*>(grid_feats_out) + voxel_index(G, xc, yc, z0) * C * kEs;
        if (((uintptr_t)dst & 15) == 0 && (run & 15) == 0) {
            for (int64_t b = (int64_t)lane * 16; b < run; b += 64 * 16)
                __builtin_nontemporal_store(f32x4{0.0f, 0.0f, 0.0f, 0.0f}, reinterpret_cast<f32x4*>(dst + b));
        } else {
            for (int64_t b = (int64_t)lane * kEs; b < run; b += 64 * kEs) {
                if constexpr (OBF16) *reinterpret_cast<unsigned short*>(dst + b) = 0;
                else *reinterpret_cast<float*>(dst + b) = 0.0f;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Tiles whose list holds at most smax <= kFsMax Gaussians, empty ones included.  k_fwd_feats keeps two
// tiles per CU (its LDS holds a 224-Gaussian K chunk), so a short list leaves that tile's chain of
// loads and barriers bare; here a 4-wave workgroup with about 10 KB of LDS takes the tile and many
// run per CU.  The weights are those of fwd_build_w (the same operations), the density their sum
// (in another order), the features float32 sums of max(w, 0) f over the list in its order, read
// straight from the caller's features.  Which kernel takes a tile depends on its list length
// alone.
// ------------------------------------------------------------------------------------------
constexpr int kFsThreads = 256;
constexpr int kFsMax = 64;          // longest list the kernel can take
constexpr int kFsStride = kFsMax + 4;   // weight row of a voxel: 16-byte aligned, few bank conflicts

struct FsSmem {
    alignas(16) float w[64][kFsStride];   // feature weights max(w, 0): [voxel row][slot]
    float dpart[kFsThreads / 64][64];
    float inv[64];
    int vlin[64];
    int gid[kFsMax];
};

template <bool OBF16>
__global__ void __launch_bounds__(kFsThreads) k_fwd_short(
    Grid G, int C, const float* __restrict__ means, const float* __restrict__ opacity,
    const float* __restrict__ cov_inv, const int* __restrict__ lb, const int* __restrict__ ub,
    const int* __restrict__ toff, const int* __restrict__ sorted_gauss, int M, const void* __restrict__ features,
    float* __restrict__ density, void* __restrict__ grid_feats_out, int smax) {
    __shared__ FsSmem sm;
    const int T = scene_tiles(G);
    const int tb = uniform(xcd_remap(blockIdx.x, gridDim.x));   // the batch's tile (its list)
    if (tb >= T * G.scenes) return;
    const int j0 = uniform(min(max(toff[tb], 0), M));
    const int Ng = uniform(min(max(toff[tb + 1], j0), M)) - j0;
    if (Ng > smax) return;   // k_fwd_feats takes the tile
    const int scene = uniform(tb / T), tile = tb - scene * T;
    {
        const int64_t vb = scene * scene_voxels(G);
        density += vb;
        grid_feats_out = static_cast<char*>(grid_feats_out) + vb * C * (OBF16 ? 2 : 4);
    }
    if (Ng == 0) {   // no Gaussian touches the tile
        fwd_zero_tile<OBF16>(G, tile, C, density, grid_feats_out);
        return;
    }
    typedef typename std::conditional<OBF16, __bf16, float>::type FT;   // element of the features
    const FT* feats = static_cast<const FT*>(features);
    const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);   // voxel row lane of the tile
    const float cx = centre(G, 0, x), cy = centre(G, 1, y), cz = centre(G, 2, z);

    // weights of voxel row lane against slots wave + 4 i (fwd_build_w's operations); every slot's
    // weight is written, 0 past the list
    float dsum = 0.0f;
#pragma unroll 1
    for (int i = 0; i < kFsMax / 4; ++i) {
        const int slot = wave + 4 * i;
        float wf = 0.0f;
        if (slot < Ng) {   // wave-uniform
            const int g = uniform(sorted_gauss[j0 + slot]);
            float A[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) A[k] = cov_inv[g * 9 + k];
            const float a00 = kq * A[0], a01 = kq * (A[1] + A[3]), a11 = kq * A[4];
            const float a02 = kq * (A[2] + A[6]), a12 = kq * (A[5] + A[7]), a22 = kq * A[8];
            const bool inxy = x >= lb[g * 3] && x <= ub[g * 3] && y >= lb[g * 3 + 1] && y <= ub[g * 3 + 1];
            const bool inz = z >= lb[g * 3 + 2] && z <= ub[g * 3 + 2];
            const float dx = cx - means[g * 3], dy = cy - means[g * 3 + 1], dz = cz - means[g * 3 + 2];
            const float fz = inz ? a22 * dz * dz : -__builtin_inff();
            float F = fmaf(fmaf(a00, dx, a01 * dy), dx, a11 * dy * dy);
            F = inxy ? F : -__builtin_inff();
            const float Gxy = fmaf(a02, dx, a12 * dy);
            const float w = opacity[g] * __builtin_amdgcn_exp2f(fmaf(Gxy, dz, F) + fz);
            dsum += w;
            wf = fmaxf(w, 0.0f);   // feature gate of the reference (.cu:936)
            if (lane == 0) sm.gid[slot] = g;
        }
        sm.w[lane][slot] = wf;
    }
    sm.dpart[wave][lane] = dsum;
    __syncthreads();
    if (wave == 0) {
        const float D = ((sm.dpart[0][lane] + sm.dpart[1][lane]) + sm.dpart[2][lane]) + sm.dpart[3][lane];
        const bool ok = in_grid(G, x, y, z);
        const int v = ok ? (int)voxel_index(G, x, y, z) : -1;
        sm.inv[lane] = 1.0f / fmaxf(D, kEps);
        sm.vlin[lane] = v;
        if (ok) density[v] = D;
    }
    __syncthreads();

    // features: wave w owns voxel rows 16 w .. 16 w + 15, lane = channel of a 64-channel block;
    // the list is taken 8 slots at a time (slots past it have weight 0 and read as 0)
    for (int cb = 0; cb < C; cb += 64) {
        const int c = cb + lane;
        const int cc = min(c, C - 1);
        float acc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        for (int s0 = 0; s0 < Ng; s0 += 8) {
            float f[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {   // every load issued before the first product
                const int sl = s0 + k;
                const int g = uniform(sm.gid[min(sl, Ng - 1)]);   // a uniform row base: one offset register for all
                f[k] = sl < Ng ? (float)feats[(int64_t)g * C + cc] : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float* wr = &sm.w[16 * wave + r][s0];
                const float4 wa = *reinterpret_cast<const float4*>(wr);
                const float4 wb = *reinterpret_cast<const float4*>(wr + 4);
                acc[r] = fmaf(wa.x, f[0], acc[r]);
                acc[r] = fmaf(wa.y, f[1], acc[r]);
                acc[r] = fmaf(wa.z, f[2], acc[r]);
                acc[r] = fmaf(wa.w, f[3], acc[r]);
                acc[r] = fmaf(wb.x, f[4], acc[r]);
                acc[r] = fmaf(wb.y, f[5], acc[r]);
                acc[r] = fmaf(wb.z, f[6], acc[r]);
                acc[r] = fmaf(wb.w, f[7], acc[r]);
            }
        }
        if (c < C) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 16 * wave + r;
                const int v = sm.vlin[row];
                if (v < 0) continue;
                const float o = acc[r] * sm.inv[row];
                if constexpr (OBF16) static_cast<__bf16*>(grid_feats_out)[(int64_t)v * C + c] = (__bf16)o;
                else __builtin_nontemporal_store(o, static_cast<float*>(grid_feats_out) + (int64_t)v * C + c);
            }
        }
    }
}

// OBF16: grid_feats is stored as bfloat16 (rounded to nearest even), else float.
template <bool OBF16>
__global__ void __launch_bounds__(kFwdThreads, 2) k_fwd_feats(
    Grid G, int C, const DenParams* __restrict__ drec, const int* __restrict__ toff,
    const int* __restrict__ sorted_gauss, int M, int n, int Cp,
    const uint32_t* __restrict__ fpk, float* __restrict__ density,
    void* __restrict__ grid_feats_out, int skip_le, const int* __restrict__ tlist, const int* __restrict__ tcount) {
    __shared__ FwdSmem sm;
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
    {
        const int64_t vb = scene * scene_voxels(G);
        density += vb;
        grid_feats_out = static_cast<char*>(grid_feats_out) + vb * C * (OBF16 ? 2 : 4);
    }
    const int j0 = uniform(min(max(toff[tb], 0), M));
    const int Ng = uniform(min(max(toff[tb + 1], j0), M)) - j0;
    if (Ng <= skip_le) return;   // k_fwd_short takes the tile
    if (Ng == 0) {   // no Gaussian touches the tile
        fwd_zero_tile<OBF16>(G, tile, C, density, grid_feats_out);
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int jl = lane & 31, kh = lane >> 5;

    int x, y, z;
    tile_voxel(G, tile, lane, x, y, z);
    if (wave == 0) sm.vlin[lane] = in_grid(G, x, y, z) ? (int)voxel_index(G, x, y, z) : -1;
    // the tile's first voxel, the z centres of its four layers and the centre of this thread's
    // W-build column (x0 + col/4, y0 + col%4)
    const int x0 = x & ~(kTile - 1), y0 = y & ~(kTile - 1), z0 = z & ~(kTile - 1);
    const float cz[4] = {centre(G, 2, z0), centre(G, 2, z0 + 1), centre(G, 2, z0 + 2), centre(G, 2, z0 + 3)};
    const int col = threadIdx.x & 15;
    const float cxl = centre(G, 0, x0 + (col >> 2)), cyl = centre(G, 1, y0 + (col & 3));

    const int nkc = (Ng + kFwdKMax - 1) / kFwdKMax;
    constexpr uint32_t kCh = OBF16 ? 2u : 4u;   // packed bytes per channel
    const uint32_t row_bytes = (uint32_t)Cp * kCh;
    const uint32_t zero_off = (uint32_t)n * row_bytes;
    const char* fbase = reinterpret_cast<const char*>(fpk);
    float dacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // density of the column's voxels, this thread's octets

    // packed quads of K step ks: rows of slots ks*16 + 8*kh + i, channels (lane offset lo)..+3
    typedef typename std::conditional<OBF16, uint2, uint4>::type Quad;   // 4 packed channels
    auto gather = [&](int ks, uint32_t lo, Quad (&u)[8]) {
        const uint32_t* rp = &sm.roff[ks * 16 + kh * 8];
        const uint4 ra = *reinterpret_cast<const uint4*>(rp);
        const uint4 rb = *reinterpret_cast<const uint4*>(rp + 4);
        const uint32_t rs[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = *reinterpret_cast<const Quad*>(fbase + (size_t)(rs[i] + lo));
    };
    // The first gather of a pass whose K chunk is already in LDS (one chunk: the weights stay for
    // every pass) is issued before the previous pass's stores: loads and stores share one in-order
    // counter, so a gather issued after the stores would wait for every store to complete.
    Quad qa[8], qb[8];
    bool qa_ready = false;

    for (int cbase = 0; cbase < C; cbase += kFwdChanPerPass) {
        const int cw0 = cbase + wave * kFwdChanPerWave;          // first channel of this wave
        const bool has_ch = cw0 < C;                               // wave-uniform
        const uint32_t lane_off = (uint32_t)(cw0 + 4 * jl) * kCh;  // byte offset of the lane's quad
        f32x16 acc[2][4];
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[vb][cb] = f32x16{};

        for (int kc = 0; kc < nkc; ++kc) {
            const int kbeg = kc * kFwdKMax;
            const int klen = min(kFwdKMax, Ng - kbeg);
            const int ksteps = ((klen + 31) >> 5) * 2;   // even: the MFMA loop takes steps in pairs
            if (nkc > 1 || cbase == 0) {
                __syncthreads();  // previous readers of W are done
                fwd_build_w(sm, j0, kbeg, klen, ksteps, dacc, drec, sorted_gauss, row_bytes, zero_off, x0, y0, z0,
                            cz, cxl, cyl);
                __syncthreads();
            }
            if (has_ch) {
                auto step = [&](int ks, const Quad (&u)[8]) {
                    const bf16x8 ah0 = sm.whi[ks][0][lane], al0 = sm.wlo[ks][0][lane];
                    const bf16x8 ah1 = sm.whi[ks][1][lane], al1 = sm.wlo[ks][1][lane];
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        bf16x8 bh, bl;
                        if constexpr (OBF16) {
                            // channel cb of rows 2j and 2j+1: half cb&1 of word cb/2 of each row
                            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                            u32x4 hv;
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const uint32_t w0 = cb < 2 ? u[2 * j].x : u[2 * j].y;
                                const uint32_t w1 = cb < 2 ? u[2 * j + 1].x : u[2 * j + 1].y;
                                hv[j] = __builtin_amdgcn_perm(w1, w0, (cb & 1) ? 0x07060302u : 0x05040100u);
                            }
                            bh = __builtin_bit_cast(bf16x8, hv);
                            bl = bf16x8{};   // zero low part: its MFMA term is left out
                        } else {
                            uint32_t q[8];
#pragma unroll
                            for (int i = 0; i < 8; ++i) q[i] = u[i][cb];
                            unpack8(q, bh, bl);
                        }
                        // bfloat16 features split into themselves and a zero low part
                        acc[0][cb] = mfma_split_32x32x16<false, OBF16>(ah0, al0, bh, bl, acc[0][cb]);
                        acc[1][cb] = mfma_split_32x32x16<false, OBF16>(ah1, al1, bh, bl, acc[1][cb]);
                    }
                };
                // loads and steps are unconditional (ksteps is even, the prefetch index is
                // clamped) so the next step's gather stays in flight across this step's MFMAs;
                // the scheduling barriers keep the compiler from sinking the gathers to their use
                const int klast = ksteps - 1;
                if (ksteps > 0) {
                    if (!qa_ready) gather(0, lane_off, qa);
                    for (int ks = 0; ks < ksteps; ks += 2) {
                        gather(ks + 1, lane_off, qb);
                        __builtin_amdgcn_sched_barrier(0);
                        step(ks, qa);
                        __builtin_amdgcn_sched_barrier(0);
                        gather(min(ks + 2, klast), lane_off, qa);
                        __builtin_amdgcn_sched_barrier(0);
                        step(ks + 1, qb);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            qa_ready = false;
        }

        if (cbase == 0) {
            // the 16 threads of a column: four per wave (lanes col, col + 16, col + 32, col + 48)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dacc[c] += __shfl_xor(dacc[c], 16);
                dacc[c] += __shfl_xor(dacc[c], 32);
            }
            int ln = lane;   // opaque, as in the epilogue below
            asm volatile("" : "+v"(ln));
            if (ln < 16)
                *reinterpret_cast<float4*>(&sm.dpart[wave][4 * ln]) = make_float4(dacc[0], dacc[1], dacc[2], dacc[3]);
            __syncthreads();
            if (wave == 0) {
                float D = 0.0f;
#pragma unroll
                for (int w = 0; w < kFwdWaves; ++w) D += sm.dpart[w][ln];
                sm.inv_den[lane] = 1.0f / fmaxf(D, kEps);
                if (sm.vlin[lane] >= 0) density[sm.vlin[lane]] = D;
            }
            __syncthreads();
        }

        {
            const int nb = cbase + kFwdChanPerPass;   // the next pass, when its weights stay in LDS
            if (nkc == 1 && Ng > 0 && nb + wave * kFwdChanPerWave < C) {
                gather(0, (uint32_t)(nb + wave * kFwdChanPerWave + 4 * jl) * kCh, qa);
                qa_ready = true;
            }
        }
        // epilogue: D row of element i = 8*(i/4) + 4*kh + i%4 (voxel), column jl -> channels
        // cw0 + 4*jl + cb for channel block cb
        if (has_ch) {
            const int c0 = cw0 + 4 * jl;
            // the lane's row offset, opaque to the compiler: the LDS addresses below are then formed
            // here, from one base and immediate offsets, instead of being hoisted out of the channel
            // pass loop and kept in registers (which spilled, and each reload waited for every
            // outstanding store)
            int khr = 4 * kh;
            asm volatile("" : "+v"(khr));
#pragma unroll
            for (int vb = 0; vb < 2; ++vb) {
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int r0 = vb * 32 + 8 * qd + khr;
                    const int4 vl = *reinterpret_cast<const int4*>(&sm.vlin[r0]);
                    const float4 iv = *reinterpret_cast<const float4*>(&sm.inv_den[r0]);
                    const int vs[4] = {vl.x, vl.y, vl.z, vl.w};
                    const float is[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int e = qd * 4 + ii;
                        const float4 v = make_float4(acc[vb][0][e] * is[ii], acc[vb][1][e] * is[ii],
                                                     acc[vb][2][e] * is[ii], acc[vb][3][e] * is[ii]);
                        if (vs[ii] < 0) continue;
                        if constexpr (OBF16) {
                            __bf16* dst = static_cast<__bf16*>(grid_feats_out) + (int64_t)vs[ii] * C + c0;
                            if ((C & 3) == 0) {
                                if (c0 < C) {
                                    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                                    const bf16x4 hv = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
                                    *reinterpret_cast<bf16x4*>(dst) = hv;
                                }
                            } else {
                                if (c0 + 0 < C) dst[0] = (__bf16)v.x;
                                if (c0 + 1 < C) dst[1] = (__bf16)v.y;
                                if (c0 + 2 < C) dst[2] = (__bf16)v.z;
                                if (c0 + 3 < C) dst[3] = (__bf16)v.w;
                            }
                            continue;
                        }
                        float* dst = static_cast<float*>(grid_feats_out) + (int64_t)vs[ii] * C + c0;
                        if ((C & 3) == 0) {
                            // written once and not read again by the forward: streaming store
                            if (c0 < C) {
                                const f32x4 nv = {v.x, v.y, v.z, v.w};
                                __builtin_nontemporal_store(nv, reinterpret_cast<f32x4*>(dst));
                            }
                        } else {
                            if (c0 + 0 < C) dst[0] = v.x;
                            if (c0 + 1 < C) dst[1] = v.y;
                            if (c0 + 2 < C) dst[2] = v.z;
                            if (c0 + 3 < C) dst[3] = v.w;
                        }
                    }
                }
            }
        }
    }
}

hipError_t launch_split_pack(int n, int C, const void* features, int fdt, uint32_t* fpk, hipStream_t s) {
    if (C <= 0 || n < 0) return hipSuccess;
    const int Cp = packed_channels(C);
    const int64_t count = (int64_t)(n + 1) * Cp;
    if (count * 4 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;   // byte offsets are 32-bit
    const unsigned pblocks = (unsigned)ceil_div(count / 4, 256);
    if (fdt == kDtBF16)
        G2V_LAUNCH(k_split_pack<__bf16>, dim3(pblocks), dim3(256), 0, s, static_cast<const __bf16*>(features), n, C,
                   Cp, fpk);
    else
        G2V_LAUNCH(k_split_pack<float>, dim3(pblocks), dim3(256), 0, s, static_cast<const float*>(features), n, C,
                   Cp, fpk);
    return hipGetLastError();
}

hipError_t launch_forward_feats(const Grid& G, int C, const float* means, const float* opacity,
                                const float* cov_inv, const int* lb, const int* ub,
                                const int* tile_offsets, const int* sorted_gauss, int M, int n,
                                const void* features, int fdt, const uint32_t* fpk, const DenParams* drec,
                                float* density, void* grid_feats, int* tl_ws, hipStream_t s) {
    const int T = scene_tiles(G) * G.scenes;
    if (T <= 0) return hipSuccess;
    if (C <= 0) return hipErrorInvalidValue;   // density only: launch_forward_density
    if (M > 0 && !drec) return hipErrorInvalidValue;
    const int Cp = packed_channels(C);
    if ((int64_t)(n + 1) * Cp * 4 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;   // byte offsets are 32-bit
    const int blocks = (int)ceil_div(T, 8) * 8;
    // lists of at most short_list_max(C) Gaussians (empty ones included) in k_fwd_short, the others
    // in k_fwd_feats.  When fewer tiles can be long than there are tiles (a sparse problem),
    // k_fwd_feats walks a compacted list of the long ones instead of the whole grid: at one
    // workgroup per CU, a grid of mostly empty workgroups costs tens of microseconds.
    const int smax = min(short_list_max(C), kFsMax);
    const int nlong = long_tiles_bound(M, T, smax);
    const int* tlist = nullptr;
    const int* tcount = nullptr;
    if (nlong < T && nlong > 0) {
        const hipError_t e = launch_long_tiles(tile_offsets, T, M, smax, tl_ws, tl_ws + 1, nlong, s);
        if (e != hipSuccess) return e;
        tcount = tl_ws;
        tlist = tl_ws + 1;
    }
    const int lblocks = (int)ceil_div(nlong, 8) * 8;
    if (fdt == kDtBF16) {
        G2V_LAUNCH(k_fwd_short<true>, dim3(blocks), dim3(kFsThreads), 0, s, G, C, means, opacity, cov_inv, lb, ub,
                   tile_offsets, sorted_gauss, M, features, density, grid_feats, smax);
        if (nlong > 0)
            G2V_LAUNCH(k_fwd_feats<true>, dim3(lblocks), dim3(kFwdThreads), 0, s, G, C, drec, tile_offsets,
                       sorted_gauss, M, n, Cp, (const uint32_t*)fpk, density, grid_feats, smax, tlist, tcount);
    } else {
        G2V_LAUNCH(k_fwd_short<false>, dim3(blocks), dim3(kFsThreads), 0, s, G, C, means, opacity, cov_inv, lb, ub,
                   tile_offsets, sorted_gauss, M, features, density, grid_feats, smax);
        if (nlong > 0)
            G2V_LAUNCH(k_fwd_feats<false>, dim3(lblocks), dim3(kFwdThreads), 0, s, G, C, drec, tile_offsets,
                       sorted_gauss, M, n, Cp, (const uint32_t*)fpk, density, grid_feats, smax, tlist, tcount);
    }
    return hipGetLastError();
}

}  // namespace g2v
