// Gaussian->Tile and Tile->Gaussian CSR build for gfx950.
//
//   k_boxes          per-Gaussian 3-sigma box, tile box, inverse covariance
//                    (reference src/cuda_gaussian_voxelizer.cu:348-536, :201-220)
//   scan_i32         device-wide scan (replaces cub::DeviceScan, reference .cu:1605-1615, :1758-1772)
//   k_fill_g2t       row-major G->T rows (reference .cu:228-286)
//   radix_sort_pairs stable LSD radix sort over only ceil(log2 T) key bits
//                    (replaces cub::DeviceRadixSort::SortPairs over 32 bits, reference .cu:1673-1691)
//   k_tile_offsets   run boundaries of the sorted tile ids for every tile, empty ones included
//                    (replaces cub::DeviceRunLengthEncode + scan, reference .cu:1708-1772)
//   k_rle_*          unique tiles / run lengths / run offsets / number of runs
#include "g2v_internal.h"

namespace g2v {

// ------------------------------------------------------------------------------------------
// Boxes
// ------------------------------------------------------------------------------------------

// float -> int32 the way the hardware converts (saturating, NaN -> 0), written out so the
// compiler cannot treat an out-of-range conversion as undefined.
__device__ __forceinline__ int cvt_sat(float f) {
    if (!(f == f)) return 0;
    if (f >= 2147483648.0f) return 2147483647;
    if (f < -2147483648.0f) return (int)0x80000000;
    return (int)f;
}

// With cell_offsets, also the number of cells of cx x cy x cz voxels that the box meets, at
// cell_offsets[g+1] (cell_offsets[0] = 0), as k_cell_count computes it from the box.  zero[0 ..
// nzero) is cleared (counts that no scan of this launch sequence writes).
__global__ void __launch_bounds__(256) k_boxes(Grid G, int n, const float* __restrict__ means,
                                               const float* __restrict__ cov,
                                               float* __restrict__ cov_inv, int* __restrict__ lb,
                                               int* __restrict__ ub, int* __restrict__ nvox,
                                               int* __restrict__ g2t_offsets, int cx, int cy, int cz,
                                               int* __restrict__ cell_offsets, long long* __restrict__ zero,
                                               int nzero) {
#pragma clang fp contract(off)
    const int g = blockIdx.x * 256 + threadIdx.x;
    if (g == 0) {
        g2t_offsets[0] = 0;
        if (cell_offsets) cell_offsets[0] = 0;
    }
    if (g < nzero) zero[g] = 0;
    if (g >= n) return;
    int lo[3], hi[3];
    bool empty = false;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float sig = sqrtf(cov[g * 9 + 4 * a]);
        const float ts = 3.0f * sig;
        const float m = means[g * 3 + a];
        float lower = m - ts;
        float upper = m + ts;
        lower = fmaxf(lower, G.r0[a]);
        upper = fminf(upper, G.r1[a]);
        const float ql = (lower - G.r0[a]) / G.s[a];
        const float qh = (upper - G.r0[a]) / G.s[a];
        lo[a] = max(cvt_sat(floorf(ql)), 0);
        hi[a] = min(cvt_sat(floorf(qh)), G.dims[a] - 1);
        empty |= lo[a] > hi[a];
    }
    if (empty) {
#pragma unroll
        for (int a = 0; a < 3; ++a) { lb[g * 3 + a] = 0; ub[g * 3 + a] = -1; }
        nvox[g] = 0;
        g2t_offsets[g + 1] = 0;
        if (cell_offsets) cell_offsets[g + 1] = 0;
#pragma unroll
        for (int k = 0; k < 9; ++k) cov_inv[g * 9 + k] = 0.0f;
        return;
    }
    int nv = 1, nt = 1;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        lb[g * 3 + a] = lo[a];
        ub[g * 3 + a] = hi[a];
        nv *= hi[a] - lo[a] + 1;
        const int tl = max(lo[a] / kTile, 0);
        const int th = min(hi[a] / kTile, G.tiles[a] - 1);
        nt *= th - tl + 1;
    }
    nvox[g] = nv;
    g2t_offsets[g + 1] = nt;
    if (cell_offsets)
        cell_offsets[g + 1] = (hi[0] / cx - lo[0] / cx + 1) * (hi[1] / cy - lo[1] / cy + 1) * (hi[2] / cz - lo[2] / cz + 1);

    float A[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) A[k] = cov[g * 9 + k];
    float det = A[0] * (A[4] * A[8] - A[5] * A[7]) - A[1] * (A[3] * A[8] - A[5] * A[6]) +
                A[2] * (A[3] * A[7] - A[4] * A[6]);
    if (fabsf(det) < 1e-6f) det = 1e-6f;
    const float inv_det = 1.0f / det;
    float* o = cov_inv + g * 9;
    o[0] = (A[4] * A[8] - A[5] * A[7]) * inv_det;
    o[1] = -(A[1] * A[8] - A[2] * A[7]) * inv_det;
    o[2] = (A[1] * A[5] - A[2] * A[4]) * inv_det;
    o[3] = -(A[3] * A[8] - A[5] * A[6]) * inv_det;
    o[4] = (A[0] * A[8] - A[2] * A[6]) * inv_det;
    o[5] = -(A[0] * A[5] - A[2] * A[3]) * inv_det;
    o[6] = (A[3] * A[7] - A[4] * A[6]) * inv_det;
    o[7] = -(A[0] * A[7] - A[1] * A[6]) * inv_det;
    o[8] = (A[0] * A[4] - A[1] * A[3]) * inv_det;
}

hipError_t launch_boxes(const Grid& G, int n, const float* means, const float* cov, float* cov_inv,
                        int* lb, int* ub, int* nvox, int* g2t_offsets, const int* cell, int* cell_offsets,
                        hipStream_t s, long long* zero, int nzero) {
    const int blocks = (int)ceil_div(n > 0 ? n : 1, 256);
    const int cx = cell ? cell[0] : 1, cy = cell ? cell[1] : 1, cz = cell ? cell[2] : 1;
    G2V_LAUNCH(k_boxes, dim3(blocks), dim3(256), 0, s, G, n, means, cov, cov_inv, lb, ub,
                       nvox, g2t_offsets, cx, cy, cz, cell ? cell_offsets : nullptr, zero, zero ? nzero : 0);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Device-wide scan: per-tile reduce -> per-tile scan with carry-in (each tile sums the totals before it).
// ------------------------------------------------------------------------------------------

// Inclusive scan of one value per thread over the block (256 threads = 4 waves).
__device__ __forceinline__ long long block_incl_scan(long long v, long long* sh /*[4]*/, long long& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const long long t = __shfl_up(v, off, 64);
        if (lane >= off) v += t;
    }
    if (lane == 63) sh[wave] = v;
    __syncthreads();
    long long carry = 0;
    for (int w = 0; w < wave; ++w) carry += sh[w];
    total = sh[0] + sh[1] + sh[2] + sh[3];
    __syncthreads();
    return v + carry;
}

__global__ void __launch_bounds__(kScanThreads) k_scan_reduce(const int* __restrict__ in, int64_t n,
                                                              long long* __restrict__ partials) {
    __shared__ long long sh[4];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    // every load is issued (clamped into the array) before any is used: a load under its own
    // bounds branch would be followed by a wait of its own
    int v[kScanItems];
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) v[r] = in[min(base + (int64_t)r * kScanThreads + threadIdx.x, n - 1)];
    long long sum = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) sum += (base + (int64_t)r * kScanThreads + threadIdx.x < n) ? v[r] : 0;
    long long total;
    block_incl_scan(sum, sh, total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Each block forms its own prefix, the sum of the tile totals before it (a block-wide sum over at most
// a few thousand values), so that no kernel scans the totals between the reduce and the apply; the
// last block also writes the grand total.
__global__ void __launch_bounds__(kScanThreads) k_scan_apply(const int* in, int* out, int64_t n,
                                                             const long long* __restrict__ partials,
                                                             int inclusive, long long* __restrict__ total_dev) {
    __shared__ long long sh[4];
    long long pre = 0;
    for (int64_t j = threadIdx.x; j < (int64_t)blockIdx.x; j += kScanThreads) pre += partials[j];
    long long ptot;
    block_incl_scan(pre, sh, ptot);   // ptot: the sum of the totals before this block
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int v[kScanItems];
    long long local = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) v[r] = in[min(base + r, n - 1)];   // clamped: no per-load branch
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        v[r] = base + r < n ? v[r] : 0;
        local += v[r];
    }
    long long total;
    const long long inc = block_incl_scan(local, sh, total);
    long long run = ptot + inc - local;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        const int64_t i = base + r;
        const long long nxt = run + v[r];
        if (i < n) out[i] = (int)(inclusive ? nxt : run);
        run = nxt;
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0 && total_dev) *total_dev = ptot + total;
}

// Single-workgroup scan for inputs up to kScanSingleMax (two tiles: beyond that the two-kernel
// scan, whose reduce and apply kernels spread over the whole chip, is faster; a tile takes one
// workgroup about 5 us).  Tiles of 1024 x 32 values: coalesced
// loads into LDS (row of 32 values per thread, padded to 33 words), a sequential scan of each
// thread's row, a workgroup scan of the row totals, and coalesced stores back from LDS; a
// running carry joins the tiles.  In-place safe (a tile is read completely before it is written).
constexpr int kScan1Threads = 1024;
constexpr int kScan1Items = 32;
constexpr int kScan1Row = kScan1Items + 1;
constexpr int64_t kScanSingleMax = int64_t(2) * kScan1Threads * kScan1Items;

struct ScanJob {
    const int* in;
    int* out;
    int n;
    int inclusive;
    long long* total;
};

// Workgroup j scans job j (one or two jobs per launch).
__global__ void __launch_bounds__(kScan1Threads) k_scan_single(ScanJob j0, ScanJob j1) {
    const ScanJob& job = blockIdx.x == 0 ? j0 : j1;
    const int* in = job.in;
    int* out = job.out;
    const int n = job.n;
    const int inclusive = job.inclusive;
    long long* total_dev = job.total;
    __shared__ int buf[kScan1Threads * kScan1Row];
    __shared__ long long wsum[kScan1Threads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kTile = kScan1Threads * kScan1Items;
    long long carry = 0;
    for (int base = 0; base < n; base += kTile) {
        // coalesced load: value e of the tile -> row e / 32, column e % 32
        // all loads issued first (indices clamped into the array), then the masked LDS stores:
        // a load under its own bounds branch would be followed by a wait of its own
        int ld[kScan1Items];
#pragma unroll
        for (int k = 0; k < kScan1Items; ++k) ld[k] = in[min(base + k * kScan1Threads + (int)threadIdx.x, n - 1)];
#pragma unroll
        for (int k = 0; k < kScan1Items; ++k) {
            const int e = k * kScan1Threads + threadIdx.x;
            buf[(e / kScan1Items) * kScan1Row + e % kScan1Items] = (base + e < n) ? ld[k] : 0;
        }
        lds_barrier();
        int* row = &buf[threadIdx.x * kScan1Row];
        long long local = 0;
#pragma unroll
        for (int r = 0; r < kScan1Items; ++r) local += row[r];
        long long x = local;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const long long t = __shfl_up(x, off, 64);
            if (lane >= off) x += t;
        }
        if (lane == 63) wsum[wave] = x;
        lds_barrier();
        long long wcarry = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < kScan1Threads / 64; ++w) {
            const long long sw = wsum[w];
            wcarry += (w < wave) ? sw : 0;
            tot += sw;
        }
        long long run = carry + wcarry + x - local;
#pragma unroll
        for (int r = 0; r < kScan1Items; ++r) {
            const long long nxt = run + row[r];
            row[r] = (int)(inclusive ? nxt : run);
            run = nxt;
        }
        lds_barrier();
#pragma unroll
        for (int k = 0; k < kScan1Items; ++k) {
            const int e = k * kScan1Threads + threadIdx.x;
            if (base + e < n) out[base + e] = buf[(e / kScan1Items) * kScan1Row + e % kScan1Items];
        }
        lds_barrier();   // buf and wsum are rewritten by the next tile
        carry += tot;
    }
    if (threadIdx.x == 0 && total_dev) *total_dev = carry;
}

size_t scan_workspace(int64_t n) {
    return (size_t)(ceil_div(n > 0 ? n : 1, kScanTile) + 1) * sizeof(long long) + 256;
}

hipError_t scan_i32(const int* in, int* out, int64_t n, bool inclusive, long long* total_dev,
                    void* ws, hipStream_t s) {
    if (n <= kScanSingleMax) {
        const ScanJob j{in, out, (int)n, inclusive ? 1 : 0, total_dev};
        G2V_LAUNCH(k_scan_single, dim3(1), dim3(kScan1Threads), 0, s, j, j);
        return hipGetLastError();
    }
    const int64_t nb = ceil_div(n > 0 ? n : 1, kScanTile);
    long long* partials = static_cast<long long*>(ws);
    G2V_LAUNCH(k_scan_reduce, dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, n, partials);
    G2V_LAUNCH(k_scan_apply, dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, out, n,
               (const long long*)partials, inclusive ? 1 : 0, total_dev);
    return hipGetLastError();
}

hipError_t scan_i32_pair(const int* in_a, int* out_a, int64_t n_a, long long* total_a, void* ws_a,
                         const int* in_b, int* out_b, int64_t n_b, long long* total_b, void* ws_b,
                         hipStream_t s) {
    if (n_a > 0 && n_b > 0 && n_a <= kScanSingleMax && n_b <= kScanSingleMax) {
        const ScanJob a{in_a, out_a, (int)n_a, 1, total_a}, b{in_b, out_b, (int)n_b, 1, total_b};
        G2V_LAUNCH(k_scan_single, dim3(2), dim3(kScan1Threads), 0, s, a, b);
        return hipGetLastError();
    }
    if (n_a > 0) {
        const hipError_t e = scan_i32(in_a, out_a, n_a, true, total_a, ws_a, s);
        if (e != hipSuccess) return e;
    }
    if (n_b > 0) return scan_i32(in_b, out_b, n_b, true, total_b, ws_b, s);
    return hipSuccess;
}

// ------------------------------------------------------------------------------------------
// G->T fill: one wave per Gaussian enumerates its tile box row-major (x slowest, z fastest).
// tile_ids may be null (only the Gaussian id of every pair is regenerated).
// ------------------------------------------------------------------------------------------
// 16 lanes per Gaussian (16 Gaussians per workgroup): a Gaussian touches about 25 to 360 tiles.
// Entry i of a row is tile box position (lx, ly, lz) = the digits of i in radix (dy, dz); a lane
// visits i = l, l + 16, ... and steps its position by the digits of 16 (at most one carry per
// digit) instead of dividing at every entry.
// keys (optional, batches): the batch's tile id of every entry (scene b T + tile), the sort key;
// tile_ids keeps the scene-local ids.
constexpr int kFillLanes = 16;

__global__ void __launch_bounds__(256) k_fill_g2t(Grid G, int n, const int* __restrict__ lb,
                                                  const int* __restrict__ ub,
                                                  const int* __restrict__ g2t_offsets,
                                                  int* __restrict__ tile_ids,
                                                  int* __restrict__ gauss_ids,
                                                  int* __restrict__ keys,
                                                  const float* __restrict__ means,
                                                  const float* __restrict__ opacity,
                                                  const float* __restrict__ cov_inv,
                                                  DenParams* __restrict__ drec) {
    const int l = threadIdx.x & (kFillLanes - 1);
    const int g = blockIdx.x * (256 / kFillLanes) + threadIdx.x / kFillLanes;
    if (g >= n) return;
    const int base = g2t_offsets[g];
    const int cnt = g2t_offsets[g + 1] - base;
    if (cnt <= 0) return;
    if (drec) {   // the Gaussian's packed record, one 32-bit word per lane (only listed Gaussians are read)
        static_assert(kFillLanes == 16, "one lane per word of DenParams");
        uint32_t w;
        if (l < 3) {
            w = __float_as_uint(means[g * 3 + l]);
        } else if (l == 3) {
            w = __float_as_uint(opacity[g]);
        } else if (l < 10) {   // a00 a01 a11 a02 a12 a22: kq (A[i0] + A[i1]) off the diagonal
            const int k = l - 4;
            const int i0 = k == 0 ? 0 : k == 1 ? 1 : k == 2 ? 4 : k == 3 ? 2 : k == 4 ? 5 : 8;
            const int i1 = k == 1 ? 3 : k == 3 ? 6 : k == 4 ? 7 : -1;
            const float* A = cov_inv + g * 9;
            w = __float_as_uint(i1 >= 0 ? kq * (A[i0] + A[i1]) : kq * A[i0]);
        } else if (l < 13) {
            w = (uint32_t)lb[g * 3 + l - 10];
        } else {
            w = (uint32_t)ub[g * 3 + l - 13];
        }
        reinterpret_cast<uint32_t*>(drec)[(size_t)g * 16 + l] = w;
    }
    const int tx0 = lb[g * 3] / kTile, ty0 = lb[g * 3 + 1] / kTile, tz0 = lb[g * 3 + 2] / kTile;
    const int dy = ub[g * 3 + 1] / kTile - ty0 + 1;
    const int dz = ub[g * 3 + 2] / kTile - tz0 + 1;
    const int dyz = dy * dz;
    int lx = l / dyz;
    int ly = (l - lx * dyz) / dz;
    int lz = l - lx * dyz - ly * dz;
    const int sx = kFillLanes / dyz;
    const int sy = (kFillLanes - sx * dyz) / dz;
    const int sz = kFillLanes - sx * dyz - sy * dz;
    const int kb = scene_of(G, g) * scene_tiles(G);
    for (int i = l; i < cnt; i += kFillLanes) {
        const int t = ((tx0 + lx) * G.tiles[1] + (ty0 + ly)) * G.tiles[2] + (tz0 + lz);
        if (tile_ids) tile_ids[base + i] = t;
        if (keys) keys[base + i] = kb + t;
        gauss_ids[base + i] = g;
        lz += sz;
        const int cz = lz >= dz ? 1 : 0;
        lz -= cz * dz;
        ly += sy + cz;
        const int cy = ly >= dy ? 1 : 0;
        ly -= cy * dy;
        lx += sx + cy;
    }
}

hipError_t launch_fill_g2t(const Grid& G, int n, const int* lb, const int* ub,
                           const int* g2t_offsets, int* tile_ids, int* gauss_ids, hipStream_t s, int* keys,
                           const float* means, const float* opacity, const float* cov_inv, DenParams* drec) {
    if (n <= 0) return hipSuccess;
    if (drec && (!means || !opacity || !cov_inv)) return hipErrorInvalidValue;
    G2V_LAUNCH(k_fill_g2t, dim3((unsigned)ceil_div(n, 256 / kFillLanes)), dim3(256), 0, s, G, n, lb, ub,
               g2t_offsets, tile_ids, gauss_ids, keys, means, opacity, cov_inv, drec);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Batches: the per-scene G->T row offsets and pair counts from the batch's offsets.
// out[b (n + 1) + k] = goff[b n + k] - goff[b n] (k = 0..n); counts[b] = goff[(b + 1) n] - goff[b n]
// for b < B and counts[B] = *mr_total (0 without it).
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_scene_offsets(int B, int n, const int* __restrict__ goff,
                                                       const long long* __restrict__ mr_total,
                                                       int* __restrict__ out, long long* __restrict__ counts) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = (int64_t)B * (n + 1);
    if (i < rows) {
        const int64_t b = i / (n + 1), k = i - b * (n + 1);
        out[i] = goff[b * n + k] - goff[b * n];
    }
    if (i < B) counts[i] = (long long)(goff[(i + 1) * n] - goff[i * n]);
    if (i == B) counts[B] = mr_total ? *mr_total : 0;
}

hipError_t launch_scene_offsets(int B, int n, const int* goff, const long long* mr_total, int* out,
                                long long* counts, hipStream_t s) {
    const int64_t items = max((int64_t)B * (n + 1), (int64_t)B + 1);
    G2V_LAUNCH(k_scene_offsets, dim3((unsigned)ceil_div(items, 256)), dim3(256), 0, s, B, n, goff, mr_total, out,
               counts);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Cells: coarser boxes of `cell` voxels per axis (the backward's regions of 2x2xRZ tiles).
// k_cell_count writes each Gaussian's cell count to offsets[g+1] (offsets[0] = 0);
// k_fill_cells enumerates each Gaussian's cell box row-major like k_fill_g2t and also writes
// the pair index of every entry (the value the sort carries).  In a batch (scene_n > 0) the cell
// id of Gaussian g's entries is offset by (g / scene_n) scene_cells.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_cell_count(int n, const int* __restrict__ lb,
                                                    const int* __restrict__ ub, int cx, int cy, int cz,
                                                    int* __restrict__ offsets) {
    const int g = blockIdx.x * 256 + threadIdx.x;
    if (g == 0) offsets[0] = 0;
    if (g >= n) return;
    const int ex = ub[g * 3] / cx - lb[g * 3] / cx + 1;
    const int ey = ub[g * 3 + 1] / cy - lb[g * 3 + 1] / cy + 1;
    const int ez = ub[g * 3 + 2] / cz - lb[g * 3 + 2] / cz + 1;
    const bool empty = ub[g * 3] < lb[g * 3] || ub[g * 3 + 1] < lb[g * 3 + 1] || ub[g * 3 + 2] < lb[g * 3 + 2];
    offsets[g + 1] = empty ? 0 : ex * ey * ez;
}

__global__ void __launch_bounds__(256) k_fill_cells(int n, const int* __restrict__ lb,
                                                    const int* __restrict__ ub,
                                                    const int* __restrict__ offsets, int cx, int cy,
                                                    int cz, int ny, int nz, int* __restrict__ cell_ids,
                                                    int* __restrict__ pair_ids,
                                                    int* __restrict__ gauss_ids, int scene_n, int scene_cells) {
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g >= n) return;
    const int base = offsets[g];
    const int cnt = offsets[g + 1] - base;
    if (cnt <= 0) return;
    const int x0 = lb[g * 3] / cx, y0 = lb[g * 3 + 1] / cy, z0 = lb[g * 3 + 2] / cz;
    const int dy = ub[g * 3 + 1] / cy - y0 + 1;
    const int dz = ub[g * 3 + 2] / cz - z0 + 1;
    const int dyz = dy * dz;
    const int kb = scene_n > 0 ? (g / scene_n) * scene_cells : 0;
    for (int i = lane; i < cnt; i += 64) {
        const int lx = i / dyz, r = i - lx * dyz;
        const int ly = r / dz, lz = r - ly * dz;
        cell_ids[base + i] = kb + ((x0 + lx) * ny + (y0 + ly)) * nz + (z0 + lz);
        pair_ids[base + i] = base + i;
        gauss_ids[base + i] = g;
    }
}

hipError_t launch_cell_count(int n, const int* lb, const int* ub, const int cell[3], int* offsets,
                             hipStream_t s) {
    G2V_LAUNCH(k_cell_count, dim3((unsigned)ceil_div(n > 0 ? n : 1, 256)), dim3(256), 0, s, n, lb, ub,
               cell[0], cell[1], cell[2], offsets);
    return hipGetLastError();
}

hipError_t launch_fill_cells(int n, const int* lb, const int* ub, const int* offsets, const int cell[3],
                             const int ncells[3], int* cell_ids, int* pair_ids, int* gauss_ids,
                             hipStream_t s, int scene_n, int scene_cells) {
    if (n <= 0) return hipSuccess;
    G2V_LAUNCH(k_fill_cells, dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, s, n, lb, ub, offsets, cell[0],
               cell[1], cell[2], ncells[1], ncells[2], cell_ids, pair_ids, gauss_ids, scene_n, scene_cells);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Stable LSD radix sort, digits of <= 8 bits, only ceil(log2 T) key bits.
//   per pass: k_radix_hist (digit counts per 4096-key block, digit-major) -> k_radix_digit_scan
//             (one workgroup per digit: exclusive scan over the blocks, and the digit's total)
//             -> k_radix_scatter (digit bases from the totals; stable rank: ballot match inside a
//             wave, LDS across waves; the block's keys sorted in LDS, then written out run by run)
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kSortThreads) k_radix_hist(const int* __restrict__ keys, int64_t M,
                                                             int shift, int dbits, int nblk,
                                                             int* __restrict__ ghist) {
    __shared__ int h[256];
    const int radix = 1 << dbits;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) h[d] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    int kv[kSortRounds];
#pragma unroll
    for (int r = 0; r < kSortRounds; ++r) kv[r] = keys[min(base + (int64_t)r * kSortThreads + threadIdx.x, M - 1)];
#pragma unroll
    for (int r = 0; r < kSortRounds; ++r)
        if (base + (int64_t)r * kSortThreads + threadIdx.x < M) atomicAdd(&h[(kv[r] >> shift) & (radix - 1)], 1);
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads) ghist[(int64_t)d * nblk + blockIdx.x] = h[d];
}

// Workgroup d: exclusive scan of digit d's block counts (row d of the digit-major histogram, in
// place) and the digit's total.  The rows are independent, so every digit's scan runs at once
// (one workgroup scanning the whole histogram would walk nblk x radix counts serially).
constexpr int kDigitItems = 8;   // counts per thread per round
__global__ void __launch_bounds__(kSortThreads) k_radix_digit_scan(int* __restrict__ ghist, int nblk,
                                                                   int* __restrict__ dtot) {
    __shared__ int wsum[kSortThreads / 64];
    const int d = blockIdx.x;
    int* row = ghist + (int64_t)d * nblk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int carry = 0;
    for (int base = 0; base < nblk; base += kSortThreads * kDigitItems) {
        // thread t takes counts base + 8t .. base + 8t + 7
        const int i0 = base + (int)threadIdx.x * kDigitItems;
        int v[kDigitItems];
        int local = 0;
#pragma unroll
        for (int k = 0; k < kDigitItems; ++k) {
            v[k] = i0 + k < nblk ? row[i0 + k] : 0;
            local += v[k];
        }
        int x = local;   // inclusive scan of the thread totals within the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(x, off, 64);
            if (lane >= off) x += t;
        }
        if (lane == 63) wsum[wave] = x;
        lds_barrier();
        int wc = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            wc += w < wave ? wsum[w] : 0;
            tot += wsum[w];
        }
        int run = carry + wc + x - local;
#pragma unroll
        for (int k = 0; k < kDigitItems; ++k) {
            if (i0 + k < nblk) row[i0 + k] = run;
            run += v[k];
        }
        carry += tot;
        lds_barrier();   // wsum is rewritten by the next round
    }
    if (threadIdx.x == 0) dtot[d] = carry;
}

// Wave w of a block owns its keys w*1024 .. w*1024 + 1023 (16 rounds of 64, in order).  Each wave
// ranks its own keys on its own (ballot match inside a round, a per-wave LDS count of each digit
// across its rounds), with no block barrier; the waves' digit counts then give every wave its base
// within each digit (waves in order: stable), the keys are placed in LDS in sorted order, and the
// block writes them out in that order: consecutive threads write consecutive positions of one
// digit's run, so a store instruction touches a few cache lines instead of one per lane.
constexpr int kSortWaveKeys = kSortTile / (kSortThreads / 64);
__global__ void __launch_bounds__(kSortThreads) k_radix_scatter(
    const int* __restrict__ keys_in, const int* __restrict__ vals_in, int* __restrict__ keys_out,
    int* __restrict__ vals_out, int64_t M, int shift, int dbits, int nblk,
    const int* __restrict__ gscan, const int* __restrict__ dtot) {
    static_assert(kSortThreads == 256 && kSortWaveKeys == 64 * kSortRounds, "one digit per thread");
    __shared__ int wcnt[4][256];   // per wave: keys of each digit seen so far, then its base
    __shared__ int gshift[256];    // global position - local position of the digit's keys
    __shared__ int dsum[2][kSortThreads / 64];
    __shared__ int lk[kSortTile], lv[kSortTile];
    const int radix = 1 << dbits;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    const int cnt = (int)min((int64_t)kSortTile, M - base);   // keys of this block
    const int w0 = wave * kSortWaveKeys;                       // the wave's first key in the block
    // the wave's keys and values are all requested up front (indices clamped into the arrays)
    int kr[kSortRounds], vr[kSortRounds];
#pragma unroll
    for (int r = 0; r < kSortRounds; ++r) {
        const int64_t i = min(base + w0 + r * 64 + lane, M - 1);
        kr[r] = keys_in[i];
        vr[r] = vals_in[i];
    }
    int lbase = 0;   // thread d: the digit's first local position
    {
        // digit d (= thread): global base = exclusive scan of the digit totals + the block's offset
        // within the digit; local base = exclusive scan of the block's own digit counts (the
        // difference of consecutive block offsets, or of the total for the last block)
        const int d = threadIdx.x;
        const int t = d < radix ? dtot[d] : 0;
        const int blk = d < radix ? gscan[(int64_t)d * nblk + blockIdx.x] : 0;
        const int nxt = d < radix ? (blockIdx.x + 1 < nblk ? gscan[(int64_t)d * nblk + blockIdx.x + 1] : t) : 0;
        const int c = nxt - blk;
        int x = t, y = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int u = __shfl_up(x, off, 64), w = __shfl_up(y, off, 64);
            if (lane >= off) {
                x += u;
                y += w;
            }
        }
        if (lane == 63) {
            dsum[0][wave] = x;
            dsum[1][wave] = y;
        }
        wcnt[0][d] = wcnt[1][d] = wcnt[2][d] = wcnt[3][d] = 0;
        lds_barrier();
        int wc = 0, wl = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            wc += w < wave ? dsum[0][w] : 0;
            wl += w < wave ? dsum[1][w] : 0;
        }
        lbase = wl + y - c;
        gshift[d] = wc + x - t + blk - lbase;
    }
    // ranks inside the wave: pre[r] = keys of the same digit before this one among the wave's keys
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int pre[kSortRounds];
#pragma unroll
    for (int r = 0; r < kSortRounds; ++r) {
        const bool valid = w0 + r * 64 + lane < cnt;
        const int d = (kr[r] >> shift) & (radix - 1);
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < dbits; ++b) {
            const bool bit = (d >> b) & 1;
            const uint64_t m = __ballot(valid && bit);
            peers &= bit ? m : ~m;
        }
        const int rank = __popcll(peers & lt_mask);
        const int seen = valid ? wcnt[wave][d] : 0;
        pre[r] = seen + rank;
        // the digit's lowest lane adds the round's count (one writer per digit; the wave's own
        // LDS operations stay in order, so the next round reads the new count)
        if (valid && rank == 0) wcnt[wave][d] = seen + __popcll(peers);
    }
    lds_barrier();
    {
        // thread d: the waves' bases within digit d, in wave order after the digit's local base
        // (the thread reads and rewrites column d only)
        const int d = threadIdx.x;
        const int c0 = wcnt[0][d], c1 = wcnt[1][d], c2 = wcnt[2][d];
        wcnt[0][d] = lbase;
        wcnt[1][d] = lbase + c0;
        wcnt[2][d] = lbase + c0 + c1;
        wcnt[3][d] = lbase + c0 + c1 + c2;
    }
    lds_barrier();
#pragma unroll
    for (int r = 0; r < kSortRounds; ++r) {
        if (w0 + r * 64 + lane < cnt) {
            const int pos = wcnt[wave][(kr[r] >> shift) & (radix - 1)] + pre[r];
            lk[pos] = kr[r];
            lv[pos] = vr[r];
        }
    }
    lds_barrier();
    // LDS position i holds the key of global position gshift[digit] + i
    for (int i = threadIdx.x; i < cnt; i += kSortThreads) {
        const int k = lk[i];
        const int pos = gshift[(k >> shift) & (radix - 1)] + i;
        keys_out[pos] = k;
        vals_out[pos] = lv[i];
    }
}

int sort_key_bits(int num_tiles) {
    int bits = 0;
    while (bits < 31 && (1ll << bits) < (long long)num_tiles) ++bits;
    return bits;
}

static void sort_plan(int num_tiles, int& passes, int& dbits) {
    const int bits = sort_key_bits(num_tiles);
    passes = (bits + 7) / 8;
    dbits = passes ? (bits + passes - 1) / passes : 0;
}

// Carves the sort workspace; with a null base it only measures it.
struct SortBufs {
    int* pk;
    int* pv;
    int* hist;
    int* dtot;    // digit totals of the pass
    size_t bytes;
};

static SortBufs carve_sort(void* ws, int64_t M, int num_tiles) {
    int passes, dbits;
    sort_plan(num_tiles, passes, dbits);
    const int64_t m = M > 0 ? M : 1;
    const int64_t nblk = ceil_div(m, kSortTile);
    const int64_t hist_n = (int64_t)(1 << dbits) * nblk;
    Carver c(ws, (size_t)-1);
    SortBufs b;
    b.pk = c.take<int>(m);
    b.pv = c.take<int>(m);
    b.hist = c.take<int>(hist_n);
    b.dtot = c.take<int>(256);
    b.bytes = c.off + 256;
    return b;
}

size_t sort_workspace(int64_t M, int num_tiles) { return carve_sort(nullptr, M, num_tiles).bytes; }

hipError_t radix_sort_pairs(const int* keys_in, const int* vals_in, int* keys_out, int* vals_out,
                            int64_t M, int num_tiles, void* ws, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    int passes, dbits;
    sort_plan(num_tiles, passes, dbits);
    if (passes == 0) {  // single tile: already sorted
        hipError_t e = hipMemcpyAsync(keys_out, keys_in, M * sizeof(int), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return e;
        return hipMemcpyAsync(vals_out, vals_in, M * sizeof(int), hipMemcpyDeviceToDevice, s);
    }
    const int nblk = (int)ceil_div(M, kSortTile);
    const SortBufs b = carve_sort(ws, M, num_tiles);
    int* pk = b.pk;
    int* pv = b.pv;
    int* hist = b.hist;
    int* dtot = b.dtot;
    const int* src_k = keys_in;
    const int* src_v = vals_in;
    for (int p = 0; p < passes; ++p) {
        // the last pass writes the caller's output; earlier passes alternate so that holds
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        int* dk = to_out ? keys_out : pk;
        int* dv = to_out ? vals_out : pv;
        const int shift = p * dbits;
        G2V_LAUNCH(k_radix_hist, dim3(nblk), dim3(kSortThreads), 0, s, src_k, M, shift, dbits,
                           nblk, hist);
        G2V_LAUNCH(k_radix_digit_scan, dim3(1 << dbits), dim3(kSortThreads), 0, s, hist, nblk, dtot);
        G2V_LAUNCH(k_radix_scatter, dim3(nblk), dim3(kSortThreads), 0, s, src_k, src_v, dk, dv,
                           M, shift, dbits, nblk, (const int*)hist, (const int*)dtot);
        src_k = dk;
        src_v = dv;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Tile offsets for every tile from the sorted keys: toff[t] = first sorted index with key >= t,
// toff[T] = M.  One lower-bound search per tile (about log2 M dependent loads), so the time does
// not depend on how the keys are spread: long runs of empty tiles cost nothing extra.  Every
// entry lies in [0, M] whatever the keys hold.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_tile_offsets(const int* __restrict__ keys, int64_t M, int T,
                                                      int* __restrict__ toff) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t > T) return;
    int64_t lo = 0, hi = M;
    if (t == T) lo = M;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (keys[mid] < t) lo = mid + 1;
        else hi = mid;
    }
    toff[t] = (int)lo;
}

hipError_t launch_tile_offsets(const int* sorted_keys, int64_t M, int T, int* tile_offsets,
                               hipStream_t s) {
    if (T < 0) return hipErrorInvalidValue;
    G2V_LAUNCH(k_tile_offsets, dim3((unsigned)ceil_div((int64_t)T + 1, 256)), dim3(256), 0, s,
               sorted_keys, M, T, tile_offsets);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Long tiles: the tiles whose list holds more than smax Gaussians, compacted into list[0 .. *count)
// (at most cap entries; a long tile holds at least smax + 1 of the M pairs, so the caller's cap of
// M / (smax + 1) always suffices).  One atomic add per wave places the wave's long tiles, in tile
// order within the wave; the order across waves is unspecified (each tile is computed alone, so the
// order changes no result).  *count must be zero beforehand.
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_long_tiles(const int* __restrict__ toff, int T, int M, int smax,
                                                    int* __restrict__ count, int* __restrict__ list, int cap) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    bool lng = false;
    if (t < T) {
        const int a = min(max(toff[t], 0), M);
        const int b = min(max(toff[t + 1], a), M);
        lng = b - a > smax;
    }
    const uint64_t m = __ballot(lng);
    if (m == 0) return;
    const int lane = threadIdx.x & 63;
    int base = 0;
    if (lane == __builtin_ctzll(m)) base = atomicAdd(count, __popcll(m));
    base = __shfl(base, __builtin_ctzll(m), 64);
    if (lng) {
        const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
        if (pos < cap) list[pos] = t;
    }
}

hipError_t launch_long_tiles(const int* toff, int T, int M, int smax, int* count, int* list, int cap,
                             hipStream_t s) {
    hipError_t e = launch_fill_i32(1, 0, count, s);
    if (e != hipSuccess || T <= 0) return e;
    G2V_LAUNCH(k_long_tiles, dim3((unsigned)ceil_div(T, 256)), dim3(256), 0, s, toff, T, M, smax, count, list, cap);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Run-length encoding of the sorted tile ids (unique tiles, run lengths, run offsets, count).
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_rle_flags(const int* __restrict__ toff, int T,
                                                   int* __restrict__ flags) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t < T) flags[t] = toff[t + 1] > toff[t] ? 1 : 0;
}

__global__ void __launch_bounds__(256) k_rle_write(const int* __restrict__ toff, int T,
                                                   const int* __restrict__ pos,
                                                   int* __restrict__ unique_tiles,
                                                   int* __restrict__ counts,
                                                   int* __restrict__ runs_offsets,
                                                   int* __restrict__ num_runs) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t < T && toff[t + 1] > toff[t]) {
        unique_tiles[pos[t]] = t;
        counts[pos[t]] = toff[t + 1] - toff[t];
        runs_offsets[pos[t]] = toff[t];
    }
    if (t == T) {
        const int U = T > 0 ? pos[T - 1] + (toff[T] > toff[T - 1] ? 1 : 0) : 0;
        runs_offsets[U] = toff[T];
        *num_runs = U;
    }
}

hipError_t launch_rle(const int* tile_offsets, int T, int* unique_tiles, int* counts,
                      int* runs_offsets, int* num_runs, void* ws, hipStream_t s) {
    Carver c(ws, (size_t)-1);
    int* flags = c.take<int>(T > 0 ? T : 1);
    void* scan_ws = c.take<char>(scan_workspace(T));
    const int blocks = (int)ceil_div(T + 1, 256);
    G2V_LAUNCH(k_rle_flags, dim3(blocks), dim3(256), 0, s, tile_offsets, T, flags);
    hipError_t e = scan_i32(flags, flags, T, false, nullptr, scan_ws, s);
    if (e != hipSuccess) return e;
    G2V_LAUNCH(k_rle_write, dim3(blocks), dim3(256), 0, s, tile_offsets, T, (const int*)flags,
                       unique_tiles, counts, runs_offsets, num_runs);
    return hipGetLastError();
}

}  // namespace g2v
