/*
 * C restatement of the reference G2V splatting path, used as the CPU oracle for
 * mid-size parity tests and as the CPU baseline of bench.py.
 *
 * TEST INFRASTRUCTURE ONLY: the product library never links or calls this file.
 *
 * It follows the reference algorithm step by step (paths relative to the
 * reference repository root):
 *   g2vo_boxes     src/cuda_gaussian_voxelizer.cu:348-536 (box, tile box), :201-220 (inverse)
 *   g2vo_g2t       src/cuda_gaussian_voxelizer.cu:1605-1615 (scan), :228-286 (row-major fill)
 *   g2vo_t2g       src/cuda_gaussian_voxelizer.cu:1673-1772 (stable sort by tile, RLE, offsets),
 *                  here as a stable counting sort
 *   g2vo_forward   src/cuda_gaussian_voxelizer.cu:7-136, :767-966 (tile-major splat), :1848-1849
 *   g2vo_backward  src/cuda_gaussian_voxelizer.cu:1304-1482 (Gaussian-major gradients), :1995-1996
 * Box and CSR are exact float32/int32 (compile with -ffp-contract=off); the splat and
 * the gradients accumulate in double.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define G2V_TILE 4
static const float kEps = 1e-6f;

static int cvt_i32(float x) {
    /* float -> int32 as the GPU converts: saturating, NaN -> 0 */
    if (x != x) return 0;
    if (x >= 2147483647.0f) return 2147483647;
    if (x <= -2147483648.0f) return (int)(-2147483647 - 1);
    return (int)x;
}

void g2vo_grid_dims(const float vs[3], const float vr[6], int dims[3], int tiles[3]) {
    for (int a = 0; a < 3; ++a) {
        float q = (vr[a + 3] - vr[a]) / vs[a];
        dims[a] = (int)q;
        tiles[a] = (dims[a] + G2V_TILE - 1) / G2V_TILE;
    }
}

static void invert3(const float* A, float* out) {
    float det = A[0] * (A[4] * A[8] - A[5] * A[7])
              - A[1] * (A[3] * A[8] - A[5] * A[6])
              + A[2] * (A[3] * A[7] - A[4] * A[6]);
    if (fabsf(det) < 1e-6f) det = 1e-6f;
    float inv_det = 1.0f / det;
    out[0] = (A[4] * A[8] - A[5] * A[7]) * inv_det;
    out[1] = -(A[1] * A[8] - A[2] * A[7]) * inv_det;
    out[2] = (A[1] * A[5] - A[2] * A[4]) * inv_det;
    out[3] = -(A[3] * A[8] - A[5] * A[6]) * inv_det;
    out[4] = (A[0] * A[8] - A[2] * A[6]) * inv_det;
    out[5] = -(A[0] * A[5] - A[2] * A[3]) * inv_det;
    out[6] = (A[3] * A[7] - A[4] * A[6]) * inv_det;
    out[7] = -(A[0] * A[7] - A[1] * A[6]) * inv_det;
    out[8] = (A[0] * A[4] - A[1] * A[3]) * inv_det;
}

void g2vo_boxes(int n, const float* means, const float* cov, const float vs[3], const float vr[6],
                int* lb, int* ub, int* nvox, int* tile_lo, int* tile_hi, int* ntiles, float* cov_inv) {
    int dims[3], tiles[3];
    g2vo_grid_dims(vs, vr, dims, tiles);
    for (int g = 0; g < n; ++g) {
        int lo[3], hi[3], empty = 0;
        for (int a = 0; a < 3; ++a) {
            float sig = sqrtf(cov[g * 9 + 4 * a]);
            float ts = 3.0f * sig;
            float lower = means[g * 3 + a] - ts;
            float upper = means[g * 3 + a] + ts;
            lower = fmaxf(lower, vr[a]);
            upper = fminf(upper, vr[a + 3]);
            float ql = (lower - vr[a]) / vs[a];
            float qh = (upper - vr[a]) / vs[a];
            lo[a] = cvt_i32(floorf(ql));
            hi[a] = cvt_i32(floorf(qh));
            if (lo[a] < 0) lo[a] = 0;
            if (hi[a] > dims[a] - 1) hi[a] = dims[a] - 1;
            if (lo[a] > hi[a]) empty = 1;
        }
        if (empty) {
            for (int a = 0; a < 3; ++a) {
                lb[g * 3 + a] = 0; ub[g * 3 + a] = -1;
                tile_lo[g * 3 + a] = 0; tile_hi[g * 3 + a] = -1;
            }
            nvox[g] = 0; ntiles[g] = 0;
            for (int k = 0; k < 9; ++k) cov_inv[g * 9 + k] = 0.0f;
            continue;
        }
        int nv = 1, nt = 1;
        for (int a = 0; a < 3; ++a) {
            lb[g * 3 + a] = lo[a]; ub[g * 3 + a] = hi[a];
            nv *= hi[a] - lo[a] + 1;
            int tl = lo[a] / G2V_TILE, th = hi[a] / G2V_TILE;
            if (tl < 0) tl = 0;
            if (th > tiles[a] - 1) th = tiles[a] - 1;
            tile_lo[g * 3 + a] = tl; tile_hi[g * 3 + a] = th;
            nt *= th - tl + 1;
        }
        nvox[g] = nv; ntiles[g] = nt;
        invert3(cov + g * 9, cov_inv + g * 9);
    }
}

/* offsets must hold n+1 ints; tile_ids/gauss_ids may be NULL to only count. Returns M. */
long long g2vo_g2t(int n, const int* tile_lo, const int* tile_hi, const int tiles[3],
                   int* offsets, int* tile_ids, int* gauss_ids) {
    long long M = 0;
    offsets[0] = 0;
    for (int g = 0; g < n; ++g) {
        int dx = tile_hi[g * 3] - tile_lo[g * 3] + 1;
        int dy = tile_hi[g * 3 + 1] - tile_lo[g * 3 + 1] + 1;
        int dz = tile_hi[g * 3 + 2] - tile_lo[g * 3 + 2] + 1;
        long long cnt = (dx > 0 && dy > 0 && dz > 0) ? (long long)dx * dy * dz : 0;
        if (tile_ids) {
            for (long long i = 0; i < cnt; ++i) {
                int lx = (int)(i / (dy * dz)), r = (int)(i % (dy * dz));
                int ly = r / dz, lz = r % dz;
                int tid = ((tile_lo[g * 3] + lx) * tiles[1] + (tile_lo[g * 3 + 1] + ly)) * tiles[2]
                          + (tile_lo[g * 3 + 2] + lz);
                tile_ids[M + i] = tid;
                gauss_ids[M + i] = g;
            }
        }
        M += cnt;
        offsets[g + 1] = (int)M;
    }
    return M;
}

/* Stable counting sort of the pairs by tile: tile_offsets (T+1), sorted_gauss (M). */
void g2vo_t2g(long long M, const int* tile_ids, const int* gauss_ids, int T,
              int* tile_offsets, int* sorted_gauss) {
    long long* cur = (long long*)calloc((size_t)T + 1, sizeof(long long));
    for (long long i = 0; i < M; ++i) cur[tile_ids[i] + 1]++;
    for (int t = 0; t < T; ++t) cur[t + 1] += cur[t];
    for (int t = 0; t <= T; ++t) tile_offsets[t] = (int)cur[t];
    for (long long i = 0; i < M; ++i) sorted_gauss[cur[tile_ids[i]]++] = gauss_ids[i];
    free(cur);
}

static inline int in_box(const int* lb, const int* ub, int g, int x, int y, int z) {
    return !(x < lb[g * 3] || x > ub[g * 3] || y < lb[g * 3 + 1] || y > ub[g * 3 + 1] ||
             z < lb[g * 3 + 2] || z > ub[g * 3 + 2]);
}

static inline double eval_w(const double* A, const float* mu, double cx, double cy, double cz,
                            double q[3]) {
    double d0 = cx - mu[0], d1 = cy - mu[1], d2 = cz - mu[2];
    q[0] = A[0] * d0 + A[1] * d1 + A[2] * d2;
    q[1] = A[3] * d0 + A[4] * d1 + A[5] * d2;
    q[2] = A[6] * d0 + A[7] * d1 + A[8] * d2;
    return exp(-0.5 * (d0 * q[0] + d1 * q[1] + d2 * q[2]));
}

/*
 * Tile-major forward (one tile at a time, its Gaussians in list order, 64 voxels).
 * cov_inv is double (N,9).  density (X*Y*Z) and grid_feats (X*Y*Z*C, may be NULL when C==0)
 * are written completely (uncovered voxels get 0).
 * tile_begin/tile_end restrict the work to a range of tiles (for timing samples);
 * pass 0, T for the full grid.
 */
void g2vo_forward(int n, int C, const float* means, const float* opacity, const double* cov_inv,
                  const int* lb, const int* ub, const float vs[3], const float vr[6],
                  const int* tile_offsets, const int* sorted_gauss, const float* features,
                  double* density, double* grid_feats, int tile_begin, int tile_end, int nthreads) {
    int dims[3], tiles[3];
    g2vo_grid_dims(vs, vr, dims, tiles);
    const int X = dims[0], Y = dims[1], Z = dims[2];
    const int Ty = tiles[1], Tz = tiles[2];
    (void)n;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 4)
#endif
    for (int t = tile_begin; t < tile_end; ++t) {
        int tx = t / (Ty * Tz), rem = t % (Ty * Tz), ty = rem / Tz, tz = rem % Tz;
        double* acc = C > 0 ? (double*)calloc((size_t)C, sizeof(double)) : NULL;
        for (int lv = 0; lv < 64; ++lv) {
            int x = tx * 4 + lv / 16, y = ty * 4 + (lv % 16) / 4, z = tz * 4 + lv % 4;
            if (x >= X || y >= Y || z >= Z) continue;
            double cx = (double)vr[0] + (x + 0.5) * (double)vs[0];
            double cy = (double)vr[1] + (y + 0.5) * (double)vs[1];
            double cz = (double)vr[2] + (z + 0.5) * (double)vs[2];
            double D = 0.0;
            if (C > 0) memset(acc, 0, sizeof(double) * (size_t)C);
            for (int j = tile_offsets[t]; j < tile_offsets[t + 1]; ++j) {
                int g = sorted_gauss[j];
                if (!in_box(lb, ub, g, x, y, z)) continue;
                double q[3];
                double w = (double)opacity[g] * eval_w(cov_inv + (size_t)g * 9, means + g * 3, cx, cy, cz, q);
                D += w;
                if (C > 0 && w > 0.0) {
                    const float* f = features + (size_t)g * C;
                    for (int c = 0; c < C; ++c) acc[c] += w * f[c];
                }
            }
            size_t v = ((size_t)x * Y + y) * Z + z;
            density[v] = D;
            if (C > 0) {
                double inv = 1.0 / (D > kEps ? D : (double)kEps);
                double* out = grid_feats + v * C;
                for (int c = 0; c < C; ++c) out[c] = acc[c] * inv;
            }
        }
        free(acc);
    }
}

/*
 * Gaussian-major backward (src/cuda_gaussian_voxelizer.cu:1304-1482): every Gaussian walks the
 * tiles of its G->T row and the voxels of its box.  density/grid_feats are the forward outputs,
 * grad_density (X*Y*Z) and grad_feats (X*Y*Z*C) the upstream gradients.  Outputs are double:
 * grad_means (N*3), grad_cov (N*9, symmetric), grad_opacity (N), grad_features (N*C).
 * g_begin/g_end restrict the work to a range of Gaussians.
 */
void g2vo_backward(int n, int C, const float* means, const float* opacity, const double* cov_inv,
                   const int* lb, const int* ub, const float vs[3], const float vr[6],
                   const int* g2t_offsets, const int* g2t_tile_ids, const float* features,
                   const float* density, const float* grid_feats, const float* grad_density,
                   const float* grad_feats, double* grad_means, double* grad_cov, double* grad_opacity,
                   double* grad_features, int g_begin, int g_end, int nthreads) {
    int dims[3], tiles[3];
    g2vo_grid_dims(vs, vr, dims, tiles);
    const int X = dims[0], Y = dims[1], Z = dims[2];
    const int Ty = tiles[1], Tz = tiles[2];
    (void)n; (void)X;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 8)
#endif
    for (int g = g_begin; g < g_end; ++g) {
        double gr[10] = {0};
        double* gf = C > 0 ? grad_features + (size_t)g * C : NULL;
        if (gf) memset(gf, 0, sizeof(double) * (size_t)C);
        const double* A = cov_inv + (size_t)g * 9;
        const float* f = C > 0 ? features + (size_t)g * C : NULL;
        for (int j = g2t_offsets[g]; j < g2t_offsets[g + 1]; ++j) {
            int t = g2t_tile_ids[j];
            int tx = t / (Ty * Tz), rem = t % (Ty * Tz), ty = rem / Tz, tz = rem % Tz;
            for (int lv = 0; lv < 64; ++lv) {
                int x = tx * 4 + lv / 16, y = ty * 4 + (lv % 16) / 4, z = tz * 4 + lv % 4;
                if (!in_box(lb, ub, g, x, y, z)) continue;
                double cx = (double)vr[0] + (x + 0.5) * (double)vs[0];
                double cy = (double)vr[1] + (y + 0.5) * (double)vs[1];
                double cz = (double)vr[2] + (z + 0.5) * (double)vs[2];
                double q[3];
                double e = eval_w(A, means + g * 3, cx, cy, cz, q);
                double w = (double)opacity[g] * e;
                size_t v = ((size_t)x * Y + y) * Z + z;
                double gw = grad_density[v];
                if (C > 0) {
                    double D = density[v];
                    double inv = 1.0 / (D > kEps ? D : (double)kEps);
                    const float* gF = grad_feats + v * C;
                    const float* Fv = grid_feats + v * C;
                    double u = 0.0, tv = 0.0;
                    for (int c = 0; c < C; ++c) {
                        u += (double)gF[c] * f[c];
                        tv += (double)gF[c] * Fv[c];
                        gf[c] += (double)gF[c] * w * inv;
                    }
                    if (!(D >= kEps)) tv = 0.0;
                    gw += (u - tv) * inv;
                }
                double gwd = gw * w;
                gr[0] += gwd * q[0]; gr[1] += gwd * q[1]; gr[2] += gwd * q[2];
                gr[3] += 0.5 * gwd * q[0] * q[0]; gr[4] += 0.5 * gwd * q[1] * q[1];
                gr[5] += 0.5 * gwd * q[2] * q[2]; gr[6] += 0.5 * gwd * q[0] * q[1];
                gr[7] += 0.5 * gwd * q[0] * q[2]; gr[8] += 0.5 * gwd * q[1] * q[2];
                gr[9] += gw * e;
            }
        }
        grad_means[g * 3] = gr[0]; grad_means[g * 3 + 1] = gr[1]; grad_means[g * 3 + 2] = gr[2];
        double* gc = grad_cov + (size_t)g * 9;
        gc[0] = gr[3]; gc[1] = gr[6]; gc[2] = gr[7];
        gc[3] = gr[6]; gc[4] = gr[4]; gc[5] = gr[8];
        gc[6] = gr[7]; gc[7] = gr[8]; gc[8] = gr[5];
        grad_opacity[g] = gr[9];
    }
}

int g2vo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
