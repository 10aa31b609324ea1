// C ABI of libg2v_hip.so (declared in include/g2v.h): argument checks, workspace carving and
// the launch sequence of each entry point.  Replaces the pybind11 binding and host
// orchestration of the reference (src/bindings.cpp:7-64, src/cuda_gaussian_voxelizer.cu:1484-2057).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/g2v.h"
#include "g2v_internal.h"

using namespace g2v;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    return fail(G2V_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

#define G2V_HIP(call)                                   \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// Grid of (voxel_size, voxel_range) in float32, truncated like the reference (.cu:1512-1519).
int make_grid(const float* vs, const float* vr, Grid& G) {
    if (!vs || !vr) return fail(G2V_ERR_INVALID, "voxel_size / voxel_range must not be null");
    G.scenes = 1;
    G.scene_n = 0;
    for (int a = 0; a < 3; ++a) {
        const float q = (vr[a + 3] - vr[a]) / vs[a];
        if (!(q >= 1.0f) || !(q < 2147483648.0f))
            return fail(G2V_ERR_INVALID, "grid axis %d has %g voxels (range %g..%g, size %g)", a,
                        (double)q, (double)vr[a], (double)vr[a + 3], (double)vs[a]);
        G.r0[a] = vr[a];
        G.r1[a] = vr[a + 3];
        G.s[a] = vs[a];
        G.dims[a] = (int)q;
        G.tiles[a] = (G.dims[a] + kTile - 1) / kTile;
    }
    const double cells = (double)G.dims[0] * G.dims[1] * G.dims[2];
    if (cells >= 2147483647.0) return fail(G2V_ERR_LIMIT, "grid has %.0f voxels (limit 2^31-1)", cells);
    return G2V_OK;
}

// Tiles of the problem (of every scene of a batch).
int num_tiles(const Grid& G) { return scene_tiles(G) * G.scenes; }

struct SplatBufs {
    int* keys;          // batches: the batch's tile id of every G->T entry (the sort key)
    int* gauss_ids;
    int* sorted_tiles;
    int* sorted_gauss;
    int* tile_offsets;
    void* sort_ws;
    uint32_t* fpk;      // features as packed bf16 (hi, lo) pairs, forward only
    int* tl;            // long-tile list of the forward (count, then the list), forward only
    DenParams* drec;    // packed per-Gaussian records of the forward's tile kernels
    size_t bytes;
};

// with_packed: room for the packed features (a caller that packs them with
// g2v_forward_pack_features passes its own buffer instead).  with_records: the forward's packed
// per-Gaussian records (written by the G->T fill).
SplatBufs carve_splat(void* ws, int n, int64_t M, const Grid& G, int feat_dim = 0, bool with_packed = true,
                      bool with_records = false) {
    const int64_t m = M > 0 ? M : 1;
    const int T = num_tiles(G);
    Carver c(ws, (size_t)-1);
    SplatBufs b;
    b.keys = G.scenes > 1 ? c.take<int>(m) : nullptr;
    b.gauss_ids = c.take<int>(m);
    b.sorted_tiles = c.take<int>(m);
    b.sorted_gauss = c.take<int>(m);
    b.tile_offsets = c.take<int>(T + 1);
    b.sort_ws = c.take<char>(sort_workspace(M, T));
    b.fpk = feat_dim > 0 && with_packed ? c.take<uint32_t>((int64_t)(n + 1) * packed_channels(feat_dim)) : nullptr;
    b.tl = feat_dim > 0 ? c.take<int>(long_list_ints(M, T, feat_dim)) : nullptr;
    b.drec = with_records ? c.take<DenParams>(n > 0 ? n : 1) : nullptr;
    b.bytes = c.off + 256;
    return b;
}

// G->T gauss ids, stable sort by tile, tile offsets: the Tile->Gaussian CSR.  A batch sorts by
// the batch's tile ids (b.keys, written beside the scene-local g2t_tile_ids_out).  With b.drec, the
// G->T fill also packs the Gaussians' records (from means, opacity and cov_inv).
int build_t2g(const Grid& G, int n, const int* lb, const int* ub, const int* g2t_offsets,
              int* g2t_tile_ids_out, const int* g2t_tile_ids_in, int64_t M, const SplatBufs& b,
              hipStream_t s, const float* means = nullptr, const float* opacity = nullptr,
              const float* cov_inv = nullptr) {
    const int T = num_tiles(G);
    if (M > 0) {
        G2V_HIP(launch_fill_g2t(G, n, lb, ub, g2t_offsets, g2t_tile_ids_out, b.gauss_ids, s, b.keys, means, opacity,
                                cov_inv, b.drec));
        const int* keys = b.keys ? b.keys : g2t_tile_ids_out ? g2t_tile_ids_out : g2t_tile_ids_in;
        G2V_HIP(radix_sort_pairs(keys, b.gauss_ids, b.sorted_tiles, b.sorted_gauss, M, T, b.sort_ws, s));
    }
    G2V_HIP(launch_tile_offsets(b.sorted_tiles, M, T, b.tile_offsets, s));
    return G2V_OK;
}

// Two counts in pinned, device-mapped host memory, one buffer per host thread (allocated on first
// use, kept until the process ends): the plan's kernels write its pair counts straight into it, so
// that the host wait is followed by no copy.  Null when pinned memory cannot be had (the plan then
// copies the counts from device memory).
long long* pinned_counts() {
    thread_local long long* p = nullptr;
    thread_local bool tried = false;
    if (!tried) {
        tried = true;
        void* q = nullptr;
        if (hipHostMalloc(&q, 64, hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess)
            p = static_cast<long long*>(q);
        else
            (void)hipGetLastError();
    }
    return p;
}

// Workspace of the backward of n Gaussians (all scenes of a batch) on G.
size_t backward_ws_bytes(const Grid& G, int n, int feat_dim, long long num_pairs, long long num_region_pairs) {
    if (feat_dim <= 0) return 256;
    Carver c(nullptr, (size_t)-1);
    c.take<char>(carve_splat(nullptr, n, num_pairs, G).bytes);
    c.take<char>(backward_feats_workspace(G, n, feat_dim, num_pairs, num_region_pairs));
    return c.off + 256;
}

int check_ws(const void* ws, size_t have, size_t need, const char* what) {
    if (need > have) return fail(G2V_ERR_INVALID, "%s workspace too small: %zu < %zu bytes", what, have, need);
    if (!ws && need > 0) return fail(G2V_ERR_INVALID, "%s workspace is null", what);
    return G2V_OK;
}

}  // namespace

extern "C" {

const char* g2v_last_error(void) { return g_err; }

int g2v_abi_version(void) { return 13; }

int g2v_grid_dims(const float voxel_size[3], const float voxel_range[6], int dims[3], int tiles[3]) {
    Grid G;
    const int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    for (int a = 0; a < 3; ++a) {
        if (dims) dims[a] = G.dims[a];
        if (tiles) tiles[a] = G.tiles[a];
    }
    return G2V_OK;
}

size_t g2v_forward_plan_workspace(int n) {
    Carver c(nullptr, (size_t)-1);
    c.take<long long>(2);
    c.take<char>(scan_workspace(n > 0 ? n : 1));
    return c.off + 256;
}

}  // extern "C"

namespace {

// Argument checks shared by the synchronous and the asynchronous plan.
int plan_checks(int n, const float* means3D, const float* covariances, const float* voxel_size,
                const float* voxel_range, float* cov_inv, int* lb, int* ub, int* nvox, int* g2t_offsets,
                void* workspace, size_t workspace_bytes, void* bwd_plan_workspace, size_t bwd_plan_workspace_bytes,
                Grid& G) {
    if (n < 0) return fail(G2V_ERR_INVALID, "n = %d", n);
    if (!g2t_offsets) return fail(G2V_ERR_INVALID, "g2t_offsets is null");
    if (bwd_plan_workspace && bwd_plan_workspace_bytes < backward_plan_workspace(n > 0 ? n : 0))
        return fail(G2V_ERR_INVALID, "backward plan workspace too small: %zu < %zu bytes",
                    bwd_plan_workspace_bytes, backward_plan_workspace(n > 0 ? n : 0));
    if (n > 0 && (!means3D || !covariances || !cov_inv || !lb || !ub || !nvox))
        return fail(G2V_ERR_INVALID, "null input/output pointer");
    int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    return check_ws(workspace, workspace_bytes, g2v_forward_plan_workspace(n), "plan");
}

// Boxes, inverse covariances and G->T row offsets, plus the backward plan's region cell offsets
// when bwd_plan_workspace is given; the pair counts land in counts[0] (M) and counts[1] (MR, or
// 0), a device-accessible pointer, when the stream reaches them.  The backward's (region,
// Gaussian) pair count rides on the same launches: the box kernel also counts each box's region
// cells, and one launch scans both count arrays.
int plan_launch(const Grid& G, int n, const float* means3D, const float* covariances, float* cov_inv, int* lb,
                int* ub, int* nvox, int* g2t_offsets, void* workspace, size_t workspace_bytes,
                void* bwd_plan_workspace, long long* counts, hipStream_t s) {
    Carver c(workspace, workspace_bytes);
    c.take<long long>(2);
    void* scan_ws = c.take<char>(scan_workspace(n > 0 ? n : 1));
    int cell[3] = {1, 1, 1};
    void* plan_scan_ws = nullptr;
    int* cell_off = bwd_plan_workspace ? backward_plan_cells(G, bwd_plan_workspace, n, cell, &plan_scan_ws) : nullptr;
    // the box kernel clears the counts that no scan writes: both without Gaussians, MR without the
    // backward plan
    long long* zero = n > 0 ? (cell_off ? nullptr : counts + 1) : counts;
    G2V_HIP(launch_boxes(G, n, means3D, covariances, cov_inv, lb, ub, nvox, g2t_offsets, cell_off ? cell : nullptr,
                         cell_off, s, zero, n > 0 ? 1 : 2));
    if (n > 0)
        G2V_HIP(scan_i32_pair(g2t_offsets + 1, g2t_offsets + 1, n, counts, scan_ws, cell_off ? cell_off + 1 : nullptr,
                              cell_off ? cell_off + 1 : nullptr, cell_off ? n : 0, counts + 1, plan_scan_ws, s));
    return G2V_OK;
}

int check_counts(long long M, long long MR) {
    if (M > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "%lld Gaussian-tile pairs exceed the int32 CSR (limit 2^31-1)", M);
    if (MR > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "%lld region-Gaussian pairs exceed the int32 CSR", MR);
    return G2V_OK;
}

}  // namespace

extern "C" {

int g2v_forward_plan(int n, const float* means3D, const float* covariances,
                     const float voxel_size[3], const float voxel_range[6], float* cov_inv,
                     int* valid_voxel_lb, int* valid_voxel_ub, int* num_voxels_per_gaussian,
                     int* g2t_offsets, void* workspace, size_t workspace_bytes,
                     long long* num_pairs, void* bwd_plan_workspace, size_t bwd_plan_workspace_bytes,
                     long long* num_region_pairs, void* stream) {
    g_err[0] = 0;
    if (!num_pairs) return fail(G2V_ERR_INVALID, "num_pairs is null");
    if (bwd_plan_workspace && !num_region_pairs)
        return fail(G2V_ERR_INVALID, "bwd_plan_workspace needs num_region_pairs");
    Grid G;
    int rc = plan_checks(n, means3D, covariances, voxel_size, voxel_range, cov_inv, valid_voxel_lb, valid_voxel_ub,
                         num_voxels_per_gaussian, g2t_offsets, workspace, workspace_bytes, bwd_plan_workspace,
                         bwd_plan_workspace_bytes, G);
    if (rc != G2V_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the counts go straight into pinned host memory when there is some (no copy before the host
    // wait), else into the workspace and are copied
    long long* hc = pinned_counts();
    long long* dc = reinterpret_cast<long long*>(Carver(workspace, workspace_bytes).take<long long>(2));
    if (hc) G2V_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&dc), hc, 0));
    rc = plan_launch(G, n, means3D, covariances, cov_inv, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian,
                     g2t_offsets, workspace, workspace_bytes, bwd_plan_workspace, dc, s);
    if (rc != G2V_OK) return rc;
    long long cnt[2] = {0, 0};
    if (!hc) G2V_HIP(hipMemcpyAsync(cnt, dc, sizeof(cnt), hipMemcpyDeviceToHost, s));
    G2V_HIP(hipStreamSynchronize(s));
    if (hc) {
        cnt[0] = hc[0];
        cnt[1] = hc[1];
    }
    rc = check_counts(cnt[0], cnt[1]);
    if (rc != G2V_OK) return rc;
    *num_pairs = cnt[0];
    if (num_region_pairs) *num_region_pairs = bwd_plan_workspace ? cnt[1] : 0;
    return G2V_OK;
}

int g2v_forward_plan_async(int n, const float* means3D, const float* covariances, const float voxel_size[3],
                           const float voxel_range[6], float* cov_inv, int* valid_voxel_lb, int* valid_voxel_ub,
                           int* num_voxels_per_gaussian, int* g2t_offsets, void* workspace, size_t workspace_bytes,
                           void* bwd_plan_workspace, size_t bwd_plan_workspace_bytes, long long* counts,
                           void* stream) {
    g_err[0] = 0;
    if (!counts) return fail(G2V_ERR_INVALID, "counts is null");
    // the kernels write the counts through a device address: that of pinned host memory is
    // looked up (it need not equal the host address), device memory is used as it is
    long long* dcounts = counts;
    {
        hipPointerAttribute_t pa;
        if (hipPointerGetAttributes(&pa, counts) != hipSuccess) {
            (void)hipGetLastError();
            return fail(G2V_ERR_INVALID, "counts is neither device memory nor pinned host memory");
        }
        if (pa.type == hipMemoryTypeHost) {
            void* d = nullptr;
            if (hipHostGetDevicePointer(&d, counts, 0) != hipSuccess || !d) {
                (void)hipGetLastError();
                return fail(G2V_ERR_INVALID, "counts: host memory without a device mapping");
            }
            dcounts = static_cast<long long*>(d);
        } else if (pa.type != hipMemoryTypeDevice && pa.type != hipMemoryTypeManaged) {
            return fail(G2V_ERR_INVALID, "counts is pageable host memory (needs device or pinned host memory)");
        }
    }
    Grid G;
    int rc = plan_checks(n, means3D, covariances, voxel_size, voxel_range, cov_inv, valid_voxel_lb, valid_voxel_ub,
                         num_voxels_per_gaussian, g2t_offsets, workspace, workspace_bytes, bwd_plan_workspace,
                         bwd_plan_workspace_bytes, G);
    if (rc != G2V_OK) return rc;
    return plan_launch(G, n, means3D, covariances, cov_inv, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian,
                       g2t_offsets, workspace, workspace_bytes, bwd_plan_workspace, dcounts,
                       static_cast<hipStream_t>(stream));
}

size_t g2v_forward_splat_workspace(int n, int feat_dim, long long num_pairs, const float voxel_size[3],
                                   const float voxel_range[6]) {
    Grid G;
    if (make_grid(voxel_size, voxel_range, G) != G2V_OK) return 0;
    return carve_splat(nullptr, n, num_pairs, G, feat_dim, false, true).bytes;
}

size_t g2v_forward_packed_bytes(int n, int feat_dim) {
    if (n < 0 || feat_dim <= 0) return 0;
    return (size_t)(n + 1) * packed_channels(feat_dim) * 4;
}

int g2v_forward_pack_features(int n, int feat_dim, const void* features, int feat_dtype, void* packed,
                              size_t packed_bytes, void* stream) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (n < 0 || feat_dim < 0) return fail(G2V_ERR_INVALID, "n = %d, feat_dim = %d", n, feat_dim);
    if (feat_dim == 0) return G2V_OK;
    if (!packed_fits(n, feat_dim))
        return fail(G2V_ERR_LIMIT, "n = %d x feat_dim = %d exceeds the packed feature rows (4 GiB)", n, feat_dim);
    if (!packed || (n > 0 && !features)) return fail(G2V_ERR_INVALID, "null features / packed pointer");
    const size_t need = g2v_forward_packed_bytes(n, feat_dim);
    if (packed_bytes < need)
        return fail(G2V_ERR_INVALID, "packed features buffer too small: %zu bytes, need %zu", packed_bytes, need);
    G2V_HIP(launch_split_pack(n, feat_dim, features, feat_dtype, static_cast<uint32_t*>(packed),
                              static_cast<hipStream_t>(stream)));
    return G2V_OK;
}

}  // extern "C"

namespace {

// The splat of n Gaussians (every scene of a batch) on G.  g2t_tile_ids (scene-local tile ids) may
// be null for a batch, whose sort keys are the batch's tile ids.
// packed: the features as g2v_forward_pack_features wrote them (queued before on the stream), or
// null: the splat packs them into its workspace (carved with_packed).
int splat_impl(const Grid& G, int n, int feat_dim, const float* means3D, const float* opacity,
               const void* features, int feat_dtype, const void* packed, const float* cov_inv, const int* valid_voxel_lb,
               const int* valid_voxel_ub, const int* g2t_offsets, long long num_pairs, int* g2t_tile_ids,
               float* density, void* grid_feats, int* t2g_tiles, int* t2g_gauss, int* t2g_offsets, void* workspace,
               size_t workspace_bytes, void* stream) {
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (n < 0 || feat_dim < 0 || num_pairs < 0)
        return fail(G2V_ERR_INVALID, "n = %d, feat_dim = %d, num_pairs = %lld", n, feat_dim, num_pairs);
    if (num_pairs > 2147483647ll) return fail(G2V_ERR_LIMIT, "num_pairs = %lld exceeds int32", num_pairs);
    if (!density) return fail(G2V_ERR_INVALID, "density is null");
    if (feat_dim > 0 && !packed_fits(n, feat_dim))
        return fail(G2V_ERR_LIMIT, "n = %d x feat_dim = %d exceeds the packed feature rows (4 GiB)", n, feat_dim);
    if (feat_dim > 0 && (!grid_feats || (n > 0 && !features)))
        return fail(G2V_ERR_INVALID, "feat_dim = %d needs features and grid_feats", feat_dim);
    if (num_pairs > 0 && ((!g2t_tile_ids && G.scenes == 1) || !g2t_offsets || !means3D || !opacity || !cov_inv ||
                          !valid_voxel_lb || !valid_voxel_ub))
        return fail(G2V_ERR_INVALID, "null input/output pointer");
    if ((double)scene_voxels(G) * G.scenes * (double)feat_dim >= 9.2e18)
        return fail(G2V_ERR_LIMIT, "grid_feats too large");
    const bool own_pack = packed == nullptr;
    const SplatBufs need = carve_splat(nullptr, n, num_pairs, G, feat_dim, own_pack, true);
    int rc = check_ws(workspace, workspace_bytes, need.bytes, "splat");
    if (rc != G2V_OK) return rc;
    SplatBufs b = carve_splat(workspace, n, num_pairs, G, feat_dim, own_pack, true);
    if (!own_pack) b.fpk = static_cast<uint32_t*>(const_cast<void*>(packed));
    if (t2g_tiles && t2g_gauss && t2g_offsets) {   // the caller keeps the Tile->Gaussian CSR
        b.sorted_tiles = t2g_tiles;
        b.sorted_gauss = t2g_gauss;
        b.tile_offsets = t2g_offsets;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (feat_dim > 0 && own_pack) G2V_HIP(launch_split_pack(n, feat_dim, features, feat_dtype, b.fpk, s));
    rc = build_t2g(G, n, valid_voxel_lb, valid_voxel_ub, g2t_offsets, g2t_tile_ids, nullptr,
                   num_pairs, b, s, means3D, opacity, cov_inv);
    if (rc != G2V_OK) return rc;
    if (feat_dim > 0)
        G2V_HIP(launch_forward_feats(G, feat_dim, means3D, opacity, cov_inv, valid_voxel_lb,
                                     valid_voxel_ub, b.tile_offsets, b.sorted_gauss, (int)num_pairs, n,
                                     features, feat_dtype, b.fpk, b.drec, density, grid_feats, b.tl, s));
    else
        G2V_HIP(launch_forward_density(G, b.drec, b.tile_offsets, b.sorted_gauss, (int)num_pairs, density, s));
    return G2V_OK;
}

}  // namespace

extern "C" {

int g2v_forward_splat(int n, int feat_dim, const float* means3D, const float* opacity,
                      const void* features, int feat_dtype, const void* packed_features, size_t packed_bytes,
                      const float voxel_size[3], const float voxel_range[6], const float* cov_inv,
                      const int* valid_voxel_lb, const int* valid_voxel_ub, const int* g2t_offsets,
                      long long num_pairs, int* g2t_tile_ids, float* density, void* grid_feats, int* t2g_tiles,
                      int* t2g_gauss, int* t2g_offsets, void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    Grid G;
    const int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    if (feat_dim > 0 && !packed_features)
        return fail(G2V_ERR_INVALID, "feat_dim = %d needs packed_features (g2v_forward_pack_features)", feat_dim);
    if (feat_dim > 0 && n > 0 && packed_bytes < g2v_forward_packed_bytes(n, feat_dim))
        return fail(G2V_ERR_INVALID, "packed features buffer too small: %zu bytes, need %zu for n = %d, feat_dim = %d",
                    packed_bytes, g2v_forward_packed_bytes(n, feat_dim), n, feat_dim);
    return splat_impl(G, n, feat_dim, means3D, opacity, features, feat_dtype, packed_features, cov_inv, valid_voxel_lb, valid_voxel_ub,
                      g2t_offsets, num_pairs, g2t_tile_ids, density, grid_feats, t2g_tiles, t2g_gauss, t2g_offsets,
                      workspace, workspace_bytes, stream);
}

size_t g2v_backward_plan_workspace(int n) { return backward_plan_workspace(n > 0 ? n : 0); }

int g2v_backward_plan(int n, int feat_dim, const float voxel_size[3], const float voxel_range[6],
                      const int* valid_voxel_lb, const int* valid_voxel_ub, void* plan_workspace,
                      size_t plan_workspace_bytes, long long* num_region_pairs, void* stream) {
    g_err[0] = 0;
    if (n < 0 || feat_dim < 0) return fail(G2V_ERR_INVALID, "n = %d, feat_dim = %d", n, feat_dim);
    if (!num_region_pairs) return fail(G2V_ERR_INVALID, "num_region_pairs is null");
    *num_region_pairs = 0;
    if (n == 0 || feat_dim == 0) return G2V_OK;
    if (!valid_voxel_lb || !valid_voxel_ub) return fail(G2V_ERR_INVALID, "null box pointer");
    Grid G;
    int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    rc = check_ws(plan_workspace, plan_workspace_bytes, backward_plan_workspace(n), "backward plan");
    if (rc != G2V_OK) return rc;
    long long MR = 0;
    G2V_HIP(backward_plan(G, n, valid_voxel_lb, valid_voxel_ub, plan_workspace, &MR,
                          static_cast<hipStream_t>(stream)));
    if (MR > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "%lld region-Gaussian pairs exceed the int32 CSR", MR);
    *num_region_pairs = MR;
    return G2V_OK;
}

size_t g2v_backward_workspace(int n, int feat_dim, long long num_pairs, long long num_region_pairs,
                              const float voxel_size[3], const float voxel_range[6]) {
    Grid G;
    if (make_grid(voxel_size, voxel_range, G) != G2V_OK) return 0;
    return backward_ws_bytes(G, n, feat_dim, num_pairs, num_region_pairs);
}

}  // extern "C"

namespace {

int backward_impl(int n, int feat_dim, const float* grad_density, const void* grad_feats,
                  const float* means3D, const float* opacity, const float* cov_inv,
                  const float voxel_size[3], const float voxel_range[6], const int* valid_voxel_lb,
                  const int* valid_voxel_ub, const int* num_voxels_per_gaussian,
                  const int* g2t_offsets, const int* g2t_tile_ids, long long num_pairs,
                  long long num_region_pairs, const float* density, const void* grid_feats,
                  const void* features, int feat_dtype, float* grad_means, float* grad_cov, float* grad_opacity,
                  void* grad_features, const int* t2g_tiles, const int* t2g_gauss,
                  const int* t2g_offsets, const void* plan_workspace, void* workspace,
                  size_t workspace_bytes, bool prepared, void* stream, const CosG* cos = nullptr,
                  int scenes = 1) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    (void)num_voxels_per_gaussian;
    if (n < 0 || feat_dim < 0 || num_pairs < 0 || num_region_pairs < 0)
        return fail(G2V_ERR_INVALID, "n = %d, feat_dim = %d, num_pairs = %lld, num_region_pairs = %lld", n,
                    feat_dim, num_pairs, num_region_pairs);
    if (num_pairs > 2147483647ll || num_region_pairs > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "pair counts exceed int32");
    if (n == 0) return G2V_OK;
    if (!grad_density || !means3D || !opacity || !cov_inv || !valid_voxel_lb || !valid_voxel_ub ||
        !grad_means || !grad_cov || !grad_opacity)
        return fail(G2V_ERR_INVALID, "null input/output pointer");
    const bool have_t2g = t2g_tiles && t2g_gauss && t2g_offsets;
    if (feat_dim > 0 && ((!grad_feats && !cos) || !grid_feats || !features || !grad_features || !density ||
                         !g2t_offsets || !plan_workspace ||
                         (num_pairs > 0 && !g2t_tile_ids && !have_t2g && scenes == 1)))
        return fail(G2V_ERR_INVALID, "feat_dim = %d needs the feature tensors, density, the CSR and the plan workspace", feat_dim);
    if (feat_dim > 0 && !split_rows_fit(n, feat_dim))
        return fail(G2V_ERR_LIMIT, "n = %d x feat_dim = %d exceeds the split feature rows (4 GiB)", n, feat_dim);
    Grid G;
    int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    if (scenes > 1) {   // n = scenes x scene_n Gaussians, scene-major
        G.scenes = scenes;
        G.scene_n = n / scenes;
    }
    if (feat_dim > 0 && !region_offsets_fit(G, feat_dim))
        return fail(G2V_ERR_LIMIT, "Y x Z x feat_dim = %d x %d x %d exceeds the 32-bit tile offsets of the "
                    "feature backward (16 Y Z C < 2^31)", G.dims[1], G.dims[2], feat_dim);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (feat_dim == 0) {
        G2V_HIP(launch_backward_density(G, n, grad_density, means3D, opacity, cov_inv, valid_voxel_lb,
                                        valid_voxel_ub, grad_means, grad_cov, grad_opacity, s));
        return G2V_OK;
    }
    rc = check_ws(workspace, workspace_bytes, backward_ws_bytes(G, n, feat_dim, num_pairs, num_region_pairs),
                  "backward");
    if (rc != G2V_OK) return rc;
    Carver c(workspace, workspace_bytes);
    void* splat_ws = c.take<char>(carve_splat(nullptr, n, num_pairs, G).bytes);
    void* feats_ws = c.take<char>(backward_feats_workspace(G, n, feat_dim, num_pairs, num_region_pairs));
    SplatBufs b = carve_splat(splat_ws, n, num_pairs, G);
    if (t2g_tiles && t2g_gauss && t2g_offsets) {   // the forward's Tile->Gaussian CSR
        b.sorted_tiles = const_cast<int*>(t2g_tiles);
        b.sorted_gauss = const_cast<int*>(t2g_gauss);
        b.tile_offsets = const_cast<int*>(t2g_offsets);
    } else {
        rc = build_t2g(G, n, valid_voxel_lb, valid_voxel_ub, g2t_offsets, nullptr, g2t_tile_ids,
                       num_pairs, b, s);
        if (rc != G2V_OK) return rc;
    }
    G2V_HIP(launch_backward_feats(G, n, feat_dim, grad_density, grad_feats, means3D, opacity, cov_inv,
                                  valid_voxel_lb, valid_voxel_ub, g2t_offsets, num_pairs,
                                  b.tile_offsets, b.sorted_tiles, b.sorted_gauss, density, grid_feats, features,
                                  feat_dtype, plan_workspace, num_region_pairs, grad_means, grad_cov, grad_opacity,
                                  grad_features, feats_ws, prepared, s, cos));
    return G2V_OK;
}

}  // namespace

extern "C" {

int g2v_backward(int n, int feat_dim, const float* grad_density, const void* grad_feats,
                 const float* means3D, const float* opacity, const float* cov_inv,
                 const float voxel_size[3], const float voxel_range[6], const int* valid_voxel_lb,
                 const int* valid_voxel_ub, const int* num_voxels_per_gaussian,
                 const int* g2t_offsets, const int* g2t_tile_ids, long long num_pairs,
                 long long num_region_pairs, const float* density, const void* grid_feats,
                 const void* features, int feat_dtype, float* grad_means, float* grad_cov, float* grad_opacity,
                 void* grad_features, const int* t2g_tiles, const int* t2g_gauss,
                 const int* t2g_offsets, const void* plan_workspace, void* workspace,
                 size_t workspace_bytes, void* stream) {
    return backward_impl(n, feat_dim, grad_density, grad_feats, means3D, opacity, cov_inv, voxel_size,
                         voxel_range, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets,
                         g2t_tile_ids, num_pairs, num_region_pairs, density, grid_feats, features, feat_dtype,
                         grad_means, grad_cov, grad_opacity, grad_features, t2g_tiles, t2g_gauss, t2g_offsets,
                         plan_workspace, workspace, workspace_bytes, false, stream);
}

}  // extern "C"

namespace {

int prepare_impl(int n, int feat_dim, const float voxel_size[3], const float voxel_range[6],
                 const int* valid_voxel_lb, const int* valid_voxel_ub, const void* features, int feat_dtype,
                 long long num_pairs, long long num_region_pairs, const int* t2g_tiles, const int* t2g_gauss,
                 const void* plan_workspace, void* workspace, size_t workspace_bytes, void* stream, int scenes) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (n < 0 || feat_dim < 0 || num_pairs < 0 || num_region_pairs < 0)
        return fail(G2V_ERR_INVALID, "n = %d, feat_dim = %d, num_pairs = %lld, num_region_pairs = %lld", n,
                    feat_dim, num_pairs, num_region_pairs);
    if (num_pairs > 2147483647ll || num_region_pairs > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "pair counts exceed int32");
    if (n == 0 || feat_dim == 0) return G2V_OK;
    if (!valid_voxel_lb || !valid_voxel_ub || !features || !plan_workspace ||
        (num_pairs > 0 && (!t2g_tiles || !t2g_gauss)))
        return fail(G2V_ERR_INVALID, "null input pointer (the Tile->Gaussian CSR of the forward is required)");
    if (!split_rows_fit(n, feat_dim))
        return fail(G2V_ERR_LIMIT, "n = %d x feat_dim = %d exceeds the split feature rows (4 GiB)", n, feat_dim);
    Grid G;
    int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    if (scenes > 1) {   // n = scenes x scene_n Gaussians, scene-major
        G.scenes = scenes;
        G.scene_n = n / scenes;
    }
    rc = check_ws(workspace, workspace_bytes, backward_ws_bytes(G, n, feat_dim, num_pairs, num_region_pairs),
                  "backward");
    if (rc != G2V_OK) return rc;
    Carver c(workspace, workspace_bytes);
    c.take<char>(carve_splat(nullptr, n, num_pairs, G).bytes);
    void* feats_ws = c.take<char>(backward_feats_workspace(G, n, feat_dim, num_pairs, num_region_pairs));
    G2V_HIP(launch_backward_prepare(G, n, feat_dim, features, feat_dtype, valid_voxel_lb, valid_voxel_ub, num_pairs,
                                    t2g_tiles, t2g_gauss, plan_workspace, num_region_pairs, feats_ws,
                                    static_cast<hipStream_t>(stream)));
    return G2V_OK;
}

}  // namespace

extern "C" {

int g2v_backward_prepare(int n, int feat_dim, const float voxel_size[3], const float voxel_range[6],
                         const int* valid_voxel_lb, const int* valid_voxel_ub, const void* features,
                         int feat_dtype, long long num_pairs, long long num_region_pairs, const int* t2g_tiles,
                         const int* t2g_gauss, const void* plan_workspace, void* workspace,
                         size_t workspace_bytes, void* stream) {
    return prepare_impl(n, feat_dim, voxel_size, voxel_range, valid_voxel_lb, valid_voxel_ub, features, feat_dtype,
                        num_pairs, num_region_pairs, t2g_tiles, t2g_gauss, plan_workspace, workspace, workspace_bytes,
                        stream, 1);
}

int g2v_backward_cosine(int n, int feat_dim, const float* grad_density, const float* grad_loss,
                        const void* pseudo_gt, const float* coef, int num_valid_voxel, const float* means3D,
                        const float* opacity, const float* cov_inv, const float voxel_size[3],
                        const float voxel_range[6], const int* valid_voxel_lb, const int* valid_voxel_ub,
                        const int* num_voxels_per_gaussian, const int* g2t_offsets, const int* g2t_tile_ids,
                        long long num_pairs, long long num_region_pairs, const float* density,
                        const void* grid_feats, const void* features, int feat_dtype, float* grad_means,
                        float* grad_cov, float* grad_opacity, void* grad_features, const int* t2g_tiles,
                        const int* t2g_gauss, const int* t2g_offsets, const void* plan_workspace, void* workspace,
                        size_t workspace_bytes, int prepared, void* stream) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d: the fused cosine gradient takes float32 features", feat_dtype);
    if (feat_dim <= 0 || (feat_dim & 3) != 0)
        return fail(G2V_ERR_INVALID, "feat_dim = %d: the fused cosine gradient needs feat_dim %% 4 == 0", feat_dim);
    if (n > 0 && (!grad_loss || !pseudo_gt || !coef))
        return fail(G2V_ERR_INVALID, "grad_loss, pseudo_gt and coef are required");
    if (((uintptr_t)pseudo_gt & 15) != 0 || ((uintptr_t)grid_feats & 15) != 0 || ((uintptr_t)coef & 7) != 0)
        return fail(G2V_ERR_INVALID, "pseudo_gt and grid_feats must be 16-byte aligned, coef 8-byte aligned");
    if (prepared && n > 0 && num_pairs > 0 && !(t2g_tiles && t2g_gauss && t2g_offsets))
        return fail(G2V_ERR_INVALID, "a prepared backward needs the forward's Tile->Gaussian CSR");
    // the scale of the loss's own backward (reference src/cuda_feats_loss.cu:319)
    const CosG cos{static_cast<const float*>(pseudo_gt), coef, grad_loss,
                   num_valid_voxel > 0 ? 1.0f / (float)num_valid_voxel : 0.0f};
    return backward_impl(n, feat_dim, grad_density, nullptr, means3D, opacity, cov_inv, voxel_size, voxel_range,
                         valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets, g2t_tile_ids,
                         num_pairs, num_region_pairs, density, grid_feats, features, feat_dtype, grad_means, grad_cov,
                         grad_opacity, grad_features, t2g_tiles, t2g_gauss, t2g_offsets, plan_workspace, workspace,
                         workspace_bytes, prepared != 0, stream, &cos);
}

int g2v_backward_prepared(int n, int feat_dim, const float* grad_density, const void* grad_feats,
                          const float* means3D, const float* opacity, const float* cov_inv,
                          const float voxel_size[3], const float voxel_range[6], const int* valid_voxel_lb,
                          const int* valid_voxel_ub, const int* num_voxels_per_gaussian,
                          const int* g2t_offsets, const int* g2t_tile_ids, long long num_pairs,
                          long long num_region_pairs, const float* density, const void* grid_feats,
                          const void* features, int feat_dtype, float* grad_means, float* grad_cov,
                          float* grad_opacity, void* grad_features, const int* t2g_tiles, const int* t2g_gauss,
                          const int* t2g_offsets, const void* plan_workspace, void* workspace,
                          size_t workspace_bytes, void* stream) {
    if (feat_dim > 0 && n > 0 && num_pairs > 0 && !(t2g_tiles && t2g_gauss && t2g_offsets)) {
        g_err[0] = 0;
        return fail(G2V_ERR_INVALID, "g2v_backward_prepared needs the forward's Tile->Gaussian CSR");
    }
    return backward_impl(n, feat_dim, grad_density, grad_feats, means3D, opacity, cov_inv, voxel_size,
                         voxel_range, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets,
                         g2t_tile_ids, num_pairs, num_region_pairs, density, grid_feats, features, feat_dtype,
                         grad_means, grad_cov, grad_opacity, grad_features, t2g_tiles, t2g_gauss, t2g_offsets,
                         plan_workspace, workspace, workspace_bytes, true, stream);
}

size_t g2v_t2g_workspace(int n, long long num_pairs, const float voxel_size[3],
                         const float voxel_range[6]) {
    Grid G;
    if (make_grid(voxel_size, voxel_range, G) != G2V_OK) return 0;
    const int T = num_tiles(G);
    Carver c(nullptr, (size_t)-1);
    c.take<char>(carve_splat(nullptr, n, num_pairs, G).bytes);
    c.take<int>(T > 0 ? T : 1);
    c.take<char>(scan_workspace(T));
    return c.off + 256;
}

int g2v_build_t2g(int n, const float voxel_size[3], const float voxel_range[6],
                  const int* valid_voxel_lb, const int* valid_voxel_ub, const int* g2t_offsets,
                  const int* g2t_tile_ids, long long num_pairs, int* sorted_tiles,
                  int* sorted_gauss, int* tile_offsets, int* unique_tiles, int* counts,
                  int* runs_offsets, int* num_runs, void* workspace, size_t workspace_bytes,
                  void* stream) {
    g_err[0] = 0;
    if (n < 0 || num_pairs < 0) return fail(G2V_ERR_INVALID, "n = %d, num_pairs = %lld", n, num_pairs);
    if (!tile_offsets || !unique_tiles || !counts || !runs_offsets || !num_runs ||
        (num_pairs > 0 && (!sorted_tiles || !sorted_gauss || !g2t_tile_ids || !g2t_offsets ||
                           !valid_voxel_lb || !valid_voxel_ub)))
        return fail(G2V_ERR_INVALID, "null pointer");
    Grid G;
    int rc = make_grid(voxel_size, voxel_range, G);
    if (rc != G2V_OK) return rc;
    rc = check_ws(workspace, workspace_bytes, g2v_t2g_workspace(n, num_pairs, voxel_size, voxel_range), "t2g");
    if (rc != G2V_OK) return rc;
    const int T = num_tiles(G);
    hipStream_t s = static_cast<hipStream_t>(stream);
    Carver c(workspace, workspace_bytes);
    void* splat_ws = c.take<char>(carve_splat(nullptr, n, num_pairs, G).bytes);
    void* rle_ws = c.take<char>(0);
    const SplatBufs b = carve_splat(splat_ws, n, num_pairs, G);
    rc = build_t2g(G, n, valid_voxel_lb, valid_voxel_ub, g2t_offsets, nullptr, g2t_tile_ids,
                   num_pairs, b, s);
    if (rc != G2V_OK) return rc;
    if (num_pairs > 0) {
        G2V_HIP(hipMemcpyAsync(sorted_tiles, b.sorted_tiles, num_pairs * sizeof(int),
                               hipMemcpyDeviceToDevice, s));
        G2V_HIP(hipMemcpyAsync(sorted_gauss, b.sorted_gauss, num_pairs * sizeof(int),
                               hipMemcpyDeviceToDevice, s));
    }
    G2V_HIP(hipMemcpyAsync(tile_offsets, b.tile_offsets, (T + 1) * sizeof(int),
                           hipMemcpyDeviceToDevice, s));
    G2V_HIP(launch_rle(b.tile_offsets, T, unique_tiles, counts, runs_offsets, num_runs, rle_ws, s));
    return G2V_OK;
}

size_t g2v_cosine_loss_workspace(long long num_voxels, int feat_dim) {
    (void)feat_dim;
    return cosine_workspace(num_voxels > 0 ? num_voxels : 0);
}

// The loss forward; coef (optional) receives the per-voxel gradient coefficients.
static int cosine_forward_impl(long long num_voxels, int feat_dim, const float* voxel_label,
                               const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                               int feat_dtype, float* loss, int* num_valid, int* num_valid_host, float* coef,
                               void* workspace, size_t workspace_bytes, void* stream) {
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (num_voxels < 0 || feat_dim < 0)
        return fail(G2V_ERR_INVALID, "num_voxels = %lld, feat_dim = %d", num_voxels, feat_dim);
    if (num_voxels > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "num_voxels = %lld exceeds the int32 valid-voxel count", num_voxels);
    if (!loss || !num_valid) return fail(G2V_ERR_INVALID, "loss / num_valid is null");
    if (num_voxels > 0 && (!voxel_label || !occ_mask || (feat_dim > 0 && (!grid_feats || !pseudo_gt))))
        return fail(G2V_ERR_INVALID, "null input pointer");
    int rc = check_ws(workspace, workspace_bytes, g2v_cosine_loss_workspace(num_voxels, feat_dim), "cosine loss");
    if (rc != G2V_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    G2V_HIP(launch_cosine_forward(num_voxels, feat_dim, voxel_label, occ_mask, grid_feats, pseudo_gt, feat_dtype,
                                  loss, num_valid, workspace, s, coef));
    if (num_valid_host) {
        int h = 0;
        G2V_HIP(hipMemcpyAsync(&h, num_valid, sizeof(int), hipMemcpyDeviceToHost, s));
        G2V_HIP(hipStreamSynchronize(s));
        *num_valid_host = h;
    }
    return G2V_OK;
}

int g2v_cosine_loss_forward(long long num_voxels, int feat_dim, const float* voxel_label,
                            const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                            int feat_dtype, float* loss, int* num_valid, int* num_valid_host, void* workspace,
                            size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    return cosine_forward_impl(num_voxels, feat_dim, voxel_label, occ_mask, grid_feats, pseudo_gt, feat_dtype, loss,
                               num_valid, num_valid_host, nullptr, workspace, workspace_bytes, stream);
}

int g2v_cosine_loss_forward_coef(long long num_voxels, int feat_dim, const float* voxel_label,
                                 const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                                 int feat_dtype, float* loss, int* num_valid, int* num_valid_host, float* coef,
                                 void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    if (num_voxels > 0 && !coef) return fail(G2V_ERR_INVALID, "coef is null");
    if (((uintptr_t)coef & 7) != 0) return fail(G2V_ERR_INVALID, "coef must be 8-byte aligned");
    return cosine_forward_impl(num_voxels, feat_dim, voxel_label, occ_mask, grid_feats, pseudo_gt, feat_dtype, loss,
                               num_valid, num_valid_host, coef, workspace, workspace_bytes, stream);
}

int g2v_cosine_loss_forward_noalloc(long long num_voxels, int feat_dim, const float* voxel_label,
                                    const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                                    int feat_dtype, float* loss, int* num_valid, void* stream) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (num_voxels < 0 || feat_dim < 0)
        return fail(G2V_ERR_INVALID, "num_voxels = %lld, feat_dim = %d", num_voxels, feat_dim);
    if (num_voxels > 2147483647ll)
        return fail(G2V_ERR_LIMIT, "num_voxels = %lld exceeds the int32 valid-voxel count", num_voxels);
    if (!loss || !num_valid) return fail(G2V_ERR_INVALID, "loss / num_valid is null");
    if (num_voxels > 0 && (!voxel_label || !occ_mask || (feat_dim > 0 && (!grid_feats || !pseudo_gt))))
        return fail(G2V_ERR_INVALID, "null input pointer");
    const hipError_t e = launch_cosine_forward_noalloc(num_voxels, feat_dim, voxel_label, occ_mask, grid_feats,
                                                       pseudo_gt, feat_dtype, loss, num_valid,
                                                       static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue)
        return fail(G2V_ERR_LIMIT, "num_voxels = %lld needs more block partials than the %zu-byte scratch holds",
                    num_voxels, cosine_scratch_bytes());
    if (e != hipSuccess) return hip_fail(e, "launch_cosine_forward_noalloc");
    return G2V_OK;
}

int g2v_cosine_loss_backward(long long num_voxels, int feat_dim, const float* grad_output,
                             const float* voxel_label, const unsigned char* occ_mask, const void* grid_feats,
                             const void* pseudo_gt, int feat_dtype, int num_valid_voxel, void* grad_grid_feats,
                             void* stream) {
    g_err[0] = 0;
    if (feat_dtype != G2V_DTYPE_F32 && feat_dtype != G2V_DTYPE_BF16)
        return fail(G2V_ERR_INVALID, "feat_dtype = %d (G2V_DTYPE_F32 or G2V_DTYPE_BF16)", feat_dtype);
    if (num_voxels < 0 || feat_dim < 0)
        return fail(G2V_ERR_INVALID, "num_voxels = %lld, feat_dim = %d", num_voxels, feat_dim);
    if (num_voxels == 0 || feat_dim == 0) return G2V_OK;
    if (!grad_output || !voxel_label || !occ_mask || !grid_feats || !pseudo_gt || !grad_grid_feats)
        return fail(G2V_ERR_INVALID, "null input/output pointer");
    // the reference's host-side scale (src/cuda_feats_loss.cu:319)
    const float inv_count = num_valid_voxel > 0 ? 1.0f / (float)num_valid_voxel : 0.0f;
    G2V_HIP(launch_cosine_backward(num_voxels, feat_dim, voxel_label, occ_mask, grid_feats, pseudo_gt, feat_dtype,
                                   grad_output, inv_count, grad_grid_feats, static_cast<hipStream_t>(stream)));
    return G2V_OK;
}

int g2v_covariance_from_scale_rotation(int n, const float* scales, const float* rotations, float* covariances,
                                       void* stream) {
    g_err[0] = 0;
    if (n < 0) return fail(G2V_ERR_INVALID, "n = %d", n);
    if (n > 0 && (!scales || !rotations || !covariances)) return fail(G2V_ERR_INVALID, "null pointer");
    if ((int64_t)n * 9 > 2147483647ll) return fail(G2V_ERR_LIMIT, "n = %d exceeds the int32 covariance index", n);
    G2V_HIP(launch_cov_from_scale_rot(n, scales, rotations, covariances, static_cast<hipStream_t>(stream)));
    return G2V_OK;
}

int g2v_covariance_from_scale_rotation_backward(int n, const float* scales, const float* rotations,
                                                const float* grad_covariances, float* grad_scales,
                                                float* grad_rotations, void* stream) {
    g_err[0] = 0;
    if (n < 0) return fail(G2V_ERR_INVALID, "n = %d", n);
    if (n > 0 && (!scales || !rotations || !grad_covariances || !grad_scales || !grad_rotations))
        return fail(G2V_ERR_INVALID, "null pointer");
    if ((int64_t)n * 9 > 2147483647ll) return fail(G2V_ERR_LIMIT, "n = %d exceeds the int32 covariance index", n);
    G2V_HIP(launch_cov_from_scale_rot_bwd(n, scales, rotations, grad_covariances, grad_scales, grad_rotations,
                                          static_cast<hipStream_t>(stream)));
    return G2V_OK;
}

// ---- batches of scenes on one grid -------------------------------------------------------------
//
// B scenes of n Gaussians each, laid out scene-major ((B, n, ...) inputs, (B, X, Y, Z[, C]) outputs),
// are planned, splatted and differentiated as one problem of B n Gaussians on B T tiles (see Grid).

}  // extern "C"

namespace {

// The batch's plan workspace: the batch's G->T row offsets (B n + 1) and pair totals, the plan's own
// workspace and the backward plan's region cell offsets, all for B n Gaussians.  The caller keeps it
// from the plan to the batch's backward.
struct BatchPlan {
    int* goff;
    long long* totals;   // pairs, region pairs of the batch
    void* plan_ws;
    size_t plan_bytes;
    void* bwd_ws;
    size_t bytes;
};

BatchPlan carve_batch_plan(void* ws, int B, int n) {
    const int nt = B * n;
    Carver c(ws, (size_t)-1);
    BatchPlan p;
    p.goff = c.take<int>((size_t)nt + 1);
    p.totals = c.take<long long>(2);
    p.plan_bytes = g2v_forward_plan_workspace(nt);
    p.plan_ws = c.take<char>(p.plan_bytes);
    p.bwd_ws = c.take<char>(backward_plan_workspace(nt));
    p.bytes = c.off + 256;
    return p;
}

bool batch_sizes_ok(int B, int n) { return B >= 1 && n >= 0 && (int64_t)B * n < 2147483647ll; }

// The batch's tile count fits the int32 tile ids (batch_setup's check, for the size queries).
bool batch_tiles_ok(const Grid& G, int B) { return (int64_t)scene_tiles(G) * B < 2147483647ll; }

// Grid of a batch of B scenes (n Gaussians each) and its plan workspace, checked.
int batch_setup(int B, int n, const float* vs, const float* vr, const void* plan_ws, size_t plan_bytes, Grid& G,
                BatchPlan& p) {
    if (!batch_sizes_ok(B, n)) return fail(G2V_ERR_INVALID, "num_scenes = %d, n = %d", B, n);
    int rc = make_grid(vs, vr, G);
    if (rc != G2V_OK) return rc;
    if (!batch_tiles_ok(G, B)) return fail(G2V_ERR_LIMIT, "%d scenes x %d tiles exceed int32", B, scene_tiles(G));
    G.scenes = B;
    G.scene_n = n;
    rc = check_ws(plan_ws, plan_bytes, carve_batch_plan(nullptr, B, n).bytes, "batch plan");
    if (rc != G2V_OK) return rc;
    p = carve_batch_plan(const_cast<void*>(plan_ws), B, n);
    return G2V_OK;
}

}  // namespace

extern "C" {

size_t g2v_batch_plan_workspace(int num_scenes, int n) {
    if (!batch_sizes_ok(num_scenes, n)) return 0;
    return carve_batch_plan(nullptr, num_scenes, n).bytes;
}

int g2v_batch_forward_plan(int num_scenes, int n, const float* means3D, const float* covariances,
                           const float voxel_size[3], const float voxel_range[6], float* cov_inv, int* valid_voxel_lb,
                           int* valid_voxel_ub, int* num_voxels_per_gaussian, int* g2t_offsets, void* plan_workspace,
                           size_t plan_workspace_bytes, int want_backward, long long* counts, void* stream) {
    g_err[0] = 0;
    if (!counts || !g2t_offsets) return fail(G2V_ERR_INVALID, "counts / g2t_offsets is null");
    Grid G;
    BatchPlan p;
    int rc = batch_setup(num_scenes, n, voxel_size, voxel_range, plan_workspace, plan_workspace_bytes, G, p);
    if (rc != G2V_OK) return rc;
    const int nt = num_scenes * n;
    if (nt > 0 && (!means3D || !covariances || !cov_inv || !valid_voxel_lb || !valid_voxel_ub || !num_voxels_per_gaussian))
        return fail(G2V_ERR_INVALID, "null input/output pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    rc = plan_launch(G, nt, means3D, covariances, cov_inv, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian,
                     p.goff, p.plan_ws, p.plan_bytes, want_backward ? p.bwd_ws : nullptr, p.totals, s);
    if (rc != G2V_OK) return rc;
    G2V_HIP(launch_scene_offsets(num_scenes, n, p.goff, want_backward ? p.totals + 1 : nullptr, g2t_offsets, counts, s));
    return G2V_OK;
}

size_t g2v_batch_forward_splat_workspace(int num_scenes, int n, int feat_dim, long long num_pairs,
                                         const float voxel_size[3], const float voxel_range[6]) {
    Grid G;
    if (!batch_sizes_ok(num_scenes, n) || make_grid(voxel_size, voxel_range, G) != G2V_OK) return 0;
    if (!batch_tiles_ok(G, num_scenes)) return 0;   // the batch's tile ids would overflow int32
    G.scenes = num_scenes;
    G.scene_n = n;
    return carve_splat(nullptr, num_scenes * n, num_pairs, G, feat_dim, true, true).bytes;
}

int g2v_batch_forward_splat(int num_scenes, int n, int feat_dim, const float* means3D, const float* opacity,
                            const void* features, int feat_dtype, const float voxel_size[3],
                            const float voxel_range[6], const float* cov_inv, const int* valid_voxel_lb,
                            const int* valid_voxel_ub, const void* plan_workspace, size_t plan_workspace_bytes,
                            long long num_pairs, int* g2t_tile_ids, float* density, void* grid_feats, int* t2g_tiles,
                            int* t2g_gauss, int* t2g_offsets, void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    Grid G;
    BatchPlan p;
    const int rc = batch_setup(num_scenes, n, voxel_size, voxel_range, plan_workspace, plan_workspace_bytes, G, p);
    if (rc != G2V_OK) return rc;
    return splat_impl(G, num_scenes * n, feat_dim, means3D, opacity, features, feat_dtype, nullptr, cov_inv, valid_voxel_lb,
                      valid_voxel_ub, p.goff, num_pairs, g2t_tile_ids, density, grid_feats, t2g_tiles, t2g_gauss,
                      t2g_offsets, workspace, workspace_bytes, stream);
}

size_t g2v_batch_backward_workspace(int num_scenes, int n, int feat_dim, long long num_pairs,
                                    long long num_region_pairs, const float voxel_size[3], const float voxel_range[6]) {
    Grid G;
    if (!batch_sizes_ok(num_scenes, n) || make_grid(voxel_size, voxel_range, G) != G2V_OK) return 0;
    if (!batch_tiles_ok(G, num_scenes)) return 0;   // the batch's tile ids would overflow int32
    G.scenes = num_scenes;
    G.scene_n = n;
    return backward_ws_bytes(G, num_scenes * n, feat_dim, num_pairs, num_region_pairs);
}

int g2v_batch_backward_prepare(int num_scenes, int n, int feat_dim, const float voxel_size[3],
                               const float voxel_range[6], const int* valid_voxel_lb, const int* valid_voxel_ub,
                               const void* features, int feat_dtype, long long num_pairs, long long num_region_pairs,
                               const int* t2g_tiles, const int* t2g_gauss, const void* plan_workspace,
                               size_t plan_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    Grid G;
    BatchPlan p;
    const int rc = batch_setup(num_scenes, n, voxel_size, voxel_range, plan_workspace, plan_workspace_bytes, G, p);
    if (rc != G2V_OK) return rc;
    return prepare_impl(num_scenes * n, feat_dim, voxel_size, voxel_range, valid_voxel_lb, valid_voxel_ub, features,
                        feat_dtype, num_pairs, num_region_pairs, t2g_tiles, t2g_gauss, p.bwd_ws, workspace,
                        workspace_bytes, stream, num_scenes);
}

int g2v_batch_backward(int num_scenes, int n, int feat_dim, const float* grad_density, const void* grad_feats,
                       const float* means3D, const float* opacity, const float* cov_inv, const float voxel_size[3],
                       const float voxel_range[6], const int* valid_voxel_lb, const int* valid_voxel_ub,
                       long long num_pairs, long long num_region_pairs, const float* density, const void* grid_feats,
                       const void* features, int feat_dtype, float* grad_means, float* grad_cov, float* grad_opacity,
                       void* grad_features, const int* t2g_tiles, const int* t2g_gauss, const int* t2g_offsets,
                       const void* plan_workspace, size_t plan_workspace_bytes, void* workspace,
                       size_t workspace_bytes, int prepared, void* stream) {
    g_err[0] = 0;
    Grid G;
    BatchPlan p;
    const int rc = batch_setup(num_scenes, n, voxel_size, voxel_range, plan_workspace, plan_workspace_bytes, G, p);
    if (rc != G2V_OK) return rc;
    if (prepared && feat_dim > 0 && n > 0 && num_pairs > 0 && !(t2g_tiles && t2g_gauss && t2g_offsets))
        return fail(G2V_ERR_INVALID, "a prepared backward needs the forward's Tile->Gaussian CSR");
    return backward_impl(num_scenes * n, feat_dim, grad_density, grad_feats, means3D, opacity, cov_inv, voxel_size,
                         voxel_range, valid_voxel_lb, valid_voxel_ub, nullptr, p.goff, nullptr, num_pairs,
                         num_region_pairs, density, grid_feats, features, feat_dtype, grad_means, grad_cov, grad_opacity,
                         grad_features, t2g_tiles, t2g_gauss, t2g_offsets, p.bwd_ws, workspace, workspace_bytes,
                         prepared != 0, stream, nullptr, num_scenes);
}

}  // extern "C"
