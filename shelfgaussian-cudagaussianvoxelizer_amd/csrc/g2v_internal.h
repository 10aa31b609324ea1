// Host-side declarations shared by the G2V translation units (not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "g2v_device.h"

namespace g2v {

// ---- workspace carving ------------------------------------------------------------------
struct Carver {
    char* base;
    size_t off = 0;
    size_t cap;
    Carver(void* p, size_t c) : base(static_cast<char*>(p)), cap(c) {}
    template <typename T>
    T* take(size_t count) {
        off = (off + 255) & ~size_t(255);
        T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
        off += count * sizeof(T);
        return p;
    }
    bool fits() const { return off <= cap; }
};

// ---- CSR build (g2v_csr.hip) ------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;
constexpr int kSortTile = kSortThreads * kSortRounds;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t scan_workspace(int64_t n);
// In-place or out-of-place scan of n int32 values (inclusive or exclusive); the int64 total
// is written to *total_dev (device pointer) when it is not null.
hipError_t scan_i32(const int* in, int* out, int64_t n, bool inclusive, long long* total_dev,
                    void* ws, hipStream_t s);

// Inclusive scans of two arrays in one launch when both fit one workgroup (else one after the
// other); the totals go to total_a / total_b (device-accessible pointers).
hipError_t scan_i32_pair(const int* in_a, int* out_a, int64_t n_a, long long* total_a, void* ws_a,
                         const int* in_b, int* out_b, int64_t n_b, long long* total_b, void* ws_b,
                         hipStream_t s);

// Boxes, inverse covariances and G->T row counts; with cell (non-null) also the cell counts of
// the boxes into cell_offsets[1..n] (cell_offsets[0] = 0), as launch_cell_count writes them.
hipError_t launch_boxes(const Grid& G, int n, const float* means, const float* cov, float* cov_inv,
                        int* lb, int* ub, int* nvox, int* g2t_offsets, const int* cell, int* cell_offsets,
                        hipStream_t s, long long* zero = nullptr, int nzero = 0);
// keys (optional): the batch's tile ids (sort keys) beside the scene-local tile_ids.
// drec (optional, with means, opacity and cov_inv): the packed record of every Gaussian that has
// G->T rows, for the forward's tile kernels.
hipError_t launch_fill_g2t(const Grid& G, int n, const int* lb, const int* ub,
                           const int* g2t_offsets, int* tile_ids, int* gauss_ids, hipStream_t s,
                           int* keys = nullptr, const float* means = nullptr, const float* opacity = nullptr,
                           const float* cov_inv = nullptr, DenParams* drec = nullptr);

// A batch of B scenes of n Gaussians: the per-scene G->T row offsets out (B x (n + 1)) and pair
// counts (counts[b], b < B; counts[B] = *mr_total, or 0 when mr_total is null) from the batch's
// offsets goff (B n + 1).
hipError_t launch_scene_offsets(int B, int n, const int* goff, const long long* mr_total, int* out,
                                long long* counts, hipStream_t s);
hipError_t launch_cell_count(int n, const int* lb, const int* ub, const int cell[3], int* offsets,
                             hipStream_t s);
// scene_n > 0 (a batch): the cells of Gaussian g are numbered from (g / scene_n) scene_cells.
hipError_t launch_fill_cells(int n, const int* lb, const int* ub, const int* offsets, const int cell[3],
                             const int ncells[3], int* cell_ids, int* pair_ids, int* gauss_ids,
                             hipStream_t s, int scene_n = 0, int scene_cells = 0);

int sort_key_bits(int num_tiles);
size_t sort_workspace(int64_t M, int num_tiles);
// Stable LSD radix sort of (key < num_tiles, value) pairs.  Inputs are not modified; the
// sorted pairs land in keys_out/vals_out.
hipError_t radix_sort_pairs(const int* keys_in, const int* vals_in, int* keys_out, int* vals_out,
                            int64_t M, int num_tiles, void* ws, hipStream_t s);
hipError_t launch_tile_offsets(const int* sorted_keys, int64_t M, int T, int* tile_offsets,
                               hipStream_t s);
hipError_t launch_rle(const int* tile_offsets, int T, int* unique_tiles, int* counts,
                      int* runs_offsets, int* num_runs, void* ws, hipStream_t s);

// The tiles whose list holds more than smax Gaussians (of the M pairs of T tiles), compacted into
// list[0 .. *count), in unspecified order; count is zeroed first.  cap >= long_tiles_bound(...).
hipError_t launch_long_tiles(const int* toff, int T, int M, int smax, int* count, int* list, int cap,
                             hipStream_t s);
// At most this many tiles hold more than smax of M pairs.
inline int long_tiles_bound(int64_t M, int T, int smax) {
    const int64_t b = M / (smax + 1);
    return (int)(b < T ? b : T);
}

// n ints of value v (a kernel, not a memset node: safe where a stream may be captured).
hipError_t launch_fill_i32(int64_t n, int v, int* dst, hipStream_t s);

// ---- forward (g2v_forward.hip) ------------------------------------------------------------
// Channels of the packed feature rows of the forward (a multiple of one wave's 128 channels).
constexpr int kPackedChannelAlign = 128;
inline int packed_channels(int C) { return (C + kPackedChannelAlign - 1) & ~(kPackedChannelAlign - 1); }
// Packed feature rows are addressed with 32-bit byte offsets.
inline bool packed_fits(int n, int C) { return (int64_t)(n + 1) * packed_channels(C) * 4 <= (int64_t)UINT32_MAX; }
// The split feature rows of the backward (32-channel chunks, 4 bytes per channel) likewise.
inline bool split_rows_fit(int n, int C) { return (int64_t)(n + 1) * ((C + 31) / 32) * 128 <= (int64_t)UINT32_MAX; }
// The feature backward reads grad_feats per tile through 32-bit byte offsets from the tile's
// origin; they span at most 4 x-slices of the grid.
inline bool region_offsets_fit(const Grid& G, int C) {
    return (int64_t)16 * G.dims[1] * G.dims[2] * C < ((int64_t)1 << 31);
}

// Longest tile list that the short-list kernels (k_fwd_short, k_bwd_tile_short) take; longer lists
// go to the matrix-core kernels.  It depends on C alone (never on the rest of the problem), so a
// tile takes the same kernel in every call: 64 Gaussians up to 256 channels, where the short
// kernels' float32 products stay cheaper than a tile slot of the matrix-core kernels, 32 above.
inline int short_list_max(int C) { return C <= 256 ? 64 : 32; }

// drec: the packed records launch_fill_g2t wrote.
hipError_t launch_forward_density(const Grid& G, const DenParams* drec, const int* tile_offsets,
                                  const int* sorted_gauss, int M, float* density, hipStream_t s);
// The features as packed bf16 (hi, lo) pairs for k_fwd_feats (packed_channels(C) 32-bit words per
// row, plus a zero row); it depends on the features alone.
hipError_t launch_split_pack(int n, int C, const void* features, int fdt, uint32_t* fpk, hipStream_t s);
// fpk: launch_split_pack's output for these features, queued before on s.
hipError_t launch_forward_feats(const Grid& G, int C, const float* means, const float* opacity,
                                const float* cov_inv, const int* lb, const int* ub,
                                const int* tile_offsets, const int* sorted_gauss, int M, int n,
                                const void* features, int fdt, const uint32_t* fpk, const DenParams* drec,
                                float* density, void* grid_feats, int* tl_ws, hipStream_t s);
// ints of the long-tile list workspace (tl_ws) of a forward or backward with features.
inline int long_list_ints(int64_t M, int T, int C) { return 1 + long_tiles_bound(M, T, short_list_max(C)); }

// ---- backward (g2v_backward.hip) ----------------------------------------------------------
hipError_t launch_backward_density(const Grid& G, int n, const float* grad_density,
                                   const float* means, const float* opacity, const float* cov_inv,
                                   const int* lb, const int* ub, float* grad_means, float* grad_cov,
                                   float* grad_opacity, hipStream_t s);
size_t backward_plan_workspace(int n);
// Counts the (region, Gaussian) pairs of the feature-gradient phase; synchronises the stream.
hipError_t backward_plan(const Grid& G, int n, const int* lb, const int* ub, void* plan_ws,
                         long long* num_region_pairs, hipStream_t s);
// The same without the synchronisation: the count lands in *mr_host once the stream reaches it.
hipError_t backward_plan_async(const Grid& G, int n, const int* lb, const int* ub, void* plan_ws,
                               long long* mr_host, hipStream_t s);
// The plan's cell counts (n + 1 ints), its scan workspace and the region cell size, for a caller
// that fills and scans them itself (the forward plan does, in its own launches).
int* backward_plan_cells(const Grid& G, void* plan_ws, int n, int cell[3], void** scan_ws);
size_t backward_feats_workspace(const Grid& G, int n, int C, int64_t M, int64_t MR);
// The part of the feature backward that needs no upstream gradient: split features, the
// Region -> Gaussian CSR and the row table of phase B (into ws).
hipError_t launch_backward_prepare(const Grid& G, int n, int C, const void* features, int fdt, const int* lb,
                                   const int* ub, int64_t M, const int* sorted_tiles, const int* sorted_gauss,
                                   const void* plan_ws, int64_t MR, void* ws, hipStream_t s);
// The cosine loss's gradient as the feature backward's upstream gradient, formed on chip per voxel
// as k1 target + k2 grid_feats with (k1, k2) = coef[2v .. 2v+1] * grad_loss[0] * inv_count: coef
// as launch_cosine_forward writes it, grad_loss a device scalar, inv_count = 1 / count (0 when
// count = 0).  float32 target and grid_feats with C % 4 == 0 and 16-byte aligned rows.
struct CosG {
    const float* tgt;
    const float* coef;
    const float* grad_loss;
    float inv_count;
};

// prepared: launch_backward_prepare already ran on ws for the same Gaussians and CSR.
// cos (optional): the upstream feature gradient is the cosine loss's (grad_feats unused).
hipError_t launch_backward_feats(const Grid& G, int n, int C, const float* grad_density,
                                 const void* grad_feats, const float* means, const float* opacity,
                                 const float* cov_inv, const int* lb, const int* ub,
                                 const int* g2t_offsets, int64_t M, const int* tile_offsets,
                                 const int* sorted_tiles, const int* sorted_gauss, const float* density,
                                 const void* grid_feats, const void* features, int fdt,
                                 const void* plan_ws, int64_t MR, float* grad_means, float* grad_cov,
                                 float* grad_opacity, void* grad_features, void* ws, bool prepared,
                                 hipStream_t s, const CosG* cos = nullptr);

// ---- feature cosine loss (g2v_cosine.hip) --------------------------------------------------
size_t cosine_workspace(int64_t V);
// 4-element vector rows: C % 4 == 0 and every non-null pointer aligned to 4 elements of esize bytes.
bool cosine_vec_ok(int C, int esize, const void* a, const void* b, const void* c);
// Mean loss over the valid voxels into *loss and their number into *count (device pointers); p and g
// hold elements of type fdt (kDtF32 or kDtBF16).  coef (V x 2 floats, optional): the unscaled gradient
// coefficients (c1, c2) of every voxel, 0 where the loss does not count the voxel.
hipError_t launch_cosine_forward(int64_t V, int C, const float* label, const uint8_t* mask, const void* p,
                                 const void* g, int fdt, float* loss, int* count, void* ws, hipStream_t s,
                                 float* coef = nullptr);
// The same forward with the block partials in a file-scope device array of
// cosine_scratch_bytes() bytes (per GPU) instead of a workspace: allocates nothing.
size_t cosine_scratch_bytes();
hipError_t launch_cosine_forward_noalloc(int64_t V, int C, const float* label, const uint8_t* mask, const void* p,
                                         const void* g, int fdt, float* loss, int* count, hipStream_t s);
// dloss/dp into grad_p (V x C, type fdt), grad_out a device scalar, inv_count = 1 / count (0 when
// count = 0).
hipError_t launch_cosine_backward(int64_t V, int C, const float* label, const uint8_t* mask, const void* p,
                                  const void* g, int fdt, const float* grad_out, float inv_count, void* grad_p,
                                  hipStream_t s);

// ---- covariances from scales and rotations (g2v_covariance.hip) ----------------------------
hipError_t launch_cov_from_scale_rot(int n, const float* scales, const float* rotations, float* cov, hipStream_t s);
hipError_t launch_cov_from_scale_rot_bwd(int n, const float* scales, const float* rotations, const float* grad_cov,
                                         float* grad_scales, float* grad_rotations, hipStream_t s);

// Brackets one kernel launch with HIP events when profiling is enabled (g2v_profile.hip).
class ProfMark {
  public:
    ProfMark(const char* name, hipStream_t s);
    ~ProfMark();
    ProfMark(const ProfMark&) = delete;
    ProfMark& operator=(const ProfMark&) = delete;

  private:
    const char* name_;
    hipStream_t s_;
    void* a_;
};

#define G2V_LAUNCH(kernel, grid, block, shmem, stream, ...)                      \
    do {                                                                        \
        ::g2v::ProfMark g2v_pm_(#kernel, stream);                               \
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);     \
    } while (0)

// XCD-aware block -> item mapping.  Workgroups are dealt to the 8 XCDs round robin (block b to XCD
// b % 8); here every run of 64 consecutive items goes to one XCD (neighbouring tiles share Gaussians,
// hence their rows in that XCD's L2), and the runs are dealt round robin, so that a grid whose work
// sits in a few places (a sparse scene) still spreads over all XCDs.  A last partial group of
// 8 x 64 blocks keeps the identity order.  A bijection on [0, nblocks).
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
    constexpr int kXcd = 8, kRun = 64, kGroup = kXcd * kRun;
    const int g = b / kGroup;
    if ((g + 1) * kGroup > nblocks) return b;
    const int r = b - g * kGroup;
    return g * kGroup + (r % kXcd) * kRun + r / kXcd;
}

}  // namespace g2v
