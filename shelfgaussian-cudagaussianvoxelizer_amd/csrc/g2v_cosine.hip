// Voxel-wise feature cosine loss and its gradient with respect to the voxel features: the consumer
// of grid_feats in ShelfGaussian (reference src/cuda_feats_loss.cu:45-367).
//
// For voxel v with p = grid_feats[v, :], g = pseudo_gt[v, :] (C channels):
//     valid_v = occ_mask[v] && label[v] > 0                                  (.cu:67-68, :255)
//     loss_v  = 1 - dot(p, g) / (sqrt(max(|p|^2, eps)) * sqrt(max(|g|^2, eps)) + eps)   (.cu:94-99)
//     loss    = sum_{valid} loss_v / count_valid   (0 when no voxel is valid)          (.cu:205-212)
//     dloss/dp = grad_out / count * (c1 g + c2 p),  c1 = -1/D,  D = a b + eps,
//                c2 = |p|^2 > eps ? dot b / (a D D) : 0,  a = |p|, b = |g| clamped  (.cu:278-291)
// and dloss/dp = 0 on invalid voxels (.cu:255-261).
//
// Layout: one group of L lanes (L a power of two, 4..64) per voxel, each lane reading 16-byte
// vectors of the voxel's row; the three row sums are combined with an xor butterfly inside the
// group.  The reference spends one 256-thread block per voxel and reduces through shared memory;
// here a 256-thread block walks a fixed range of voxels with 256/L groups and the loss is summed
// in a fixed order (group, then block, then one final workgroup), so it is deterministic (the
// reference sums with float atomics).  Everything is a single streaming pass over HBM: the
// forward reads p and g once (8 C bytes per valid voxel), the backward reads them once more and
// writes the gradient with non-temporal stores (12 C bytes per valid voxel, 4 C per other voxel).
#include "../../include/g2v.h"
#include "g2v_internal.h"

#include <type_traits>

namespace g2v {
namespace {

constexpr int kCosThreads = 256;
constexpr int kCosMaxBlocks = 4096;     // forward partial sums (one per block)
constexpr int kCosFinalThreads = 1024;
constexpr int kCosMaxNv = 8;            // 16-byte vectors per lane kept in registers (C <= 2048)

__device__ __forceinline__ bool cos_valid(const float* __restrict__ label, const uint8_t* __restrict__ mask,
                                          int64_t v) {
    return mask[v] != 0 && label[v] > 0.0f;
}

// Sum over the L lanes of a group (xor butterfly; every lane of the group gets the total).
template <int L>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
    for (int m = L / 2; m > 0; m >>= 1) x += __shfl_xor(x, m, kWave);
    return x;
}

__device__ __forceinline__ float cos_loss(float dot, float pp, float gg) {
    const float pn = sqrtf(fmaxf(pp, kEps));
    const float gn = sqrtf(fmaxf(gg, kEps));
    return 1.0f - dot / (pn * gn + kEps);
}

// Gradient coefficients of (g, p), already scaled by grad_out / count (reference .cu:278-291).
__device__ __forceinline__ void cos_coefs(float dot, float pp, float gg, float scale, float& k1, float& k2) {
    const float a = sqrtf(fmaxf(pp, kEps));
    const float b = sqrtf(fmaxf(gg, kEps));
    const float D = a * b + kEps;
    const float c1 = -1.0f / D;
    const float c2 = pp > kEps ? (dot * b) / (a * D * D) : 0.0f;
    k1 = c1 * scale;
    k2 = c2 * scale;
}

// Row sums dot(p,g), |p|^2, |g|^2 of one voxel by a group of L lanes (lane gl of the group).
template <int L, bool VEC>
__device__ __forceinline__ void row_sums(const float* __restrict__ p, const float* __restrict__ g, int C,
                                         int gl, float& dot, float& pp, float& gg) {
    float d = 0.0f, a = 0.0f, b = 0.0f;
    if constexpr (VEC) {
        const f32x4* p4 = reinterpret_cast<const f32x4*>(p);
        const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
        const int C4 = C >> 2;
#pragma unroll 4
        for (int c = gl; c < C4; c += L) {
            const f32x4 x = __builtin_nontemporal_load(p4 + c);
            const f32x4 y = __builtin_nontemporal_load(g4 + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                d += x[i] * y[i];
                a += x[i] * x[i];
                b += y[i] * y[i];
            }
        }
    } else {
#pragma unroll 4
        for (int c = gl; c < C; c += L) {
            const float x = p[c], y = g[c];
            d += x * y;
            a += x * x;
            b += y * y;
        }
    }
    dot = group_sum<L>(d);
    pp = group_sum<L>(a);
    gg = group_sum<L>(b);
}

// Forward: block b sums the losses and counts the valid voxels of voxels [b vpb, (b+1) vpb).
template <int L, bool VEC>
__global__ void __launch_bounds__(kCosThreads) k_cos_fwd(int64_t V, int C, int vpb,
                                                          const float* __restrict__ label,
                                                          const uint8_t* __restrict__ mask,
                                                          const float* __restrict__ p,
                                                          const float* __restrict__ g,
                                                          float* __restrict__ part_loss,
                                                          int* __restrict__ part_cnt) {
    constexpr int G = kCosThreads / L;
    __shared__ float s_loss[G];
    __shared__ int s_cnt[G];
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    float lsum = 0.0f;
    int cnt = 0;
    for (int64_t v = v0 + grp; v < v1; v += G) {
        if (!cos_valid(label, mask, v)) continue;
        float dot, pp, gg;
        row_sums<L, VEC>(p + v * C, g + v * C, C, gl, dot, pp, gg);
        lsum += cos_loss(dot, pp, gg);
        ++cnt;
    }
    if (gl == 0) {
        s_loss[grp] = lsum;
        s_cnt[grp] = cnt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        int n = 0;
#pragma unroll
        for (int k = 0; k < G; ++k) {
            t += s_loss[k];
            n += s_cnt[k];
        }
        part_loss[blockIdx.x] = t;
        part_cnt[blockIdx.x] = n;
    }
}

// Sum of the block partials in a fixed order; loss = sum / count (0 without valid voxels).
__global__ void __launch_bounds__(kCosFinalThreads) k_cos_final(int nparts, const float* __restrict__ part_loss,
                                                                 const int* __restrict__ part_cnt,
                                                                 float* __restrict__ loss, int* __restrict__ count) {
    __shared__ double s_l[kCosFinalThreads];
    __shared__ long long s_n[kCosFinalThreads];
    double t = 0.0;
    long long n = 0;
    for (int i = threadIdx.x; i < nparts; i += kCosFinalThreads) {
        t += (double)part_loss[i];
        n += part_cnt[i];
    }
    s_l[threadIdx.x] = t;
    s_n[threadIdx.x] = n;
    __syncthreads();
    for (int w = kCosFinalThreads / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) {
            s_l[threadIdx.x] += s_l[threadIdx.x + w];
            s_n[threadIdx.x] += s_n[threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int c = (int)s_n[0];
        *count = c;
        *loss = c > 0 ? (float)s_l[0] / (float)c : 0.0f;
    }
}

// Backward, rows held in registers (C <= 4 L NV, 16-byte aligned rows): one voxel per group and
// iteration over the block's voxel range.
template <int L, int NV>
__global__ void __launch_bounds__(kCosThreads) k_cos_bwd(int64_t V, int C, int vpb,
                                                          const float* __restrict__ label,
                                                          const uint8_t* __restrict__ mask,
                                                          const float* __restrict__ p,
                                                          const float* __restrict__ g,
                                                          const float* __restrict__ grad_out, float inv_count,
                                                          float* __restrict__ grad_p) {
    constexpr int G = kCosThreads / L;
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const int C4 = C >> 2;
    const float scale = grad_out[0] * inv_count;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    for (int64_t v = v0 + grp; v < v1; v += G) {
        f32x4* out = reinterpret_cast<f32x4*>(grad_p + v * C);
        if (!cos_valid(label, mask, v)) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int c = gl + L * j;
                if (c < C4) __builtin_nontemporal_store(f32x4{}, out + c);
            }
            continue;
        }
        const f32x4* p4 = reinterpret_cast<const f32x4*>(p + v * C);
        const f32x4* g4 = reinterpret_cast<const f32x4*>(g + v * C);
        f32x4 x[NV], y[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = gl + L * j;
            x[j] = c < C4 ? __builtin_nontemporal_load(p4 + c) : f32x4{};
            y[j] = c < C4 ? __builtin_nontemporal_load(g4 + c) : f32x4{};
        }
        float d = 0.0f, a = 0.0f, b = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                d += x[j][i] * y[j][i];
                a += x[j][i] * x[j][i];
                b += y[j][i] * y[j][i];
            }
        float k1, k2;
        cos_coefs(group_sum<L>(d), group_sum<L>(a), group_sum<L>(b), scale, k1, k2);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = gl + L * j;
            if (c < C4) __builtin_nontemporal_store(k1 * y[j] + k2 * x[j], out + c);
        }
    }
}

// Backward for any C and alignment: row sums first, then a second pass over the row (re-read).
template <int L>
__global__ void __launch_bounds__(kCosThreads) k_cos_bwd_any(int64_t V, int C, int vpb,
                                                              const float* __restrict__ label,
                                                              const uint8_t* __restrict__ mask,
                                                              const float* __restrict__ p,
                                                              const float* __restrict__ g,
                                                              const float* __restrict__ grad_out,
                                                              float inv_count, float* __restrict__ grad_p) {
    constexpr int G = kCosThreads / L;
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const float scale = grad_out[0] * inv_count;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    for (int64_t v = v0 + grp; v < v1; v += G) {
        float* out = grad_p + v * C;
        if (!cos_valid(label, mask, v)) {
            for (int c = gl; c < C; c += L) out[c] = 0.0f;
            continue;
        }
        const float* pr = p + v * C;
        const float* gr = g + v * C;
        float dot, pp, gg;
        row_sums<L, false>(pr, gr, C, gl, dot, pp, gg);
        float k1, k2;
        cos_coefs(dot, pp, gg, scale, k1, k2);
        for (int c = gl; c < C; c += L) out[c] = k1 * gr[c] + k2 * pr[c];
    }
}

// Lanes per voxel: the smallest power of two in [4, 64] covering the row's vectors (or scalars).
int lanes_for(int units) {
    int L = 4;
    while (L < 64 && L < units) L <<= 1;
    return L;
}

// Voxels per block: a multiple of the group count, with at most kCosMaxBlocks blocks.
int voxels_per_block(int64_t V, int L) {
    const int G = kCosThreads / L;
    const int64_t per = ceil_div(V, kCosMaxBlocks);
    return (int)(ceil_div(per > 0 ? per : 1, G) * G);
}

template <typename F>
hipError_t dispatch_lanes(int L, F&& f) {
    switch (L) {
        case 4: return f(std::integral_constant<int, 4>{});
        case 8: return f(std::integral_constant<int, 8>{});
        case 16: return f(std::integral_constant<int, 16>{});
        case 32: return f(std::integral_constant<int, 32>{});
        default: return f(std::integral_constant<int, 64>{});
    }
}

template <int L, int NV>
hipError_t launch_bwd_nv(int64_t V, int C, int vpb, unsigned blocks, const float* label, const uint8_t* mask,
                         const float* p, const float* g, const float* grad_out, float inv_count, float* grad_p,
                         hipStream_t s) {
    G2V_LAUNCH((k_cos_bwd<L, NV>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask, p, g,
               grad_out, inv_count, grad_p);
    return hipGetLastError();
}

}  // namespace

size_t cosine_workspace(int64_t V) {
    (void)V;
    return (size_t)kCosMaxBlocks * (sizeof(float) + sizeof(int)) + 512;
}

bool cosine_vec_ok(int C, const void* a, const void* b, const void* c) {
    const auto al = [](const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return (C & 3) == 0 && al(a) && al(b) && al(c);
}

hipError_t launch_cosine_forward(int64_t V, int C, const float* label, const uint8_t* mask, const float* p,
                                 const float* g, float* loss, int* count, void* ws, hipStream_t s) {
    Carver c(ws, (size_t)-1);
    float* part_loss = c.take<float>(kCosMaxBlocks);
    int* part_cnt = c.take<int>(kCosMaxBlocks);
    const bool vec = cosine_vec_ok(C, p, g, nullptr);
    const int L = lanes_for(vec ? C / 4 : C);
    const int vpb = voxels_per_block(V, L);
    const int blocks = V > 0 ? (int)ceil_div(V, vpb) : 0;
    if (blocks > 0) {
        const hipError_t e = dispatch_lanes(L, [&](auto Lc) -> hipError_t {
            constexpr int LL = decltype(Lc)::value;
            if (vec)
                G2V_LAUNCH((k_cos_fwd<LL, true>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask,
                           p, g, part_loss, part_cnt);
            else
                G2V_LAUNCH((k_cos_fwd<LL, false>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask,
                           p, g, part_loss, part_cnt);
            return hipGetLastError();
        });
        if (e != hipSuccess) return e;
    }
    G2V_LAUNCH(k_cos_final, dim3(1), dim3(kCosFinalThreads), 0, s, blocks, (const float*)part_loss,
               (const int*)part_cnt, loss, count);
    return hipGetLastError();
}

hipError_t launch_cosine_backward(int64_t V, int C, const float* label, const uint8_t* mask, const float* p,
                                  const float* g, const float* grad_out, float inv_count, float* grad_p,
                                  hipStream_t s) {
    if (V == 0 || C == 0) return hipSuccess;
    const bool vec = cosine_vec_ok(C, p, g, grad_p);
    const int L = lanes_for(vec ? C / 4 : C);
    const int NV = vec ? (int)ceil_div(C / 4, L) : 0;
    const int vpb = voxels_per_block(V, L);
    const unsigned blocks = (unsigned)ceil_div(V, vpb);
    if (vec && NV <= kCosMaxNv) {
        return dispatch_lanes(L, [&](auto Lc) -> hipError_t {
            constexpr int LL = decltype(Lc)::value;
            if constexpr (LL < 64) {
                // small rows: one vector per lane
                return launch_bwd_nv<LL, 1>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
            } else {
                switch (NV) {
                    case 1: return launch_bwd_nv<64, 1>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 2: return launch_bwd_nv<64, 2>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 3: return launch_bwd_nv<64, 3>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 4: return launch_bwd_nv<64, 4>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 5: return launch_bwd_nv<64, 5>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 6: return launch_bwd_nv<64, 6>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    case 7: return launch_bwd_nv<64, 7>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    default: return launch_bwd_nv<64, 8>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                }
            }
        });
    }
    return dispatch_lanes(L, [&](auto Lc) -> hipError_t {
        constexpr int LL = decltype(Lc)::value;
        G2V_LAUNCH((k_cos_bwd_any<LL>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask, p, g,
                   grad_out, inv_count, grad_p);
        return hipGetLastError();
    });
}

}  // namespace g2v
