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
// grid_feats, pseudo_gt and the gradient share one element type T, float or bfloat16 (half the
// bytes); the arithmetic is float, and a bfloat16 gradient is the float value rounded to nearest
// even.
#include "../../include/g2v.h"
#include "g2v_internal.h"

#include <mutex>
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

// Four consecutive elements 4q..4q+3 as floats (one 16-byte or 8-byte non-temporal load), and the
// matching store; single elements for the unaligned path.
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ f32x4 load4(const T* __restrict__ p, int64_t q) {
    if constexpr (std::is_same<T, float>::value) return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + q);
    else return __builtin_convertvector(__builtin_nontemporal_load(reinterpret_cast<const bf16x4_t*>(p) + q), f32x4);
}
template <typename T>
__device__ __forceinline__ void store4(T* __restrict__ p, int64_t q, f32x4 v) {
    if constexpr (std::is_same<T, float>::value) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p) + q);
    else __builtin_nontemporal_store(__builtin_convertvector(v, bf16x4_t), reinterpret_cast<bf16x4_t*>(p) + q);
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
template <int L, bool VEC, typename T>
__device__ __forceinline__ void row_sums(const T* __restrict__ p, const T* __restrict__ g, int C,
                                         int gl, float& dot, float& pp, float& gg) {
    float d = 0.0f, a = 0.0f, b = 0.0f;
    if constexpr (VEC) {
        const int C4 = C >> 2;
#pragma unroll 4
        for (int c = gl; c < C4; c += L) {
            const f32x4 x = load4(p, c);
            const f32x4 y = load4(g, c);
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
            const float x = (float)p[c], y = (float)g[c];
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
// With coef, the unscaled gradient coefficients (c1, c2) of every voxel of the range are written
// as well ((0, 0) for a voxel the loss does not count), for a backward that forms the gradient
// c1 g + c2 p itself.
template <int L, bool VEC, typename T>
__global__ void __launch_bounds__(kCosThreads) k_cos_fwd(int64_t V, int C, int vpb,
                                                          const float* __restrict__ label,
                                                          const uint8_t* __restrict__ mask,
                                                          const T* __restrict__ p,
                                                          const T* __restrict__ g,
                                                          float* __restrict__ part_loss,
                                                          int* __restrict__ part_cnt,
                                                          float* __restrict__ coef) {
    constexpr int G = kCosThreads / L;
    __shared__ float s_loss[G];
    __shared__ int s_cnt[G];
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    float lsum = 0.0f;
    int cnt = 0;
    for (int64_t v = v0 + grp; v < v1; v += G) {
        if (!cos_valid(label, mask, v)) {
            if (coef && gl == 0) *reinterpret_cast<float2*>(coef + 2 * v) = make_float2(0.0f, 0.0f);
            continue;
        }
        float dot, pp, gg;
        row_sums<L, VEC, T>(p + v * C, g + v * C, C, gl, dot, pp, gg);
        lsum += cos_loss(dot, pp, gg);
        ++cnt;
        if (coef && gl == 0) {
            float c1, c2;
            cos_coefs(dot, pp, gg, 1.0f, c1, c2);
            *reinterpret_cast<float2*>(coef + 2 * v) = make_float2(c1, c2);
        }
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
template <int L, int NV, typename T>
__global__ void __launch_bounds__(kCosThreads) k_cos_bwd(int64_t V, int C, int vpb,
                                                          const float* __restrict__ label,
                                                          const uint8_t* __restrict__ mask,
                                                          const T* __restrict__ p,
                                                          const T* __restrict__ g,
                                                          const float* __restrict__ grad_out, float inv_count,
                                                          T* __restrict__ grad_p) {
    constexpr int G = kCosThreads / L;
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const int C4 = C >> 2;
    const float scale = grad_out[0] * inv_count;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    for (int64_t v = v0 + grp; v < v1; v += G) {
        T* out = grad_p + v * C;
        if (!cos_valid(label, mask, v)) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int c = gl + L * j;
                if (c < C4) store4(out, c, f32x4{});
            }
            continue;
        }
        const T* pr = p + v * C;
        const T* gr = g + v * C;
        f32x4 x[NV], y[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = gl + L * j;
            x[j] = c < C4 ? load4(pr, c) : f32x4{};
            y[j] = c < C4 ? load4(gr, c) : f32x4{};
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
            if (c < C4) store4(out, c, k1 * y[j] + k2 * x[j]);
        }
    }
}

// Backward for any C and alignment: row sums first, then a second pass over the row (re-read).
template <int L, typename T>
__global__ void __launch_bounds__(kCosThreads) k_cos_bwd_any(int64_t V, int C, int vpb,
                                                              const float* __restrict__ label,
                                                              const uint8_t* __restrict__ mask,
                                                              const T* __restrict__ p,
                                                              const T* __restrict__ g,
                                                              const float* __restrict__ grad_out,
                                                              float inv_count, T* __restrict__ grad_p) {
    constexpr int G = kCosThreads / L;
    const int grp = threadIdx.x / L, gl = threadIdx.x % L;
    const float scale = grad_out[0] * inv_count;
    const int64_t v0 = (int64_t)blockIdx.x * vpb;
    const int64_t v1 = min(v0 + vpb, V);
    for (int64_t v = v0 + grp; v < v1; v += G) {
        T* out = grad_p + v * C;
        if (!cos_valid(label, mask, v)) {
            for (int c = gl; c < C; c += L) out[c] = (T)0.0f;
            continue;
        }
        const T* pr = p + v * C;
        const T* gr = g + v * C;
        float dot, pp, gg;
        row_sums<L, false, T>(pr, gr, C, gl, dot, pp, gg);
        float k1, k2;
        cos_coefs(dot, pp, gg, scale, k1, k2);
        for (int c = gl; c < C; c += L) out[c] = (T)(k1 * (float)gr[c] + k2 * (float)pr[c]);
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

template <int L, int NV, typename T>
hipError_t launch_bwd_nv(int64_t V, int C, int vpb, unsigned blocks, const float* label, const uint8_t* mask,
                         const T* p, const T* g, const float* grad_out, float inv_count, T* grad_p,
                         hipStream_t s) {
    G2V_LAUNCH((k_cos_bwd<L, NV, T>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask, p, g,
               grad_out, inv_count, grad_p);
    return hipGetLastError();
}

// f on the element type of fdt (float or bfloat16).
template <typename F>
hipError_t dispatch_type(int fdt, F&& f) {
    if (fdt == kDtBF16) return f(__bf16{});
    return f(float{});
}

}  // namespace

size_t cosine_workspace(int64_t V) {
    (void)V;
    return (size_t)kCosMaxBlocks * (sizeof(float) + sizeof(int)) + 512;
}

bool cosine_vec_ok(int C, int esize, const void* a, const void* b, const void* c) {
    // 4-element vectors: 16-byte (float) or 8-byte (bfloat16) aligned rows
    const uintptr_t m = (uintptr_t)(4 * esize - 1);
    const auto al = [m](const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & m) == 0; };
    return (C & 3) == 0 && al(a) && al(b) && al(c);
}

hipError_t launch_cosine_forward(int64_t V, int C, const float* label, const uint8_t* mask, const void* p_,
                                 const void* g_, int fdt, float* loss, int* count, void* ws, hipStream_t s,
                                 float* coef) {
    Carver c(ws, (size_t)-1);
    float* part_loss = c.take<float>(kCosMaxBlocks);
    int* part_cnt = c.take<int>(kCosMaxBlocks);
    const int esize = fdt == kDtBF16 ? 2 : 4;
    const bool vec = cosine_vec_ok(C, esize, p_, g_, nullptr);
    const int L = lanes_for(vec ? C / 4 : C);
    const int vpb = voxels_per_block(V, L);
    const int blocks = V > 0 ? (int)ceil_div(V, vpb) : 0;
    if (blocks > 0) {
        const hipError_t e = dispatch_type(fdt, [&](auto tv) -> hipError_t {
            using T = decltype(tv);
            const T* p = static_cast<const T*>(p_);
            const T* g = static_cast<const T*>(g_);
            return dispatch_lanes(L, [&](auto Lc) -> hipError_t {
                constexpr int LL = decltype(Lc)::value;
                if (vec)
                    G2V_LAUNCH((k_cos_fwd<LL, true, T>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label,
                               mask, p, g, part_loss, part_cnt, coef);
                else
                    G2V_LAUNCH((k_cos_fwd<LL, false, T>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label,
                               mask, p, g, part_loss, part_cnt, coef);
                return hipGetLastError();
            });
        });
        if (e != hipSuccess) return e;
    }
    G2V_LAUNCH(k_cos_final, dim3(1), dim3(kCosFinalThreads), 0, s, blocks, (const float*)part_loss,
               (const int*)part_cnt, loss, count);
    return hipGetLastError();
}

hipError_t launch_cosine_backward(int64_t V, int C, const float* label, const uint8_t* mask, const void* p_,
                                  const void* g_, int fdt, const float* grad_out, float inv_count, void* grad_p_,
                                  hipStream_t s) {
    if (V == 0 || C == 0) return hipSuccess;
    const int esize = fdt == kDtBF16 ? 2 : 4;
    const bool vec = cosine_vec_ok(C, esize, p_, g_, grad_p_);
    const int L = lanes_for(vec ? C / 4 : C);
    const int NV = vec ? (int)ceil_div(C / 4, L) : 0;
    const int vpb = voxels_per_block(V, L);
    const unsigned blocks = (unsigned)ceil_div(V, vpb);
    return dispatch_type(fdt, [&](auto tv) -> hipError_t {
        using T = decltype(tv);
        const T* p = static_cast<const T*>(p_);
        const T* g = static_cast<const T*>(g_);
        T* grad_p = static_cast<T*>(grad_p_);
        if (vec && NV <= kCosMaxNv) {
            return dispatch_lanes(L, [&](auto Lc) -> hipError_t {
                constexpr int LL = decltype(Lc)::value;
                if constexpr (LL < 64) {
                    // small rows: one vector per lane
                    return launch_bwd_nv<LL, 1, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                } else {
                    switch (NV) {
                        case 1: return launch_bwd_nv<64, 1, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 2: return launch_bwd_nv<64, 2, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 3: return launch_bwd_nv<64, 3, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 4: return launch_bwd_nv<64, 4, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 5: return launch_bwd_nv<64, 5, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 6: return launch_bwd_nv<64, 6, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        case 7: return launch_bwd_nv<64, 7, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                        default: return launch_bwd_nv<64, 8, T>(V, C, vpb, blocks, label, mask, p, g, grad_out, inv_count, grad_p, s);
                    }
                }
            });
        }
        return dispatch_lanes(L, [&](auto Lc) -> hipError_t {
            constexpr int LL = decltype(Lc)::value;
            G2V_LAUNCH((k_cos_bwd_any<LL, T>), dim3(blocks), dim3(kCosThreads), 0, s, V, C, vpb, label, mask, p, g,
                       grad_out, inv_count, grad_p);
            return hipGetLastError();
        });
    });
}

// ---- forward without allocation ------------------------------------------------------------
// The per-block partial sums of a forward live in this file-scope array instead of a caller's
// workspace: one copy per GPU, held until the process ends.  A forward launches at most
// kCosMaxBlocks blocks whatever the voxel count (voxels_per_block grows with it), and every block
// writes its own partial, so a call never reads what an earlier call left.  Calls that overlap on
// one GPU share the array and race.
constexpr size_t kCosPartBytes = (size_t)kCosMaxBlocks * sizeof(float);
constexpr size_t kCosScratchBytes = 2 * ((kCosPartBytes + 255) & ~size_t(255));
static __device__ __align__(256) unsigned char scratch[kCosScratchBytes];

size_t cosine_scratch_bytes() { return kCosScratchBytes; }

// Device address of `scratch` on the current device, looked up once per device with that device
// current (in host code the array's name is not a device address).
static hipError_t scratch_address(void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = p;
    }
    *out = addr[dev];
    return hipSuccess;
}

hipError_t launch_cosine_forward_noalloc(int64_t V, int C, const float* label, const uint8_t* mask, const void* p,
                                         const void* g, int fdt, float* loss, int* count, hipStream_t s) {
    // the partials of the largest grid a forward can see fit the array (checked, not assumed)
    const int esize = fdt == kDtBF16 ? 2 : 4;
    const bool vec = cosine_vec_ok(C, esize, p, g, nullptr);
    const int L = lanes_for(vec ? C / 4 : C);
    const int64_t blocks = V > 0 ? ceil_div(V, voxels_per_block(V, L)) : 0;
    if (blocks > kCosMaxBlocks) return hipErrorInvalidValue;
    void* ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return e;
    return launch_cosine_forward(V, C, label, mask, p, g, fdt, loss, count, ws, s);
}

}  // namespace g2v
