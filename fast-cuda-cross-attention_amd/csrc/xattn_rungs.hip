// The fp32 "ladder" entry points behind launch_naive_kernel,
// launch_parallel_kernel and launch_tiled_kernel.  They exist for API
// completeness and as readable correctness baselines; the fast path is the
// MFMA kernel in xattn_flash_f32.hip.  All three are written for 64-lane
// wavefronts and any dim in [1, 768] (naive: any dim >= 1).
#include "xattn_common.h"
#include "xattn_launch.h"

namespace xattn {
namespace rungs {

constexpr int kMaxPerLane = kDim / kWave;  // 12 elements of a 768-wide row per lane
constexpr int kTile = 16;

// One thread per output element (b, i, d); online softmax over the keys with
// the exact 1/sum normaliser (kernel_naive.cu:16-66 computes the same
// quantity with a stored score row, which caps NI at 784; this one has no
// cap).  The q.k dot products are recomputed by every d -- that is the
// baseline's defining cost.
__global__ __launch_bounds__(256) void naive_kernel(const float* __restrict__ Q,
                                                    const float* __restrict__ K,
                                                    const float* __restrict__ V,
                                                    float* __restrict__ out, int NL, int NI,
                                                    int dim, int row_blocks, int d_blocks) {
    const int d = (blockIdx.x % d_blocks) * kWave + threadIdx.x;
    const int rest = blockIdx.x / d_blocks;
    const int i = (rest % row_blocks) * 4 + threadIdx.y;
    const int b = rest / row_blocks;
    if (i >= NL || d >= dim) return;
    const float* q = Q + ((size_t)b * NL + i) * dim;
    const float* Kb = K + (size_t)b * NI * dim;
    const float* Vb = V + (size_t)b * NI * dim;
    const float sq = sqrtf((float)dim);
    float m = -FLT_MAX, l = 0.f, acc = 0.f;
    for (int k = 0; k < NI; ++k) {
        const float* kr = Kb + (size_t)k * dim;
        float s = 0.f;
        for (int e = 0; e < dim; ++e) s += q[e] * kr[e];
        s = s / sq;
        if (s > m) {
            const float a = expf(m - s);
            l *= a;
            acc *= a;
            m = s;
        }
        const float p = expf(s - m);
        l += p;
        acc += p * Vb[(size_t)k * dim + d];
    }
    out[((size_t)b * NL + i) * dim + d] = NI > 0 ? acc * (1.0f / l) : 0.f;
}

// One wavefront per latent, four per workgroup; the full score row of each
// latent lives in LDS, (4 * NI + 4) floats per workgroup
// (kernel_warp_parallel.cu:16-111).  Scores: lane-strided partial dot
// products and a 64-lane butterfly; softmax: lane-parallel over keys;
// P.V: lane-strided over d.  Exact 1/sum normaliser.
__global__ __launch_bounds__(256) void warp_kernel(const float* __restrict__ Q,
                                                   const float* __restrict__ K,
                                                   const float* __restrict__ V,
                                                   float* __restrict__ out, int NL, int NI,
                                                   int dim, int row_blocks) {
    extern __shared__ float smem[];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x / row_blocks;
    const int i = (blockIdx.x % row_blocks) * 4 + w;
    if (i >= NL) return;  // waves never synchronise with each other
    float* sc = smem + (size_t)w * NI;
    float* ssum = smem + (size_t)4 * NI;

    float q[kMaxPerLane];
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) {
        const int d = lane + kWave * k;
        q[k] = d < dim ? Q[((size_t)b * NL + i) * dim + d] : 0.f;
    }
    const float* Kb = K + (size_t)b * NI * dim;
    const float* Vb = V + (size_t)b * NI * dim;
    const float sq = sqrtf((float)dim);

    float mx = -FLT_MAX;
    for (int key = 0; key < NI; ++key) {
        float part = 0.f;
#pragma unroll
        for (int k = 0; k < kMaxPerLane; ++k) {
            const int d = lane + kWave * k;
            if (d < dim) part += q[k] * Kb[(size_t)key * dim + d];
        }
        const float s = wave_sum(part) / sq;
        if (lane == 0) sc[key] = s;
        mx = fmaxf(mx, s);
    }
    float sum = 0.f;
    for (int key = lane; key < NI; key += kWave) {
        const float e = expf(sc[key] - mx);
        sc[key] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) ssum[w] = sum;
    const float norm = NI > 0 ? 1.0f / sum : 0.f;

    float o[kMaxPerLane];
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) o[k] = 0.f;
    for (int key = 0; key < NI; ++key) {
        const float wgt = sc[key] * norm;
#pragma unroll
        for (int k = 0; k < kMaxPerLane; ++k) {
            const int d = lane + kWave * k;
            if (d < dim) o[k] += wgt * Vb[(size_t)key * dim + d];
        }
    }
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) {
        const int d = lane + kWave * k;
        if (d < dim) out[((size_t)b * NL + i) * dim + d] = o[k];
    }
}

// One wavefront per latent, four per workgroup sharing a 16-key K tile in LDS;
// online softmax with running max / sum and a 1/(sum + 1e-6) normaliser
// (kernel_tiled.cu:16-167).  Every wavefront -- including ones whose latent
// is past NL -- takes part in the tile loads and both barriers, and the tile
// is not overwritten before all wavefronts are done with it.
__global__ __launch_bounds__(256) void tiled_kernel(const float* __restrict__ Q,
                                                    const float* __restrict__ K,
                                                    const float* __restrict__ V,
                                                    float* __restrict__ out, int NL, int NI,
                                                    int dim, int row_blocks) {
    __shared__ float tk[kTile * kDim];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x / row_blocks;
    const int i = (blockIdx.x % row_blocks) * 4 + w;
    const int ic = min(i, NL - 1);

    float q[kMaxPerLane];
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) {
        const int d = lane + kWave * k;
        q[k] = d < dim ? Q[((size_t)b * NL + ic) * dim + d] : 0.f;
    }
    const float* Kb = K + (size_t)b * NI * dim;
    const float* Vb = V + (size_t)b * NI * dim;
    const float sq = sqrtf((float)dim);

    float m = -FLT_MAX, l = 0.f;
    float o[kMaxPerLane];
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) o[k] = 0.f;

    for (int t0 = 0; t0 < NI; t0 += kTile) {
        for (int e = threadIdx.x; e < kTile * dim; e += 256) {
            const int r = e / dim, c = e - r * dim;
            const int key = t0 + r;
            tk[r * kDim + c] = key < NI ? Kb[(size_t)key * dim + c] : 0.f;
        }
        __syncthreads();
        float s[kTile];
        float tmax = -FLT_MAX;
#pragma unroll
        for (int r = 0; r < kTile; ++r) {
            float part = 0.f;
#pragma unroll
            for (int k = 0; k < kMaxPerLane; ++k) {
                const int d = lane + kWave * k;
                if (d < dim) part += q[k] * tk[r * kDim + d];
            }
            s[r] = wave_sum(part) / sq;
            if (t0 + r < NI) tmax = fmaxf(tmax, s[r]);
        }
        const float nm = fmaxf(m, tmax);
        const float scale = expf(m - nm);
        l *= scale;
#pragma unroll
        for (int k = 0; k < kMaxPerLane; ++k) o[k] *= scale;
        m = nm;
#pragma unroll
        for (int r = 0; r < kTile; ++r) {
            if (t0 + r >= NI) break;
            const float p = expf(s[r] - m);
            l += p;
#pragma unroll
            for (int k = 0; k < kMaxPerLane; ++k) {
                const int d = lane + kWave * k;
                if (d < dim) o[k] += p * Vb[(size_t)(t0 + r) * dim + d];
            }
        }
        __syncthreads();
    }
    if (i >= NL) return;
    const float norm = 1.0f / (l + 1e-6f);
#pragma unroll
    for (int k = 0; k < kMaxPerLane; ++k) {
        const int d = lane + kWave * k;
        if (d < dim) out[((size_t)b * NL + i) * dim + d] = o[k] * norm;
    }
}

}  // namespace rungs

static bool grid_ok(const char* who, long long blocks) {
    if (blocks > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: grid of %lld workgroups too large", who, blocks);
        return false;
    }
    return true;
}

bool launch_naive(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                  int NI, int dim, hipStream_t stream) {
    const int row_blocks = (NL + 3) / 4, d_blocks = (dim + kWave - 1) / kWave;
    const long long nblk = (long long)B * row_blocks * d_blocks;
    if (nblk <= 0) return true;
    if (!grid_ok("launch_naive_kernel", nblk)) return false;
    hipLaunchKernelGGL(rungs::naive_kernel, dim3((unsigned)nblk), dim3(kWave, 4), 0, stream, Q,
                       K, V, out, NL, NI, dim, row_blocks, d_blocks);
    return check_launch("launch_naive_kernel");
}

bool launch_warp(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                 int NI, int dim, hipStream_t stream) {
    const int row_blocks = (NL + 3) / 4;
    const long long nblk = (long long)B * row_blocks;
    if (nblk <= 0) return true;
    if (!grid_ok("launch_parallel_kernel", nblk)) return false;
    const size_t lds = ((size_t)4 * NI + 4) * sizeof(float);
    if (lds > 64 * 1024)
        (void)hipFuncSetAttribute((const void*)rungs::warp_kernel,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(rungs::warp_kernel, dim3((unsigned)nblk), dim3(256), lds, stream, Q, K,
                       V, out, NL, NI, dim, row_blocks);
    return check_launch("launch_parallel_kernel");
}

bool launch_tiled(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                  int NI, int dim, hipStream_t stream) {
    const int row_blocks = (NL + 3) / 4;
    const long long nblk = (long long)B * row_blocks;
    if (nblk <= 0) return true;
    if (!grid_ok("launch_tiled_kernel", nblk)) return false;
    hipLaunchKernelGGL(rungs::tiled_kernel, dim3((unsigned)nblk), dim3(256), 0, stream, Q, K, V,
                       out, NL, NI, dim, row_blocks);
    return check_launch("launch_tiled_kernel");
}

}  // namespace xattn
