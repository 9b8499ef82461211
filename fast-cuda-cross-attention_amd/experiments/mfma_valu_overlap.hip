// Does vector-ALU work run while the MFMA pipe of the same SIMD is busy?
// One CU-filling launch of 256 workgroups x 8 wavefronts; wavefronts w and
// w + 4 of a workgroup share SIMD w % 4.  Wavefronts 0-3 ("MFMA waves") run a
// loop of back-to-back MFMAs (4 independent accumulators): per iteration 4
// v_mfma_f32_16x16x4_f32 (32 cycles each) or 8 v_mfma_f32_16x16x32_bf16
// (16 cycles each), 128 MFMA cycles either way.  Wavefronts 4-7 ("VALU
// waves") run the same number of iterations of 12 independent-chain VALU
// instructions (4 v_exp_f32, 8 FMAs: what a softmax issues).  Modes:
//
//   0  fp32 MFMA waves only          4  bf16 MFMA waves only
//   1  VALU waves only
//   2  fp32 MFMA waves + VALU waves  5  bf16 MFMA waves + VALU waves
//   3  fp32 MFMA with the VALU work interleaved in the same waves
//   6  bf16 MFMA with the VALU work interleaved in the same waves
//   7  fp32 MFMA with 12 scalar-ALU instructions per iteration in the same
//      waves (wave-uniform multiply-adds: what DMA address arithmetic issues)
//
// Prints, per mode, the launch time (HIP events) and the mean shader-clock
// cycles (s_memtime) that the MFMA waves and the VALU waves take.  If the
// two kinds of work overlap, mode 2 / 5 take about as long as the longer of
// modes 0 / 4 and 1; if they serialise, about the sum.
//
//   make -C fast-cuda-cross-attention_amd probes
//   fast-cuda-cross-attention_amd/experiments/mfma_valu_overlap
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

constexpr int kGroups = 256, kWaves = 8, kIters = 2048;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

// 12 VALU instructions on four independent chains.
__device__ inline void valu_step(float& x0, float& x1, float& x2, float& x3) {
    x0 = __builtin_amdgcn_exp2f(x0 * 0.5f - 0.25f);
    x1 = x1 * 0.999f + 0.001f;
    x2 = __builtin_amdgcn_exp2f(x2 * 0.5f - 0.25f);
    x3 = x3 * 0.999f + 0.001f;
    x0 = x0 * 0.999f + 0.002f;
    x1 = __builtin_amdgcn_exp2f(x1 * 0.5f - 0.25f);
    x2 = x2 * 0.999f + 0.002f;
    x3 = __builtin_amdgcn_exp2f(x3 * 0.5f - 0.25f);
}

template <int MODE>
__global__ __launch_bounds__(512) void probe(float* sink, unsigned long long* cycles) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    const float a = 1.0f + lane * 1e-3f, b = 0.5f - lane * 1e-4f;
    f4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0;
    float x0 = lane * 1e-3f, x1 = x0 + 0.1f, x2 = x0 + 0.2f, x3 = x0 + 0.3f;
    constexpr bool f32 = MODE == 0 || MODE == 2 || MODE == 3;
    constexpr bool bf16 = MODE >= 4 && MODE <= 6;
    constexpr bool mixed = MODE == 3 || MODE == 6;
    constexpr bool valu_waves = MODE == 1 || MODE == 2 || MODE == 5;
    if (w < 4 && f32) {
        for (int i = 0; i < kIters; ++i) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, c1, 0, 0, 0);
            if (mixed) valu_step(x0, x1, x2, x3);
            c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(b, b, c3, 0, 0, 0);
        }
    }
    if (w < 4 && bf16) {
        bf8 ha, hb;
        for (int k = 0; k < 8; ++k) {
            ha[k] = (__bf16)(a + k * 1e-3f);
            hb[k] = (__bf16)(b - k * 1e-3f);
        }
        for (int i = 0; i < kIters; ++i) {
            for (int r = 0; r < 2; ++r) {
                c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha, hb, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hb, ha, c1, 0, 0, 0);
                if (mixed && r == 0) valu_step(x0, x1, x2, x3);
                c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha, ha, c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hb, hb, c3, 0, 0, 0);
            }
        }
    }
    if (w >= 4 && valu_waves) {
        for (int i = 0; i < kIters; ++i) valu_step(x0, x1, x2, x3);
    }
    unsigned su = __builtin_amdgcn_readfirstlane(blockIdx.x + 1u);
    if (w < 4 && MODE == 7) {
        // fp32 MFMAs with 12 scalar-ALU instructions per iteration (a
        // shift-xor-multiply hash of a wave-uniform value, four times; written
        // out so the compiler cannot fold it) between the second and third
        // MFMA.
        for (int i = 0; i < kIters; ++i) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, c1, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            unsigned tmp;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                asm volatile("s_lshr_b32 %1, %0, 7\n\ts_xor_b32 %0, %0, %1\n\t"
                             "s_mul_i32 %0, %0, 0x9e3779b1"
                             : "+s"(su), "=&s"(tmp));
            __builtin_amdgcn_sched_barrier(0);
            c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(b, b, c3, 0, 0, 0);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    sink[blockIdx.x * 512 + threadIdx.x] =
        c0[0] + c1[1] + c2[2] + c3[3] + x0 + x1 + x2 + x3 + (float)(su & 0xff);
    if (lane == 0) cycles[blockIdx.x * kWaves + w] = t1 - t0;
}

typedef void (*Kernel)(float*, unsigned long long*);

}  // namespace

int main() {
    const Kernel kernels[8] = {probe<0>, probe<1>, probe<2>, probe<3>,
                               probe<4>, probe<5>, probe<6>, probe<7>};
    const char* names[8] = {"fp32 MFMA waves only",
                            "VALU waves only",
                            "fp32 MFMA waves + VALU waves",
                            "fp32 MFMA + VALU in the same waves",
                            "bf16 MFMA waves only",
                            "bf16 MFMA waves + VALU waves",
                            "bf16 MFMA + VALU in the same waves",
                            "fp32 MFMA + SALU in the same waves"};
    float* sink;
    unsigned long long* cyc;
    check(hipMalloc(&sink, sizeof(float) * kGroups * 512), "hipMalloc");
    check(hipMalloc(&cyc, sizeof(unsigned long long) * kGroups * kWaves), "hipMalloc");
    std::vector<unsigned long long> h(kGroups * kWaves);
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    printf("%-36s %10s %14s %14s\n", "mode", "us", "MFMA waves", "VALU waves");
    for (int rep = 0; rep < 2; ++rep) {
        for (int m = 0; m < 8; ++m) {
            hipLaunchKernelGGL(kernels[m], dim3(kGroups), dim3(512), 0, 0, sink, cyc);
            check(hipEventRecord(e0, 0), "hipEventRecord");
            hipLaunchKernelGGL(kernels[m], dim3(kGroups), dim3(512), 0, 0, sink, cyc);
            check(hipEventRecord(e1, 0), "hipEventRecord");
            check(hipDeviceSynchronize(), "launch");
            float ms = 0.f;
            check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
            check(hipMemcpy(h.data(), cyc, h.size() * sizeof(h[0]), hipMemcpyDeviceToHost),
                  "hipMemcpy");
            double mw = 0.0, vw = 0.0;
            for (int g = 0; g < kGroups; ++g)
                for (int w = 0; w < kWaves; ++w) (w < 4 ? mw : vw) += (double)h[g * kWaves + w];
            printf("%d %-34s %10.1f %14.0f %14.0f\n", m, names[m], ms * 1e3, mw / (kGroups * 4),
                   vw / (kGroups * 4));
        }
    }
    check(hipGetLastError(), "launches");
    check(hipEventDestroy(e0), "hipEventDestroy");
    check(hipEventDestroy(e1), "hipEventDestroy");
    check(hipFree(sink), "hipFree");
    check(hipFree(cyc), "hipFree");
    return 0;
}
