// LDS and LDS-DMA rates of one gfx950 CU, for the access patterns the 16-bit
// flash kernel uses.  One 512-thread workgroup per CU (150 KiB of dynamic
// LDS keeps it alone there), 256 workgroups; every wavefront times its own
// loop with the shader clock (s_memtime) and the 100 MHz real-time clock.
//
//   make -C fast-cuda-cross-attention_amd probes
//   fast-cuda-cross-attention_amd/experiments/lds_rates
//
// Prints, per case, bytes per shader clock per CU (and per wavefront).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u4 lds_u4;
typedef __attribute__((address_space(3))) s4 lds_s4;

constexpr int kLds = 150 * 1024;
constexpr int kBlocks = 256;
constexpr int kSrcBytes = 64 * 1024;  // DMA source per group of workgroups
constexpr int kSrcGroups = 32;

// An address the optimiser cannot tie to the previous iteration's, so every
// read is issued.
__device__ inline unsigned opaque(unsigned x) {
    asm volatile("" : "+v"(x));
    return x;
}

enum Pattern : int {
    kLinear = 0,    // ds_read_b128, lane-contiguous 1 KiB per instruction
    kKFrag = 1,     // ds_read_b128, 16 rows (stride 1568) x 64 B: a K fragment
    kTrOld = 2,     // ds_read_b64_tr_b16, 16 rows (stride 1568) x 32 B
    kTr1600 = 3,    // ds_read_b64_tr_b16, rows 0-3 and 8-11 (stride 1600) x 64 B
    kTr1568 = 4,    // the same rows at stride 1568
};

// Wavefronts w < nread issue `depth` reads of `pat` per iteration, `iters`
// times; wavefronts w >= nread (when src is set) stream 1 KiB LDS-DMA chunks
// of a 48 KiB window of src, sixteen in flight.
template <int DEPTH>
__global__ __launch_bounds__(512) void rates(int pat, int iters, int nread, const char* src,
                                             unsigned long long* clocks, unsigned* sink) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    for (int i = tid; i < kLds / 4; i += 512) ((unsigned*)lds)[i] = i * 2654435761u;
    __syncthreads();
    const unsigned l0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
    const unsigned long long t0 = clock64(), r0 = wall_clock64();
    unsigned acc = 0;
    if (w < nread) {
        const int j = lane & 15, g = lane >> 4, h = g & 1, kg = g >> 1;
        unsigned base = 0, step = 0;
        switch (pat) {
            case kLinear: base = 16384 * w + 16 * lane, step = 1024; break;
            case kKFrag: base = 8192 * w + 1568 * j + 16 * g, step = 64; break;
            case kTrOld: base = 384 * w + 1568 * (4 * g + (j >> 2)) + 8 * (j & 3), step = 64; break;
            case kTr1600: base = 384 * w + 1600 * (8 * kg + (j >> 2)) + 2 * (16 * h + 4 * (j & 3)), step = 64; break;
            default: base = 384 * w + 1568 * (8 * kg + (j >> 2)) + 2 * (16 * h + 4 * (j & 3)), step = 64; break;
        }
        for (int it = 0; it < iters; ++it) {
            const unsigned a = opaque(l0 + base);
            if (pat <= kKFrag) {
                u4 v[DEPTH];
#pragma unroll
                for (int r = 0; r < DEPTH; ++r) v[r] = *(const lds_u4*)(uintptr_t)(a + step * (r % 16));
#pragma unroll
                for (int r = 0; r < DEPTH; ++r) acc ^= v[r].x ^ v[r].w;
            } else {
                s4 v[DEPTH];
#pragma unroll
                for (int r = 0; r < DEPTH; ++r)
                    v[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(uintptr_t)(a + step * (r % 8)));
#pragma unroll
                for (int r = 0; r < DEPTH; ++r) acc ^= (unsigned short)v[r].x ^ (unsigned short)v[r].w;
            }
        }
    } else if (src) {
        // chunk r of an iteration lands in this wavefront's 8 KiB of the
        // upper LDS half; sources cycle over 48 KiB of this group's window
        const unsigned dst = l0 + 65536 + 8192 * ((w - nread) & 7);
        const char* s = src + (size_t)(blockIdx.x % kSrcGroups) * kSrcBytes;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int r = 0; r < 8; ++r)
                __builtin_amdgcn_global_load_lds(
                    s + 16 * lane + 1024 * ((it * 8 + r) % 48),
                    (__attribute__((address_space(3))) void*)(uintptr_t)(dst + 1024 * r), 16, 0, 0);
            __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));  // vmcnt(8)
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    }
    const unsigned long long t1 = clock64(), r1 = wall_clock64();
    sink[blockIdx.x * 512 + tid] = acc;
    if (lane == 0) {
        clocks[(blockIdx.x * 8 + w) * 2] = t1 - t0;
        clocks[(blockIdx.x * 8 + w) * 2 + 1] = r1 - r0;
    }
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

struct Result {
    double read_cyc, dma_cyc, ghz;
};

template <int DEPTH>
Result run(int pat, int iters, int nread, bool dma, const char* src, unsigned long long* clocks,
           unsigned* sink) {
    check(hipFuncSetAttribute((const void*)rates<DEPTH>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds),
          "hipFuncSetAttribute");
    for (int rep = 0; rep < 2; ++rep) {  // the first launch warms clocks and caches
        hipLaunchKernelGGL((rates<DEPTH>), dim3(kBlocks), dim3(512), kLds, 0, pat, iters, nread,
                           dma ? src : nullptr, clocks, sink);
        check(hipDeviceSynchronize(), "rates kernel");
    }
    std::vector<unsigned long long> h(kBlocks * 16);
    check(hipMemcpy(h.data(), clocks, h.size() * 8, hipMemcpyDeviceToHost), "hipMemcpy");
    double rc = 0, dc = 0, cyc = 0, rt = 0;
    int nr = 0, nd = 0;
    for (int b = 0; b < kBlocks; ++b)
        for (int w = 0; w < 8; ++w) {
            const double c = (double)h[(b * 8 + w) * 2];
            if (w < nread) rc += c, ++nr;
            else if (dma) dc += c, ++nd;
            else continue;
            cyc += c, rt += (double)h[(b * 8 + w) * 2 + 1];
        }
    return {nr ? rc / nr : 0.0, nd ? dc / nd : 0.0, cyc / rt * 0.1};
}

template <int DEPTH>
void read_case(const char* name, int pat, int nread, unsigned long long* clocks, unsigned* sink) {
    const int iters = 16000 / DEPTH;
    const Result r = run<DEPTH>(pat, iters, nread, false, nullptr, clocks, sink);
    const double per_read = pat <= kKFrag ? 1024.0 : 512.0;
    const double bytes = per_read * DEPTH * iters;
    printf("%-34s waves %d depth %2d: %6.1f B/clk/CU  %5.1f B/clk/wave  %5.1f cyc/read  (%.2f GHz)\n",
           name, nread, DEPTH, bytes * nread / r.read_cyc, bytes / r.read_cyc,
           r.read_cyc / (DEPTH * iters), r.ghz);
}

}  // namespace

int main() {
    unsigned long long* clocks;
    unsigned* sink;
    char* src;
    check(hipMalloc(&clocks, kBlocks * 16 * 8), "hipMalloc");
    check(hipMalloc(&sink, kBlocks * 512 * 4), "hipMalloc");
    check(hipMalloc(&src, kSrcGroups * kSrcBytes), "hipMalloc");
    check(hipMemset(src, 1, kSrcGroups * kSrcBytes), "hipMemset");

    printf("-- ds_read_b128, lane-contiguous: reads in flight per wavefront\n");
    for (int nr : {1, 4, 8}) {
        read_case<1>("b128 linear", kLinear, nr, clocks, sink);
        read_case<2>("b128 linear", kLinear, nr, clocks, sink);
        read_case<4>("b128 linear", kLinear, nr, clocks, sink);
        read_case<8>("b128 linear", kLinear, nr, clocks, sink);
        read_case<16>("b128 linear", kLinear, nr, clocks, sink);
    }
    printf("-- the 16-bit kernel's read patterns, 8 wavefronts, 8 in flight\n");
    read_case<8>("b128 K fragment, stride 1568", kKFrag, 8, clocks, sink);
    read_case<8>("tr_b16 16 rows x 32 B, stride 1568", kTrOld, 8, clocks, sink);
    read_case<8>("tr_b16 rows 0-3,8-11 x 64 B, 1600", kTr1600, 8, clocks, sink);
    read_case<8>("tr_b16 rows 0-3,8-11 x 64 B, 1568", kTr1568, 8, clocks, sink);

    printf("-- LDS DMA (global_load_lds_dwordx4), 1 KiB chunks, 16 in flight per wavefront\n");
    const int dma_iters = 500;
    const double dma_bytes = 8.0 * 1024 * dma_iters;
    {
        const Result r = run<1>(kLinear, dma_iters, 0, true, src, clocks, sink);
        printf("%-34s waves 8: %6.1f B/clk/CU  (%.2f GHz)\n", "DMA only", dma_bytes * 8 / r.dma_cyc,
               r.ghz);
    }
    {
        const Result r = run<8>(kLinear, 2000, 4, true, src, clocks, sink);
        printf("%-34s 4 + 4 waves: reads %6.1f B/clk/CU, DMA %6.1f B/clk/CU  (%.2f GHz)\n",
               "b128 linear beside DMA", 8.0 * 1024 * 2000 * 4 / r.read_cyc,
               8.0 * 1024 * 2000 * 4 / r.dma_cyc, r.ghz);
    }
    check(hipFree(clocks), "hipFree");
    check(hipFree(sink), "hipFree");
    check(hipFree(src), "hipFree");
    return 0;
}
