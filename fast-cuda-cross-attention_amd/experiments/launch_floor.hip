// The fixed cost of a launch as the per-call event timing sees it: empty
// kernels (one or two per call, small and full grids, with and without a
// large LDS allocation) timed exactly as bench.py times a call (an event
// pair around each launch, the pairs recorded back to back) and as the
// reference's drivers do (the same, waiting for each call's closing event
// before the next), beside launch_optimized_kernel at B=1 N_latent=64
// N_input=784 (loaded from kernels.so) under both.
//
//   make -C fast-cuda-cross-attention_amd probes
//   fast-cuda-cross-attention_amd/experiments/launch_floor
//
// Prints, per case and protocol, the mean and median µs per call over 300
// calls after 50 untimed ones.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <random>
#include <vector>

namespace {

__global__ void empty_kernel() {}

// Same, but each workgroup holds the launch's dynamic LDS (150 KiB, untouched),
// about what the flash kernels hold: one workgroup per CU.
__global__ void empty_lds_kernel() {
    extern __shared__ char lds[];
    (void)lds;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

typedef void (*F32Launch)(const float*, const float*, const float*, float*, int, int, int, int,
                          hipStream_t);

struct Stat {
    double mean, median;
};

// n calls of fn, each between two events on the null stream; `sync`: wait
// for each call's closing event before the next call.
Stat time_calls(const std::function<void()>& fn, int n, bool sync) {
    std::vector<hipEvent_t> a(n), b(n);
    for (int i = 0; i < n; ++i) {
        check(hipEventCreate(&a[i]), "hipEventCreate");
        check(hipEventCreate(&b[i]), "hipEventCreate");
    }
    for (int i = 0; i < 50; ++i) fn();
    check(hipDeviceSynchronize(), "warmup");
    for (int i = 0; i < n; ++i) {
        check(hipEventRecord(a[i], 0), "hipEventRecord");
        fn();
        check(hipEventRecord(b[i], 0), "hipEventRecord");
        if (sync) check(hipEventSynchronize(b[i]), "hipEventSynchronize");
    }
    check(hipDeviceSynchronize(), "timed calls");
    std::vector<double> us(n);
    double sum = 0.0;
    for (int i = 0; i < n; ++i) {
        float ms;
        check(hipEventElapsedTime(&ms, a[i], b[i]), "hipEventElapsedTime");
        us[i] = 1e3 * ms;
        sum += us[i];
        check(hipEventDestroy(a[i]), "hipEventDestroy");
        check(hipEventDestroy(b[i]), "hipEventDestroy");
    }
    std::sort(us.begin(), us.end());
    return {sum / n, us[n / 2]};
}

}  // namespace

int main() {
    const char* libpath = getenv("XATTN_KERNELS_SO");
    if (!libpath) libpath = "fast-cuda-cross-attention_amd/kernels.so";
    void* lib = dlopen(libpath, RTLD_NOW);
    if (!lib) {
        fprintf(stderr, "dlopen %s: %s\n", libpath, dlerror());
        return 1;
    }
    const F32Launch opt = (F32Launch)dlsym(lib, "launch_optimized_kernel");
    if (!opt) {
        fprintf(stderr, "no launch_optimized_kernel in %s\n", libpath);
        return 1;
    }
    const int B = 1, NL = 64, NI = 784, D = 768;
    std::mt19937 rng(0);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> hq((size_t)B * NL * D), hk((size_t)B * NI * D), hv(hk.size());
    for (auto& x : hq) x = nd(rng);
    for (auto& x : hk) x = nd(rng);
    for (auto& x : hv) x = nd(rng);
    float *q, *k, *v, *o;
    check(hipMalloc(&q, hq.size() * 4), "hipMalloc");
    check(hipMalloc(&k, hk.size() * 4), "hipMalloc");
    check(hipMalloc(&v, hv.size() * 4), "hipMalloc");
    check(hipMalloc(&o, hq.size() * 4), "hipMalloc");
    check(hipMemcpy(q, hq.data(), hq.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    check(hipMemcpy(k, hk.data(), hk.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    check(hipMemcpy(v, hv.data(), hv.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");

    const size_t lds_bytes = 150 * 1024;
    check(hipFuncSetAttribute((const void*)empty_lds_kernel,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes),
          "hipFuncSetAttribute");

    struct Case {
        const char* name;
        std::function<void()> fn;
    };
    const Case cases[] = {
        {"empty, 1 x 64 threads", [] { hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0); }},
        {"empty, 256 x 256", [] { hipLaunchKernelGGL(empty_kernel, dim3(256), dim3(256), 0, 0); }},
        {"empty, 100 x 256, 150 KiB LDS",
         [=] { hipLaunchKernelGGL(empty_lds_kernel, dim3(100), dim3(256), lds_bytes, 0); }},
        {"two empty: 100 x 256 then 64 x 256",
         [] {
             hipLaunchKernelGGL(empty_kernel, dim3(100), dim3(256), 0, 0);
             hipLaunchKernelGGL(empty_kernel, dim3(64), dim3(256), 0, 0);
         }},
        {"launch_optimized_kernel B=1 NL=64 NI=784",
         [=] { opt(q, k, v, o, B, NL, NI, D, 0); }},
    };
    printf("%-44s %22s %22s\n", "case (us per call: mean / median)", "back-to-back pairs",
           "sync after each call");
    for (const Case& c : cases) {
        const Stat a = time_calls(c.fn, 300, false);
        const Stat s = time_calls(c.fn, 300, true);
        printf("%-44s %10.2f / %8.2f %10.2f / %8.2f\n", c.name, a.mean, a.median, s.mean, s.median);
    }
    check(hipGetLastError(), "launches");
    check(hipFree(q), "hipFree");
    check(hipFree(k), "hipFree");
    check(hipFree(v), "hipFree");
    check(hipFree(o), "hipFree");
    return 0;
}
