/*
 * A C program that uses kernels.so through include/xattn.h alone (no Python,
 * no torch): the fp32 entry point, split-K with caller-owned scratch, the
 * bf16 entry point, the two plan-override entry points and the no-allocation
 * entry point on a small ragged problem, each checked against a
 * double-precision softmax(Q K^T / sqrt(D)) V computed here.
 *
 *   gcc -std=c11 -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -Iinclude \
 *       tests/c/abi_client.c -L<dir of kernels.so> -l:kernels.so \
 *       -L/opt/rocm/lib -lamdhip64 -lm -o abi_client
 *
 * Exit status 0 and a last line "ok" when every check passes.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "xattn.h"

enum { B = 2, NL = 70, NI = 300, D = 768, SPLITS = 7 };

static float frand(unsigned* state) {
    /* xorshift32 mapped to a standard-normal-ish value (sum of 4 uniforms) */
    float acc = 0.f;
    for (int i = 0; i < 4; ++i) {
        *state ^= *state << 13;
        *state ^= *state >> 17;
        *state ^= *state << 5;
        acc += (float)(*state & 0xffffff) / 16777216.f;
    }
    return (acc - 2.f) * 1.7320508f;
}

static void reference(const float* q, const float* k, const float* v, double* o) {
    double* w = malloc(sizeof(double) * NI);
    const double scale = 1.0 / sqrt((double)D);
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < NL; ++i) {
            const float* qi = q + ((size_t)b * NL + i) * D;
            double m = -INFINITY, l = 0.0;
            for (int j = 0; j < NI; ++j) {
                const float* kj = k + ((size_t)b * NI + j) * D;
                double s = 0.0;
                for (int d = 0; d < D; ++d) s += (double)qi[d] * kj[d];
                w[j] = s * scale;
                if (w[j] > m) m = w[j];
            }
            for (int j = 0; j < NI; ++j) l += (w[j] = exp(w[j] - m));
            double* oi = o + ((size_t)b * NL + i) * D;
            memset(oi, 0, sizeof(double) * D);
            for (int j = 0; j < NI; ++j) {
                const float* vj = v + ((size_t)b * NI + j) * D;
                for (int d = 0; d < D; ++d) oi[d] += w[j] / l * vj[d];
            }
        }
    free(w);
}

/* float -> bfloat16 bits, round to nearest even (finite inputs) */
static uint16_t to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static int check(const char* what, const float* got, const double* ref, double max_abs_gate,
                 double rel_gate) {
    double ma = 0.0, mref = 0.0;
    for (size_t i = 0; i < (size_t)B * NL * D; ++i) {
        if (!isfinite(got[i])) {
            printf("%s: non-finite output at %zu\n", what, i);
            return 1;
        }
        const double e = fabs(got[i] - ref[i]);
        if (e > ma) ma = e;
        if (fabs(ref[i]) > mref) mref = fabs(ref[i]);
    }
    const double rel = ma / (mref + 1e-6);
    printf("%-28s max_abs %.3e  rel %.3e\n", what, ma, rel);
    return (ma <= max_abs_gate && rel <= rel_gate) ? 0 : 1;
}

static int status(const char* what) {
    const int e = xattn_get_last_error();
    const hipError_t h = hipDeviceSynchronize();
    if (e != XATTN_OK || h != hipSuccess) {
        printf("%s: library error %d (%s), hip %d\n", what, e, xattn_get_last_error_string(),
               (int)h);
        return 1;
    }
    return 0;
}

#define HIP_OK(x)                                                   \
    do {                                                            \
        if ((x) != hipSuccess) {                                    \
            printf("%s failed at line %d\n", #x, __LINE__);         \
            return 2;                                               \
        }                                                           \
    } while (0)

int main(void) {
    const size_t nq = (size_t)B * NL * D, nk = (size_t)B * NI * D;
    float* q = malloc(nq * 4);
    float* k = malloc(nk * 4);
    float* v = malloc(nk * 4);
    float* out = malloc(nq * 4);
    double* ref = malloc(nq * 8);
    uint16_t* h16 = malloc(nk * 2);
    unsigned seed = 12345u;
    for (size_t i = 0; i < nq; ++i) q[i] = frand(&seed);
    for (size_t i = 0; i < nk; ++i) k[i] = frand(&seed);
    for (size_t i = 0; i < nk; ++i) v[i] = frand(&seed);
    reference(q, k, v, ref);

    float *dq, *dk, *dv, *dout, *po, *pm, *pl;
    HIP_OK(hipMalloc((void**)&dq, nq * 4));
    HIP_OK(hipMalloc((void**)&dk, nk * 4));
    HIP_OK(hipMalloc((void**)&dv, nk * 4));
    HIP_OK(hipMalloc((void**)&dout, nq * 4));
    HIP_OK(hipMalloc((void**)&po, nq * SPLITS * 4));
    HIP_OK(hipMalloc((void**)&pm, (size_t)B * NL * SPLITS * 4));
    HIP_OK(hipMalloc((void**)&pl, (size_t)B * NL * SPLITS * 4));
    HIP_OK(hipMemcpy(dq, q, nq * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dk, k, nk * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv, v, nk * 4, hipMemcpyHostToDevice));
    int fails = 0;

    launch_optimized_kernel(dq, dk, dv, dout, B, NL, NI, D, NULL);
    fails += status("launch_optimized_kernel");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_optimized_kernel", out, ref, 1e-4, 1e-3);

    HIP_OK(hipMemset(dout, 0, nq * 4));
    launch_splitk_kernel(dq, dk, dv, dout, po, pm, pl, B, NL, NI, D, SPLITS, NULL);
    fails += status("launch_splitk_kernel");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_splitk_kernel", out, ref, 1e-4, 1e-3);

    /* bf16: Q pre-scaled by 1/sqrt(D) before rounding, as the entry point's
     * contract asks; the output is checked against the fp32-input reference */
    uint16_t *bq, *bk, *bv;
    HIP_OK(hipMalloc((void**)&bq, nq * 2));
    HIP_OK(hipMalloc((void**)&bk, nk * 2));
    HIP_OK(hipMalloc((void**)&bv, nk * 2));
    const float qs = 1.0f / sqrtf((float)D);
    for (size_t i = 0; i < nq; ++i) h16[i] = to_bf16(q[i] * qs);
    HIP_OK(hipMemcpy(bq, h16, nq * 2, hipMemcpyHostToDevice));
    for (size_t i = 0; i < nk; ++i) h16[i] = to_bf16(k[i]);
    HIP_OK(hipMemcpy(bk, h16, nk * 2, hipMemcpyHostToDevice));
    for (size_t i = 0; i < nk; ++i) h16[i] = to_bf16(v[i]);
    HIP_OK(hipMemcpy(bv, h16, nk * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemset(dout, 0, nq * 4));
    launch_wmma_bf16_kernel(bq, bk, bv, dout, B, NL, NI, D, NULL);
    fails += status("launch_wmma_bf16_kernel");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_wmma_bf16_kernel", out, ref, 1.0, 2e-2);

    /* the plan-override entry points with plans of their own choosing:
     * 64 latents in two column halves, 3 key splits (bf16); 16 latents, 5
     * splits (fp32) */
    HIP_OK(hipMemset(dout, 0, nq * 4));
    launch_wmma_plan_kernel(1, bq, bk, bv, dout, B, NL, NI, D, 64, 2, 3, NULL);
    fails += status("launch_wmma_plan_kernel");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_wmma_plan_kernel", out, ref, 1.0, 2e-2);
    HIP_OK(hipMemset(dout, 0, nq * 4));
    launch_optimized_plan_kernel(dq, dk, dv, dout, B, NL, NI, D, 16, 5, NULL);
    fails += status("launch_optimized_plan_kernel");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_optimized_plan_kernel", out, ref, 1e-4, 1e-3);
    /* the no-allocation twin of launch_optimized_kernel (static scratch) */
    HIP_OK(hipMemset(dout, 0, nq * 4));
    launch_optimized_kernel_noalloc(dq, dk, dv, dout, B, NL, NI, D, NULL);
    fails += status("launch_optimized_kernel_noalloc");
    HIP_OK(hipMemcpy(out, dout, nq * 4, hipMemcpyDeviceToHost));
    fails += check("launch_optimized_kernel_noalloc", out, ref, 1e-4, 1e-3);

    /* an argument the kernels cannot run with is refused, not launched */
    launch_optimized_kernel(dq, dk, dv, dout, B, NL, NI, 64, NULL);
    if (xattn_get_last_error() != XATTN_ERR_UNSUPPORTED) {
        printf("dim=64 was not refused\n");
        ++fails;
    }

    hipFree(dq); hipFree(dk); hipFree(dv); hipFree(dout);
    hipFree(po); hipFree(pm); hipFree(pl); hipFree(bq); hipFree(bk); hipFree(bv);
    free(q); free(k); free(v); free(out); free(ref); free(h16);
    printf("%s\n", fails ? "FAILED" : "ok");
    return fails ? 1 : 0;
}
