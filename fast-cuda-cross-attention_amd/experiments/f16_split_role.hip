// A tried and dropped design for the 16-bit cross-attention kernel, kept as a
// runnable experiment: split wavefront roles, 64 latents per workgroup,
// 16-key tiles.  The program times it against the library's
// launch_wmma_bf16_kernel / launch_wmma_kernel (loaded from kernels.so) on
// the same inputs, interleaved, and compares the two outputs.
//
//   make -C fast-cuda-cross-attention_amd probes
//   fast-cuda-cross-attention_amd/experiments/f16_split_role [bf16|fp16] [B NL NI]
//   fast-cuda-cross-attention_amd/experiments/f16_split_role_clock ...  (per-step role times)
//
// Eight wavefronts in two roles, one of each per SIMD:
//   score wavefront c (0..3): latent block c (16 latents), Q block in
//     registers; per tile S^T[16 keys x 16 q] = K_tile . Q_c^T (24
//     v_mfma_f32_16x16x32), the block's softmax over the tile's keys, and
//     P^T (16-bit) into a double-buffered P buffer;
//   output wavefront a (0..3): columns 192a .. 192a + 191 of all 64 latents;
//     per tile O^T[192 x 64] += V_tile^T . P^T (12 v_mfma_f32_32x32x16), V^T
//     from two transposing LDS reads per fragment.
// The output wavefronts run one tile behind: in step i the score wavefronts
// work on tile i and the output wavefronts on tile i - 1, one barrier per
// step.  K and V each have a ring of three 16-key slots in LDS (K(i + 2) and
// V(i + 1) requested during step i).  In-loop DMA goes where each role has
// slack: a score wavefront issues its quarter of K(i + 2) after writing its
// weights, an output wavefront its quarter of V(i + 1), one chunk per MFMA.
// Odd row blocks take their tiles one step ahead of even ones, so half of a
// tile's readers find it in L2.  Softmax by restart passes, as in the
// library's kernels.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "xattn_common.h"

namespace sr {

using namespace xattn;

constexpr int BN = 16;                           // keys per tile
constexpr int BM = 64;                           // latents per workgroup
constexpr int NWAVE = 8;
constexpr int ROWB = kDim * 2;                   // bytes per K / V row in memory
constexpr int LROW = ROWB + 32;                  // K row stride in LDS (32 mod 512)
constexpr int LROWV = ROWB + 64;                 // V row stride in LDS (64 mod 512)
constexpr int PIECES = LROW / 16;                // 16-byte pieces per K row (98)
constexpr int PIECESV = LROWV / 16;              // ... per V row (100)
constexpr int CHUNKS = (BN * PIECES + kWave - 1) / kWave;  // 1 KiB DMA chunks per tile (25)
constexpr int SLOT = CHUNKS * 1024;
constexpr int NSLOT = 3;
constexpr int KRING = 0;
constexpr int VRING = NSLOT * SLOT;
constexpr int PBYTES = BM * BN * 2;
constexpr int PBUF = 2 * NSLOT * SLOT;
constexpr int STATS = PBUF + 2 * PBYTES;
constexpr int FLAG = STATS + BM * 16;
constexpr int LDS_BYTES = FLAG + 16;
constexpr int KSF = kDim / 32;
constexpr int KPF = 4;
constexpr int OCB = 6;
constexpr int OCOLS = 32 * OCB;
constexpr int SROW = OCOLS * 4 + 16;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(CHUNKS * 1024 >= BN * LROW && CHUNKS * 1024 == BN * LROWV, "chunks");
static_assert(32 * SROW <= SLOT && 4 * SLOT <= PBUF, "output staging");

template <typename T> constexpr float tau_log2 = 64.0f;
template <> constexpr float tau_log2<_Float16> = 15.0f;

struct Params {
    const u16* Q;
    const u16* K;
    const u16* V;
    float* out;
    int B, NL, NI, row_blocks;
    unsigned long long* clock;  // per (workgroup, wavefront): 8 values, or null
};

typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned int u2v __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) char lds_char;

template <typename T> struct Vec8;
template <> struct Vec8<_Float16> { typedef h8 type; };
template <> struct Vec8<__bf16> { typedef bf8 type; };

template <typename T>
__device__ inline f4 mfma16(typename Vec8<T>::type a, typename Vec8<T>::type b, f4 c) {
    if constexpr (__is_same(T, _Float16))
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ inline f16v mfma32(typename Vec8<T>::type a, typename Vec8<T>::type b, f16v c) {
    if constexpr (__is_same(T, _Float16))
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ inline unsigned pack2(float lo, float hi) {
    const T a = (T)lo, b = (T)hi;
    return (unsigned)__builtin_bit_cast(u16, a) | ((unsigned)__builtin_bit_cast(u16, b) << 16);
}

__device__ inline s4 tr_read(const lds_char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
}

__device__ inline lds_char* opaque_lds(unsigned byte_addr) {
    asm volatile("" : "+v"(byte_addr));
    return (lds_char*)(uintptr_t)byte_addr;
}

#ifdef STEP_CLOCK
#define STAMP(var)                                         \
    __builtin_amdgcn_sched_barrier(0);                     \
    const unsigned long long var = __builtin_amdgcn_s_memtime(); \
    __builtin_amdgcn_sched_barrier(0)
#define ACC(dst, a, b) dst += (b) - (a)
#else
#define STAMP(var) [[maybe_unused]] const unsigned long long var = 0
#define ACC(dst, a, b) (void)0
#endif

template <typename T>
__global__ __launch_bounds__(NWAVE * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void split_role_kernel(Params p) {
    typedef typename Vec8<T>::type v8;
    __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
    STAMP(clk0);

    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int rb = item % p.row_blocks;
    const int b = item / p.row_blocks;
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int q0 = rb * BM;

    const char* Kb = (const char*)(p.K + (size_t)b * p.NI * kDim);
    const char* Vb = (const char*)(p.V + (size_t)b * p.NI * kDim);
    const int nk = p.NI;
    const int ntiles = (nk + BN - 1) / BN;
    auto row_lo = [&](int t) { return (t == ntiles - 1 && nk >= BN) ? BN - (nk - t * BN) : 0; };
    const int rot = ntiles > 1 ? (rb & 1) : 0;
    auto step_tile = [&](int i) { return i + rot < ntiles ? i + rot : i + rot - ntiles; };

    // DMA: chunk m of a tile fills LDS bytes [1024 m, +1024) of its slot;
    // lane i lands on 16-byte piece u = 64 m + i: row u / P, piece u % P
    // (pieces past 96 are padding and re-read piece 95).  Before the loop,
    // wavefront w issues chunks m = w (mod 8) of K and m = w + 4 (mod 8) of V;
    // in the loop, role wavefront r = w mod 4 issues chunks m = r (mod 4).
    const int mk = w, mv = (w + 4) % NWAVE;
    const int nck = (CHUNKS - 1 - mk) / NWAVE + 1, ncv = (CHUNKS - 1 - mv) / NWAVE + 1;
    unsigned doffk[4], doffv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int uk = 64 * (mk + NWAVE * t) + lane, uv = 64 * (mv + NWAVE * t) + lane;
        doffk[t] = (unsigned)(min(min(uk / PIECES, BN - 1), nk - 1) * ROWB +
                              16 * min(uk % PIECES, ROWB / 16 - 1));
        doffv[t] = (unsigned)(min(uv / PIECESV, nk - 1) * ROWB + 16 * min(uv % PIECESV, ROWB / 16 - 1));
    }
    const int r4 = w & 3;
    const int noc = (CHUNKS - 1 - r4) / 4 + 1;
    unsigned roff[7];
#pragma unroll
    for (int c = 0; c < 7; ++c) {
        const int u = 64 * (r4 + 4 * c) + lane;
        roff[c] = w < 4 ? (unsigned)(min(min(u / PIECES, BN - 1), nk - 1) * ROWB +
                                     16 * min(u % PIECES, ROWB / 16 - 1))
                        : (unsigned)(min(u / PIECESV, nk - 1) * ROWB +
                                     16 * min(u % PIECESV, ROWB / 16 - 1));
    }
    const unsigned lds0 = lds_u32(lds);
    struct Dma {
        const char* src;
        unsigned m0;
    };
    auto dma_setup = [&](bool isv, int tile, int slot) {
        const int t = step_tile(min(tile, ntiles - 1));
        Dma d;
        d.src = uniform_ptr((isv ? Vb : Kb) + (size_t)(t * BN - row_lo(t)) * ROWB);
        d.m0 = lds0 + (unsigned)((isv ? VRING : KRING) + slot * SLOT);
        return d;
    };
    auto issue = [&](bool isv, int tile, int slot) {
        const Dma d = dma_setup(isv, tile, slot);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (c < (isv ? ncv : nck))
                dma16_untracked(d.src, isv ? doffv[c] : doffk[c],
                                d.m0 + 1024u * ((isv ? mv : mk) + NWAVE * c));
    };
    auto rchunk = [&](const Dma& d, int c) {
        if (c < noc) dma16_untracked(d.src, roff[c], d.m0 + 1024u * (r4 + 4 * c));
    };

    int* const restart_flag = (int*)(lds + FLAG);
    f4* const stats = (f4*)(lds + STATS);
    if (tid == 0) *restart_flag = 0;
    const float tau_raw = tau_log2<T> / kLog2e;
    [[maybe_unused]] unsigned long long ph[3] = {0, 0, 0};  // per-step role phases (STEP_CLOCK)
    STAMP(clk_loop);

    if (w < 4) {
        // score wavefront c = w
        const int c = w;
        const int j = lane & 15, g = lane >> 4;
        issue(false, 0, 0);
        v8 qr[KSF];
        {
            const int qc = min(q0 + 16 * c + j, p.NL - 1);
            const u16* qrow = p.Q + ((size_t)b * p.NL + qc) * kDim + 8 * g;
#pragma unroll
            for (int s = 0; s < KSF; ++s) qr[s] = *(const v8*)(qrow + 32 * s);
        }
        const int kread = LROW * j + 16 * g;
        lds_char* const pw_dst = (lds_char*)lds + PBUF + (16 * c + j) * (BN * 2) + 8 * g;
        float m_true = -FLT_MAX, m_ref = -FLT_MAX, lsum;
        bool ref_set = false;
        unsigned long long over;
        for (bool first = true;; first = false) {
            if (!first) issue(false, 0, 0);
            wait_vmcnt<0>();
            issue(false, 1, 1);
            issue(true, 0, 0);
            lds_barrier();
            lsum = 0.f;
            over = 0;
            for (int i = 0; i <= ntiles; ++i) {
                STAMP(t0);
                [[maybe_unused]] unsigned long long t1v = t0;
                if (i < ntiles) {
                    const lds_char* kr =
                        opaque_lds(lds0 + (unsigned)(KRING + (i % NSLOT) * SLOT + kread));
                    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
                    v8 kf[KSF];
#pragma unroll
                    for (int s = 0; s < KPF; ++s) kf[s] = *(const v8*)(kr + 64 * s);
#pragma unroll
                    for (int s = 0; s < KSF; ++s) {
                        if (s + KPF < KSF) kf[s + KPF] = *(const v8*)(kr + 64 * (s + KPF));
                        if (s % 2 == 0) s0 = mfma16<T>(kf[s], qr[s], s0);
                        else s1 = mfma16<T>(kf[s], qr[s], s1);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    STAMP(t1);
                    t1v = t1;
                    const f4 sv = s0 + s1;
                    const int ti = step_tile(i), n0 = ti * BN, lo = row_lo(ti);
                    float x[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * g + e;
                        x[e] = (r >= lo && n0 - lo + r < nk) ? sv[e] : -INFINITY;
                    }
                    const float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
                    m_true = fmaxf(m_true, tmax);
                    if (!ref_set) {
                        m_ref = wave_max16_groups(tmax);
                        ref_set = true;
                    }
                    over |= __ballot(tmax > m_ref + tau_raw);
                    float pw[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pw[e] = fast_exp2((x[e] - m_ref) * kLog2e);
                        lsum += pw[e];
                    }
                    *(u2v*)(pw_dst + (i % 2) * PBYTES) =
                        (u2v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3])};
                }
                STAMP(t2);
                {
                    const Dma dk = dma_setup(false, i + 2, (i + 2) % NSLOT);
#pragma unroll
                    for (int cc = 0; cc < 7; ++cc) rchunk(dk, cc);
                }
                if (c == 0) wait_vmcnt<7>();
                else wait_vmcnt<6>();
                lds_barrier();
                STAMP(t3);
                ACC(ph[0], t0, t1v);
                ACC(ph[1], t1v, t2);
                ACC(ph[2], t2, t3);
            }
            if (over != 0 && lane == 0) *restart_flag = 1;
            lds_barrier();
            if (!__builtin_amdgcn_readfirstlane(*restart_flag)) break;
            wait_vmcnt<0>();
            lds_barrier();
            if (tid == 0) *restart_flag = 0;
            m_ref = wave_max16_groups(m_true);
            lds_barrier();
        }
        wait_vmcnt<0>();
        const float mt = wave_max16_groups(m_true);
        const float l = wave_sum16_groups(lsum);
        if (g == 0) stats[16 * c + j] = (f4){mt, l, m_ref, 0.f};
        lds_barrier();
    } else {
        // output wavefront a = w - 4
        const int a = w - 4;
        const int G = lane >> 4, ii = lane & 15;
        const int h = G & 1, kg = G >> 1;
        const int vread = LROWV * (8 * kg + (ii >> 2)) + 2 * (OCOLS * a + 16 * h + 4 * (ii & 3));
        const int pread = PBUF + (lane & 31) * (BN * 2) + 16 * kg;
        f16v acc[OCB][2];
        for (;;) {
            issue(false, 0, 0);
            wait_vmcnt<0>();
            issue(false, 1, 1);
            issue(true, 0, 0);
#pragma unroll
            for (int cb = 0; cb < OCB; ++cb)
#pragma unroll
                for (int b2 = 0; b2 < 2; ++b2)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[cb][b2][r] = 0.f;
            lds_barrier();
            for (int i = 0; i <= ntiles; ++i) {
                STAMP(t0);
                if (i >= 1) {
                    const int t = i - 1;
                    const lds_char* vr =
                        opaque_lds(lds0 + (unsigned)(VRING + (t % NSLOT) * SLOT + vread));
                    const Dma dv = dma_setup(true, i + 1, (i + 1) % NSLOT);
                    const lds_char* pr = opaque_lds(lds0 + (unsigned)(pread + (t % 2) * PBYTES));
                    const v8 pt0 = *(const v8*)(pr);
                    const v8 pt1 = *(const v8*)(pr + 32 * (BN * 2));
                    s4 va[OCB], vb[OCB];
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        va[cb] = tr_read(vr + 64 * cb);
                        vb[cb] = tr_read(vr + 4 * LROWV + 64 * cb);
                    }
#pragma unroll
                    for (int cb = 0; cb < OCB; ++cb) {
                        if (cb + 2 < OCB) {
                            va[cb + 2] = tr_read(vr + 64 * (cb + 2));
                            vb[cb + 2] = tr_read(vr + 4 * LROWV + 64 * (cb + 2));
                        }
                        const v8 vt = __builtin_bit_cast(
                            v8, __builtin_shufflevector(va[cb], vb[cb], 0, 1, 2, 3, 4, 5, 6, 7));
                        if (cb < 4) rchunk(dv, 2 * cb);
                        acc[cb][0] = mfma32<T>(vt, pt0, acc[cb][0]);
                        if (cb < 3) rchunk(dv, 2 * cb + 1);
                        acc[cb][1] = mfma32<T>(vt, pt1, acc[cb][1]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    const Dma dv = dma_setup(true, i + 1, (i + 1) % NSLOT);
#pragma unroll
                    for (int cc = 0; cc < 7; ++cc) rchunk(dv, cc);
                }
                STAMP(t1);
                if (a == 0) wait_vmcnt<7>();
                else wait_vmcnt<6>();
                lds_barrier();
                STAMP(t2);
                ACC(ph[0], t0, t1);
                ACC(ph[2], t1, t2);
            }
            lds_barrier();
            if (!__builtin_amdgcn_readfirstlane(*restart_flag)) break;
            wait_vmcnt<0>();
            lds_barrier();
            lds_barrier();
        }
        wait_vmcnt<0>();
        lds_barrier();
        // normalise and store through the free tile ring (row-contiguous)
        lds_char* const stage = (lds_char*)lds + a * SLOT;
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2) {
            const int n = lane & 31, hh = lane >> 5;
            const f4 st = stats[32 * b2 + n];
            const float factor = fast_exp2((st.z - st.x) * kLog2e);
            const float rsc = factor / (st.y * factor + 1e-6f);
#pragma unroll
            for (int cb = 0; cb < OCB; ++cb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const f4 o = (f4){acc[cb][b2][4 * jj], acc[cb][b2][4 * jj + 1],
                                      acc[cb][b2][4 * jj + 2], acc[cb][b2][4 * jj + 3]} * rsc;
                    *(f4*)(stage + n * SROW + 4 * (32 * cb + 8 * jj + 4 * hh)) = o;
                }
            const int qb = q0 + 32 * b2;
#pragma unroll
            for (int k = 0; k < 32 * (OCOLS / 4) / kWave; ++k) {
                const int pc = k * kWave + lane;
                const int r = pc / (OCOLS / 4), cc = pc % (OCOLS / 4);
                const f4 o = *(const f4*)(stage + r * SROW + 16 * cc);
                if (qb + r >= p.NL) continue;
                __builtin_nontemporal_store(
                    o, (f4*)(p.out + ((size_t)b * p.NL + qb + r) * kDim + OCOLS * a + 4 * cc));
            }
        }
    }
#ifdef STEP_CLOCK
    STAMP(clk_end);
    if (lane == 0 && p.clock) {
        unsigned long long* o = p.clock + ((size_t)blockIdx.x * NWAVE + w) * 8;
        o[0] = clk_loop - clk0, o[1] = clk_end - clk_loop, o[2] = ph[0], o[3] = ph[1],
        o[4] = ph[2], o[5] = (unsigned long long)(ntiles + 1);
    }
#endif
}

}  // namespace sr

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

unsigned short to16(float x, bool bf16) {
    if (bf16) {
        unsigned u;
        memcpy(&u, &x, 4);
        return (unsigned short)((u + 0x7fff + ((u >> 16) & 1)) >> 16);  // round to nearest even
    }
    const _Float16 h = (_Float16)x;
    unsigned short s;
    memcpy(&s, &h, 2);
    return s;
}

typedef void (*LaunchFn)(const uint16_t*, const uint16_t*, const uint16_t*, float*, int, int,
                         int, int, hipStream_t);

}  // namespace

int main(int argc, char** argv) {
    const bool bf16 = argc < 2 || strcmp(argv[1], "fp16") != 0;
    const int B = argc > 4 ? atoi(argv[2]) : 32, NL = argc > 4 ? atoi(argv[3]) : 1024,
              NI = argc > 4 ? atoi(argv[4]) : 784;
    const char* libpath = getenv("XATTN_KERNELS_SO");
    if (!libpath) libpath = "fast-cuda-cross-attention_amd/kernels.so";
    if (B < 1 || NL < 1 || NI < 1) {
        fprintf(stderr, "usage: %s [bf16|fp16] [B NL NI]\n", argv[0]);
        return 2;
    }
    void* lib = dlopen(libpath, RTLD_NOW);
    if (!lib) {
        fprintf(stderr, "dlopen %s: %s\n", libpath, dlerror());
        return 1;
    }
    const LaunchFn ref = (LaunchFn)dlsym(lib, bf16 ? "launch_wmma_bf16_kernel" : "launch_wmma_kernel");
    if (!ref) {
        fprintf(stderr, "no launch_wmma entry point in %s\n", libpath);
        return 1;
    }
    const int D = xattn::kDim;
    std::mt19937 rng(0);
    std::normal_distribution<float> nd(0.f, 1.f);
    const float qs = 1.0f / std::sqrt((float)D);  // the entry points take Q pre-scaled
    std::vector<unsigned short> hq((size_t)B * NL * D), hk((size_t)B * NI * D), hv(hk.size());
    for (auto& x : hq) x = to16(nd(rng) * qs, bf16);
    for (auto& x : hk) x = to16(nd(rng), bf16);
    for (auto& x : hv) x = to16(nd(rng), bf16);
    uint16_t *q, *k, *v;
    float *o_ref, *o_sr;
    unsigned long long* clk = nullptr;
    const size_t on = (size_t)B * NL * D;
    check(hipMalloc(&q, hq.size() * 2), "hipMalloc");
    check(hipMalloc(&k, hk.size() * 2), "hipMalloc");
    check(hipMalloc(&v, hv.size() * 2), "hipMalloc");
    check(hipMalloc(&o_ref, on * 4), "hipMalloc");
    check(hipMalloc(&o_sr, on * 4), "hipMalloc");
    check(hipMemcpy(q, hq.data(), hq.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    check(hipMemcpy(k, hk.data(), hk.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    check(hipMemcpy(v, hv.data(), hv.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");

    sr::Params p;
    p.Q = q, p.K = k, p.V = v, p.out = o_sr, p.B = B, p.NL = NL, p.NI = NI;
    p.row_blocks = (NL + sr::BM - 1) / sr::BM;
    const int nblk = B * p.row_blocks;
#ifdef STEP_CLOCK
    check(hipMalloc(&clk, (size_t)nblk * sr::NWAVE * 8 * 8), "hipMalloc");
#endif
    p.clock = clk;
    auto run_sr = [&]() {
        if (bf16) hipLaunchKernelGGL(sr::split_role_kernel<__bf16>, dim3(nblk), dim3(512), 0, 0, p);
        else hipLaunchKernelGGL(sr::split_role_kernel<_Float16>, dim3(nblk), dim3(512), 0, 0, p);
    };
    auto run_ref = [&]() { ref(q, k, v, o_ref, B, NL, NI, D, 0); };

    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    auto time = [&](auto&& fn, int n) {
        check(hipEventRecord(e0, 0), "hipEventRecord");
        for (int i = 0; i < n; ++i) fn();
        check(hipEventRecord(e1, 0), "hipEventRecord");
        check(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms;
        check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        return 1e3 * ms / n;
    };
    for (int i = 0; i < 50; ++i) run_ref(), run_sr();
    check(hipDeviceSynchronize(), "warmup");
    double t_ref = 0, t_sr = 0;
    const int reps = 4, n = 100;
    for (int r = 0; r < reps; ++r) t_ref += time(run_ref, n), t_sr += time(run_sr, n);
    check(hipDeviceSynchronize(), "timed launches");

    std::vector<float> a(on), bref(on);
    check(hipMemcpy(a.data(), o_sr, on * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    check(hipMemcpy(bref.data(), o_ref, on * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    double maxabs = 0, num = 0, den = 0;
    for (size_t i = 0; i < on; ++i) {
        const double d = (double)a[i] - bref[i];
        maxabs = std::fmax(maxabs, std::fabs(d));
        num += d * d, den += (double)bref[i] * bref[i];
    }
    printf("%s B=%d NL=%d NI=%d: library %.2f us, split-role %.2f us per call "
           "(%d x %d interleaved); outputs differ by max-abs %.3g, rel %.3g\n",
           bf16 ? "bf16" : "fp16", B, NL, NI, t_ref / reps, t_sr / reps, reps, n, maxabs,
           std::sqrt(num / (den > 0 ? den : 1)));
#ifdef STEP_CLOCK
    std::vector<unsigned long long> c((size_t)nblk * sr::NWAVE * 8);
    check(hipMemcpy(c.data(), clk, c.size() * 8, hipMemcpyDeviceToHost), "hipMemcpy");
    double s[2][5] = {};
    for (int bk = 0; bk < nblk; ++bk)
        for (int w = 0; w < sr::NWAVE; ++w)
            for (int f = 0; f < 5; ++f) s[w / 4][f] += (double)c[((size_t)bk * sr::NWAVE + w) * 8 + f];
    const double steps = (double)((NI + sr::BN - 1) / sr::BN + 1), per = 4.0 * nblk;
    printf("score wavefronts:  K reads + MFMA %.0f, softmax + P write %.0f, DMA issue + wait + "
           "barrier %.0f cycles per step\n",
           s[0][2] / per / steps, s[0][3] / per / steps, s[0][4] / per / steps);
    printf("output wavefronts: reads + MFMA + V DMA issue %.0f, wait + barrier %.0f cycles per step\n",
           s[1][2] / per / steps, s[1][4] / per / steps);
    printf("lifetime: %.0f cycles before the loop, %.0f from the loop to the end (per wavefront)\n",
           (s[0][0] + s[1][0]) / (2 * per), (s[0][1] + s[1][1]) / (2 * per));
    check(hipFree(clk), "hipFree");
#endif
    check(hipFree(q), "hipFree");
    check(hipFree(k), "hipFree");
    check(hipFree(v), "hipFree");
    check(hipFree(o_ref), "hipFree");
    check(hipFree(o_sr), "hipFree");
    return 0;
}
