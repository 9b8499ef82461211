// fp16 / bf16 fused cross-attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}),
// fp32 accumulate, fp32 online softmax, fp32 output.
//
// Contract (kernel_wmma.cu:42-137): Q arrives pre-scaled by 1/sqrt(D), so a
// score is the plain dot product q.k.
//
// Work item = (batch, key split, 64 latents); 4 wavefronts x 16 latents, the
// same S^T formulation as the fp32 kernel:
//
//   S^T[32 keys x 16 q] = K_tile . Q^T       2 x 24 MFMA (k = 32)
//   O[16 q x 768]     += P[16 q x 32 keys] . V_tile     48 MFMA (k = 32)
//
// After the two S^T MFMAs (keys 0..15 and 16..31 of the tile), lane (j, g)
// holds S[q = j][4g + i] and S[q = j][16 + 4g + i], i < 4: eight scores, which
// become the eight k-values of its P operand directly.  The matching V operand
// needs those eight keys contiguous for one d, so V is written into LDS
// transposed, Vt[d][pos] with pos = 8g + e for key 4g + e (e < 4) and
// 16 + 4g + (e - 4) (e >= 4): one 16-byte read per lane per MFMA.
//
// K tile (32 x 768, 48 KiB) arrives by global->LDS DMA into a row-major layout
// whose 16-byte blocks are XOR-swizzled by (row & 15), which keeps the 16 rows
// read by one MFMA on distinct banks without padding (padding would break the
// 1 KiB DMA chunks).  K is double-buffered; V goes global -> VGPR -> transpose
// -> LDS one tile ahead.  LDS: 2 x 48 KiB (K) + 60 KiB (Vt) = 156 KiB.
#include "xattn_common.h"

namespace xattn {
namespace h16 {

constexpr int BN = 32;                 // keys per tile
constexpr int QW = 16;                 // latents per wavefront
constexpr int NW = 4;
constexpr int BM = QW * NW;            // 64 latents per workgroup
constexpr int KBLK = kDim / 8;         // 16-byte blocks per K row (96)
constexpr int KBUF = BN * kDim;        // halves per K buffer
constexpr int VT_ROW = BN + 8;         // Vt row stride in halves (80 B: conflict-free reads)
constexpr int VT_BUF = kDim * VT_ROW;  // halves
constexpr int K_CHUNKS = BN * KBLK / kWave;  // 1 KiB DMA chunks per K tile (48)
constexpr int K_CPW = K_CHUNKS / NW;         // per wavefront (12)
constexpr int V_UNITS = (BN / 4) * KBLK;     // 4 keys x 8 d units per tile (768)
constexpr int V_UPT = V_UNITS / (NW * kWave);  // per thread (3)
constexpr float kTauLog2 = 8.0f;

static_assert((2 * KBUF + VT_BUF) * 2 <= 160 * 1024, "LDS budget");
static_assert(V_UNITS % (NW * kWave) == 0, "V units per thread");

struct Params {
    const u16* Q;
    const u16* K;
    const u16* V;
    float* out;
    float* po;
    float* pm;
    float* pl;
    int B, NL, NI, S, chunk, row_blocks;
};

typedef unsigned int u4v __attribute__((ext_vector_type(4)));

// Operand vector type of the MFMA for element type T (8 x 16-bit).
template <typename T> struct Vec8;
template <> struct Vec8<_Float16> { typedef h8 type; };
template <> struct Vec8<__bf16> { typedef bf8 type; };

template <typename T>
__device__ inline f4 mfma32(typename Vec8<T>::type a, typename Vec8<T>::type b, f4 c) {
    if constexpr (__is_same(T, _Float16))
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ inline unsigned pack2(float lo, float hi) {
    const T a = (T)lo, b = (T)hi;
    return (unsigned)__builtin_bit_cast(u16, a) | ((unsigned)__builtin_bit_cast(u16, b) << 16);
}

// Swizzled position (in 16-byte blocks) of block c of K-tile row r.
__device__ inline int kpos(int r, int c) { return r * KBLK + (c ^ (r & 15)); }

template <typename T, bool PARTIAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void flash16_kernel(Params p) {
    typedef typename Vec8<T>::type v8;
    __shared__ __attribute__((aligned(16))) u16 lds[2 * KBUF + VT_BUF];
    u16* const vt = lds + 2 * KBUF;

    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int rb = item % p.row_blocks;
    const int bs = item / p.row_blocks;
    const int split = bs % p.S;
    const int b = bs / p.S;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int j = lane & 15, g = lane >> 4;
    const int q0 = rb * BM + w * QW;

    int k0 = 0, k1 = p.NI;
    if (PARTIAL) {
        k0 = split * p.chunk;
        k1 = min(k0 + p.chunk, p.NI);
    }

    if (k0 >= k1) {
        // empty key range: sentinel partials (kernel_wmma_splitk.cu:65-76) or zeros
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = q0 + 4 * g + i;
            if (q >= p.NL) continue;
            float* dst = PARTIAL ? p.po + (((size_t)b * p.NL + q) * p.S + split) * kDim
                                 : p.out + ((size_t)b * p.NL + q) * kDim;
#pragma unroll
            for (int t = 0; t < 48; ++t) dst[16 * t + j] = 0.f;
        }
        if (PARTIAL && g == 0 && q0 + j < p.NL) {
            const size_t pi = ((size_t)b * p.NL + q0 + j) * p.S + split;
            p.pm[pi] = -FLT_MAX;
            p.pl[pi] = 0.f;
        }
        return;
    }

    const u16* Kb = p.K + (size_t)b * p.NI * kDim;
    const u16* Vb = p.V + (size_t)b * p.NI * kDim;
    const int ntiles = (k1 - k0 + BN - 1) / BN;

    // K tile -> LDS by DMA: chunk m of the tile fills swizzled blocks
    // [64m, 64m + 64); lane i fetches the global block that belongs at 64m + i.
    auto issue_k = [&](int tile) {
        u16* buf = lds + (tile & 1) * KBUF;
        const int n0 = k0 + tile * BN;
#pragma unroll
        for (int t = 0; t < K_CPW; ++t) {
            const int m = w * K_CPW + t;
            const int P = 64 * m + lane;
            const int r = P / KBLK;
            const int c = (P - r * KBLK) ^ (r & 15);
            const int key = min(n0 + r, k1 - 1);
            dma16(Kb + (size_t)key * kDim + 8 * c, buf + 64 * 8 * m);
        }
    };

    // V tile -> registers: unit u = tid + 256 x covers keys 4kg..4kg+3 and
    // d = 8db..8db+7 with kg = u % 8, db = u / 8: per load, 8 lanes read 128
    // contiguous bytes of one row, and the transposed 8-byte writes of one
    // instruction fall on 32 distinct banks (4-way instead of 32-way).
    u4v vreg[V_UPT][4];
    auto load_v = [&](int tile) {
        const int n0 = k0 + tile * BN;
#pragma unroll
        for (int x = 0; x < V_UPT; ++x) {
            const int u = tid + 256 * x;
            const int kg = u & 7, db = u >> 3;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = min(n0 + 4 * kg + e, k1 - 1);
                vreg[x][e] = *(const u4v*)(Vb + (size_t)key * kDim + 8 * db);
            }
        }
    };
    // registers -> Vt[d][pos(key)], 4 keys (8 bytes) per write
    auto store_vt = [&]() {
#pragma unroll
        for (int x = 0; x < V_UPT; ++x) {
            const int u = tid + 256 * x;
            const int kg = u & 7, db = u >> 3;
            const int pos = kg < 4 ? 8 * kg : 8 * (kg - 4) + 4;
#pragma unroll
            for (int h = 0; h < 4; ++h) {  // column pair (2h, 2h+1) of the 8 columns
                const unsigned r0 = vreg[x][0][h], r1 = vreg[x][1][h];
                const unsigned r2 = vreg[x][2][h], r3 = vreg[x][3][h];
                // low halves -> column 2h, high halves -> column 2h+1
                const unsigned lo01 = __builtin_amdgcn_perm(r1, r0, 0x05040100u);
                const unsigned lo23 = __builtin_amdgcn_perm(r3, r2, 0x05040100u);
                const unsigned hi01 = __builtin_amdgcn_perm(r1, r0, 0x07060302u);
                const unsigned hi23 = __builtin_amdgcn_perm(r3, r2, 0x07060302u);
                const int d = 8 * db + 2 * h;
                typedef unsigned u2v __attribute__((ext_vector_type(2)));
                *(u2v*)(vt + (size_t)d * VT_ROW + pos) = (u2v){lo01, lo23};
                *(u2v*)(vt + (size_t)(d + 1) * VT_ROW + pos) = (u2v){hi01, hi23};
            }
        }
    };

    // Q^T operand: Q[q0 + j][32s + 8g .. +7], s < 24 (96 registers).
    v8 qr[24];
    {
        const int qc = min(q0 + j, p.NL - 1);
        const u16* qrow = p.Q + ((size_t)b * p.NL + qc) * kDim + 8 * g;
#pragma unroll
        for (int s = 0; s < 24; ++s) qr[s] = *(const v8*)(qrow + 32 * s);
    }
    issue_k(0);
    load_v(0);

    f4 acc[48];
#pragma unroll
    for (int t = 0; t < 48; ++t) acc[t] = (f4){0.f, 0.f, 0.f, 0.f};

    const float tau_raw = kTauLog2 / kLog2e;
    float m_true = -FLT_MAX, m_used = -FLT_MAX, lsum = 0.f;

    for (int tile = 0; tile < ntiles; ++tile) {
        const int n0 = k0 + tile * BN;
        wait_vmcnt<V_UPT * 4>();  // K(tile) landed; V(tile) loads may be in flight
        lds_barrier();            // and every wave is done with Vt and K(tile-1)
        if (tile + 1 < ntiles) issue_k(tile + 1);
        store_vt();
        if (tile + 1 < ntiles) load_v(tile + 1);

        // ---------------- QK: two 16-key halves ----------------
        f4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
        {
            const u16* kb = lds + (tile & 1) * KBUF;
            v8 ka[3], kbv[3];
            ka[0] = *(const v8*)(kb + 8 * kpos(j, g));
            kbv[0] = *(const v8*)(kb + 8 * kpos(16 + j, g));
            ka[1] = *(const v8*)(kb + 8 * kpos(j, 4 + g));
            kbv[1] = *(const v8*)(kb + 8 * kpos(16 + j, 4 + g));
#pragma unroll
            for (int s = 0; s < 24; ++s) {
                if (s + 2 < 24) {
                    ka[(s + 2) % 3] = *(const v8*)(kb + 8 * kpos(j, 4 * (s + 2) + g));
                    kbv[(s + 2) % 3] = *(const v8*)(kb + 8 * kpos(16 + j, 4 * (s + 2) + g));
                }
                sa = mfma32<T>(ka[s % 3], qr[s], sa);
                sb = mfma32<T>(kbv[s % 3], qr[s], sb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---------------- online softmax (raw-dot units) ----------------
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = (n0 + 4 * g + i < k1) ? sa[i] : -INFINITY;
            x[4 + i] = (n0 + 16 + 4 * g + i < k1) ? sb[i] : -INFINITY;
        }
        float tmax = x[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, x[i]);
        tmax = wave_max16_groups(tmax);
        m_true = fmaxf(m_true, tmax);
        const bool grow = tmax > m_used + tau_raw;
        if (__any(grow)) {
            const float m_new = grow ? tmax : m_used;
            const float alpha = fast_exp2((m_used - m_new) * kLog2e);
            lsum *= alpha;
            m_used = m_new;
            float a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int t = 0; t < 48; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] *= a[i];
        }
        float pw[8];
        float rs = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pw[i] = fast_exp2((x[i] - m_used) * kLog2e);
            rs += pw[i];
        }
        lsum += wave_sum16_groups(rs);
        const v8 pa = __builtin_bit_cast(
            v8, ((u4v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3]), pack2<T>(pw[4], pw[5]),
                       pack2<T>(pw[6], pw[7])}));

        // ---------------- PV ----------------
        lds_barrier();  // Vt of this tile written by every wave
        {
            const u16* vb = vt + (size_t)j * VT_ROW + 8 * g;
            v8 vv[3];
            vv[0] = *(const v8*)(vb);
            vv[1] = *(const v8*)(vb + 16 * VT_ROW);
#pragma unroll
            for (int t = 0; t < 48; ++t) {
                if (t + 2 < 48) vv[(t + 2) % 3] = *(const v8*)(vb + (size_t)16 * (t + 2) * VT_ROW);
                acc[t] = mfma32<T>(pa, vv[t % 3], acc[t]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    const float factor = fast_exp2((m_used - m_true) * kLog2e);
    const float rowscale = PARTIAL ? factor : factor / (lsum * factor + 1e-6f);
    float rsc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rsc[i] = __shfl(rowscale, 4 * g + i);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = q0 + 4 * g + i;
        if (q >= p.NL) continue;
        float* dst = PARTIAL ? p.po + (((size_t)b * p.NL + q) * p.S + split) * kDim
                             : p.out + ((size_t)b * p.NL + q) * kDim;
#pragma unroll
        for (int t = 0; t < 48; ++t) dst[16 * t + j] = acc[t][i] * rsc[i];
    }
    if (PARTIAL && g == 0 && q0 + j < p.NL) {
        const size_t pi = ((size_t)b * p.NL + q0 + j) * p.S + split;
        p.pm[pi] = m_true;  // scores are q.k with Q pre-scaled
        p.pl[pi] = lsum * factor;
    }
}

}  // namespace h16

int h16_row_blocks(int NL) { return (NL + h16::BM - 1) / h16::BM; }

bool launch_flash16(bool bf16, const void* Q, const void* K, const void* V, float* out, float* po,
                    float* pm, float* pl, int B, int NL, int NI, int S, int chunk,
                    hipStream_t stream) {
    h16::Params p;
    p.Q = (const u16*)Q; p.K = (const u16*)K; p.V = (const u16*)V;
    p.out = out; p.po = po; p.pm = pm; p.pl = pl;
    p.B = B; p.NL = NL; p.NI = NI; p.S = S; p.chunk = chunk;
    p.row_blocks = h16_row_blocks(NL);
    const long long nblk = (long long)B * p.row_blocks * S;
    if (nblk <= 0) return true;
    if (nblk > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "grid of %lld workgroups too large", nblk);
        return false;
    }
    const dim3 grid((unsigned)nblk), block(256);
    if (bf16) {
        if (po) hipLaunchKernelGGL((h16::flash16_kernel<__bf16, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((h16::flash16_kernel<__bf16, false>), grid, block, 0, stream, p);
    } else {
        if (po) hipLaunchKernelGGL((h16::flash16_kernel<_Float16, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((h16::flash16_kernel<_Float16, false>), grid, block, 0, stream, p);
    }
    return check_launch(bf16 ? "flash_bf16" : "flash_f16");
}

}  // namespace xattn
