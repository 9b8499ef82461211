// fp16 / bf16 fused cross-attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}),
// fp32 accumulate, fp32 online softmax, fp32 output.
//
// Contract (kernel_wmma.cu:42-137): Q arrives pre-scaled by 1/sqrt(D), so a
// score is the plain dot product q.k.
//
// Work item = (batch, key split, 64 latents); 4 wavefronts x 16 latents, the
// S^T formulation of the fp32 kernel with 32-key tiles:
//
//   S^T[32 keys x 16 q] = K_tile . Q^T       2 x 24 MFMA (k = 32)
//   O[16 q x 768]     += P[16 q x 32 keys] . V_tile     48 MFMA (k = 32)
//
// After the two S^T MFMAs (tile keys 0..15 and 16..31), lane (j, g) holds
// S[q = j][4g + i] and S[q = j][16 + 4g + i], i < 4: the eight k-values of its
// P operand.  The V operand needs, in lane (j, g), V[4g + e][d0 + j] and
// V[16 + 4g + e][d0 + j]: eight keys of one column.  gfx950's transposing LDS
// read (ds_read_b64_tr_b16) delivers exactly that from a row-major V tile:
// within each 16-lane group, lane i receives element (i mod 4) of the 8-byte
// rows read by lanes 4e + i/4 (e < 4), so lane 4e + q of group g points at
// V[4g + e][d0 + 4q] and lane j gets V[4g + e][d0 + j] for e = 0..3.
//
// K and V therefore both arrive by global->LDS DMA into row-major tiles, one
// pipeline for both (as in the fp32 kernel): phases alternate QK(t) / PV(t),
// phase p reads buffer p % 3 and requests phase p + 2.  Tiles are 32 x 768
// (48 KiB); 3 buffers = 144 KiB.  The 16-byte blocks of row r are XOR-swizzled
// by f(r) = 2(r & 7) + ((r >> 3) & 1), which is distinct for 16 consecutive
// rows (the 16 rows of one b128 K read hit 16 different 4-bank groups) and
// keeps the 32-byte column pairs of 8 consecutive rows apart (one transposed V
// read of 32 lanes covers all 64 banks once), so neither reader conflicts and
// no padding breaks the contiguous 1 KiB DMA chunks.  K and V tiles share the
// layout, hence the per-lane DMA offsets.
#include "xattn_common.h"

namespace xattn {
namespace h16 {

constexpr int BN = 32;                 // keys per tile
constexpr int QW = 16;                 // latents per wavefront
constexpr int NW = 4;
constexpr int BM = QW * NW;            // 64 latents per workgroup
constexpr int KBLK = kDim / 8;         // 16-byte blocks per row (96)
constexpr int BUF = BN * kDim;         // halves per tile buffer
constexpr int NBUF = 3;
constexpr int CHUNKS = BN * KBLK / kWave;  // 1 KiB DMA chunks per tile (48)
constexpr int CPW = CHUNKS / NW;           // per wavefront (12)
// A row's weights are exp2(s - m_ref) with m_ref fixed for a whole pass over
// the keys; a pass restarts when some score exceeds m_ref by tau_log2<T> (in
// exp2 units), which bounds every weight by 2^tau_log2<T> in the MFMA's input
// type: 2^15 for fp16 (largest finite 65504), 2^64 for bf16 (fp32's range).
template <typename T> constexpr float tau_log2 = 64.0f;
template <> constexpr float tau_log2<_Float16> = 15.0f;

static_assert(NBUF * BUF * 2 <= 160 * 1024, "LDS budget");

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
typedef short s4 __attribute__((ext_vector_type(4)));
typedef short s8v __attribute__((ext_vector_type(8)));

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

// swizzle of the 16-byte blocks of tile row r
__device__ inline int swz(int r) { return 2 * (r & 7) + ((r >> 3) & 1); }

__device__ inline s4 tr_read(const u16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4*)(p));
}

template <typename T, bool PARTIAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void flash16_kernel(Params p) {
    typedef typename Vec8<T>::type v8;
    __shared__ __attribute__((aligned(16))) u16 lds[NBUF * BUF];

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
    const int nphase = 2 * ntiles;

    // DMA: chunk m of a tile fills swizzled blocks [64m, 64m + 64); lane i
    // fetches the global block that belongs at 64m + i.  For a full tile the
    // per-lane element offset of chunk w*CPW + t is dofs[t].
    unsigned dofs[CPW];
#pragma unroll
    for (int t = 0; t < CPW; ++t) {
        const int P = 64 * (w * CPW + t) + lane;
        const int r = P / KBLK;
        dofs[t] = (unsigned)(r * kDim + 8 * ((P - r * KBLK) ^ swz(r)));
    }
    auto issue = [&](int ph) {
        const int n0 = k0 + (ph >> 1) * BN;
        const u16* src = uniform_ptr(((ph & 1) ? Vb : Kb) + (size_t)n0 * kDim);
        u16* buf = lds + (ph % NBUF) * BUF;
        const int last = k1 - 1 - n0;  // last valid row of this tile
        if (last >= BN - 1) {
#pragma unroll
            for (int t = 0; t < CPW; ++t) dma16(src + dofs[t], buf + 64 * 8 * (w * CPW + t));
        } else {
            // partial tile: rows past k1 re-read the last valid row (their
            // scores are masked to -inf and their weights are 0)
#pragma unroll
            for (int t = 0; t < CPW; ++t) {
                const int P = 64 * (w * CPW + t) + lane;
                const int r = P / KBLK;
                const int c = (P - r * KBLK) ^ swz(r);
                dma16(src + (unsigned)(min(r, last) * kDim + 8 * c),
                      buf + 64 * 8 * (w * CPW + t));
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

    // LDS read bases (in halves, relative to a tile buffer).  f(r) < 16, so
    // the swizzle only touches the low 4 bits of a block index.
    // K (QK, A operand): row j, block 4s + g, s = 4a + bb ->
    //   j*768 + 128a + 8((4bb + g) ^ f(j)); rows 16 + j (f(16 + j) = f(j)) are
    //   16*768 further.
    int kofs[4];
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) kofs[bb] = j * kDim + 8 * ((4 * bb + g) ^ swz(j));
    // V (PV, transposed read): lane 4e + q of group g reads row 4g + e at
    // column 16t + 4q, i.e. block 2t + (q >> 1) at byte 8 (q & 1) ->
    //   row*768 + 128(t >> 3) + 8((2(t & 7) + (q >> 1)) ^ f(row)) + 4(q & 1).
    int vofs[8];
    {
        const int e = j >> 2, q = j & 3;
        const int row = 4 * g + e;
#pragma unroll
        for (int t8 = 0; t8 < 8; ++t8)
            vofs[t8] = row * kDim + 8 * ((2 * t8 + (q >> 1)) ^ swz(row)) + 4 * (q & 1);
    }

    __shared__ int restart_flag;
    if (tid == 0) restart_flag = 0;

    const float tau_raw = tau_log2<T> / kLog2e;
    // m_true: exact running max of this lane's latent; m_ref: the reference
    // of the weights, fixed for a pass (set on the first tile of the first
    // pass, raised to m_true when a pass restarts).
    float m_true = -FLT_MAX, m_ref = -FLT_MAX, lsum;
    f4 acc[48];

    for (;;) {  // passes over the key range; the second one is rare
        issue(0);
        issue(1);
#pragma unroll
        for (int t = 0; t < 48; ++t) acc[t] = (f4){0.f, 0.f, 0.f, 0.f};
        lsum = 0.f;
        bool restart = false;

        for (int tile = 0; tile < ntiles; ++tile) {
            const int n0 = k0 + tile * BN;
            int ph = 2 * tile;

            // ---------------- QK phase ----------------
            wait_vmcnt<CPW>();
            lds_barrier();
            if (ph + 2 < nphase) issue(ph + 2);
            f4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
            {
                const u16* kb = lds + (ph % NBUF) * BUF;
                v8 ka[3], kv[3];
                ka[0] = *(const v8*)(kb + kofs[0]);
                kv[0] = *(const v8*)(kb + kofs[0] + 16 * kDim);
                ka[1] = *(const v8*)(kb + kofs[1]);
                kv[1] = *(const v8*)(kb + kofs[1] + 16 * kDim);
#pragma unroll
                for (int s = 0; s < 24; ++s) {
                    if (s + 2 < 24) {
                        const int sn = s + 2;
                        const u16* pk = kb + kofs[sn & 3] + 128 * (sn >> 2);
                        ka[sn % 3] = *(const v8*)(pk);
                        kv[sn % 3] = *(const v8*)(pk + 16 * kDim);
                    }
                    sa = mfma32<T>(ka[s % 3], qr[s], sa);
                    sb = mfma32<T>(kv[s % 3], qr[s], sb);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }

            // ---------------- softmax weights (raw-dot units) ----------------
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
            if (m_ref == -FLT_MAX) m_ref = tmax;
            if (__any(tmax > m_ref + tau_raw) && lane == 0) restart_flag = 1;
            float pw[8];
            float rs = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pw[i] = fast_exp2((x[i] - m_ref) * kLog2e);
                rs += pw[i];
            }
            lsum += wave_sum16_groups(rs);
            const v8 pa = __builtin_bit_cast(
                v8, ((u4v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3]),
                           pack2<T>(pw[4], pw[5]), pack2<T>(pw[6], pw[7])}));

            // ---------------- PV phase ----------------
            ph += 1;
            if (ph + 1 < nphase) wait_vmcnt<CPW>();
            else wait_vmcnt<0>();
            lds_barrier();
            if (__builtin_amdgcn_readfirstlane(restart_flag)) {  // uniform over the workgroup
                restart = true;
                break;
            }
            if (ph + 2 < nphase) issue(ph + 2);
            {
                const u16* vb = lds + (ph % NBUF) * BUF;
                s4 va[3], vc[3];
                va[0] = tr_read(vb + vofs[0]);
                vc[0] = tr_read(vb + vofs[0] + 16 * kDim);
                va[1] = tr_read(vb + vofs[1]);
                vc[1] = tr_read(vb + vofs[1] + 16 * kDim);
#pragma unroll
                for (int t = 0; t < 48; ++t) {
                    if (t + 2 < 48) {
                        const int tn = t + 2;
                        const u16* pv = vb + vofs[tn & 7] + 128 * (tn >> 3);
                        va[tn % 3] = tr_read(pv);
                        vc[tn % 3] = tr_read(pv + 16 * kDim);
                    }
                    const s8v both = __builtin_shufflevector(va[t % 3], vc[t % 3], 0, 1, 2, 3,
                                                             4, 5, 6, 7);
                    acc[t] = mfma32<T>(pa, __builtin_bit_cast(v8, both), acc[t]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (!restart) break;
        // Some latent's scores outgrew its reference: drain the DMA, clear the
        // flag, and run the keys again with the reference raised to the max
        // seen so far.
        wait_vmcnt<0>();
        lds_barrier();
        if (tid == 0) restart_flag = 0;
        m_ref = m_true;
        lds_barrier();
    }

    const float factor = fast_exp2((m_ref - m_true) * kLog2e);
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
