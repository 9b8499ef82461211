// fp16 / bf16 fused cross-attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}),
// fp32 accumulate, fp32 online softmax, fp32 output.
//
// Contract (kernel_wmma.cu:42-137): Q arrives pre-scaled by 1/sqrt(D), so a
// score is the plain dot product q.k.
//
// Work item = (batch, key split, 64 latents) on 4 wavefronts; tiles of 32 keys.
// Every wavefront owns a 192-column slice of D, for the scores and for the
// output alike, so a K or V element read from LDS feeds four MFMAs (one per
// 16-latent block) instead of one:
//
//   partial S^T[32 keys x 64 q] = K[:, slice] . Q[:, slice]^T   2 x 4 x 6 MFMA
//   O^T[slice x 64 q]         += V[:, slice]^T . P^T            12 x 4 MFMA
//
// The four partial score blocks are summed through LDS (in the buffer the K
// tile just left); wavefront c then owns the softmax of latents 16c..16c+15
// and publishes their P operand (1 KiB) for all four wavefronts.
//
// Layouts.  In the S^T MFMA (A = K rows, B = Q^T) lane (j, g) ends with
// S[q = j][4g + i] and S[q = j][16 + 4g + i], i < 4: the eight k-values of the
// P^T operand, whose k order {4g..4g+3, 16+4g..16+4g+3} the V^T operand must
// follow.  V^T's A operand needs, in lane (j, g), V[4g + e][d0 + j] and
// V[16 + 4g + e][d0 + j]: eight keys of one column.  gfx950's transposing LDS
// read (ds_read_b64_tr_b16) delivers exactly that from a row-major V tile:
// within each 16-lane group, lane i receives element (i mod 4) of the 8-byte
// rows read by lanes 4e + i/4 (e < 4), so lane 4e + q of group g points at
// V[4g + e][d0 + 4q] and lane j gets V[4g + e][d0 + j] for e = 0..3.  The O^T
// accumulator puts O[q = j][d0 + 4g .. d0 + 4g + 3] in lane (j, g): one
// 16-byte store per (latent block, column block).
//
// K and V both arrive by global->LDS DMA into row-major 32 x 768 tiles (48 KiB)
// on one pipeline: phases alternate QK(t) / PV(t), phase p reads buffer p % 3
// and requests phase p + 2; 3 buffers = 144 KiB.  The 16-byte blocks of row r
// are XOR-swizzled by f(r) = 2(r & 7) + ((r >> 3) & 1), which is distinct for
// 16 consecutive rows (the 16 rows of one b128 K read hit 16 different 4-bank
// groups) and keeps the 32-byte column pairs of 8 consecutive rows apart (one
// transposed V read of 32 lanes covers all 64 banks once), so neither reader
// conflicts and no padding breaks the contiguous 1 KiB DMA chunks.
#include "xattn_common.h"

namespace xattn {
namespace h16 {

constexpr int BN = 32;                 // keys per tile
constexpr int NW = 4;                  // wavefronts per workgroup
constexpr int QB = 16;                 // latents per MFMA block
constexpr int BM = QB * NW;            // 64 latents per workgroup
constexpr int DW = kDim / NW;          // columns of D per wavefront (192)
constexpr int KS = DW / 32;            // k-steps of a score MFMA chain (6)
constexpr int DB = DW / 16;            // 16-column output blocks per wavefront (12)
constexpr int KBLK = kDim / 8;         // 16-byte blocks per row (96)
constexpr int BUF = BN * kDim;         // halves per tile buffer
constexpr int NBUF = 3;
constexpr int CHUNKS = BN * KBLK / kWave;  // 1 KiB DMA chunks per tile (48)
constexpr int CPW = CHUNKS / NW;           // per wavefront (12)

static_assert(NBUF * BUF * 2 + NW * kWave * 16 + BM * 4 + 4 <= 160 * 1024, "LDS budget");
static_assert(NW * NW * 2 * kWave * 16 <= BUF * 2, "score exchange fits in a tile buffer");

// A row's weights are exp2(s - m_ref) with m_ref fixed for a whole pass over
// the keys; a pass restarts when some score exceeds m_ref by tau_log2<T> (in
// exp2 units), which bounds every weight by 2^tau_log2<T> in the MFMA's input
// type: 2^15 for fp16 (largest finite 65504), 2^64 for bf16 (fp32's range).
template <typename T> constexpr float tau_log2 = 64.0f;
template <> constexpr float tau_log2<_Float16> = 15.0f;

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
    __shared__ __attribute__((aligned(16))) u4v pbuf[NW * kWave];  // P^T operand per latent block
    __shared__ float rowscale_lds[BM];
    __shared__ int restart_flag;

    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int rb = item % p.row_blocks;
    const int bs = item / p.row_blocks;
    const int split = bs % p.S;
    const int b = bs / p.S;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int j = lane & 15, g = lane >> 4;
    const int q0 = rb * BM;      // first latent of the workgroup
    const int d0 = w * DW;       // first column of this wavefront's slice

    int k0 = 0, k1 = p.NI;
    if (PARTIAL) {
        k0 = split * p.chunk;
        k1 = min(k0 + p.chunk, p.NI);
    }

    // output row of latent q (this split's partial row when PARTIAL)
    auto out_row = [&](int q) {
        return PARTIAL ? p.po + (((size_t)b * p.NL + q) * p.S + split) * kDim
                       : p.out + ((size_t)b * p.NL + q) * kDim;
    };

    if (k0 >= k1) {
        // empty key range: sentinel partials (kernel_wmma_splitk.cu:65-76) or zeros
#pragma unroll
        for (int c = 0; c < NW; ++c) {
            const int q = q0 + QB * c + j;
            if (q >= p.NL) continue;
            float* dst = out_row(q) + d0 + 4 * g;
#pragma unroll
            for (int e = 0; e < DB; ++e) *(f4*)(dst + 16 * e) = (f4){0.f, 0.f, 0.f, 0.f};
        }
        if (PARTIAL && g == 0 && q0 + QB * w + j < p.NL) {
            const size_t pi = ((size_t)b * p.NL + q0 + QB * w + j) * p.S + split;
            p.pm[pi] = -FLT_MAX;
            p.pl[pi] = 0.f;
        }
        return;
    }

    // K and V rows of this split's key range; keys are counted from k0 below.
    const u16* Kb = p.K + ((size_t)b * p.NI + k0) * kDim;
    const u16* Vb = p.V + ((size_t)b * p.NI + k0) * kDim;
    const int nk = k1 - k0;
    // Non-empty (the early return above); without these facts the compiler
    // guards the tile loop for zero trips and the split-K instantiation no
    // longer fits the 512 registers.
    __builtin_assume(nk >= 1);
    const int ntiles = (nk + BN - 1) / BN;
    __builtin_assume(ntiles >= 1);
    const int nphase = 2 * ntiles;

    // DMA: chunk m of a tile fills swizzled blocks [64m, 64m + 64); lane i
    // fetches the global block that belongs at 64m + i.  For a full tile the
    // per-lane byte offset of chunk w*CPW + t is dofs[t].  The DMA is issued
    // untracked (dma16_untracked): the phase waits below order it.
    unsigned dofs[CPW];
#pragma unroll
    for (int t = 0; t < CPW; ++t) {
        const int P = 64 * (w * CPW + t) + lane;
        const int r = P / KBLK;
        dofs[t] = (unsigned)(2 * (r * kDim + 8 * ((P - r * KBLK) ^ swz(r))));
    }
    const unsigned lds0 = lds_u32(lds);
    auto issue = [&](int ph) {
        const int n0 = (ph >> 1) * BN;
        const u16* src = uniform_ptr(((ph & 1) ? Vb : Kb) + (size_t)n0 * kDim);
        const unsigned buf = lds0 + (unsigned)((ph % NBUF) * BUF * 2 + 1024 * w * CPW);
        const int last = nk - 1 - n0;  // last valid row of this tile
        if (last >= BN - 1) {
#pragma unroll
            for (int t = 0; t < CPW; ++t) dma16_untracked(src, dofs[t], buf + 1024 * t);
        } else {
            // partial tile: rows past the range re-read its last row (their
            // scores are masked to -inf and their weights are 0).  The row of
            // a full-tile offset is offset / 1536 (a row is 1536 bytes and
            // the block part stays below that).  The empty asm hides the
            // offset's origin, so none of this is hoisted out of the loop as
            // extra per-lane state.
#pragma unroll
            for (int t = 0; t < CPW; ++t) {
                unsigned o = dofs[t];
                asm volatile("" : "+v"(o));
                const int r = (int)(o / (2 * kDim));
                dma16_untracked(src, o - (unsigned)(max(r - last, 0) * 2 * kDim), buf + 1024 * t);
            }
        }
    };

    // Q^T operand of latent block c, k-step s: Q[q0 + 16c + j][d0 + 32s + 8g .. +7]
    // (96 registers).  Latents past NL repeat the last one; they are not stored.
    // K(0) is requested first; the full wait after the Q loads leaves no
    // compiler-visible load pending, so the compiler adds no waits inside the
    // tile loop (where only untracked DMA is in flight).
    issue(0);
    v8 qr[NW][KS];
#pragma unroll
    for (int c = 0; c < NW; ++c) {
        const int qc = min(q0 + QB * c + j, p.NL - 1);
        const u16* qrow = p.Q + ((size_t)b * p.NL + qc) * kDim + d0 + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s) qr[c][s] = *(const v8*)(qrow + 32 * s);
    }
    wait_vmcnt<0>();

    // LDS read offsets (in halves, relative to a tile buffer).  A block index
    // X < 96 XOR f < 16 stays inside its row.
    // K (A operand of the scores): row j (16 + j for keys 16..31; f(16 + j) =
    // f(j)), block (d0 + 32s + 8g) / 8.
    int kofs[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) kofs[s] = j * kDim + 8 * ((d0 / 8 + 4 * s + g) ^ swz(j));
    // V (transposed read): lane 4e + q of group g reads row 4g + e at column
    // d0 + 16t + 4q, i.e. block (d0 + 16t)/8 + (q >> 1), byte 8(q & 1).
    int vofs[DB];
    {
        const int row = 4 * g + (j >> 2), q = j & 3;
#pragma unroll
        for (int t = 0; t < DB; ++t)
            vofs[t] = row * kDim + 8 * (((d0 + 16 * t) / 8 + (q >> 1)) ^ swz(row)) + 4 * (q & 1);
    }

    if (tid == 0) restart_flag = 0;

    const float tau_raw = tau_log2<T> / kLog2e;
    // Softmax state of latent q0 + 16w + j (this wavefront's block), replicated
    // over g.  m_true: exact running max; m_ref: the reference of the weights,
    // fixed for a pass (set on the first tile of the first pass, raised to
    // m_true when a pass restarts).
    float m_true = -FLT_MAX, m_ref = -FLT_MAX, lsum;
    f4 acc[NW][DB];  // O^T[d0 + 16t + 4g + i][q0 + 16c + j]

    for (bool first = true;; first = false) {  // passes over the key range; a second is rare
        if (!first) issue(0);
        issue(1);
#pragma unroll
        for (int c = 0; c < NW; ++c)
#pragma unroll
            for (int t = 0; t < DB; ++t) acc[c][t] = (f4){0.f, 0.f, 0.f, 0.f};
        lsum = 0.f;
        bool restart = false;

        for (int tile = 0; tile < ntiles; ++tile) {
            const int n0 = tile * BN;
            int ph = 2 * tile;

            // ---------------- partial scores over this wavefront's slice ----------------
            wait_vmcnt<CPW>();
            lds_barrier();
            if (ph + 2 < nphase) issue(ph + 2);
            u16* kb = lds + (ph % NBUF) * BUF;
            f4 sacc[2][NW];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int c = 0; c < NW; ++c) sacc[h][c] = (f4){0.f, 0.f, 0.f, 0.f};
            {
                // fragment f: k-step f >> 1, keys 16 (f & 1) .. +15
                auto kfrag = [&](int f) {
                    return *(const v8*)(kb + kofs[f >> 1] + (f & 1) * 16 * kDim);
                };
                // one fragment read ahead: each one feeds four MFMAs
                v8 kf[2];
                kf[0] = kfrag(0);
#pragma unroll
                for (int f = 0; f < 2 * KS; ++f) {
                    if (f + 1 < 2 * KS) kf[(f + 1) & 1] = kfrag(f + 1);
#pragma unroll
                    for (int c = 0; c < NW; ++c)
                        sacc[f & 1][c] = mfma32<T>(kf[f & 1], qr[c][f >> 1], sacc[f & 1][c]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // Every wavefront is done with K(t): its buffer carries the partial
            // sums, slot ((c * 4 + source) * 2 + h), 64 lanes x 16 B each.
            lds_barrier();
            f4* xs = (f4*)kb;
#pragma unroll
            for (int c = 0; c < NW; ++c)
#pragma unroll
                for (int h = 0; h < 2; ++h) xs[((c * NW + w) * 2 + h) * kWave + lane] = sacc[h][c];
            lds_barrier();
            f4 sa = xs[((w * NW) * 2 + 0) * kWave + lane];
            f4 sb = xs[((w * NW) * 2 + 1) * kWave + lane];
#pragma unroll
            for (int src = 1; src < NW; ++src) {
                sa += xs[((w * NW + src) * 2 + 0) * kWave + lane];
                sb += xs[((w * NW + src) * 2 + 1) * kWave + lane];
            }

            // ---------------- softmax weights of latent block w (raw-dot units) ----------------
            float x[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = (n0 + 4 * g + i < nk) ? sa[i] : -INFINITY;
                x[4 + i] = (n0 + 16 + 4 * g + i < nk) ? sb[i] : -INFINITY;
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
            pbuf[w * kWave + lane] = (u4v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3]),
                                           pack2<T>(pw[4], pw[5]), pack2<T>(pw[6], pw[7])};

            // ---------------- O^T += V^T . P^T over this wavefront's slice ----------------
            ph += 1;
            if (ph + 1 < nphase) wait_vmcnt<CPW>();
            else wait_vmcnt<0>();
            lds_barrier();
            // Every wavefront sets the flag (if at all) before this barrier, so
            // all read the same value.
            if (__builtin_amdgcn_readfirstlane(restart_flag)) {
                restart = true;
                break;
            }
            if (ph + 2 < nphase) issue(ph + 2);
            v8 pt[NW];
#pragma unroll
            for (int c = 0; c < NW; ++c) pt[c] = __builtin_bit_cast(v8, pbuf[c * kWave + lane]);
            {
                const u16* vb = lds + (ph % NBUF) * BUF;
                s4 va[2], vc[2];
                va[0] = tr_read(vb + vofs[0]);
                vc[0] = tr_read(vb + vofs[0] + 16 * kDim);
#pragma unroll
                for (int t = 0; t < DB; ++t) {
                    if (t + 1 < DB) {
                        va[(t + 1) & 1] = tr_read(vb + vofs[t + 1]);
                        vc[(t + 1) & 1] = tr_read(vb + vofs[t + 1] + 16 * kDim);
                    }
                    const v8 vt = __builtin_bit_cast(
                        v8, __builtin_shufflevector(va[t & 1], vc[t & 1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                    for (int c = 0; c < NW; ++c) acc[c][t] = mfma32<T>(vt, pt[c], acc[c][t]);
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

    // Normalisation (or the partial's rescale to m_true) of latent block w,
    // shared with the wavefronts that hold its other columns.
    const float factor = fast_exp2((m_ref - m_true) * kLog2e);
    const float rowscale = PARTIAL ? factor : factor / (lsum * factor + 1e-6f);
    if (g == 0) rowscale_lds[QB * w + j] = rowscale;
    if (PARTIAL && g == 0 && q0 + QB * w + j < p.NL) {
        const size_t pi = ((size_t)b * p.NL + q0 + QB * w + j) * p.S + split;
        p.pm[pi] = m_true;  // scores are q.k with Q pre-scaled
        p.pl[pi] = lsum * factor;
    }
    lds_barrier();
#pragma unroll
    for (int c = 0; c < NW; ++c) {
        const int q = q0 + QB * c + j;
        if (q >= p.NL) continue;
        const float sc = rowscale_lds[QB * c + j];
        float* dst = out_row(q) + d0 + 4 * g;
#pragma unroll
        for (int t = 0; t < DB; ++t) *(f4*)(dst + 16 * t) = acc[c][t] * sc;
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
