// fp16 / bf16 fused cross-attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}),
// fp32 accumulate, fp32 online softmax, fp32 output.
//
// Contract (kernel_wmma.cu:42-137): Q arrives pre-scaled by 1/sqrt(D), so a
// score is the plain dot product q.k.
//
// Work item = (batch, key split, 64 latents = four 16-latent blocks) on 8
// wavefronts (two per SIMD); tiles of 32 keys.  Wavefront w has two roles:
//
//   scores:  unit (block c = w / 2, key half k = w % 2):
//            S^T[16 keys x 16 q] = K[16k.., :] . Q[block c, :]^T       24 MFMA
//            over all of D, then the unit's softmax and its half of the
//            block's P^T operand, in the wavefront's own registers;
//   output:  column slice w (96 columns) of all four latent blocks:
//            O^T[slice x 64 q] += V[:, slice]^T . P^T[blocks]           6 x 4 MFMA
//
// so scores never cross wavefronts: the only exchange is the P operand (one
// LDS write and read per block) plus, on the first tile and at restarts, the
// weights' reference of a block's two owners.  Each V^T fragment feeds one
// MFMA per latent block, so the CU reads each V tile from LDS once.  Per
// tile, each SIMD issues 96 MFMAs; registers per lane: the Q block (96), the
// O^T accumulators (96).  (NW = 4: two latent blocks, 192-column slices,
// 12 x 2 MFMA.)
//
// Softmax by passes: a row's weights are exp2(s - m_ref) with m_ref fixed for
// a pass (the row max of the first tile, shared by the two owners of the
// block); when some score exceeds m_ref by tau_log2<T> (in exp2 units) the
// pass is discarded at its end and the keys run again, so every weight of a
// kept pass is bounded by 2^tau_log2<T> in the MFMA's input type.  The exact
// running max is kept apart and folded in at the end, so
// the normalised output and the split partials (pm = exact max) follow the
// reference algorithm (kernel_wmma.cu:88-131, kernel_wmma_splitk.cu:80-139).
//
// Operand layouts.  In the S^T MFMA (A = K rows, B = Q^T) lane (j, g) ends
// with S[q = j][4g + i], i < 4, of its 16-key half: four of the eight k-values
// of the P^T operand, whose k order {4g..4g+3, 16+4g..16+4g+3} the V^T
// operand must follow.  V^T's A operand needs, in lane (j, g), V[4g + e][d + j]
// and V[16 + 4g + e][d + j]: eight keys of one column.  gfx950's transposing
// LDS read (ds_read_b64_tr_b16) delivers exactly that: within each 16-lane
// group, lane i receives element (i mod 4) of the 8-byte pieces read by lanes
// 4e + i/4 (e < 4), so lane 4e + q of group g reads V[4g + e][d + 4q .. +3].
// The O^T accumulator puts O[q = j][d + 4g .. d + 4g + 3] in lane (j, g): one
// 16-byte store per (latent block, column block).
//
// Tiles in LDS are row-major with a 1568-byte row stride (1536 bytes of data
// and 32 of padding).  A stride of 32 mod 512 bytes spreads the 16 rows of a
// K fragment read and the 16 rows of a transposed V read over distinct banks
// (measured at the rate of a plain sequential read), and every MFMA operand
// read is one per-lane base register plus an immediate offset: a wave64 VALU
// instruction holds its SIMD for four cycles, so per-read address arithmetic
// would cost the MFMA sections more than the reads themselves.  The tile
// (32 rows, 49 KiB) is filled by 49 global->LDS DMA chunks of 1 KiB whose
// lanes read consecutive 16-byte pieces of a row (coalesced; the lanes that
// land on padding re-read the row's last piece).  K and V tiles share one
// pipeline: phases alternate QK(t) / PV(t), phase p reads buffer p % 3 and
// requests phase p + 2 (into the buffer phase p - 1 just left); 3 buffers =
// 147 KiB.  Two barriers per tile.
#include "xattn_common.h"

namespace xattn {
namespace h16 {

constexpr int BN = 32;                 // keys per tile
constexpr int QB = 16;                 // latents per MFMA block
constexpr int KSF = kDim / 32;         // k-steps of a full-D score chain (24)
constexpr int ROWB = kDim * 2;         // bytes per K / V row in memory (1536)
constexpr int LROW = ROWB + 32;        // bytes per tile row in LDS (1568)
constexpr int BUFB = BN * LROW;        // bytes per tile buffer (49 KiB)
constexpr int NBUF = 3;
constexpr int CHUNKS = BUFB / 1024;    // 1 KiB DMA chunks per tile (49)

// Workgroup shapes.  NW = 8: two wavefronts per SIMD, 64 latents; NW = 4: one
// per SIMD, 32 latents (twice the workgroups for a given NL, for shapes whose
// 64-latent blocks cannot fill the device: no key split, no merge pass).
// CP = 2 (NW = 8 only): the workgroup computes the scores of its 64 latents
// over all of D but only half of the output columns, and its twin the other
// half: twice the workgroups again, each streaming all of K but half of V
// (74 instead of 98 KiB per tile), for 1.5x the MFMA work per output.
// Either way each wavefront owns one score unit and one output slice.
template <int NW, int CP>
struct Shape {
    static constexpr int BM = 8 * NW;          // latents per workgroup
    static constexpr int NCB = BM / QB;        // latent blocks (4 or 2)
    static constexpr int DWC = kDim / CP;      // output columns per workgroup (768 or 384)
    static constexpr int DW = DWC / NW;        // output columns per wavefront (96, 192 or 48)
    static constexpr int DB = DW / 16;         // 16-column output blocks per wavefront
    static constexpr int LROWV = DWC * 2 + 32;  // bytes per V tile row in LDS (1568 or 800)
    static constexpr int CHUNKSV = BN * LROWV / 1024;  // DMA chunks per V tile (49 or 25)
    static constexpr int CPW = CHUNKS / NW;    // DMA chunks per wavefront per K tile (6 or 12) ...
    static constexpr int CPWV = CHUNKSV / NW;  // ... and per V tile (6, 12 or 3); wavefront
    // 0 also issues the last chunk of each
    // Read-ahead depths and score chains, each timed at every form: the
    // 32-latent form runs 2-3 % faster with two chains and two fragments of
    // read-ahead than with four of each.
    static constexpr int KPF = NW == 8 ? 3 : 2;  // K fragments read ahead of their MFMAs
    static constexpr int VPF = 2;                // V column blocks read ahead of theirs
    static constexpr int NCH = 2;                // score accumulator chains
    static_assert(NCB * 2 == NW && NCB * DB * CP == 24 && (CP == 1 || NW == 8),
                  "one score unit and one output slice (all latents) per wavefront");
    static_assert(CHUNKS * 1024 == BUFB && CHUNKS == CPW * NW + 1, "DMA split");
    static_assert(CHUNKSV * 1024 == BN * LROWV && CHUNKSV == CPWV * NW + 1 && DB % CPWV == 0,
                  "V DMA split");
    static_assert(NBUF * BUFB + NCB * kWave * 16 + NW * QB * 8 + NCB * QB * 4 + 4 <= 160 * 1024,
                  "LDS budget");
};

template <typename T> constexpr float tau_log2 = 64.0f;
template <> constexpr float tau_log2<_Float16> = 15.0f;  // fp16's largest finite is 65504

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
typedef unsigned int u2v __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));

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

typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) char lds_char;

// Offsets are applied to LDS-typed pointers, which lets the compiler fold
// them into the instruction's immediate offset.
__device__ inline s4 tr_read(lds_s4* p) { return __builtin_amdgcn_ds_read_tr16_b64_v4i16(p); }

// LDS byte address of a per-lane read base, opaque to the optimiser: without
// the empty asm the compiler re-associates (buffer + lane base + fragment
// offset), hoists one register per fragment out of the tile loop and adds the
// buffer offset to each, instead of one base register plus immediates.
__device__ inline lds_char* opaque_lds(unsigned byte_addr) {
    asm volatile("" : "+v"(byte_addr));
    return (lds_char*)(uintptr_t)byte_addr;
}

// The lane index read again from the lane counter, opaque to the optimiser:
// indices derived from threadIdx.x before the tile loop and used only after
// it would otherwise stay live across the loop (and spill where the
// registers are full).
__device__ inline int fresh_lane_id() {
    int v;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(v));
    return v;
}

#ifdef XATTN_PHASE_CLOCK
// lifetime stamps and per-tile sums of the last 16-bit launch: waits at the
// two barriers, the score phase (with the softmax and the P write), the
// output phase
__device__ unsigned long long phase_clock[kClockBlocks][8][kClockFields];
#endif

template <typename T, bool PARTIAL, int NW, int CP>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void flash16_kernel(Params p) {
    typedef typename Vec8<T>::type v8;
    typedef Shape<NW, CP> Sh;
    constexpr int BM = Sh::BM, NCB = Sh::NCB, CPW = Sh::CPW, KPF = Sh::KPF;
    // The split 64-latent form reads V one column block ahead: with two, its
    // registers overflow and a Q fragment is reloaded from scratch every tile
    // (a wait for all memory operations, the DMA included).
    constexpr int VPF = PARTIAL && NW == 8 && CP == 1 ? 1 : Sh::VPF;
    constexpr int DW = Sh::DW, DB = Sh::DB, DWC = Sh::DWC, LROWV = Sh::LROWV;
    constexpr int CPWV = Sh::CPWV, CHUNKSV = Sh::CHUNKSV;
    __shared__ __attribute__((aligned(16))) char lds[NBUF * BUFB];
    __shared__ __attribute__((aligned(16))) u4v pbuf[NCB * kWave];  // P^T operand per latent block
    __shared__ float2 stats[NW * QB];  // per owner and latent: (max, sum) or the reference
    __shared__ float sref[NCB * QB];   // the reference m_ref of each latent
    __shared__ int restart_flag;

    XATTN_STAMP(clk_start);
#ifdef XATTN_PHASE_CLOCK
    const unsigned long long rt_start = __builtin_amdgcn_s_memrealtime();
#endif
    // The CP column parts of a row block are consecutive items, so they run
    // on one XCD and share its K tiles and Q block in L2.
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int ch = CP == 1 ? 0 : item % CP;  // output column part
    const int rb = (item / CP) % p.row_blocks;
    const int bs = item / CP / p.row_blocks;
    const int split = bs % p.S;
    const int b = bs / p.S;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int j = lane & 15, g = lane >> 4;
    const int q0 = rb * BM;                     // first latent of the workgroup
    const int cbo = w >> 1, kbo = w & 1;        // score unit: latent block, key half
    const int d0 = ch * DWC + w * DW;           // output role: first column of the slice

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
        // empty key range: sentinel partials (kernel_wmma_splitk.cu:65-76) or
        // zeros (the lane indices recomputed: this exit joins the main one)
        const int lane_z = fresh_lane_id(), jz = lane_z & 15, gz = lane_z >> 4;
#pragma unroll
        for (int cl = 0; cl < NCB; ++cl) {
            const int q = q0 + QB * cl + jz;
            if (q >= p.NL) continue;
            float* dst = out_row(q) + d0 + 4 * gz;
#pragma unroll
            for (int e = 0; e < DB; ++e) *(f4*)(dst + 16 * e) = (f4){0.f, 0.f, 0.f, 0.f};
        }
        const int qz = q0 + QB * cbo + jz;
        if (PARTIAL && ch == 0 && kbo == 0 && gz == 0 && qz < p.NL) {
            const size_t pi = ((size_t)b * p.NL + qz) * p.S + split;
            p.pm[pi] = -FLT_MAX;
            p.pl[pi] = 0.f;
        }
        return;
    }

    // K rows and this column part's V columns of the split's key range; keys
    // are counted from k0 below.
    const char* Kb = (const char*)(p.K + ((size_t)b * p.NI + k0) * kDim);
    const char* Vb = (const char*)(p.V + ((size_t)b * p.NI + k0) * kDim + ch * DWC);
    const int nk = k1 - k0;
    // Non-empty (the early return above); without these facts the compiler
    // guards the tile loop for zero trips and the split-K instantiation no
    // longer fits the register budget.
    __builtin_assume(nk >= 1);
    const int ntiles = (nk + BN - 1) / BN;
    __builtin_assume(ntiles >= 1);
    const int nphase = 2 * ntiles;

    // The key window of tile t starts at row n0 - lo(t): a partial last tile
    // is shifted back to end at the range's last key (its first lo rows
    // repeat keys of the previous tile and are masked), so no DMA lane ever
    // reads past the range.  A range shorter than a tile has one tile whose
    // rows past the range re-read its last row instead (clamped below).
    auto row_lo = [&](int tile) { return (tile == ntiles - 1 && nk >= BN) ? BN - (nk - tile * BN) : 0; };

    // DMA.  Chunk m of a K tile covers LDS bytes [1024 m, 1024 m + 1024): lane
    // i lands on 16-byte slot u = 64 m + i, row u / 98, piece u % 98 (pieces
    // 96 and 97 are padding, which re-read piece 95).  Wavefront w issues
    // chunks CPW w .. CPW w + CPW - 1, and wavefront 0 also chunk 48.  A V
    // tile is laid out the same way at its own row stride (LROWV: 50 pieces
    // and 25 chunks when the workgroup holds half of the columns).  The
    // per-lane source offsets are the same for every tile; the DMA is
    // untracked inline assembly (dma16_m0: the compiler sets M0, with no save
    // and restore around each chunk), ordered by the phase waits.  Phases past the
    // end re-read the last phase of the same kind into the buffer of phase
    // ph - 3, whose readers are done, so every tile issues the same way; the
    // DMA is drained after the loop.
    auto chunk_offset = [&](int m, int row_pieces, int data_pieces) {
        const int u = 64 * m + lane;
        const int r = u / row_pieces, piece = min(u - r * row_pieces, data_pieces - 1);
        return (unsigned)(min(r, nk - 1) * ROWB + 16 * piece);
    };
    unsigned doff[CPW + 1];
#pragma unroll
    for (int t = 0; t <= CPW; ++t)  // t = CPW: chunk 48
        doff[t] = chunk_offset(t < CPW ? CPW * w + t : CHUNKS - 1, LROW / 16, ROWB / 16);
    unsigned doffv[CP == 1 ? 1 : CPWV + 1];
    if constexpr (CP > 1) {
#pragma unroll
        for (int t = 0; t <= CPWV; ++t)
            doffv[t] = chunk_offset(t < CPWV ? CPWV * w + t : CHUNKSV - 1, LROWV / 16, DWC / 8);
    }
    const unsigned lds0 = lds_u32(lds);
    struct Dma {
        const char* src;
        unsigned m0;
    };
    auto dma_setup = [&](int ph) {
        const int pr = ph < nphase ? ph : ph - 2;
        const int tile = pr >> 1;
        // the first row as a scalar, so the address stays in SGPRs (a
        // per-lane copy would hold VGPRs across the tile loop)
        const int row0 = __builtin_amdgcn_readfirstlane(tile * BN - row_lo(tile));
        Dma d;
        d.src = uniform_ptr(((ph & 1) ? Vb : Kb) + (size_t)row0 * ROWB);
        d.m0 = lds0 + (unsigned)((ph % NBUF) * BUFB);
        return d;
    };
    // chunk t (< CPW) of a K phase / (< CPWV) of a V phase
    auto dma_chunk_k = [&](const Dma& d, int t) {
        dma16_m0<0>(d.src, doff[t], d.m0 + 1024 * (CPW * w + t));
    };
    auto dma_chunk_v = [&](const Dma& d, int t) {
        if constexpr (CP == 1) dma16_m0<0>(d.src, doff[t], d.m0 + 1024 * (CPW * w + t));
        else dma16_m0<0>(d.src, doffv[t], d.m0 + 1024 * (CPWV * w + t));
    };
    auto dma_last_k = [&](const Dma& d) {
        if (w == 0) dma16_m0<0>(d.src, doff[CPW], d.m0 + 1024 * (CHUNKS - 1));
    };
    auto dma_last_v = [&](const Dma& d) {
        if constexpr (CP == 1) dma_last_k(d);
        else if (w == 0) dma16_m0<0>(d.src, doffv[CPWV], d.m0 + 1024 * (CHUNKSV - 1));
    };
    auto issue = [&](int ph) {
        const Dma d = dma_setup(ph);
        if (ph & 1) {
#pragma unroll
            for (int t = 0; t < CPWV; ++t) dma_chunk_v(d, t);
            dma_last_v(d);
        } else {
#pragma unroll
            for (int t = 0; t < CPW; ++t) dma_chunk_k(d, t);
            dma_last_k(d);
        }
    };

    // Q^T operand of the score unit's block, k-step s:
    // Q[q0 + 16 cbo + j][32s + 8g .. +7] (96 registers).  K(0) is requested
    // first; no compiler-visible load is pending in the tile loop (where
    // only untracked DMA is in flight).
    // The Q block arrives by the same DMA as the tiles, row-contiguous 1 KiB
    // chunks into the buffer of phase 2 (32 latents) or of phases 1 and 2
    // (64), free until the loop starts, and every wavefront then reads its
    // operand from LDS.  With 32 latents V(0) is requested at once, behind
    // K(0) and the Q block; with 64 it waits for the staging buffer.
    constexpr bool Q_ONE_BUF = BM * LROW <= BUFB;
    constexpr unsigned QSTAGE = Q_ONE_BUF ? 2 * BUFB : BUFB;
    issue(0);
    {
        // Latents past NL repeat the last one.
        constexpr int QCH = BM * (LROW / 16) / kWave;  // 1 KiB chunks of the block
        static_assert(QCH * 1024 == BM * LROW && BM * LROW <= 2 * BUFB, "Q staging");
        const char* qsrc = uniform_ptr((const char*)(p.Q + ((size_t)b * p.NL + q0) * kDim));
        const int qrows = p.NL - q0;  // >= 1
        for (int m = w; m < QCH; m += NW) {
            const int u = kWave * m + lane;
            const int r = min(u / (LROW / 16), qrows - 1);
            const int piece = min(u % (LROW / 16), ROWB / 16 - 1);
            dma16_untracked(qsrc, (unsigned)(r * ROWB + 16 * piece), lds0 + QSTAGE + 1024u * m);
        }
    }
    if constexpr (Q_ONE_BUF) {
        issue(1);
        wait_vmcnt<CPWV>();  // K(0) and Q landed (wavefront 0: and its first V(0) chunk)
    } else {
        wait_vmcnt<0>();
    }
    lds_barrier();
    v8 qr[KSF];
    {
        const lds_char* qrd = opaque_lds(lds0 + (unsigned)(QSTAGE + LROW * (QB * cbo + j) + 16 * g));
#pragma unroll
        for (int s = 0; s < KSF; ++s) qr[s] = *(const v8*)(qrd + 64 * s);
    }
    lds_barrier();  // the staging buffer(s) take the tiles of phases 1 and 2 next

    // Per-lane LDS read bases within a tile buffer (fragments differ by
    // immediate offsets): K row 16 kbo + j at byte 16 g (k-step s adds 64 s);
    // V row 4g + e at byte 2 (w DW + 4q) of the tile (the workgroup's columns)
    // for lane 16g + 4e + q (column block t adds 32 t, key half 16 rows).
    const int kread = LROW * (16 * kbo + j) + 16 * g;
    const int vread = LROWV * (4 * g + (j >> 2)) + 2 * (w * DW + 4 * (j & 3));

    if (tid == 0) restart_flag = 0;

    const float tau_raw = tau_log2<T> / kLog2e;
    // Softmax state of the owned unit, for latent q0 + 16 cbo + j: m_true: exact running
    // max over this lane's keys of the half; m_ref: the reference of the
    // weights, the same for both halves of the latent and fixed for a pass;
    // lsum: the sum of this lane's weights.  The four lanes of a latent are
    // combined only where a whole-half value is needed (the first tile, a
    // restart, the end), so the per-tile softmax has no cross-lane step.
    float m_true = -FLT_MAX, m_ref = -FLT_MAX, lsum;
    bool ref_set = false;  // the same at every lane of the workgroup
    // Lanes with a score over the pass's bound (a lane mask, so scalar):
    // the pass is checked once, at its end.  Its weights may then have
    // overflowed, but the whole pass is discarded and run again.
    unsigned long long over;
    f4 acc[NCB][DB];  // O^T[d0 + 16t + 4g + i][q0 + 16cl + j]

    XATTN_STAMP(clk_loop);
    XATTN_CLOCK_DECL(pc_wait = 0, pc_qk = 0, pc_pv = 0);
    for (bool first = true;; first = false) {  // passes over the key range; a second is rare
        if (!first) issue(0);
        if (!first || !Q_ONE_BUF) issue(1);
#pragma unroll
        for (int cl = 0; cl < NCB; ++cl)
#pragma unroll
            for (int t = 0; t < DB; ++t) acc[cl][t] = (f4){0.f, 0.f, 0.f, 0.f};
        lsum = 0.f;
        over = 0;

        for (int tile = 0; tile < ntiles; ++tile) {
            const int n0 = tile * BN, lo = row_lo(tile);
            int ph = 2 * tile;

            // ---------------- scores of the owned unit over all of D ----------------
            // K(t) has landed for every wavefront (only this wavefront's chunks
            // of V(t) may still be in flight), and every wavefront is done with
            // V(t - 1), whose buffer takes K(t + 1).
            XATTN_STAMP(pc_a);
            wait_vmcnt<CPWV>();
            lds_barrier();
            XATTN_STAMP(pc_b);
            f4 sacc[Sh::NCH];
#pragma unroll
            for (int c = 0; c < Sh::NCH; ++c) sacc[c] = (f4){0.f, 0.f, 0.f, 0.f};
            {
                const lds_char* kr = opaque_lds(lds0 + (unsigned)((ph % NBUF) * BUFB + kread));
                const Dma dk = dma_setup(ph + 2);
                v8 kf[KSF];
#pragma unroll
                for (int s = 0; s < KPF; ++s) kf[s] = *(const v8*)(kr + 64 * s);
#pragma unroll
                for (int s = 0; s < KSF; ++s) {
                    if (s + KPF < KSF) kf[s + KPF] = *(const v8*)(kr + 64 * (s + KPF));
                    constexpr int KSTEP = KSF / CPW;  // one chunk per KSTEP k-steps
                    if (s % KSTEP == 1) dma_chunk_k(dk, s / KSTEP);
                    if (s == KSF - 1) dma_last_k(dk);
                    sacc[s % Sh::NCH] = mfma32<T>(kf[s], qr[s], sacc[s % Sh::NCH]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            f4 sv = sacc[0];
#pragma unroll
            for (int c = 1; c < Sh::NCH; ++c) sv += sacc[c];

            // ------ softmax weights of the owned unit (raw-dot units) ------
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * kbo + 4 * g + i;  // tile row; its key is n0 - lo + r
                x[i] = (r >= lo && n0 - lo + r < nk) ? sv[i] : -INFINITY;
            }
            const float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
            m_true = fmaxf(m_true, tmax);
            if (!ref_set) {
                // First tile of the kernel: the two owners of a latent block
                // agree on the reference, the row max of the tile.
                const float hmax = wave_max16_groups(tmax);
                if (g == 0) stats[w * QB + j].x = hmax;
                lds_barrier();
                m_ref = fmaxf(hmax, stats[(w ^ 1) * QB + j].x);
                lds_barrier();
                ref_set = true;
            }
            // any lane over the bound <=> the latent's row max over the bound
            over |= __ballot(tmax > m_ref + tau_raw);
            float pw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pw[i] = fast_exp2((x[i] - m_ref) * kLog2e);
                lsum += pw[i];
            }
            // this half of block cbo's P^T operand: bytes 8 kbo .. 8 kbo + 7 of each lane
            *(u2v*)((char*)pbuf + (size_t)(cbo * kWave + lane) * 16 + 8 * kbo) =
                (u2v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3])};

            // ---------------- O^T += V^T . P^T over this wavefront's slice ----------------
            // V(t) has landed (only this wavefront's chunks of K(t + 1) may
            // still be in flight), P is complete, and every wavefront is done
            // with K(t), whose buffer takes V(t + 1).
            ph += 1;
            XATTN_STAMP(pc_c);
            wait_vmcnt<CPW>();
            lds_barrier();
            XATTN_STAMP(pc_d);
            v8 pt[NCB];
#pragma unroll
            for (int cl = 0; cl < NCB; ++cl)
                pt[cl] = __builtin_bit_cast(v8, pbuf[cl * kWave + lane]);
            {
                lds_s4* vr = (lds_s4*)opaque_lds(lds0 + (unsigned)((ph % NBUF) * BUFB + vread));  // 4 per 32 B
                const Dma dv = dma_setup(ph + 2);
                s4 va[DB], vc[DB];
#pragma unroll
                for (int t = 0; t < VPF; ++t) {
                    va[t] = tr_read(vr + 4 * t);
                    vc[t] = tr_read(vr + 2 * LROWV + 4 * t);
                }
#pragma unroll
                for (int t = 0; t < DB; ++t) {
                    if (t + VPF < DB) {
                        va[t + VPF] = tr_read(vr + 4 * (t + VPF));
                        vc[t + VPF] = tr_read(vr + 2 * LROWV + 4 * (t + VPF));
                    }
                    constexpr int VSTEP = DB / CPWV;  // one chunk per VSTEP column blocks
                    if (t % VSTEP == 0) dma_chunk_v(dv, t / VSTEP);
                    if (t == DB - 1) dma_last_v(dv);
                    const v8 vt = __builtin_bit_cast(
                        v8, __builtin_shufflevector(va[t], vc[t], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                    for (int cl = 0; cl < NCB; ++cl) acc[cl][t] = mfma32<T>(vt, pt[cl], acc[cl][t]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            XATTN_STAMP(pc_e);
            XATTN_CLOCK_ADD(pc_wait, pc_a, pc_b);
            XATTN_CLOCK_ADD(pc_wait, pc_c, pc_d);
            XATTN_CLOCK_ADD(pc_qk, pc_b, pc_c);
            XATTN_CLOCK_ADD(pc_pv, pc_d, pc_e);
        }
        // Every wavefront raises the flag (if at all) before this barrier, so
        // all of them read the same value.
        if (over != 0 && lane == 0) restart_flag = 1;
        lds_barrier();
        if (!__builtin_amdgcn_readfirstlane(restart_flag)) break;
        // Some latent's scores outgrew its reference: drain the DMA (the
        // re-reads past the last phase may be in flight), clear the flag, and
        // run the keys again with the reference raised to the max seen so far
        // over both halves.
        wait_vmcnt<0>();
        lds_barrier();
        if (tid == 0) restart_flag = 0;
        const float hmax = wave_max16_groups(m_true);
        if (g == 0) stats[w * QB + j].x = hmax;
        lds_barrier();
        m_ref = fmaxf(hmax, stats[(w ^ 1) * QB + j].x);
        lds_barrier();
    }
    XATTN_STAMP(clk_loop_end);
    wait_vmcnt<0>();  // the re-reads issued past the last phase
    // lane (je, ge) as before the loop, recomputed rather than kept live
    const int lane_e = fresh_lane_id(), je = lane_e & 15, ge = lane_e >> 4;

    // Combine the two key halves of each latent (max and sum, both against
    // the shared m_ref), then normalise (or, for a partial, rescale to the
    // exact max).  A wavefront's m_ref is that of the block of its score
    // unit; the output blocks it accumulates are weighted by their own
    // blocks' m_ref.
    m_true = wave_max16_groups(m_true);
    lsum = wave_sum16_groups(lsum);
    if (ge == 0) stats[w * QB + je] = make_float2(m_true, lsum);
    if (ge == 0 && kbo == 0) sref[cbo * QB + je] = m_ref;
    lds_barrier();
    float rsc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const float2 s0 = stats[(2 * cb) * QB + je], s1 = stats[(2 * cb + 1) * QB + je];
        const float mt = fmaxf(s0.x, s1.x);
        const float factor = fast_exp2((sref[cb * QB + je] - mt) * kLog2e);
        const float l = s0.y + s1.y;
        rsc[cb] = PARTIAL ? factor : factor / (l * factor + 1e-6f);
        if (PARTIAL && ch == 0 && w == 0 && ge == 0) {
            const int q = q0 + QB * cb + je;
            if (q < p.NL) {
                const size_t pi = ((size_t)b * p.NL + q) * p.S + split;
                p.pm[pi] = mt;  // scores are q.k with Q pre-scaled
                p.pl[pi] = l * factor;
            }
        }
    }
    // The output leaves through the tile ring, free since the barrier above
    // (the DMA was drained after the loop): per latent block, each
    // wavefront writes its 16-row slice row-major into its own area, then
    // reads it back row-contiguous, so every store instruction covers whole
    // 128-byte lines of a row (the accumulator layout gives 64-byte halves).
    constexpr int SROW = DW * 4 + 16;  // padded staging row (bytes)
    static_assert(NW * QB * SROW <= NBUF * BUFB, "staging area");
    char* const stage = lds + w * (QB * SROW);
#pragma unroll
    for (int cl = 0; cl < NCB; ++cl) {
#pragma unroll
        for (int t = 0; t < DB; ++t)
            *(f4*)(stage + je * SROW + (16 * t + 4 * ge) * 4) = acc[cl][t] * rsc[cl];
        const int qb = q0 + QB * cl;
#pragma unroll
        for (int k = 0; k < QB * DW / 4 / kWave; ++k) {
            const int pc = k * kWave + lane_e;  // 16-byte piece of the slice
            const int r = pc / (DW / 4), c = pc % (DW / 4);
            const f4 o = *(const f4*)(stage + r * SROW + 16 * c);
            if (qb + r >= p.NL) continue;
            f4* const at = (f4*)(out_row(qb + r) + d0 + 4 * c);
            // streamed past the caches: the output is not read again, and
            // the split partials only by the merge, another launch
            __builtin_nontemporal_store(o, at);
        }
    }
#ifdef XATTN_PHASE_CLOCK
    XATTN_STAMP(clk_end);
    const unsigned long long rt_end = __builtin_amdgcn_s_memrealtime();
    if (lane == 0 && blockIdx.x < (unsigned)kClockBlocks) {
        unsigned long long* c = phase_clock[blockIdx.x][w];
        c[0] = clk_start, c[1] = clk_loop, c[2] = clk_loop_end, c[3] = clk_end;
        c[4] = rt_start, c[5] = rt_end, c[6] = pc_wait, c[7] = pc_qk, c[8] = pc_pv;
    }
#endif
}

}  // namespace h16

int h16_row_blocks(int NL, int nw) { return (NL + 8 * nw - 1) / (8 * nw); }

#ifdef XATTN_PHASE_CLOCK
// The 16-bit kernel's stamps: [kClockBlocks][8 wavefronts][kClockFields]
// unsigned 64-bit values.  Clear before a launch, read after.  0 on success.
extern "C" int xattn_phase_clock_read_f16(void* dst, size_t bytes) {
    const size_t n = bytes < sizeof(h16::phase_clock) ? bytes : sizeof(h16::phase_clock);
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(h16::phase_clock), n) == hipSuccess ? 0 : 1;
}
extern "C" int xattn_phase_clock_clear_f16(void) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(h16::phase_clock)) != hipSuccess) return 1;
    if (hipMemset(ptr, 0, sizeof(h16::phase_clock)) != hipSuccess) return 1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : 1;
}
#endif

template <typename T, bool PARTIAL>
static void launch16(int nw, int cp, dim3 grid, hipStream_t stream, const h16::Params& p) {
    if (nw == 4)
        hipLaunchKernelGGL((h16::flash16_kernel<T, PARTIAL, 4, 1>), grid, dim3(4 * kWave), 0, stream, p);
    else if (cp == 2)
        hipLaunchKernelGGL((h16::flash16_kernel<T, PARTIAL, 8, 2>), grid, dim3(8 * kWave), 0, stream, p);
    else
        hipLaunchKernelGGL((h16::flash16_kernel<T, PARTIAL, 8, 1>), grid, dim3(8 * kWave), 0, stream, p);
}

bool launch_flash16(bool bf16, int nw, int cp, const void* Q, const void* K, const void* V,
                    float* out, float* po, float* pm, float* pl, int B, int NL, int NI, int S,
                    int chunk, hipStream_t stream) {
    if ((nw != 4 && nw != 8) || (cp != 1 && cp != 2) || (nw == 4 && cp != 1)) {
        set_error(XATTN_ERR_INVALID_VALUE, "flash16: %d wavefronts per workgroup, %d column parts",
                  nw, cp);
        return false;
    }
    h16::Params p;
    p.Q = (const u16*)Q; p.K = (const u16*)K; p.V = (const u16*)V;
    p.out = out; p.po = po; p.pm = pm; p.pl = pl;
    p.B = B; p.NL = NL; p.NI = NI; p.S = S; p.chunk = chunk;
    p.row_blocks = h16_row_blocks(NL, nw);
    const long long nblk = (long long)B * p.row_blocks * S * cp;
    if (nblk <= 0) return true;
    if (nblk > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "grid of %lld workgroups too large", nblk);
        return false;
    }
    const dim3 grid((unsigned)nblk);
    if (bf16) {
        if (po) launch16<__bf16, true>(nw, cp, grid, stream, p);
        else launch16<__bf16, false>(nw, cp, grid, stream, p);
    } else {
        if (po) launch16<_Float16, true>(nw, cp, grid, stream, p);
        else launch16<_Float16, false>(nw, cp, grid, stream, p);
    }
    return check_launch(bf16 ? "flash_bf16" : "flash_f16");
}

}  // namespace xattn
