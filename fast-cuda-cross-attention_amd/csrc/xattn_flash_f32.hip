// fp32 fused cross-attention on fp32 MFMA (v_mfma_f32_16x16x4_f32), gfx950.
//
// Work item = (batch b, key split s, block of 64 latents).  A workgroup is 4
// wavefronts; wavefront w owns 16 latents q0..q0+15 for the whole key range,
// so there is no cross-wave reduction.  Per 16-key tile:
//
//   S^T[16 keys x 16 q] = K_tile[16 x 768] . Q^T          192 MFMA (k = 4)
//   online softmax on S^T (running max / sum per latent)
//   O[16 q x 768]     += P[16 q x 16 keys] . V_tile[16 x 768]   192 MFMA
//
// Computing S^T (keys on the MFMA M axis) leaves lane (j, g) holding
// S[q = j][key = 4g + i] in accumulator register i -- exactly the A-operand
// layout P[q = j][k = g] of the P.V MFMA for k-slab i, so P never moves.
//
// Registers per lane: Q^T operand 192 VGPRs (Q[q0+j][16u + 4g + c], u < 48,
// c < 4), O accumulator 192 AGPRs (O[q0 + 4g + i][64T + 4j + c], T < 12),
// written only by MFMA, so neither operand is ever copied between register
// files inside the loop.  One wavefront per SIMD; the MFMA pipe is kept busy
// by a single wave.
//
// Column-split forms (DS = 2 or 4) for batch sizes and latent counts whose
// 64-latent workgroups would leave compute units idle: DS wavefronts share
// one 16-latent block, each holding 768 / DS columns of Q^T and O (so a
// workgroup covers 32 or 16 latents); after QK each writes its share of S^T
// to LDS and, after the next barrier, every wavefront of the block adds the
// DS shares in the same order before its softmax.  The launch planner picks
// the form and the key splits (xattn_abi.hip, f32_plan).
//
// K and V tiles are shared by the 4 wavefronts through LDS and arrive by
// global->LDS DMA (16 B per lane, 1 KiB per wave instruction).  Phases
// alternate QK(t), PV(t); phase p reads buffer p % 3, and the data of phase
// p + 2 is requested during phase p, spread over it (one chunk per 16 MFMAs
// in the 64-latent form: a burst of 48 chunks per CU at the start of a phase
// stalls every wavefront on the full DMA queue), so every tile has about two
// phases (~12k cycles in the 64-latent form) to arrive.
// Phases past the end re-read the last phase of the same kind into the
// buffer of phase p - 1, whose readers are done, so the loop issues the same
// way on every tile; the DMA is drained after the loop.  One barrier per
// phase.
//
// Softmax in raw dot-product units by passes: a row's weights are
// exp2((s - m_ref) c2) with m_ref fixed for the whole pass (the row max of
// the first tile), so the accumulator is never rescaled.  If a score
// exceeds m_ref by 2^64 in exp2 space the workgroup discards the pass at its
// end (a flag in LDS, read by every wavefront after the same barrier) and
// runs the keys again with m_ref = the max seen so far; unit-variance scores
// never need a second pass.  The exact max is tracked separately and folded in at
// the end, so the normalised output and the split partials (pm = exact max
// score) match the reference algorithm (kernel_vectorized.cu:58-181,
// kernel_splitk.cu:94-180).

#include "xattn_common.h"
#include "xattn_launch.h"

namespace xattn {
namespace f32 {

constexpr int BN = 16;                 // keys per tile
constexpr int QW = 16;                 // latents per wavefront
constexpr int NW = 4;                  // wavefronts per workgroup
constexpr int BM = QW * NW;            // latents per workgroup
constexpr int ROW = kDim + 4;          // padded LDS row (floats): conflict-free b128 reads
constexpr int BUF = BN * ROW;          // floats per LDS tile buffer
constexpr int NBUF = 3;
constexpr int CHUNKS = BN * kDim / (kWave * 4);  // 1 KiB DMA chunks per tile (48)
constexpr int CPW = CHUNKS / NW;                 // per wavefront (12)
constexpr int ROW_CHUNKS = kDim / (kWave * 4);   // 3 chunks per key row
// a pass restarts when a score exceeds its reference by 2^kTauLog2 (exp2 units)
constexpr float kTauLog2 = 64.0f;

static_assert(CHUNKS % NW == 0, "chunks per wave");
static_assert((NBUF * BUF + 4) * 4 <= 160 * 1024, "LDS budget");

struct Params {
    const float* Q;
    const float* K;
    const float* V;
    float* out;
    float* po;
    float* pm;
    float* pl;
    int B, NL, NI, S, chunk, row_blocks;
};

typedef __attribute__((address_space(3))) const float lds_cfloat;
typedef __attribute__((address_space(3))) const f4 lds_cf4;

// An LDS read base opaque to the optimiser (its float index within the tile
// array): without it the compiler may re-associate (ring buffer + lane base
// + fragment offset), hoist one register per fragment out of the tile loop
// and add the buffer offset to each of them every phase, VALU work that an
// fp32 MFMA stream cannot hide, instead of one base register plus immediates.
__device__ inline lds_cfloat* opaque_lds_f(const float* lds, int index) {
    unsigned a = lds_u32(lds) + 4u * (unsigned)index;
    asm volatile("" : "+v"(a));
    return (lds_cfloat*)(uintptr_t)a;
}

// Maxima of scores as single instructions: fmaxf would first canonicalise
// each input (v_max_f32 x, x, x) against signalling NaNs, which MFMA results
// never are; a quiet NaN input is dropped by both alike.
__device__ inline float vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ inline float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <bool B>
struct Peel {
    static constexpr bool value = B;
};

__device__ inline f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

#ifdef XATTN_PHASE_CLOCK
// lifetime stamps and per-tile sums of the last fp32 launch: waits at the
// two barriers, the QK phase (with the softmax when DS = 1), the PV phase
__device__ unsigned long long phase_clock[kClockBlocks][8][kClockFields];
#endif

template <bool PARTIAL, int DS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void flash_f32_kernel(Params p) {
    static_assert(DS == 1 || DS == 2 || DS == 4, "column parts per latent block");
    constexpr int BMW = BM / DS;     // latents per workgroup
    constexpr int NU = 48 / DS;      // 16-column K-operand groups per wavefront
    constexpr int NT = 12 / DS;      // 64-column output tiles per wavefront
    constexpr int DSTEP = NU / CPW;  // MFMA groups per DMA chunk
    // Score accumulator chains: two in the 64-latent form; one in the
    // column-split forms, whose scores then stay in VGPRs for the exchange
    // (no AGPR reads and adds; 0-1.5 % faster there, 0.2 % slower in the
    // 64-latent form).
    constexpr int SCH = DS == 1 ? 2 : 1;
    constexpr int XCH = DS > 1 ? NW * kWave * 4 : 0;  // partial-score exchange (floats)
    static_assert(NU % CPW == 0, "DMA spread");
    static_assert((NBUF * BUF + XCH + 4) * 4 <= 160 * 1024, "LDS budget");

    // tile buffers, the score exchange, then the restart flag (one LDS object)
    __shared__ __attribute__((aligned(16))) float lds[NBUF * BUF + XCH + 4];

    XATTN_STAMP(clk_start);
#ifdef XATTN_PHASE_CLOCK
    const unsigned long long rt_start = __builtin_amdgcn_s_memrealtime();
#endif
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int rb = item % p.row_blocks;
    const int bs = item / p.row_blocks;
    const int split = bs % p.S;
    const int b = bs / p.S;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int j = lane & 15, g = lane >> 4;
    // Wavefront w: latent block w / DS, output columns [768 dp / DS, ...).
    const int dp = w % DS;
    const int q0 = rb * BMW + (w / DS) * QW;

    int k0 = 0, k1 = p.NI;
    if (PARTIAL) {
        k0 = split * p.chunk;
        k1 = min(k0 + p.chunk, p.NI);
    }

    if (k0 >= k1) {
        // Empty key range: sentinel partials (kernel_splitk.cu:62-71) or, for
        // a full-range launch with N_input == 0, a zero output.
        const f4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = q0 + 4 * g + i;
            if (q >= p.NL) continue;
            float* dst = PARTIAL
                ? p.po + (((size_t)b * p.NL + q) * p.S + split) * kDim
                : p.out + ((size_t)b * p.NL + q) * kDim;
#pragma unroll
            for (int T = 0; T < NT; ++T) *(f4*)(dst + 64 * (NT * dp + T) + 4 * j) = z;
        }
        if (PARTIAL && dp == 0 && g == 0 && q0 + j < p.NL) {
            const size_t pi = ((size_t)b * p.NL + q0 + j) * p.S + split;
            p.pm[pi] = -FLT_MAX;
            p.pl[pi] = 0.f;
        }
        return;
    }

    const float* Kb = p.K + (size_t)b * p.NI * kDim;
    const float* Vb = p.V + (size_t)b * p.NI * kDim;
    const int ntiles = (k1 - k0 + BN - 1) / BN;
    // Non-empty (the early return above); without this the compiler guards
    // the tile loop for zero trips and the split-K instantiation spills.
    __builtin_assume(k1 - k0 >= 1);
    __builtin_assume(ntiles >= 1);

    // Phase ph (even: K of tile ph/2, odd: V of tile ph/2) -> buffer ph % 3.
    // Wavefront w's chunks cover tile rows r0 .. r0 + 3, three 1 KiB chunks
    // per row; chunk t of the phase is rows r0 + t / 3, floats 256 (t % 3)...
    // Tile t's rows are the keys from win(t) on: k0 + 16 t, except that a
    // partial last tile is shifted back to end at k1 (its first rows repeat
    // keys of the tile before; the softmax masks them), and a range shorter
    // than a tile keeps its window at k0 with the rows past the range
    // re-reading its last row (masked too).  Every row read is a key of
    // [k0, k1).  A chunk's source is one scalar base per phase (the window's
    // first byte), the row's offset in a per-lane register set up once, and
    // the column as the instruction's immediate; M0 (set by the compiler) is
    // the buffer's base plus the row's, and the tile loop rotates the three
    // buffer bases instead of reducing phase numbers modulo 3: every scalar
    // instruction costs issue time here (an fp32 MFMA holds the SIMD while
    // it runs).  The DMA is untracked; the phase waits below order it.
    const unsigned lds0 = lds_u32(lds);
    const int r0 = w * (CPW / ROW_CHUNKS);
    const unsigned lane16 = 16u * lane;
    const float* const Ks = uniform_ptr(Kb);
    const float* const Vs = uniform_ptr(Vb);
    const int nk = k1 - k0;
    auto win = [&](int n0) {  // n0 = k0 + 16 t
        return nk >= BN ? min(n0, k1 - BN) : n0;
    };
    // lane16 plus the byte offset of each of this wavefront's rows in a window
    unsigned voff[CPW / ROW_CHUNKS];
#pragma unroll
    for (int r = 0; r < CPW / ROW_CHUNKS; ++r)
        voff[r] = lane16 + (unsigned)(min(r0 + r, min(nk, BN) - 1) * (kDim * 4));
    // Chunk t of a phase whose window starts at src (wave-uniform) and whose
    // LDS buffer starts at byte lds_buf; chunk c of a row adds c KiB to the
    // row's source and LDS addresses (the instruction's immediate).
    auto dma_chunk = [&](const char* src, unsigned lds_buf, int t) {
        const int r = t / ROW_CHUNKS, c = t % ROW_CHUNKS;
        const unsigned row_lds = lds_buf + 4u * (unsigned)((r0 + r) * ROW);
        if (c == 0) dma16_m0<0>(src, voff[r], row_lds);
        else if (c == 1) dma16_m0<kWave * 16>(src, voff[r], row_lds);
        else dma16_m0<2 * kWave * 16>(src, voff[r], row_lds);
    };
    // the first byte of tile t's window in K or V
    auto tile_src = [&](const float* base, int t) {
        return (const char*)base + (size_t)win(k0 + t * BN) * (kDim * 4);
    };
    auto issue = [&](int ph) {  // phase 0 or 1 (the first tile's K or V) into buffer ph
        const char* src = tile_src((ph & 1) ? Vs : Ks, 0);
#pragma unroll
        for (int t = 0; t < CPW; ++t) dma_chunk(src, lds0 + 4u * (unsigned)(ph * BUF), t);
    };

    // Q^T operand (this wavefront's columns), kept in registers for the whole
    // key loop, requested behind the first tile's K and V.  The first tile's
    // QK phase (peeled out of the tile loop) waits for each fragment as it
    // uses it, so its MFMAs run while the rest of Q arrives, and no
    // compiler-visible load is pending in the loop itself.
    issue(0);
    issue(1);
    f4 qr[NU];
    {
        const int qc = min(q0 + j, p.NL - 1);
        const float* qrow = p.Q + ((size_t)b * p.NL + qc) * kDim + 4 * g + 16 * NU * dp;
#pragma unroll
        for (int u = 0; u < NU; ++u) qr[u] = *(const f4*)(qrow + 16 * u);
    }

    // The exchange and the flag live in the tile array: a second LDS object
    // would give the LDS reads alias-scope metadata and make the compiler
    // drain the DMA before each of them.
    float* const xch = lds + NBUF * BUF;
    int* restart_flag = (int*)(lds + NBUF * BUF + XCH);
    if (tid == 0) *restart_flag = 0;
    const float c2 = kLog2e / sqrtf((float)kDim);
    const float tau_raw = kTauLog2 / c2;
    // m_true and lsum cover this lane's keys only (4g + i of every tile):
    // the four lanes of a latent are combined once, at the end of the pass,
    // so the per-tile softmax has no cross-lane step except on the tile
    // that sets the pass's reference.
    float m_true = -FLT_MAX, m_ref = -FLT_MAX, bound = -FLT_MAX, lsum;
    bool ref_set = false;  // the same at every lane of the workgroup
    // Lanes with a score over the pass's bound (a lane mask, so scalar):
    // the pass is checked once, at its end.  Its weights may then have
    // overflowed, but the whole pass is discarded and run again.
    unsigned long long over;
    f4 acc[NT][4];
    float pw[4];

    // Online softmax of one tile's scores s (lane (j, g): latent j, keys
    // n0 + 4g + i) into the P operand pw; notes the lanes whose scores
    // outgrow the pass's reference.
    auto softmax = [&](f4 s, int n0) {
        float x[4];
        if (n0 + BN <= k1) {  // a full tile (uniform branch): no key to mask
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = s[i];
        } else {
            // the window's keys are ws + 4g + i; those before n0 were scored
            // by the tile before, those from k1 on are past the range
            const int ws = win(n0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = ws + 4 * g + i;
                x[i] = (key >= n0 && key < k1) ? s[i] : -INFINITY;
            }
        }
        const float tmax = vmax(vmax3(x[0], x[1], x[2]), x[3]);
        if (!ref_set) {
            // first tile of the kernel: the reference is the latent's row max
            m_ref = wave_max16_groups(tmax);
            bound = m_ref + tau_raw;
            ref_set = true;
        }
        m_true = vmax(m_true, tmax);
        // any lane over the bound <=> the latent's row max over the bound
        over |= __ballot(tmax > bound);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pw[i] = fast_exp2((x[i] - m_ref) * c2);
            lsum += pw[i];
        }
    };

    // Per-lane LDS read bases of the tile loop.  The column-split forms take
    // them opaque (their loops otherwise re-associate the fragment offsets
    // as above); the 64-latent form's loop is compiled well without.
    auto lds_base = [&](int index) -> lds_cfloat* {
        if constexpr (DS == 1) return (lds_cfloat*)(lds + index);
        else return opaque_lds_f(lds, index);
    };

    XATTN_STAMP(clk_loop);
    XATTN_CLOCK_DECL(pc_wait = 0, pc_qk = 0, pc_pv = 0);
    // K and V operand fragments share one ring of three f4, read two 4-MFMA
    // groups ahead, so the first two fragments of a phase can be read before
    // it starts.  A QK phase's barrier sits two groups before the end of the
    // PV phase before it, after the wavefront's last read of that phase's V
    // buffer: past it, every read of the V buffer is done (the next phase's
    // DMA refills it) and the next K tile has landed (its DMA was issued a
    // phase earlier; the chunks issued so far in this phase may still be in
    // flight), and the first K fragments are read under the last two groups'
    // MFMAs.  A PV phase's barrier stays after the softmax (the column-split
    // forms exchange their scores across it; moved into the 64-latent form's
    // QK phase it measured 0.2-0.5 % slower) and the first V fragments are
    // read right after it.
    f4 fr[3];
    static_assert(NU % 3 == 0, "the fragment ring runs on across phases");
    constexpr int ISSUED = (NU - 2) / DSTEP + 1 < CPW ? (NU - 2) / DSTEP + 1 : CPW;
    auto tail_barrier = [&]() {
        XATTN_STAMP(tw0);
        wait_vmcnt<ISSUED>();
        lds_barrier();
        XATTN_STAMP(tw1);
        XATTN_CLOCK_ADD(pc_wait, tw0, tw1);
        XATTN_CLOCK_ADD(pc_pv, tw1, tw0);  // a wait, not PV phase time
    };
    // LDS read bases of the K fragments of phase ph (lane (j, g): key j,
    // columns 16 u + 4 g of this wavefront's part) and the V fragments of
    // phase ph (group n = NT r + T: V[4 g + r][64 (NT dp + T) + 4 j ..]).
    auto k_base = [&](int buf) {  // buf: the buffer's first float
        return lds_base(buf + j * ROW + 4 * g + 16 * NU * dp);
    };
    auto v_base = [&](int buf) {
        return lds_base(buf + 4 * j + 4 * g * ROW + 64 * NT * dp);
    };
    auto v_frag = [&](lds_cfloat* vb, int n) {
        return *(lds_cf4*)(vb + (n / NT) * ROW + 64 * (n % NT));
    };

    // One pass over the keys (a second is rare); FIRST: the first pass,
    // whose first tile may still be waiting for Q.  Returns whether some
    // latent's scores outgrew the pass's reference.
    auto pass = [&](auto first_pass) -> bool {
        constexpr bool FIRST = decltype(first_pass)::value;
        if constexpr (!FIRST) {
            issue(0);
            issue(1);
        }
#pragma unroll
        for (int T = 0; T < NT; ++T)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[T][c] = (f4){0.f, 0.f, 0.f, 0.f};
        lsum = 0.f;
        over = 0;
        if constexpr (FIRST) wait_vmcnt<NU>();  // phases 0 and 1 landed; Q may be in flight
        else wait_vmcnt<CPW>();                 // phase 0 landed; phase 1 may be in flight
        lds_barrier();
        {
            lds_cfloat* kb = k_base(0);
            fr[0] = *(lds_cf4*)(kb);
            fr[1] = *(lds_cf4*)(kb + 16);
        }
        // The buffers of phases 2 tile, 2 tile + 1 and 2 tile + 2 (first
        // floats), rotated per tile: phase ph reads buffer ph % 3 and refills
        // buffer (ph + 2) % 3 with the data of phase ph + 2.
        int bk = 0, bv = BUF, bn = 2 * BUF;
        // One tile: its QK phase, softmax and PV phase.  PEEL: the first
        // pass's first tile, whose QK phase may still be waiting for Q (the
        // compiler waits for each fragment before its MFMAs); it requests
        // the next tile's K after its MFMAs, so those waits never hold it up.
        auto tile_body = [&](int tile, auto peel) {
            constexpr bool PEEL = decltype(peel)::value;
            const int n0 = k0 + tile * BN;
            // the next tile's K and V windows (the last tile re-reads its
            // own: phases past the end, loaded but never read)
            const int tnext = min(tile + 1, ntiles - 1);
            const char* const ksrc = tile_src(Ks, tnext);
            const char* const vsrc = tile_src(Vs, tnext);

            // ---------------- QK phase ----------------
            XATTN_STAMP(pc_b);
            lds_cfloat* const vb = v_base(bv);
            f4 s;
            {
                // the sched_barrier keeps the scheduler from hoisting the
                // fragment reads out of their groups
                lds_cfloat* kb = k_base(bk);
                f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    if (u + 2 < NU) fr[(u + 2) % 3] = *(lds_cf4*)(kb + 16 * (u + 2));
                    if (!PEEL && u % DSTEP == 0) dma_chunk(ksrc, lds0 + 4u * (unsigned)bn, u / DSTEP);
                    const f4 k4 = fr[u % 3];
                    s0 = mfma4(k4[0], qr[u][0], s0);
                    if constexpr (SCH == 2) s1 = mfma4(k4[1], qr[u][1], s1);
                    else s0 = mfma4(k4[1], qr[u][1], s0);
                    s0 = mfma4(k4[2], qr[u][2], s0);
                    if constexpr (SCH == 2) s1 = mfma4(k4[3], qr[u][3], s1);
                    else s0 = mfma4(k4[3], qr[u][3], s0);
                    __builtin_amdgcn_sched_barrier(0);
                }
                s = SCH == 2 ? s0 + s1 : s0;
                if constexpr (PEEL) {
#pragma unroll
                    for (int t = 0; t < CPW; ++t) dma_chunk(ksrc, lds0 + 4u * (unsigned)bn, t);
                }
            }

            if constexpr (DS == 1) {
                softmax(s, n0);
            } else {
                // this wavefront's share of the block's scores, summed after
                // the barrier (the previous tile's shares were all read
                // before the last phase's barrier)
                *(f4*)(xch + (w * kWave + lane) * 4) = s;
            }
            XATTN_STAMP(tw0);
            wait_vmcnt<CPW>();  // the V tile landed; the next K tile may be in flight
            lds_barrier();
            XATTN_STAMP(tw1);
            XATTN_CLOCK_ADD(pc_wait, tw0, tw1);
            fr[0] = v_frag(vb, 0);
            fr[1] = v_frag(vb, 1);
            if constexpr (DS > 1) {
                // Every wavefront of the block sums the shares in the same
                // order, so all of them hold bit-identical scores and weights
                // (the first V fragments are in flight meanwhile).
                const float* xs = xch + ((w - dp) * kWave + lane) * 4;
                f4 st = *(const f4*)(xs);
#pragma unroll
                for (int d = 1; d < DS; ++d) st += *(const f4*)(xs + d * kWave * 4);
                softmax(st, n0);
            }

            // ---------------- PV phase ----------------
            {
                lds_cfloat* const kn = k_base(bn);  // the next tile's K (read in the tail)
#pragma unroll
                for (int n = 0; n < 4 * NT; ++n) {
                    if (n + 2 < 4 * NT) fr[(n + 2) % 3] = v_frag(vb, n + 2);
                    if (n % DSTEP == 0) dma_chunk(vsrc, lds0 + 4u * (unsigned)bk, n / DSTEP);
                    if (n == 4 * NT - 2) {
                        tail_barrier();
                        fr[0] = *(lds_cf4*)(kn);
                    }
                    if (n == 4 * NT - 1) fr[1] = *(lds_cf4*)(kn + 16);
                    const int r = n / NT, T = n % NT;
                    const f4 v4 = fr[n % 3];
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[T][c] = mfma4(pw[r], v4[c], acc[T][c]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            XATTN_STAMP(pc_e);
            XATTN_CLOCK_ADD(pc_qk, pc_b, tw0);
            XATTN_CLOCK_ADD(pc_pv, tw1, pc_e);
            const int b0 = bk;
            bk = bn;
            bn = bv;
            bv = b0;
        };
        tile_body(0, Peel<FIRST>{});
        for (int tile = 1; tile < ntiles; ++tile) tile_body(tile, Peel<false>{});

        // Every wavefront raises the flag (if at all) before this barrier, so
        // all of them read the same value.  (The last tail read the K buffer
        // of the phase past the end: data re-read from the range, unused.)
        if (over != 0 && lane == 0) *restart_flag = 1;
        lds_barrier();
        return __builtin_amdgcn_readfirstlane(*restart_flag) != 0;
    };
    // The first pass runs outside any loop, so the compiler's waits for the
    // Q fragments stay in its first tile (inside a loop it would wait for
    // most of Q before entering it).
    if (pass(Peel<true>{})) {
        do {
            // Some latent's scores outgrew its reference: drain the DMA (the
            // re-reads past the last phase may be in flight), clear the
            // flag, and run the keys again with the reference raised to the
            // max seen so far.
            wait_vmcnt<0>();
            lds_barrier();
            if (tid == 0) *restart_flag = 0;
            m_ref = wave_max16_groups(m_true);
            bound = m_ref + tau_raw;
            lds_barrier();
        } while (pass(Peel<false>{}));
    }

    XATTN_STAMP(clk_loop_end);
    wait_vmcnt<0>();  // the re-reads issued past the last phase

    // The latent's exact max and sum of weights over its four lanes.
    m_true = wave_max16_groups(m_true);
    lsum = wave_sum16_groups(lsum);
    // Fold the exact max back in: factor = exp(m_ref - m_true) <= 1.
    const float factor = fast_exp2((m_ref - m_true) * c2);
    float rowscale;
    if (PARTIAL) rowscale = factor;
    else rowscale = factor / (lsum * factor + 1e-6f);
    float rsc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rsc[i] = __shfl(rowscale, 4 * g + i);

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = q0 + 4 * g + i;
        if (q >= p.NL) continue;
        float* dst = PARTIAL
            ? p.po + (((size_t)b * p.NL + q) * p.S + split) * kDim
            : p.out + ((size_t)b * p.NL + q) * kDim;
#pragma unroll
        for (int T = 0; T < NT; ++T) {
            const f4 o = (f4){acc[T][0][i], acc[T][1][i], acc[T][2][i], acc[T][3][i]} * rsc[i];
            f4* const at = (f4*)(dst + 64 * (NT * dp + T) + 4 * j);
            // Streamed past the caches: the output is not read again by this
            // launch (measured 1 % faster at 64 latents x 784 keys), and the
            // split partials are read by the merge, another launch whose
            // workgroups mostly sit on other XCDs, so caching them here only
            // leaves dirty lines for the end-of-kernel write-back (0.5-2.8 %
            // faster on split plans, config 1 2.8 %).
            __builtin_nontemporal_store(o, at);
        }
    }
    if (PARTIAL && dp == 0 && g == 0 && q0 + j < p.NL) {
        const size_t pi = ((size_t)b * p.NL + q0 + j) * p.S + split;
        p.pm[pi] = m_true / sqrtf((float)kDim);
        p.pl[pi] = lsum * factor;
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

// Log-sum-exp merge of split partials (kernel_splitk.cu:186-236).  Each
// (batch, latent) row is merged by C workgroups, each owning 768 / C of its
// columns, in P groups of 192 / C threads: every wave reduces M = max pm and
// L = sum exp(pm - M) pl over the splits (lane-strided), and thread c of
// group p accumulates float4 column c over splits p, p + P, ... with 8
// partial rows in flight at a time; the P group sums are added in group
// order through LDS.  Neither C nor the thread count changes any column's
// arithmetic or its order, so the output is bit-identical for every C.  The
// first 8 partial rows and each lane's first pm / pl are requested before
// the reductions (the partials do not depend on M), so a row with few
// splits waits for one round of loads, not three.  P = 1 when there are rows
// enough to fill the device twice (HBM-bound: S * 3 KiB of po per row); P = 4
// for fewer rows, where one group's loads in flight would set the time, and
// then C > 1 spreads the rows' loads over more compute units.
constexpr int kCombineThreads = kDim / 4;  // float4 columns of a row (192)

template <int P, int C>
__global__ __launch_bounds__(kCombineThreads / C * P)
void lse_combine_kernel(const float* __restrict__ po, const float* __restrict__ pm,
                        const float* __restrict__ pl, float* __restrict__ out, int S) {
    constexpr int G = kCombineThreads / C;  // threads (float4 columns) per group
    static_assert(kCombineThreads % C == 0, "column parts");
    __shared__ f4 part[P > 1 ? (P - 1) * G : 1];
    const size_t row = blockIdx.x / C;
    const int lane = threadIdx.x & 63;
    const int cl = threadIdx.x % G;
    const int c = (int)(blockIdx.x % C) * G + cl;  // float4 column of the row
    const int grp = threadIdx.x / G;
    const float* pmr = pm + row * S;
    const float* plr = pl + row * S;
    const f4* src = (const f4*)(po + row * S * kDim) + c;

    // Batches of 8 splits per thread; a partial last batch re-reads split
    // S - 1 with weight 0, so every batch issues its 8 loads before the first
    // use (no chain of dependent single loads).
    f4 v[8];
    float mv[8];
    auto load_batch = [&](int s) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = s + u * P;
            const int ic = i < S ? i : S - 1;
            v[u] = src[(size_t)ic * (kDim / 4)];
            mv[u] = pmr[ic];
        }
    };
    if (grp < S) load_batch(grp);
    const float m_first = lane < S ? pmr[lane] : -FLT_MAX;
    const float l_first = lane < S ? plr[lane] : 0.f;

    float M = m_first;
    for (int s = lane + kWave; s < S; s += kWave) M = fmaxf(M, pmr[s]);
    M = wave_max(M);
    float L = m_first > -FLT_MAX ? expf(m_first - M) * l_first : 0.f;
    for (int s = lane + kWave; s < S; s += kWave) {
        const float m = pmr[s];
        if (m > -FLT_MAX) L += expf(m - M) * plr[s];
    }
    L = wave_sum(L);

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = grp; s < S; s += 8 * P) {
        if (s != grp) load_batch(s);
        float wgt[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            wgt[u] = (s + u * P >= S || mv[u] == -FLT_MAX) ? 0.f : expf(mv[u] - M);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += wgt[u] * v[u];
    }
    if constexpr (P > 1) {
        if (grp > 0) part[(grp - 1) * G + cl] = acc;
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int q = 1; q < P; ++q) acc += part[(q - 1) * G + cl];
    }
    ((f4*)(out + row * kDim))[c] = acc * (1.0f / (L + 1e-6f));
}

}  // namespace f32

// --------------------------------------------------------------------------
// Host launch helpers (used by the C entry points in xattn_abi.hip)
// --------------------------------------------------------------------------

int f32_row_blocks(int NL, int ds) { return (NL + f32::BM / ds - 1) / (f32::BM / ds); }

#ifdef XATTN_PHASE_CLOCK
// The fp32 kernel's stamps: [kClockBlocks][8][kClockFields] unsigned 64-bit
// values (four wavefronts used).  Clear before a launch, read after.  0 on
// success.
extern "C" int xattn_phase_clock_read_f32(void* dst, size_t bytes) {
    const size_t n = bytes < sizeof(f32::phase_clock) ? bytes : sizeof(f32::phase_clock);
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(f32::phase_clock), n) == hipSuccess ? 0 : 1;
}
extern "C" int xattn_phase_clock_clear_f32(void) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(f32::phase_clock)) != hipSuccess) return 1;
    if (hipMemset(ptr, 0, sizeof(f32::phase_clock)) != hipSuccess) return 1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : 1;
}
#endif

template <bool PARTIAL>
static void launch_f32(int ds, unsigned nblk, hipStream_t stream, const f32::Params& p) {
    if (ds == 4)
        hipLaunchKernelGGL((f32::flash_f32_kernel<PARTIAL, 4>), dim3(nblk), dim3(256), 0, stream, p);
    else if (ds == 2)
        hipLaunchKernelGGL((f32::flash_f32_kernel<PARTIAL, 2>), dim3(nblk), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((f32::flash_f32_kernel<PARTIAL, 1>), dim3(nblk), dim3(256), 0, stream, p);
}

bool launch_flash_f32(int ds, const float* Q, const float* K, const float* V, float* out,
                      float* po, float* pm, float* pl, int B, int NL, int NI,
                      int S, int chunk, hipStream_t stream) {
    if (ds != 1 && ds != 2 && ds != 4) {
        set_error(XATTN_ERR_INVALID_VALUE, "flash_f32: column parts %d not in {1, 2, 4}", ds);
        return false;
    }
    f32::Params p;
    p.Q = Q; p.K = K; p.V = V; p.out = out; p.po = po; p.pm = pm; p.pl = pl;
    p.B = B; p.NL = NL; p.NI = NI; p.S = S; p.chunk = chunk;
    p.row_blocks = f32_row_blocks(NL, ds);
    const long long nblk = (long long)B * p.row_blocks * S;
    if (nblk <= 0) return true;
    if (nblk > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "grid of %lld workgroups too large", nblk);
        return false;
    }
    if (po) launch_f32<true>(ds, (unsigned)nblk, stream, p);
    else launch_f32<false>(ds, (unsigned)nblk, stream, p);
    return check_launch("flash_f32");
}

// Column parts of the merge: the most (1, 2 or 4) that still leave at most
// one workgroup per CU.  The merge's time is its launch and one round trip
// of loads; more parts help only while they reach CUs that would otherwise
// stay idle (measured on MI355X: 64 rows, 4 parts 4.04 against 4.16 µs;
// 256 rows, 2 parts 6.13 against 5.85 µs).
int lse_combine_parts(int rows, int S, int cu) {
    if (rows <= 0 || S <= 1 || rows >= 2 * cu) return 1;
    int c = 1;
    while (c < 4 && (long long)rows * (2 * c) <= cu) c *= 2;
    return c;
}

bool launch_lse_combine(const float* po, const float* pm, const float* pl, float* out,
                        int rows, int S, hipStream_t stream, int parts) {
    if (rows <= 0) return true;
    const bool few = rows < 2 * device_cu_count() && S > 1;
    if (parts <= 0) parts = few ? lse_combine_parts(rows, S, device_cu_count()) : 1;
    if (!few) parts = 1;
    const long long nblk = (long long)rows * parts;
    if (nblk > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "lse_combine: grid of %lld workgroups too large", nblk);
        return false;
    }
    const dim3 grid((unsigned)nblk);
    const int G = f32::kCombineThreads / parts;
    if (!few)
        hipLaunchKernelGGL((f32::lse_combine_kernel<1, 1>), grid, dim3(f32::kCombineThreads), 0,
                           stream, po, pm, pl, out, S);
    else if (parts == 4)
        hipLaunchKernelGGL((f32::lse_combine_kernel<4, 4>), grid, dim3(4 * G), 0, stream, po, pm,
                           pl, out, S);
    else if (parts == 2)
        hipLaunchKernelGGL((f32::lse_combine_kernel<4, 2>), grid, dim3(4 * G), 0, stream, po, pm,
                           pl, out, S);
    else
        hipLaunchKernelGGL((f32::lse_combine_kernel<4, 1>), grid, dim3(4 * G), 0, stream, po, pm,
                           pl, out, S);
    return check_launch("lse_combine");
}

}  // namespace xattn
