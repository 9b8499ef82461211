// fp16 / bf16 fused cross-attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}),
// fp32 accumulate, fp32 online softmax, fp32 output.
//
// Contract (kernel_wmma.cu:42-137): Q arrives pre-scaled by 1/sqrt(D), so a
// score is the plain dot product q.k.
//
// Work item = (batch, key split, 64 latents) on 8 wavefronts (two per SIMD);
// tiles of 32 keys.  Wavefront w = (a, h), a = w & 3, h = w >> 2, owns the
// 192-column slice a of D and the latent half h (two 16-latent blocks), for
// the scores and for the output alike:
//
//   partial S^T[32 keys x 32 q] = K[:, slice] . Q[half, slice]^T   2 x 2 x 6 MFMA
//   O^T[slice x 32 q]         += V[:, slice]^T . P^T[half]         12 x 2 MFMA
//
// The four column slices' partial scores of a (latent block, 16-key half)
// unit are summed through LDS (in the buffer the K tile just left); each of
// the eight units has an owner wavefront that runs its softmax and writes its
// half of the P operand.  The two owners of a latent block share the weights'
// reference m_ref (exchanged on the first tile and at restarts); their running
// maxima and sums are combined at the end.  Two wavefronts per SIMD double
// the LDS read rate a single wavefront reaches, which bounds the MFMA
// sections (the transposed V reads run at half the b128 rate).
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
// Tiles in LDS are fragment-major: every MFMA operand read is one contiguous
// run indexed by the lane, so each read is a base register plus an immediate
// offset (no per-read address arithmetic: a wave64 VALU instruction holds its
// SIMD for four cycles, which is what the MFMA sections would wait on) and
// the reads are conflict-free.
//   K tile: fragment (key half kh, 32-column group c) at (24 kh + c) KiB;
//           lane 16g + j at +16 lanes holds K[16kh + j][32c + 8g .. +7].
//   V tile: piece (key half kh, 16-column block c) at (48 kh + c) * 512 B;
//           lane 16g + 4e + q at +8 lanes holds V[16kh + 4g + e][16c + 4q .. +3].
// The global->LDS DMA does the gather: each 1 KiB chunk is 16 rows x 64 bytes
// of the row-major K or V (chunk n of a tile lies at n KiB for both).  K and
// V tiles (48 KiB each) share one pipeline: phases alternate QK(t) / PV(t),
// phase p reads buffer p % 3 and requests phase p + 2; 3 buffers = 144 KiB.
#include "xattn_common.h"

namespace xattn {
namespace h16 {

constexpr int BN = 32;                 // keys per tile
constexpr int NA = 4;                  // column slices
constexpr int NH = 2;                  // latent halves
constexpr int NW = NA * NH;            // wavefronts per workgroup (8)
constexpr int QB = 16;                 // latents per MFMA block
constexpr int BM = 64;                 // latents per workgroup
constexpr int NCB = BM / QB;           // latent blocks per workgroup (4)
constexpr int CBW = NCB / NH;          // latent blocks per wavefront (2)
constexpr int DW = kDim / NA;          // columns of D per wavefront (192)
constexpr int KS = DW / 32;            // k-steps of a score MFMA chain (6)
constexpr int DB = DW / 16;            // 16-column output blocks per wavefront (12)
constexpr int ROWB = kDim * 2;         // bytes per K / V row (1536)
constexpr int BUFB = BN * ROWB;        // bytes per tile buffer (48 KiB)
constexpr int NBUF = 3;
constexpr int CHUNKS = BUFB / 1024;        // 1 KiB DMA chunks per tile (48)
constexpr int CPW = CHUNKS / NW;           // per wavefront (6)
constexpr int NUNIT = NCB * 2;             // (latent block, key half) softmax units (8)
constexpr int KPF = 4;                     // K fragments read ahead of their MFMAs
constexpr int VPF = 3;                     // V column blocks read ahead of their MFMAs

static_assert(NUNIT == NW, "one softmax unit per wavefront");
static_assert(CHUNKS % NW == 0, "DMA split");
static_assert(NBUF * BUFB + NCB * kWave * 16 + NW * QB * 8 + NCB * QB * 4 + 4 <= 160 * 1024,
              "LDS budget");
static_assert(NUNIT * NA * kWave * 16 <= BUFB, "score exchange fits in a tile buffer");
static_assert(CPW * NA == 24 && NW == 2 * NA, "a wavefront's chunks: one key half, 6 column groups");

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
typedef unsigned int u2v __attribute__((ext_vector_type(2)));
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
    return (lds_char*)byte_addr;
}

template <typename T, bool PARTIAL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash16_kernel(Params p) {
    typedef typename Vec8<T>::type v8;
    __shared__ __attribute__((aligned(16))) char lds[NBUF * BUFB];
    __shared__ __attribute__((aligned(16))) u4v pbuf[NCB * kWave];  // P^T operand per latent block
    __shared__ float2 stats[NW * QB];  // per owner and latent: (max, sum) or the reference
    __shared__ float sref[NCB * QB];   // the reference m_ref of each latent
    __shared__ int restart_flag;

    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int rb = item % p.row_blocks;
    const int bs = item / p.row_blocks;
    const int split = bs % p.S;
    const int b = bs / p.S;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int a = w & (NA - 1), h = w / NA;      // column slice, latent half
    const int j = lane & 15, g = lane >> 4;
    const int q0 = rb * BM;                     // first latent of the workgroup
    const int d0 = a * DW;                      // first column of this wavefront's slice
    const int cbo = w >> 1, kbo = w & 1;        // the softmax unit this wavefront owns
    const int qo = q0 + QB * cbo + j;           // ... and the latent of lane (j, *) in it

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
        for (int cl = 0; cl < CBW; ++cl) {
            const int q = q0 + QB * (CBW * h + cl) + j;
            if (q >= p.NL) continue;
            float* dst = out_row(q) + d0 + 4 * g;
#pragma unroll
            for (int e = 0; e < DB; ++e) *(f4*)(dst + 16 * e) = (f4){0.f, 0.f, 0.f, 0.f};
        }
        if (PARTIAL && kbo == 0 && g == 0 && qo < p.NL) {
            const size_t pi = ((size_t)b * p.NL + qo) * p.S + split;
            p.pm[pi] = -FLT_MAX;
            p.pl[pi] = 0.f;
        }
        return;
    }

    // K and V rows of this split's key range; keys are counted from k0 below.
    const char* Kb = (const char*)(p.K + ((size_t)b * p.NI + k0) * kDim);
    const char* Vb = (const char*)(p.V + ((size_t)b * p.NI + k0) * kDim);
    const int nk = k1 - k0;
    // Non-empty (the early return above); without these facts the compiler
    // guards the tile loop for zero trips and the split-K instantiation no
    // longer fits the register budget.
    __builtin_assume(nk >= 1);
    const int ntiles = (nk + BN - 1) / BN;
    __builtin_assume(ntiles >= 1);
    const int nphase = 2 * ntiles;

    // DMA.  Wavefront w fills chunks 6w .. 6w + 5 of each tile: key half
    // kh = w / 4, 64-byte column groups 6 (w % 4) + t.  Lane i of a K chunk
    // fetches row 16kh + i % 16 at byte 16 (i / 16) of the group; lane i of a V
    // chunk row 16kh + (i % 32) / 2 at byte 32 (i / 32) + 16 (i % 2).  Rows past
    // the key range re-read the range's last row (their scores are masked to
    // -inf, their weights are 0).  Phases past the end re-read the last phase
    // of the same kind into the ring slot of phase ph - 3, whose readers are
    // done, so every tile issues the same way; the DMA is drained after the
    // loop.  The DMA is untracked (dma16_untracked): the phase waits order it.
    const int dkh = w / NA, dcol = 64 * CPW * (w % NA);
    const int rowK = 16 * dkh + (lane & 15), colK = dcol + 16 * (lane >> 4);
    const int rowV = 16 * dkh + ((lane & 31) >> 1), colV = dcol + 32 * (lane >> 5) + 16 * (lane & 1);
    const unsigned lds0 = lds_u32(lds);
    struct Dma {
        const char* src;
        unsigned voff, m0;
    };
    auto dma_setup = [&](int ph) {
        const bool isv = ph & 1;
        const int pr = ph < nphase ? ph : ph - 2;
        const int n0 = (pr >> 1) * BN;
        const int last = nk - 1 - n0;  // last valid row of the tile
        Dma d;
        d.src = (isv ? Vb : Kb) + (size_t)n0 * ROWB;
        d.voff = (unsigned)(min(isv ? rowV : rowK, last) * ROWB + (isv ? colV : colK));
        d.m0 = lds0 + (unsigned)((ph % NBUF) * BUFB + 1024 * CPW * w);
        return d;
    };
    auto dma_chunk = [&](const Dma& d, int t) { dma16_untracked(d.src + 64 * t, d.voff, d.m0 + 1024 * t); };
    auto issue = [&](int ph) {
        const Dma d = dma_setup(ph);
#pragma unroll
        for (int t = 0; t < CPW; ++t) dma_chunk(d, t);
    };

    // Q^T operand of latent block 2h + cl, k-step s:
    // Q[q0 + 16(2h + cl) + j][d0 + 32s + 8g .. +7] (48 registers).  Latents past
    // NL repeat the last one; they are not stored.  K(0) is requested first;
    // the full wait after the Q loads leaves no compiler-visible load pending,
    // so the compiler adds no waits inside the tile loop (where only untracked
    // DMA is in flight).
    issue(0);
    v8 qr[CBW][KS];
#pragma unroll
    for (int cl = 0; cl < CBW; ++cl) {
        const int qc = min(q0 + QB * (CBW * h + cl) + j, p.NL - 1);
        const u16* qrow = p.Q + ((size_t)b * p.NL + qc) * kDim + d0 + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s) qr[cl][s] = *(const v8*)(qrow + 32 * s);
    }
    wait_vmcnt<0>();

    // Per-lane LDS read bases within a tile buffer: the K fragments of this
    // wavefront's column groups 6a .. 6a + 5, the V pieces of its column
    // blocks 12a .. 12a + 11; fragments differ by immediate offsets.
    const int kread = 1024 * CPW * a + 16 * lane;
    const int vread = 512 * DB * a + 8 * lane;

    if (tid == 0) restart_flag = 0;

    const float tau_raw = tau_log2<T> / kLog2e;
    // Softmax state of the owned unit, for latent qo (replicated over g):
    // m_true: exact running max over this key half; m_ref: the reference of
    // the weights, the same for both halves of the latent and fixed for a
    // pass; lsum: the half's sum of weights.
    float m_true = -FLT_MAX, m_ref = -FLT_MAX, lsum;
    bool ref_set = false;  // the same at every lane of the workgroup
    f4 acc[CBW][DB];  // O^T[d0 + 16t + 4g + i][q0 + 16(2h + cl) + j]

    for (bool first = true;; first = false) {  // passes over the key range; a second is rare
        if (!first) issue(0);
        issue(1);
#pragma unroll
        for (int cl = 0; cl < CBW; ++cl)
#pragma unroll
            for (int t = 0; t < DB; ++t) acc[cl][t] = (f4){0.f, 0.f, 0.f, 0.f};
        lsum = 0.f;
        bool restart = false;

        for (int tile = 0; tile < ntiles; ++tile) {
            const int n0 = tile * BN;
            int ph = 2 * tile;

            // ---------------- partial scores over this wavefront's slice ----------------
            wait_vmcnt<CPW>();
            lds_barrier();
            char* kb = lds + (ph % NBUF) * BUFB;
            f4 sacc[2][CBW];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int cl = 0; cl < CBW; ++cl) sacc[kh][cl] = (f4){0.f, 0.f, 0.f, 0.f};
            {
                // fragment f: k-step f >> 1, keys 16 (f & 1) .. +15
                const lds_char* kr = opaque_lds(lds0 + (unsigned)((ph % NBUF) * BUFB + kread));
                auto kfrag = [&](int f) { return *(const v8*)(kr + 1024 * ((f & 1) * 24 + (f >> 1))); };
                const Dma dk = dma_setup(ph + 2);
                // K fragments run KPF ahead of the MFMAs that use them; the
                // phase-(ph + 2) DMA goes out one chunk per two fragments, so
                // the address unit drains between issues.
                v8 kf[2 * KS];
#pragma unroll
                for (int f = 0; f < KPF; ++f) kf[f] = kfrag(f);
#pragma unroll
                for (int f = 0; f < 2 * KS; ++f) {
                    if (f + KPF < 2 * KS) kf[f + KPF] = kfrag(f + KPF);
                    if ((f & 1) == 0) dma_chunk(dk, f >> 1);
#pragma unroll
                    for (int cl = 0; cl < CBW; ++cl)
                        sacc[f & 1][cl] = mfma32<T>(kf[f], qr[cl][f >> 1], sacc[f & 1][cl]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // Every wavefront is done with K(t): its buffer carries the partial
            // sums, slot (unit * 4 + slice), unit = block * 2 + key half,
            // 64 lanes x 16 B each.
            lds_barrier();
            f4* xs = (f4*)kb;
#pragma unroll
            for (int cl = 0; cl < CBW; ++cl)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
                    xs[(((CBW * h + cl) * 2 + kh) * NA + a) * kWave + lane] = sacc[kh][cl];
            lds_barrier();
            f4 sv = xs[(w * NA) * kWave + lane];
#pragma unroll
            for (int src = 1; src < NA; ++src) sv += xs[(w * NA + src) * kWave + lane];

            // ------ softmax weights of the owned unit (raw-dot units) ------
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = (n0 + 16 * kbo + 4 * g + i < nk) ? sv[i] : -INFINITY;
            float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
            tmax = wave_max16_groups(tmax);
            m_true = fmaxf(m_true, tmax);
            if (!ref_set) {
                // First tile of the kernel: the two owners of a latent block
                // agree on the reference, the row max of the tile.
                if (g == 0) stats[w * QB + j].x = tmax;
                lds_barrier();
                m_ref = fmaxf(tmax, stats[(w ^ 1) * QB + j].x);
                lds_barrier();
                ref_set = true;
            }
            if (__any(tmax > m_ref + tau_raw) && lane == 0) restart_flag = 1;
            float pw[4];
            float rs = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pw[i] = fast_exp2((x[i] - m_ref) * kLog2e);
                rs += pw[i];
            }
            lsum += wave_sum16_groups(rs);
            // this half of block cbo's P^T operand: bytes 8 kbo .. 8 kbo + 7 of each lane
            *(u2v*)((char*)pbuf + (size_t)(cbo * kWave + lane) * 16 + 8 * kbo) =
                (u2v){pack2<T>(pw[0], pw[1]), pack2<T>(pw[2], pw[3])};

            // ---------------- O^T += V^T . P^T over this wavefront's slice ----------------
            ph += 1;
            wait_vmcnt<CPW>();
            lds_barrier();
            // Every wavefront sets the flag (if at all) before this barrier, so
            // all read the same value.
            if (__builtin_amdgcn_readfirstlane(restart_flag)) {
                restart = true;
                break;
            }
            v8 pt[CBW];
#pragma unroll
            for (int cl = 0; cl < CBW; ++cl)
                pt[cl] = __builtin_bit_cast(v8, pbuf[(CBW * h + cl) * kWave + lane]);
            {
                lds_s4* vr = (lds_s4*)opaque_lds(lds0 + (unsigned)((ph % NBUF) * BUFB + vread));  // 64 per 512 B
                const Dma dv = dma_setup(ph + 2);
                s4 va[DB], vc[DB];
#pragma unroll
                for (int t = 0; t < VPF; ++t) {
                    va[t] = tr_read(vr + 64 * t);
                    vc[t] = tr_read(vr + 64 * (48 + t));
                }
#pragma unroll
                for (int t = 0; t < DB; ++t) {
                    if (t + VPF < DB) {
                        va[t + VPF] = tr_read(vr + 64 * (t + VPF));
                        vc[t + VPF] = tr_read(vr + 64 * (48 + t + VPF));
                    }
                    if ((t & 1) == 0) dma_chunk(dv, t >> 1);
                    const v8 vt = __builtin_bit_cast(
                        v8, __builtin_shufflevector(va[t], vc[t], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                    for (int cl = 0; cl < CBW; ++cl) acc[cl][t] = mfma32<T>(vt, pt[cl], acc[cl][t]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (!restart) break;
        // Some latent's scores outgrew its reference: drain the DMA (phases up
        // to ph + 2 may be in flight), clear the flag, and run the keys again
        // with the reference raised to the max seen so far over both halves.
        wait_vmcnt<0>();
        lds_barrier();
        if (tid == 0) restart_flag = 0;
        if (g == 0) stats[w * QB + j].x = m_true;
        lds_barrier();
        m_ref = fmaxf(m_true, stats[(w ^ 1) * QB + j].x);
        lds_barrier();
    }
    wait_vmcnt<0>();  // the re-reads issued past the last phase

    // Combine the two key halves of each latent (max and sum, both against
    // the shared m_ref), then normalise (or, for a partial, rescale to the
    // exact max).
    // A wavefront's m_ref is that of the latent block it owns a unit of; the
    // output blocks it accumulates are weighted by their own blocks' m_ref.
    if (g == 0) stats[w * QB + j] = make_float2(m_true, lsum);
    if (g == 0 && kbo == 0) sref[cbo * QB + j] = m_ref;
    lds_barrier();
    float rsc[CBW];
#pragma unroll
    for (int cl = 0; cl < CBW; ++cl) {
        const int cb = CBW * h + cl;
        const float2 s0 = stats[(2 * cb) * QB + j], s1 = stats[(2 * cb + 1) * QB + j];
        const float mt = fmaxf(s0.x, s1.x);
        const float factor = fast_exp2((sref[cb * QB + j] - mt) * kLog2e);
        const float l = s0.y + s1.y;
        rsc[cl] = PARTIAL ? factor : factor / (l * factor + 1e-6f);
        if (PARTIAL && a == 0 && g == 0) {
            const int q = q0 + QB * cb + j;
            if (q < p.NL) {
                const size_t pi = ((size_t)b * p.NL + q) * p.S + split;
                p.pm[pi] = mt;  // scores are q.k with Q pre-scaled
                p.pl[pi] = l * factor;
            }
        }
    }
#pragma unroll
    for (int cl = 0; cl < CBW; ++cl) {
        const int q = q0 + QB * (CBW * h + cl) + j;
        if (q >= p.NL) continue;
        float* dst = out_row(q) + d0 + 4 * g;
#pragma unroll
        for (int t = 0; t < DB; ++t) *(f4*)(dst + 16 * t) = acc[cl][t] * rsc[cl];
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
    const dim3 grid((unsigned)nblk), block(h16::NW * kWave);
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
