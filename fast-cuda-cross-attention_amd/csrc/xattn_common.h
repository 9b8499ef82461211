// Shared device/host helpers for the gfx950 cross-attention kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, MFMA builtins,
// LDS DMA (global_load_lds) and the 8-XCD dispatch order of MI355X.
#pragma once

#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

#include "xattn.h"

namespace xattn {

constexpr int kWave = 64;
constexpr int kDim = 768;              // model dimension every MFMA path is built for
constexpr int kNumXcd = 8;             // MI355X: 8 XCDs, workgroups dealt round-robin

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef short s8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16;

// log2(e) / sqrt(768): turns a raw q.k dot product into a base-2 exponent.
constexpr float kLog2e = 1.4426950408889634f;

// --------------------------------------------------------------------------
// Workgroup -> work-item mapping that keeps co-operating workgroups on one
// XCD.  The dispatcher deals block b to XCD (b % 8); this returns a logical
// index such that logical ids [off(x), off(x) + count(x)) all live on XCD x.
// It is a bijection on [0, n) for every n (tested on the host).
// --------------------------------------------------------------------------
__host__ __device__ inline int xcd_remap(int bid, int n) {
    int per = n / kNumXcd, rem = n % kNumXcd;
    int x = bid % kNumXcd, local = bid / kNumXcd;
    return x * per + (x < rem ? x : rem) + local;
}

// --------------------------------------------------------------------------
// Wave-level helpers
// --------------------------------------------------------------------------
// Reductions over the 4 lanes {l, l^16, l^32, l^48} with the gfx950 row
// swaps (v_permlane16_swap / v_permlane32_swap): each returns the pair
// (own value, value of the partner row), so no LDS round trip is involved.
__device__ inline float xor16_partner_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_partner_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_max16_groups(float v) {
    return xor32_partner_max(xor16_partner_max(v));
}
__device__ inline float wave_sum16_groups(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                              false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ inline float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt with only a vmcnt limit (expcnt / lgkmcnt left unconstrained).
// gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14].
// The waits and barriers below are also compiler fences: no memory access
// (LDS read, DMA issue) may be moved across them, at IR level (asm memory
// clobber) or by the machine scheduler (sched_barrier).
__device__ inline void compiler_fence() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    compiler_fence();
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    compiler_fence();
}

// Workgroup barrier for LDS hand-off: waits for this wave's own LDS
// operations, then s_barrier.  Unlike __syncthreads() it carries no release
// fence, so global->LDS DMA issued for later phases stays in flight; the
// caller makes the DMA of the phase being consumed visible with wait_vmcnt
// before calling this.
__device__ inline void lds_barrier() {
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    compiler_fence();
}

// A wave-uniform pointer re-materialised through readfirstlane: the compiler
// cannot re-associate (uniform base + per-lane offset) across it and hoist
// per-lane 64-bit sums out of a loop, and the base lands in SGPRs.
template <typename T>
__device__ inline const T* uniform_ptr(const T* p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (const T*)(((unsigned long long)hi << 32) | lo);
}

// 16-byte global -> LDS DMA for one lane.  The 64 lanes of the wave land at
// lds_base + 16 * lane (lds_base must be wave-uniform).
__device__ inline void dma16(const void* gptr, void* lds_base) {
    __builtin_amdgcn_global_load_lds(
        gptr, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// Byte address of an LDS location (the value M0 takes for an LDS DMA).
__device__ inline unsigned lds_u32(const void* p) {
    return (unsigned)(uintptr_t)((const __attribute__((address_space(3))) char*)p);
}

// The same DMA issued as inline assembly: lane i reads sbase + voff_i (sbase
// wave-uniform, in SGPRs) and writes LDS bytes [lds_byte + 16 i, +16).  The
// compiler does not see it, so it inserts no vmcnt waits of its own before
// later LDS reads (it drains every outstanding DMA before a transposing LDS
// read, and before any LDS read once a kernel has more than one LDS object);
// the caller orders it with wait_vmcnt + lds_barrier, which count it like any
// vector memory load.  M0 (reserved to the compiler) is saved and restored
// around the load and written one wait state before the load reads it.
__device__ inline void dma16_untracked(const void* sbase, unsigned voff, unsigned lds_byte) {
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(lds_byte)
        : "memory");
}

// The same DMA with M0 an input operand of the assembly: the compiler sets M0
// itself (no save and restore around each load) and knows it changed.  OFF,
// a constant byte offset below 4096, is the instruction's immediate: the
// hardware adds it to every lane's source address and to the LDS
// destination alike, so lds_byte is the destination minus OFF.  The one wait
// state between the write of M0 and the load is the s_nop.
template <int OFF>
__device__ inline void dma16_m0(const void* sbase, unsigned voff, unsigned lds_byte) {
    static_assert(OFF >= 0 && OFF < 4096, "global instruction offset range");
    asm volatile(
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:%3"
        :
        : "v"(voff), "s"(sbase), "{m0}"(lds_byte), "i"(OFF)
        : "memory");
}

// --------------------------------------------------------------------------
// Phase clock: instrumented builds only (`make phaseclock` defines
// XATTN_PHASE_CLOCK; the product build compiles none of it).  A kernel
// keeps, per workgroup (the first kClockBlocks of a launch) and wavefront,
// kClockFields 64-bit values: the shader clock at kernel start, tile-loop
// start, tile-loop end and kernel end; the 100 MHz real-time clock at start
// and end; then, summed over the tiles (kernels that record them), the
// cycles spent waiting for tiles at barriers, in the first phase of a tile
// and in the second.  Each stamp sits where the wavefront has no LDS or
// scalar load in flight, so its wait changes no overlap; the scheduling
// barriers around it do pin the instruction order.
// --------------------------------------------------------------------------
constexpr int kClockBlocks = 4096;
constexpr int kClockFields = 9;
#ifdef XATTN_PHASE_CLOCK
#define XATTN_STAMP(var)                                         \
    __builtin_amdgcn_sched_barrier(0);                           \
    const unsigned long long var = __builtin_amdgcn_s_memtime(); \
    __builtin_amdgcn_sched_barrier(0)
#define XATTN_CLOCK_DECL(...) unsigned long long __VA_ARGS__
#define XATTN_CLOCK_ADD(acc, from, to) acc += (to) - (from)
#else
#define XATTN_STAMP(var) (void)0
#define XATTN_CLOCK_DECL(...) (void)0
#define XATTN_CLOCK_ADD(acc, from, to) (void)0
#endif

}  // namespace xattn

// --------------------------------------------------------------------------
// Host-side error reporting shared by every launcher (xattn_abi.hip).
// --------------------------------------------------------------------------
namespace xattn {
void set_error(int code, const char* fmt, ...);
bool check_launch(const char* who);
}  // namespace xattn
