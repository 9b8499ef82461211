// C entry points of kernels.so: argument validation, error state, device
// queries, workspace and launch planning.  The kernels live in the other
// translation units; every launcher here is host code only.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "xattn_common.h"
#include "xattn_launch.h"

namespace xattn {

// --------------------------------------------------------------------------
// Error state (per host thread, first error wins until read)
// --------------------------------------------------------------------------
static thread_local int g_err = XATTN_OK;
static thread_local char g_msg[512] = "";

void set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    // The message belongs to the error xattn_get_last_error() will return.
    if (g_err != XATTN_OK) return;
    g_err = code;
    snprintf(g_msg, sizeof(g_msg), "%s", buf);
}

bool check_launch(const char* who) {
    const hipError_t e = hipPeekAtLastError();
    if (e != hipSuccess) {
        set_error(XATTN_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
        return false;
    }
    return true;
}

// --------------------------------------------------------------------------
// Device properties (cached per device)
// --------------------------------------------------------------------------
static std::mutex g_dev_mu;
static int g_cu[256];
static int g_lds[256];

int device_max_lds() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return 64 * 1024;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (g_lds[dev] <= 0) {
        int lds = 0;
        if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
                hipSuccess ||
            lds <= 0)
            lds = 64 * 1024;
        g_lds[dev] = lds;
    }
    return g_lds[dev];
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return 256;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (g_cu[dev] <= 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cu <= 0)
            cu = 256;
        g_cu[dev] = cu;
    }
    return g_cu[dev];
}

// --------------------------------------------------------------------------
// Library-owned split workspaces of launch_optimized_kernel and
// launch_wmma_kernel / launch_wmma_bf16_kernel: one block per (device,
// stream), so split launches on different streams never share memory and
// need no cross-stream ordering; on one stream, stream order serialises
// them.  hipStreamPerThread names a different stream in every host thread,
// so for that handle the calling thread is part of the key.  A block is
// allocated (hipMalloc) on a stream's first split launch and replaced by a
// larger one, at least twice the size, when a launch needs more.  A
// replaced block is never freed: launches already enqueued, or kernels
// recorded into a graph, may still use it (its memory comes back at process
// exit); geometric growth bounds the retired blocks' total by the live
// block's size.  No launcher synchronises.
//
// Graphs.  Under stream capture a launch whose stream has a large enough
// block proceeds, and the block then belongs to the graph: the next launch
// on that stream outside capture retires it and takes a fresh block, so a
// replay of the graph (on any stream) never shares partials with later
// eager launches on the capturing stream.  A capturing launch that would
// have to allocate is refused with XATTN_ERR_CAPTURE before anything is
// enqueued.  Two graphs captured on one stream with no eager split launch
// between the captures share a block, so their replays must not overlap.
// --------------------------------------------------------------------------
struct StreamWorkspace {
    int dev;
    hipStream_t stream;
    uint64_t thread;         // the owning thread for hipStreamPerThread, else 0
    void* ptr;
    size_t bytes;
    bool captured;           // a graph recorded launches that use this block
};
static std::mutex g_ws_mu;
static std::vector<StreamWorkspace> g_ws;  // a handful of (device, stream) entries
static std::vector<void*> g_ws_retired;     // replaced blocks, kept to process exit

// A number of the calling host thread, never reused within the process (a
// finished thread's std::thread::id can be).
static uint64_t thread_number() {
    static std::atomic<uint64_t> next{1};
    thread_local const uint64_t mine = next++;
    return mine;
}

// Is `stream` recording a graph?  A query that fails counts as capturing
// (the launcher then refuses rather than allocate blindly).
static bool stream_capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return st != hipStreamCaptureStatusNone;
}

class WorkspaceLease {
  public:
    // The workspace of (current device, stream) with at least `bytes`;
    // nullptr with an error recorded on failure.  The lock is held until
    // release(), so no other host thread replaces the block between this
    // launch's pointer lookup and its enqueue.
    void* acquire(size_t bytes, hipStream_t stream) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) {
            (void)hipGetLastError();
            set_error(XATTN_ERR_ALLOC, "workspace: no current device");
            return nullptr;
        }
        const uint64_t owner = stream == hipStreamPerThread ? thread_number() : 0;
        const bool capturing = stream_capturing(stream);
        lk_.lock();
        StreamWorkspace* w = nullptr;
        for (StreamWorkspace& e : g_ws)
            if (e.dev == dev && e.stream == stream && e.thread == owner) w = &e;
        if (w && w->bytes >= bytes) {
            if (capturing) {
                w->captured = true;
                return w->ptr;
            }
            if (!w->captured) return w->ptr;
            // an eager launch after a capture used this block: the graph
            // keeps it, this stream takes a fresh one of the same size
        } else if (capturing) {
            set_error(XATTN_ERR_CAPTURE,
                      "workspace: this split launch needs %zu bytes of workspace on a stream "
                      "that is capturing a graph and has %zu; make one launch of this (or a "
                      "larger) shape on the stream before capturing, or use "
                      "launch_splitk_kernel with caller-owned scratch",
                      bytes, w ? w->bytes : (size_t)0);
            return nullptr;
        }
        size_t want = bytes;
        if (w && want < w->bytes) want = w->bytes;
        if (w && !w->captured && want < 2 * w->bytes) want = 2 * w->bytes;
        void* p = nullptr;
        if (hipMalloc(&p, want) != hipSuccess) {
            (void)hipGetLastError();
            set_error(XATTN_ERR_ALLOC, "workspace: hipMalloc(%zu) failed", want);
            return nullptr;
        }
        if (w) {
            g_ws_retired.push_back(w->ptr);
            w->ptr = p;
            w->bytes = want;
            w->captured = false;
        } else {
            g_ws.push_back(StreamWorkspace{dev, stream, owner, p, want, false});
        }
        return p;
    }
    // The launch using the workspace has been enqueued.
    void release() {
        if (lk_.owns_lock()) lk_.unlock();
    }
    ~WorkspaceLease() { release(); }

  private:
    std::unique_lock<std::mutex> lk_{g_ws_mu, std::defer_lock};
};

// --------------------------------------------------------------------------
// Static scratch of launch_optimized_kernel_noalloc: split partials live in a
// file-scope device array instead of an allocated workspace.  Each GPU the
// library runs on holds its own copy from module load until the process
// ends.  On the host, `scratch` names a host-side stand-in, not device
// memory: the device address is looked up once per device with
// hipGetSymbolAddress (that device current, in xattn_noalloc_prepare) and
// only that address is handed to kernels.  Each launch overwrites every
// partial it merges (an empty split writes its sentinel), so nothing has to
// be cleared between calls.
//
// Every call on a GPU shares its copy.  Outside stream capture, split calls
// are ordered on the device by a library event per GPU: each call's stream
// waits for the event (hipStreamWaitEvent: no host wait, no allocation),
// the call enqueues its two kernels, and the event is recorded after the
// merge, all under one lock, so overlapping calls from other streams or
// host threads run one after the other.  A call under capture neither waits
// nor records (a captured graph cannot depend on work outside it): a graph
// replay that overlaps another split call on the same GPU races with it.
// --------------------------------------------------------------------------
constexpr size_t kNoallocScratchBytes = (size_t)64 << 20;  // 64 MiB per device
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

struct NoallocDevice {
    std::mutex mu;             // held across (wait, launches, record)
    void* ptr = nullptr;       // device address of this GPU's `scratch`
    hipEvent_t done = nullptr;  // recorded after the last split call's merge
    bool recorded = false;
};
static NoallocDevice g_noalloc[256];

// Resolve `scratch` and create the ordering event for device `dev` (the
// caller holds g_noalloc[dev].mu and has made `dev` current).  0 on success.
static int noalloc_setup(int dev, const char* who) {
    NoallocDevice& d = g_noalloc[dev];
    if (!d.ptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            (void)hipGetLastError();
            set_error(XATTN_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", who,
                      hipGetErrorString(e));
            return (int)(e != hipSuccess ? e : hipErrorInvalidSymbol);
        }
        d.ptr = ptr;
    }
    if (!d.done) {
        hipEvent_t ev = nullptr;
        const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error(XATTN_ERR_LAUNCH, "%s: hipEventCreateWithFlags failed: %s", who,
                      hipGetErrorString(e));
            return (int)e;
        }
        d.done = ev;
    }
    return 0;
}

// --------------------------------------------------------------------------
// Validation
// --------------------------------------------------------------------------
bool validate_common(const char* who, const void* Q, const void* K, const void* V,
                     const void* out, int B, int NL, int NI, int dim) {
    if (B < 0 || NL < 0 || NI < 0 || dim < 0) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: negative size (B=%d NL=%d NI=%d dim=%d)", who, B,
                  NL, NI, dim);
        return false;
    }
    if ((long long)B * NL > 0 && (!Q || !out)) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: NULL Q/output", who);
        return false;
    }
    if ((long long)B * NI > 0 && (!K || !V)) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: NULL K/V", who);
        return false;
    }
    return true;
}

bool validate_dim768(const char* who, int dim) {
    if (dim != kDim) {
        set_error(XATTN_ERR_UNSUPPORTED, "%s: dim=%d unsupported (built for dim=%d)", who, dim,
                  kDim);
        return false;
    }
    return true;
}

// The MFMA paths move Q/K/V and the fp32 rows in 16-byte vectors (and K/V by
// 16-byte global->LDS DMA); hipMalloc returns 256-byte aligned memory.
bool validate_aligned16(const char* who, const void* Q, const void* K, const void* V,
                        const void* out, const void* po) {
    const void* ptr[5] = {Q, K, V, out, po};
    const char* name[5] = {"Q", "K", "V", "output", "partial output"};
    for (int i = 0; i < 5; ++i) {
        if ((reinterpret_cast<uintptr_t>(ptr[i]) & 15) != 0) {
            set_error(XATTN_ERR_INVALID_VALUE, "%s: %s pointer %p is not 16-byte aligned", who,
                      name[i], ptr[i]);
            return false;
        }
    }
    return true;
}

bool validate_splits(const char* who, const void* po, const void* pm, const void* pl, int B,
                     int NL, int S) {
    if (S < 1) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: num_splits=%d must be >= 1", who, S);
        return false;
    }
    if ((long long)B * NL > 0 && (!po || !pm || !pl)) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: NULL split scratch", who);
        return false;
    }
    return true;
}

// Key splits that let B * row_blocks workgroups fill `cu` compute units, with
// every split a whole number of `tile`-key tiles.
int plan_splits(int B, int NL, int NI, int cu, int bm, int tile) {
    if (B <= 0 || NL <= 0 || NI <= 0) return 1;
    const long long items = (long long)B * ((NL + bm - 1) / bm);
    if (items >= cu) return 1;
    const int tiles = (NI + tile - 1) / tile;
    long long s = (cu + items - 1) / items;
    if (s > tiles) s = tiles;
    if (s < 1) s = 1;
    // tile-aligned chunks: recompute the count that chunk implies
    const int chunk_tiles = (int)((tiles + s - 1) / s);
    return (tiles + chunk_tiles - 1) / chunk_tiles;
}

// Modelled time (µs) of one fp32 launch with ds wavefronts per 16-latent
// block (64/ds-latent workgroups) and S key splits of ct 16-key tiles each,
// fitted (least squares on relative error, coefficients >= 0) to 803 timed
// launches on MI355X (every workgroup size and split count the planner weighs
// at 31 shapes, B = 1..32, N_latent = 64..1024, N_input = 784..50176): a
// 16-key tile costs a workgroup 5.62 µs at 64 latents, 2.99 at 32 and 1.72 at
// 16 (smaller workgroups stream more K/V from L2 and run the softmax more
// often per FLOP), plus 0.68 µs per round of workgroups; a split launch adds
// the LSE merge, 10.67 µs + 0.36 µs per MB of partials written and read back,
// + 0.08 µs per split while there are fewer merge rows (B * N_latent) than
// CUs.  Its choice is the fastest timed plan at 27 of the 31 shapes, 0.48 %
// slower on average and 4.4 % at worst.
static double f32_cost(int B, int NL, int cu, int ds, long long S, long long ct) {
    const double tile_us = ds == 1 ? 5.620 : ds == 2 ? 2.986 : 1.716;
    const long long W = (long long)B * f32_row_blocks(NL, ds) * S;
    const long long rounds = (W + cu - 1) / cu;
    double t = (double)rounds * (0.675 + (double)ct * tile_us);
    if (S > 1) {
        const double rows = (double)B * NL;
        t += 10.668 + 0.355 * rows * (double)S * (kDim * 4) * 1e-6 +
             0.08 * (double)S * std::max(0.0, 1.0 - rows / cu);
    }
    return t;
}

// Wavefronts per 16-latent block (1, 2 or 4) for a launch of S key splits of
// `chunk` keys each: the cheapest by f32_cost.
static int f32_parts(int B, int NL, int NI, int S, int chunk, int cu) {
    const long long ct = NI > 0 ? ((long long)std::min(chunk, NI) + 15) / 16 : 0;
    int best = 1;
    double best_t = 0.0;
    for (int ds = 1; ds <= 4; ds *= 2) {
        const double t = f32_cost(B, NL, cu, ds, S, ct);
        if (ds == 1 || t < best_t) best = ds, best_t = t;
    }
    return best;
}

// Launch shape of launch_optimized_kernel: the (ds, S) pair of least
// f32_cost over ds in {1, 2, 4} and S up to min(tiles, cu), with every split
// a whole number of tiles.  The last shape is cached per thread.
static void f32_plan(int B, int NL, int NI, int cu, int* ds, int* S) {
    thread_local int key[4] = {-1, -1, -1, -1}, val[2] = {1, 1};
    if (key[0] == B && key[1] == NL && key[2] == NI && key[3] == cu) {
        *ds = val[0];
        *S = val[1];
        return;
    }
    int bd = 1, bs = 1;
    const long long tiles = NI > 0 ? ((long long)NI + 15) / 16 : 0;
    if (B > 0 && NL > 0 && tiles > 0) {
        double best_t = -1.0;
        const long long smax = std::min<long long>(tiles, cu);
        for (int d = 1; d <= 4; d *= 2) {
            for (long long s = 1; s <= smax; ++s) {
                const long long ct = (tiles + s - 1) / s;
                if ((tiles + ct - 1) / ct != s) continue;  // same chunks as a smaller s
                const double t = f32_cost(B, NL, cu, d, s, ct);
                if (best_t < 0.0 || t < best_t) best_t = t, bd = d, bs = (int)s;
            }
        }
    }
    key[0] = B, key[1] = NL, key[2] = NI, key[3] = cu;
    val[0] = bd, val[1] = bs;
    *ds = bd;
    *S = bs;
}

int optimized_num_splits(int B, int NL, int NI, int cu) {
    int ds = 1, S = 1;
    f32_plan(B, NL, NI, cu, &ds, &S);
    return S;
}

// Launch forms of the 16-bit kernel: 64 latents on 8 wavefronts, 32 on 4,
// and 64 latents on 8 wavefronts in two column halves (two workgroups per
// row block, each computing the scores over all of D and half of the output).
struct H16Form {
    int nw, cp;
};
constexpr H16Form kH16Forms[] = {{8, 1}, {8, 2}, {4, 1}};

// Modelled time (µs) of one 16-bit launch of form f with S key splits of ct
// 32-key tiles each, fitted (least squares on relative error, coefficients
// >= 0) to 1,164 timed launches on MI355X, bf16 and fp16: every form and
// split count the planner weighs at 27 shapes, B = 1..32, N_latent =
// 64..1024, N_input = 784..50176, each timed through launch_wmma_plan_kernel.
// Per launch 4.87 µs; per round of workgroups 1.26 µs, and per 32-key tile
// and round 1.30 µs at 64 latents, 1.08 µs at 64 latents and half the
// columns, 1.15 µs at 32 latents, plus 0.56 / 0.31 / 0.13 µs when an
// unsplit launch fills every CU (its workgroups then all stream K and V from
// L2 at once).  A split launch adds the LSE merge, 6.21 µs + 0.33 µs per MB
// of partials written and read back.  Its choice is the fastest timed plan
// for 40 of the 54 (type, shape) pairs and within 4.3 % of it for the others
// (0.54 % mean), and the same in a later session the fit did not see (41 of
// 54, 0.51 %); repeated timings of one plan spread by a few per cent.
static double h16_cost(int B, int NL, int cu, H16Form f, long long S, long long ct) {
    const long long W = (long long)B * h16_row_blocks(NL, f.nw) * S * f.cp;
    const long long rounds = (W + cu - 1) / cu;
    const bool full = S == 1 && W >= cu;
    double tile_us = f.nw == 4 ? 1.149 : f.cp == 2 ? 1.082 : 1.298;
    if (full) tile_us += f.nw == 4 ? 0.128 : f.cp == 2 ? 0.311 : 0.556;
    double t = 4.868 + (double)rounds * (1.263 + (double)ct * tile_us);
    if (S > 1) t += 6.210 + 0.331 * (double)B * NL * (double)S * (kDim * 4) * 1e-6;
    return t;
}

// Launch form of a 16-bit launch of S key splits of `chunk` keys each: the
// cheapest by h16_cost.
static H16Form h16_form_for(int B, int NL, int NI, int S, int chunk, int cu) {
    const long long ct = NI > 0 ? ((long long)std::min(chunk, NI) + 31) / 32 : 0;
    H16Form best = kH16Forms[0];
    double best_t = -1.0;
    for (const H16Form& f : kH16Forms) {
        const double t = h16_cost(B, NL, cu, f, S, ct);
        if (best_t < 0.0 || t < best_t) best_t = t, best = f;
    }
    return best;
}

// Launch plan of the 16-bit entry points: the (form, S) pair of least
// h16_cost, S up to min(tiles, cu) whole 32-key tiles per split.  The last
// plan is cached per thread.
static void wmma_plan(int B, int NL, int NI, int cu, H16Form* form, int* S) {
    thread_local int key[4] = {-1, -1, -1, -1}, val[3] = {8, 1, 1};
    if (key[0] == B && key[1] == NL && key[2] == NI && key[3] == cu) {
        *form = {val[0], val[1]};
        *S = val[2];
        return;
    }
    H16Form bf = kH16Forms[0];
    int bs = 1;
    const long long tiles = NI > 0 ? ((long long)NI + 31) / 32 : 0;
    if (B > 0 && NL > 0 && tiles > 0) {
        double best_t = -1.0;
        const long long smax = std::min<long long>(tiles, cu);
        for (const H16Form& f : kH16Forms) {
            for (long long s = 1; s <= smax; ++s) {
                const long long ct = (tiles + s - 1) / s;
                if ((tiles + ct - 1) / ct != s) continue;  // same chunks as a smaller s
                const double t = h16_cost(B, NL, cu, f, s, ct);
                if (best_t < 0.0 || t < best_t) best_t = t, bf = f, bs = (int)s;
            }
        }
    }
    key[0] = B, key[1] = NL, key[2] = NI, key[3] = cu;
    val[0] = bf.nw, val[1] = bf.cp, val[2] = bs;
    *form = bf;
    *S = bs;
}

// Library-workspace split launch shared by the fp32 and 16-bit entry points.
struct SplitScratch {
    float* po;
    float* pm;
    float* pl;
};

static bool split_scratch(SplitScratch* s, WorkspaceLease& lease, int B, int NL, int S,
                          hipStream_t stream) {
    const size_t rows = (size_t)B * NL;
    const size_t po_bytes = rows * S * kDim * sizeof(float);
    const size_t ml_bytes = rows * S * sizeof(float);
    char* ws = (char*)lease.acquire(po_bytes + 2 * ml_bytes + 256, stream);
    if (!ws) return false;
    s->po = (float*)ws;
    s->pm = (float*)(ws + po_bytes);
    s->pl = (float*)(ws + po_bytes + ml_bytes);
    return true;
}

}  // namespace xattn

using namespace xattn;

extern "C" {

int xattn_get_last_error(void) {
    const int e = g_err;
    g_err = XATTN_OK;
    return e;
}

const char* xattn_get_last_error_string(void) { return g_msg; }

int xattn_device_info(int device, int* cu_count, int* lds_bytes_per_block) {
    int cu = 0, lds = 0;
    hipError_t e = hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return (int)e;
    e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
    if (e != hipSuccess) return (int)e;
    if (cu_count) *cu_count = cu;
    if (lds_bytes_per_block) *lds_bytes_per_block = lds;
    return 0;
}

int xattn_device_arch(int device, char* arch, int arch_len, int* clock_khz) {
    hipDeviceProp_t prop;
    const hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return (int)e;
    if (arch && arch_len > 0) {
        strncpy(arch, prop.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    if (clock_khz) *clock_khz = prop.clockRate;
    return 0;
}

int xattn_xcd_remap(int block, int num_blocks) { return xcd_remap(block, num_blocks); }

int xattn_optimized_num_splits(int batch_size, int N_latent, int N_input, int cu_count) {
    return optimized_num_splits(batch_size, N_latent, N_input, cu_count);
}

int xattn_plan_splits(int batch_size, int N_latent, int N_input, int cu_count,
                      int latents_per_workgroup, int keys_per_tile) {
    if (latents_per_workgroup < 1 || keys_per_tile < 1 || cu_count < 1) return 1;
    return plan_splits(batch_size, N_latent, N_input, cu_count, latents_per_workgroup,
                       keys_per_tile);
}

void xattn_f32_plan(int batch_size, int N_latent, int N_input, int cu_count,
                    int* latents_per_workgroup, int* num_splits) {
    int ds = 1, S = 1;
    f32_plan(batch_size, N_latent, N_input, cu_count < 1 ? 1 : cu_count, &ds, &S);
    if (latents_per_workgroup) *latents_per_workgroup = 64 / ds;
    if (num_splits) *num_splits = S;
}

int xattn_f32_split_latents(int batch_size, int N_latent, int N_input, int num_splits,
                            int cu_count) {
    if (batch_size < 1 || N_latent < 1 || num_splits < 1) return 64;
    const int chunk = (int)(((long long)std::max(N_input, 0) + num_splits - 1) / num_splits);
    return 64 / f32_parts(batch_size, N_latent, N_input, num_splits, chunk,
                          cu_count < 1 ? 1 : cu_count);
}

int xattn_wmma_split_latents(int batch_size, int N_latent, int N_input, int num_splits,
                             int cu_count) {
    if (batch_size < 1 || N_latent < 1 || num_splits < 1) return 64;
    long long chunk = ((long long)std::max(N_input, 0) + num_splits - 1) / num_splits;
    chunk = (chunk + 15) / 16 * 16;
    return 8 * h16_form_for(batch_size, N_latent, N_input, num_splits, (int)chunk,
                            cu_count < 1 ? 1 : cu_count).nw;
}

void xattn_wmma_plan(int batch_size, int N_latent, int N_input, int cu_count,
                     int* latents_per_workgroup, int* num_splits) {
    H16Form f;
    int S = 1;
    wmma_plan(batch_size, N_latent, N_input, cu_count < 1 ? 1 : cu_count, &f, &S);
    if (latents_per_workgroup) *latents_per_workgroup = 8 * f.nw;
    if (num_splits) *num_splits = S;
}

void xattn_wmma_plan_ex(int batch_size, int N_latent, int N_input, int cu_count,
                        int* latents_per_workgroup, int* column_parts, int* num_splits) {
    H16Form f;
    int S = 1;
    wmma_plan(batch_size, N_latent, N_input, cu_count < 1 ? 1 : cu_count, &f, &S);
    if (latents_per_workgroup) *latents_per_workgroup = 8 * f.nw;
    if (column_parts) *column_parts = f.cp;
    if (num_splits) *num_splits = S;
}

int xattn_lse_combine_parts(int rows, int num_splits, int cu_count) {
    return lse_combine_parts(rows, num_splits, cu_count < 1 ? 1 : cu_count);
}

void xattn_lse_combine(const float* po, const float* pm, const float* pl, float* output,
                       int rows, int num_splits, int column_parts, hipStream_t stream) {
    const char* who = "xattn_lse_combine";
    if (rows < 0) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: negative row count %d", who, rows);
        return;
    }
    if (!validate_splits(who, po, pm, pl, 1, rows, num_splits)) return;
    if (rows > 0 && !output) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: NULL output", who);
        return;
    }
    if (column_parts != 0 && column_parts != 1 && column_parts != 2 && column_parts != 4) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: column_parts %d (0, 1, 2 or 4)", who,
                  column_parts);
        return;
    }
    if (!validate_aligned16(who, po, po, po, output, po)) return;
    if ((long long)rows * num_splits > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: rows*num_splits too large", who);
        return;
    }
    launch_lse_combine(po, pm, pl, output, rows, num_splits, stream, column_parts);
}

void launch_naive_kernel(const float* Q, const float* K, const float* V, float* output,
                         int batch_size, int N_latent, int N_input, int dim, hipStream_t stream) {
    const char* who = "launch_naive_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (dim < 1) {
        set_error(XATTN_ERR_UNSUPPORTED, "%s: dim=%d must be >= 1", who, dim);
        return;
    }
    launch_naive(Q, K, V, output, batch_size, N_latent, N_input, dim, stream);
}

static bool validate_rung_dim(const char* who, int dim) {
    if (dim < 1 || dim > kDim) {
        set_error(XATTN_ERR_UNSUPPORTED, "%s: dim=%d outside [1, %d]", who, dim, kDim);
        return false;
    }
    return true;
}

void launch_parallel_kernel(const float* Q, const float* K, const float* V, float* output,
                            int batch_size, int N_latent, int N_input, int dim,
                            hipStream_t stream) {
    const char* who = "launch_parallel_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_rung_dim(who, dim)) return;
    const long long lds = (4LL * N_input + 4) * 4;
    if (lds > device_max_lds()) {
        set_error(XATTN_ERR_UNSUPPORTED,
                  "%s: score row needs %lld B of LDS for N_input=%d, device allows %d", who, lds,
                  N_input, device_max_lds());
        return;
    }
    launch_warp(Q, K, V, output, batch_size, N_latent, N_input, dim, stream);
}

void launch_tiled_kernel(const float* Q, const float* K, const float* V, float* output,
                         int batch_size, int N_latent, int N_input, int dim, hipStream_t stream) {
    const char* who = "launch_tiled_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_rung_dim(who, dim)) return;
    launch_tiled(Q, K, V, output, batch_size, N_latent, N_input, dim, stream);
}

// An fp32 launch with a given plan: ds wavefronts per 16-latent block
// (64 / ds latents per workgroup), S key splits of whole 16-key tiles
// (partials in the stream's library workspace when S > 1).
static void optimized_run(const float* Q, const float* K, const float* V, float* output,
                          int batch_size, int N_latent, int N_input, int ds, int S,
                          hipStream_t stream) {
    if (S <= 1) {
        launch_flash_f32(ds, Q, K, V, output, nullptr, nullptr, nullptr, batch_size, N_latent,
                         N_input, 1, N_input, stream);
        return;
    }
    const int tiles = (N_input + 15) / 16;
    const int chunk = ((tiles + S - 1) / S) * 16;
    SplitScratch sc;
    WorkspaceLease lease;
    if (!split_scratch(&sc, lease, batch_size, N_latent, S, stream)) return;
    if (launch_flash_f32(ds, Q, K, V, nullptr, sc.po, sc.pm, sc.pl, batch_size, N_latent,
                         N_input, S, chunk, stream))
        launch_lse_combine(sc.po, sc.pm, sc.pl, output, batch_size * N_latent, S, stream);
    lease.release();
}

void launch_optimized_kernel(const float* Q, const float* K, const float* V, float* output,
                             int batch_size, int N_latent, int N_input, int dim,
                             hipStream_t stream) {
    const char* who = "launch_optimized_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_aligned16(who, Q, K, V, output, nullptr)) return;
    if (batch_size == 0 || N_latent == 0) return;
    int ds = 1, S = 1;
    f32_plan(batch_size, N_latent, N_input, device_cu_count(), &ds, &S);
    optimized_run(Q, K, V, output, batch_size, N_latent, N_input, ds, S, stream);
}

void launch_optimized_plan_kernel(const float* Q, const float* K, const float* V,
                                  float* output, int batch_size, int N_latent, int N_input,
                                  int dim, int latents_per_workgroup, int num_splits,
                                  hipStream_t stream) {
    const char* who = "launch_optimized_plan_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_aligned16(who, Q, K, V, output, nullptr)) return;
    if (latents_per_workgroup != 64 && latents_per_workgroup != 32 &&
        latents_per_workgroup != 16) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: %d latents per workgroup (64, 32 or 16)", who,
                  latents_per_workgroup);
        return;
    }
    const int tiles = (N_input + 15) / 16;
    if (num_splits < 1 || num_splits > std::max(tiles, 1)) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: num_splits %d outside 1..%d (16-key tiles)", who,
                  num_splits, std::max(tiles, 1));
        return;
    }
    if (batch_size == 0 || N_latent == 0) return;
    optimized_run(Q, K, V, output, batch_size, N_latent, N_input, 64 / latents_per_workgroup,
                  N_input == 0 ? 1 : num_splits, stream);
}

int xattn_noalloc_prepare(int device) {
    if (device < 0 || device >= 256) return (int)hipErrorInvalidDevice;
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e != hipSuccess) return (int)e;
    if ((e = hipSetDevice(device)) != hipSuccess) return (int)e;
    int rc;
    {
        std::lock_guard<std::mutex> lk(g_noalloc[device].mu);
        rc = noalloc_setup(device, "xattn_noalloc_prepare");
    }
    e = hipSetDevice(prev);
    return rc != 0 ? rc : (int)e;
}

void launch_optimized_kernel_noalloc(const float* Q, const float* K, const float* V,
                                     float* output, int batch_size, int N_latent, int N_input,
                                     int dim, hipStream_t stream) {
    const char* who = "launch_optimized_kernel_noalloc";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_aligned16(who, Q, K, V, output, nullptr)) return;
    if (batch_size == 0 || N_latent == 0) return;
    // The plan of launch_optimized_kernel, so both give identical results.
    int ds = 1, S = 1;
    f32_plan(batch_size, N_latent, N_input, device_cu_count(), &ds, &S);
    if (S <= 1) {
        launch_flash_f32(ds, Q, K, V, output, nullptr, nullptr, nullptr, batch_size, N_latent,
                         N_input, 1, N_input, stream);
        return;
    }
    const size_t rows = (size_t)batch_size * N_latent;
    const size_t po_bytes = rows * S * kDim * sizeof(float);
    const size_t ml_bytes = rows * S * sizeof(float);
    if (po_bytes + 2 * ml_bytes > kNoallocScratchBytes) {
        set_error(XATTN_ERR_UNSUPPORTED,
                  "%s: the plan for B=%d N_latent=%d N_input=%d takes %d key splits, whose "
                  "partials need %zu bytes; the static scratch holds %zu (use "
                  "launch_splitk_kernel with caller-owned scratch)",
                  who, batch_size, N_latent, N_input, S, po_bytes + 2 * ml_bytes,
                  kNoallocScratchBytes);
        return;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) {
        (void)hipGetLastError();
        set_error(XATTN_ERR_LAUNCH, "%s: no current device", who);
        return;
    }
    const bool capturing = stream_capturing(stream);
    NoallocDevice& nd = g_noalloc[dev];
    std::lock_guard<std::mutex> lk(nd.mu);
    if (!nd.ptr || !nd.done) {
        if (capturing) {
            set_error(XATTN_ERR_CAPTURE,
                      "%s: first split call on device %d inside a stream capture; call "
                      "xattn_noalloc_prepare(%d) (or make one call) before capturing",
                      who, dev, dev);
            return;
        }
        if (noalloc_setup(dev, who) != 0) return;
    }
    if (!capturing && nd.recorded && hipStreamWaitEvent(stream, nd.done, 0) != hipSuccess) {
        const hipError_t e = hipGetLastError();
        set_error(XATTN_ERR_LAUNCH, "%s: hipStreamWaitEvent failed: %s", who,
                  hipGetErrorString(e));
        return;
    }
    char* base = (char*)nd.ptr;
    float* po = (float*)base;
    float* pm = (float*)(base + po_bytes);
    float* pl = (float*)(base + po_bytes + ml_bytes);
    const int tiles = (N_input + 15) / 16;
    const int chunk = ((tiles + S - 1) / S) * 16;
    if (!launch_flash_f32(ds, Q, K, V, nullptr, po, pm, pl, batch_size, N_latent, N_input, S,
                          chunk, stream))
        return;
    if (!launch_lse_combine(po, pm, pl, output, (int)rows, S, stream)) return;
    if (!capturing) {
        if (hipEventRecord(nd.done, stream) != hipSuccess) {
            const hipError_t e = hipGetLastError();
            set_error(XATTN_ERR_LAUNCH, "%s: hipEventRecord failed: %s", who,
                      hipGetErrorString(e));
            return;
        }
        nd.recorded = true;
    }
}

void launch_splitk_kernel(const float* Q, const float* K, const float* V, float* output,
                          float* po, float* pm, float* pl, int batch_size, int N_latent,
                          int N_input, int dim, int num_splits, hipStream_t stream) {
    const char* who = "launch_splitk_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_splits(who, po, pm, pl, batch_size, N_latent, num_splits)) return;
    if (!validate_aligned16(who, Q, K, V, output, po)) return;
    if (batch_size == 0 || N_latent == 0) return;
    if ((long long)batch_size * N_latent * num_splits > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: B*NL*num_splits too large", who);
        return;
    }
    // kernel_splitk.cu:59: chunk = ceil(NI / S)
    const int chunk = (int)(((long long)N_input + num_splits - 1) / num_splits);
    const int ds = f32_parts(batch_size, N_latent, N_input, num_splits, chunk,
                             device_cu_count());
    if (!launch_flash_f32(ds, Q, K, V, nullptr, po, pm, pl, batch_size, N_latent, N_input,
                          num_splits, chunk, stream))
        return;
    launch_lse_combine(po, pm, pl, output, batch_size * N_latent, num_splits, stream);
}

// A 16-bit launch with a given plan: form f, S key splits of whole 32-key
// tiles (partials in the stream's library workspace when S > 1).
static void wmma_run(bool bf16, const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                     float* output, int batch_size, int N_latent, int N_input, H16Form f, int S,
                     hipStream_t stream) {
    if (S <= 1) {
        launch_flash16(bf16, f.nw, f.cp, Q, K, V, output, nullptr, nullptr, nullptr, batch_size,
                       N_latent, N_input, 1, N_input, stream);
        return;
    }
    const int tiles = (N_input + 31) / 32;
    const int chunk = ((tiles + S - 1) / S) * 32;
    SplitScratch sc;
    WorkspaceLease lease;
    if (!split_scratch(&sc, lease, batch_size, N_latent, S, stream)) return;
    if (launch_flash16(bf16, f.nw, f.cp, Q, K, V, nullptr, sc.po, sc.pm, sc.pl, batch_size,
                       N_latent, N_input, S, chunk, stream))
        launch_lse_combine(sc.po, sc.pm, sc.pl, output, batch_size * N_latent, S, stream);
    lease.release();
}

static void wmma_common(bool bf16, const char* who, const uint16_t* Q, const uint16_t* K,
                        const uint16_t* V, float* output, int batch_size, int N_latent,
                        int N_input, int dim, hipStream_t stream) {
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_aligned16(who, Q, K, V, output, nullptr)) return;
    if (batch_size == 0 || N_latent == 0) return;
    H16Form f;
    int S = 1;
    wmma_plan(batch_size, N_latent, N_input, device_cu_count(), &f, &S);
    wmma_run(bf16, Q, K, V, output, batch_size, N_latent, N_input, f, S, stream);
}

static void wmma_splitk_common(bool bf16, const char* who, const uint16_t* Q, const uint16_t* K,
                               const uint16_t* V, float* output, float* po, float* pm,
                               float* pl, int batch_size, int N_latent, int N_input, int dim,
                               int num_splits, hipStream_t stream) {
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_splits(who, po, pm, pl, batch_size, N_latent, num_splits)) return;
    if (!validate_aligned16(who, Q, K, V, output, po)) return;
    if (batch_size == 0 || N_latent == 0) return;
    if ((long long)batch_size * N_latent * num_splits > 0x7fffffffLL) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: B*NL*num_splits too large", who);
        return;
    }
    // kernel_wmma_splitk.cu:52: chunk = ceil(NI / S) rounded up to a multiple of 16
    long long chunk = ((long long)N_input + num_splits - 1) / num_splits;
    chunk = (chunk + 15) / 16 * 16;
    const H16Form f = h16_form_for(batch_size, N_latent, N_input, num_splits, (int)chunk,
                                   device_cu_count());
    if (!launch_flash16(bf16, f.nw, f.cp, Q, K, V, nullptr, po, pm, pl, batch_size, N_latent,
                        N_input, num_splits, (int)chunk, stream))
        return;
    launch_lse_combine(po, pm, pl, output, batch_size * N_latent, num_splits, stream);
}

void launch_wmma_kernel(const uint16_t* Q, const uint16_t* K, const uint16_t* V, float* output,
                        int batch_size, int N_latent, int N_input, int dim,
                        hipStream_t stream) {
    wmma_common(false, "launch_wmma_kernel", Q, K, V, output, batch_size, N_latent, N_input,
                dim, stream);
}

void launch_wmma_bf16_kernel(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                             float* output, int batch_size, int N_latent, int N_input, int dim,
                             hipStream_t stream) {
    wmma_common(true, "launch_wmma_bf16_kernel", Q, K, V, output, batch_size, N_latent,
                N_input, dim, stream);
}

void launch_wmma_plan_kernel(int bf16, const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                             float* output, int batch_size, int N_latent, int N_input, int dim,
                             int latents_per_workgroup, int column_parts, int num_splits,
                             hipStream_t stream) {
    const char* who = "launch_wmma_plan_kernel";
    if (!validate_common(who, Q, K, V, output, batch_size, N_latent, N_input, dim)) return;
    if (!validate_dim768(who, dim)) return;
    if (!validate_aligned16(who, Q, K, V, output, nullptr)) return;
    const bool form_ok = (latents_per_workgroup == 64 && (column_parts == 1 || column_parts == 2)) ||
                         (latents_per_workgroup == 32 && column_parts == 1);
    if (!form_ok) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: no form of %d latents per workgroup in %d column "
                  "parts (64 in 1 or 2, 32 in 1)", who, latents_per_workgroup, column_parts);
        return;
    }
    const int tiles = (N_input + 31) / 32;
    if (num_splits < 1 || num_splits > std::max(tiles, 1)) {
        set_error(XATTN_ERR_INVALID_VALUE, "%s: num_splits %d outside 1..%d (32-key tiles)", who,
                  num_splits, std::max(tiles, 1));
        return;
    }
    if (batch_size == 0 || N_latent == 0) return;
    wmma_run(bf16 != 0, Q, K, V, output, batch_size, N_latent, N_input,
             H16Form{latents_per_workgroup / 8, column_parts}, N_input == 0 ? 1 : num_splits,
             stream);
}

void launch_wmma_splitk_kernel(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                               float* output, float* po, float* pm, float* pl, int batch_size,
                               int N_latent, int N_input, int dim, int num_splits,
                               hipStream_t stream) {
    wmma_splitk_common(false, "launch_wmma_splitk_kernel", Q, K, V, output, po, pm, pl,
                       batch_size, N_latent, N_input, dim, num_splits, stream);
}

void launch_wmma_splitk_bf16_kernel(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                    float* output, float* po, float* pm, float* pl,
                                    int batch_size, int N_latent, int N_input, int dim,
                                    int num_splits, hipStream_t stream) {
    wmma_splitk_common(true, "launch_wmma_splitk_bf16_kernel", Q, K, V, output, po, pm, pl,
                       batch_size, N_latent, N_input, dim, num_splits, stream);
}

}  // extern "C"
