/*
 * xattn.h -- C ABI of kernels.so, the MI355X (gfx950) fused cross-attention
 * library.  O = softmax(Q K^T / sqrt(dim)) V, single head.
 *
 * Layouts (all row-major, contiguous, device pointers):
 *   Q   [batch_size, N_latent, dim]
 *   K,V [batch_size, N_input,  dim]
 *   out [batch_size, N_latent, dim]  (always fp32)
 *
 * The first seven entry points keep the names, argument order and C types of
 * the reference's kernels.so so that its ctypes bindings
 * (cuda_wrappers.py:83-175) bind unchanged; cudaStream_t becomes hipStream_t
 * (both opaque pointers; NULL is the null stream).
 *
 * Error behaviour: launchers return void and only enqueue work on `stream`;
 * none calls hipDeviceSynchronize, hipStreamSynchronize, hipFree or any
 * other synchronising function.  A launch the hardware rejects is reported
 * through hipGetLastError() as in the reference.  In addition, arguments a
 * kernel cannot run with (dim other than the kernel's supported dim, negative
 * sizes, num_splits < 1, NULL data pointers with non-zero sizes) are refused
 * before anything is launched and recorded for xattn_get_last_error().
 *
 * Allocation: every entry point works on caller-owned buffers, except that
 * launch_optimized_kernel, launch_wmma_kernel and launch_wmma_bf16_kernel,
 * when their plan splits the keys, keep the split partials in a
 * library-owned workspace, one per (device, stream; and host thread for
 * hipStreamPerThread, which names a different stream in each thread).  It
 * is allocated with hipMalloc on the first such launch on a stream and
 * replaced (hipMalloc of at least twice the size; the old block is kept,
 * never freed, until the process exits) when a later launch on that
 * stream needs more.  Launches on different streams never share a
 * workspace.  While `stream` is capturing a graph, such a launch proceeds
 * only if the stream's workspace is already large enough (otherwise it is
 * refused with XATTN_ERR_CAPTURE and nothing is enqueued), and the block
 * then belongs to the graph: the next launch on that stream outside capture
 * takes a fresh block, so replays of the graph, on any stream, never share
 * partials with later eager launches.  Two graphs captured on one stream
 * with no eager split launch on it between the captures share a block:
 * their replays must not overlap.  launch_splitk_kernel and its 16-bit
 * twins never allocate.
 */
#ifndef XATTN_H
#define XATTN_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp32 ladder ------------------------------------------------------- */

/* Replaces launch_naive_kernel, kernel_naive.cu:68-78.
 * One thread per output element; any dim >= 1, any N_input. */
void launch_naive_kernel(const float* Q, const float* K, const float* V,
                         float* output, int batch_size, int N_latent,
                         int N_input, int dim, hipStream_t stream);

/* Replaces launch_parallel_kernel, kernel_warp_parallel.cu:113-123.
 * One 64-lane wavefront per latent; the full score row lives in LDS,
 * (4 * N_input + 4) * 4 bytes per workgroup (refused when that exceeds the
 * device's per-workgroup LDS).  1 <= dim <= 768. */
void launch_parallel_kernel(const float* Q, const float* K, const float* V,
                            float* output, int batch_size, int N_latent,
                            int N_input, int dim, hipStream_t stream);

/* Replaces launch_tiled_kernel, kernel_tiled.cu:169-179.
 * 16-key K tiles staged in LDS, online softmax.  1 <= dim <= 768. */
void launch_tiled_kernel(const float* Q, const float* K, const float* V,
                         float* output, int batch_size, int N_latent,
                         int N_input, int dim, hipStream_t stream);

/* Replaces launch_optimized_kernel, kernel_vectorized.cu:198-208 (the
 * 'vectorized' entry of cuda_wrappers.py:352-357).  Both GEMMs on fp32 MFMA
 * (v_mfma_f32_16x16x4_f32), online softmax in registers.  dim == 768.
 * Workgroups of 64, 32 or 16 latents and, where those cannot fill the device
 * cheaply, key splits merged by a log-sum-exp pass, as xattn_f32_plan
 * reports; split partials live in the stream's library-owned workspace (see
 * "Allocation" above). */
void launch_optimized_kernel(const float* Q, const float* K, const float* V,
                             float* output, int batch_size, int N_latent,
                             int N_input, int dim, hipStream_t stream);

/* No reference counterpart: launch_optimized_kernel with the caller's
 * launch plan instead of xattn_f32_plan's, for plan tuning and for
 * measuring the planner's cost model: latents_per_workgroup 64, 32 or 16,
 * num_splits key splits of whole 16-key tiles (1 .. ceil(N_input / 16);
 * split partials in the stream's library workspace).  Any other plan is
 * refused with XATTN_ERR_INVALID_VALUE before anything is enqueued.  Results
 * match launch_optimized_kernel's within the fp32 tolerance (different
 * splits and workgroup sizes sum in different orders). */
void launch_optimized_plan_kernel(const float* Q, const float* K, const float* V,
                                  float* output, int batch_size, int N_latent,
                                  int N_input, int dim, int latents_per_workgroup,
                                  int num_splits, hipStream_t stream);

/* No counterpart in the reference: launch_optimized_kernel for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same plan, kernels and
 * results, bit for bit; split partials go to a static scratch array of
 * 64 MiB per device instead of the stream's workspace, and the call never
 * allocates or frees device memory.  A plan whose partials
 * (batch_size * N_latent * splits * (dim + 2) * 4 bytes, splits from
 * xattn_f32_plan) exceed 64 MiB is refused with XATTN_ERR_UNSUPPORTED.
 * All calls on one GPU share its scratch.  Outside stream capture, calls
 * whose plan splits the keys are ordered on the GPU by a library event
 * (each call's stream waits for the previous split call's merge; no host
 * wait), so calls from several streams or host threads do not race.  A
 * call made under capture is not ordered against others: a replay of that
 * graph must not overlap another split call on the same GPU.  The first
 * split call on a device resolves the scratch address and creates the
 * event (xattn_noalloc_prepare); made under capture it is refused with
 * XATTN_ERR_CAPTURE instead. */
void launch_optimized_kernel_noalloc(const float* Q, const float* K, const float* V,
                                     float* output, int batch_size, int N_latent,
                                     int N_input, int dim, hipStream_t stream);
/* No counterpart in the reference, for the callers of
 * launch_optimized_kernel_noalloc: resolve device `device`'s scratch
 * address and create its ordering event now (idempotent), e.g. before
 * capturing a graph that calls it.  Allocates no device memory.  Returns a
 * hipError_t value (0 on success); the current device is left unchanged. */
int xattn_noalloc_prepare(int device);

/* ---- split-K (key-parallel) fp32 -------------------------------------- */

/* Replaces launch_splitk_kernel, kernel_splitk.cu:238-251.
 * Split s covers keys [s*chunk, min((s+1)*chunk, N_input)) with
 * chunk = ceil(N_input / num_splits).  Caller-owned scratch:
 *   po [batch_size, N_latent, num_splits, dim]  sum exp(s - pm) * V
 *   pm [batch_size, N_latent, num_splits]       max score of the split
 *   pl [batch_size, N_latent, num_splits]       sum exp(s - pm)
 * An empty split holds (pm, pl, po) = (-FLT_MAX, 0, 0).  dim == 768. */
void launch_splitk_kernel(const float* Q, const float* K, const float* V,
                          float* output, float* po, float* pm, float* pl,
                          int batch_size, int N_latent, int N_input, int dim,
                          int num_splits, hipStream_t stream);

/* No reference counterpart (the merge pass of launch_splitk_kernel on its
 * own, kernel_splitk.cu:186-236): output[r, :] = sum_s exp(pm[r,s] - M)
 * po[r,s,:] / (sum_s exp(pm[r,s] - M) pl[r,s] + 1e-6), M = max_s pm[r,s],
 * for rows r < rows (a row is one (batch, latent) pair; the layouts of
 * launch_splitk_kernel's scratch with batch_size * N_latent = rows), dim
 * 768; splits with pm = -FLT_MAX are skipped.  column_parts: workgroups
 * per row, 1, 2 or 4, or 0 for the library's choice
 * (xattn_lse_combine_parts); every choice gives bit-identical output.
 * Refused with XATTN_ERR_INVALID_VALUE for other values, num_splits < 1 or
 * NULL pointers with rows > 0. */
void xattn_lse_combine(const float* po, const float* pm, const float* pl,
                       float* output, int rows, int num_splits,
                       int column_parts, hipStream_t stream);
/* Workgroups per row the merge uses for rows rows of num_splits splits on a
 * device of cu_count compute units (no reference counterpart). */
int xattn_lse_combine_parts(int rows, int num_splits, int cu_count);

/* ---- fp16 / bf16 MFMA (fp32 accumulate, fp32 softmax, fp32 output) ----- */

/* Replaces launch_wmma_kernel, kernel_wmma.cu:139-154.  Q, K, V are IEEE
 * binary16 bit patterns; Q is pre-scaled by 1/sqrt(dim) by the caller
 * (cuda_wrappers.py:635-640).  dim == 768.  Launch shape and internal key
 * splits (stream's library workspace, as above) as xattn_wmma_plan reports. */
void launch_wmma_kernel(const uint16_t* Q, const uint16_t* K,
                        const uint16_t* V, float* output, int batch_size,
                        int N_latent, int N_input, int dim,
                        hipStream_t stream);

/* Replaces launch_wmma_splitk_kernel, kernel_wmma_splitk.cu:201-219.
 * fp16 inputs as launch_wmma_kernel; splits as launch_splitk_kernel except
 * that chunk is rounded up to a multiple of 16 (kernel_wmma_splitk.cu:52). */
void launch_wmma_splitk_kernel(const uint16_t* Q, const uint16_t* K,
                               const uint16_t* V, float* output, float* po,
                               float* pm, float* pl, int batch_size,
                               int N_latent, int N_input, int dim,
                               int num_splits, hipStream_t stream);

/* Additive (no reference counterpart): bfloat16 twins of the two entry
 * points above, same contract with bf16 bit patterns for Q, K, V. */
void launch_wmma_bf16_kernel(const uint16_t* Q, const uint16_t* K,
                             const uint16_t* V, float* output, int batch_size,
                             int N_latent, int N_input, int dim,
                             hipStream_t stream);
void launch_wmma_splitk_bf16_kernel(const uint16_t* Q, const uint16_t* K,
                                    const uint16_t* V, float* output,
                                    float* po, float* pm, float* pl,
                                    int batch_size, int N_latent, int N_input,
                                    int dim, int num_splits,
                                    hipStream_t stream);

/* No reference counterpart: launch_wmma_kernel (bf16 == 0) or
 * launch_wmma_bf16_kernel (bf16 != 0) with the caller's launch plan instead
 * of xattn_wmma_plan's, for plan tuning and for measuring the planner's cost
 * model: latents_per_workgroup 64 (column_parts 1 or 2) or 32 (column_parts
 * 1), num_splits key splits of whole 32-key tiles (1 .. ceil(N_input / 32);
 * split partials in the stream's library workspace, as above).  Any other
 * plan is refused with XATTN_ERR_INVALID_VALUE before anything is
 * enqueued.  Results match the planned entry points' within the 16-bit
 * tolerance (different splits round differently). */
void launch_wmma_plan_kernel(int bf16, const uint16_t* Q, const uint16_t* K,
                             const uint16_t* V, float* output, int batch_size,
                             int N_latent, int N_input, int dim,
                             int latents_per_workgroup, int column_parts,
                             int num_splits, hipStream_t stream);

/* ---- library status / device queries (additive) ----------------------- */

enum {
    XATTN_OK = 0,
    XATTN_ERR_INVALID_VALUE = 1, /* negative size, NULL pointer, bad splits */
    XATTN_ERR_UNSUPPORTED = 2,   /* shape the kernel is not built for      */
    XATTN_ERR_LAUNCH = 3,        /* the HIP runtime rejected the launch     */
    XATTN_ERR_ALLOC = 4,         /* workspace allocation failed             */
    XATTN_ERR_CAPTURE = 5        /* would allocate while the stream captures */
};

/* Returns the first error recorded on this host thread since the last call,
 * and clears it (like hipGetLastError). */
int xattn_get_last_error(void);
/* Message of the error xattn_get_last_error() returns (or last returned):
 * the first one recorded since the code was last read; "" if none. */
const char* xattn_get_last_error_string(void);

/* Replaces the ordinal-based cudaDeviceGetAttribute query of
 * cuda_wrappers.py:187-194: compute-unit count and maximum LDS bytes one
 * workgroup may use.  Returns a hipError_t value (0 on success). */
int xattn_device_info(int device, int* cu_count, int* lds_bytes_per_block);

/* Additive (no reference counterpart; the reference names its GPU from
 * nvidia-smi, experiments/gpu_specs.py:60-109): the device's architecture
 * name as the HIP runtime reports it (e.g. "gfx950:sramecc+:xnack-"), NUL
 * terminated within arch_len bytes, and its peak engine clock in kHz.  The
 * product name alone does not identify the part on hosts without libdrm's
 * ASIC table.  Returns a hipError_t value (0 on success). */
int xattn_device_arch(int device, char* arch, int arch_len, int* clock_khz);

/* Host copies of the launch planning, for inspection and tests. */
int xattn_xcd_remap(int block, int num_blocks);
/* Number of key splits launch_optimized_kernel uses internally. */
int xattn_optimized_num_splits(int batch_size, int N_latent, int N_input,
                               int cu_count);
/* Key splits that make batch_size * ceil(N_latent / latents_per_workgroup)
 * workgroups fill cu_count compute units once, each split a whole number of
 * keys_per_tile-key tiles.  The fp32 kernel uses 64, 32 or 16 latents per
 * workgroup (xattn_f32_plan), the 16-bit one 64 or 32 (xattn_wmma_plan);
 * tiles are 16 keys (fp32) and
 * 32 keys (fp16/bf16).  Replaces the
 * block-count heuristic of cuda_wrappers.py:456-467 for these kernels. */
int xattn_plan_splits(int batch_size, int N_latent, int N_input, int cu_count,
                      int latents_per_workgroup, int keys_per_tile);
/* Launch shape launch_optimized_kernel uses (no reference counterpart):
 * latents per workgroup (64, or 32 / 16 when two / four wavefronts share a
 * 16-latent block, each holding 384 / 192 of the 768 columns) and key splits
 * (16-key tiles, whole tiles per split), chosen by a cost model of the fp32
 * kernel and the merge fitted to MI355X launches: larger workgroups cost
 * less per FLOP, smaller ones and splits fill the device at small
 * batch_size * N_latent, splits add the partials' round trip to memory. */
void xattn_f32_plan(int batch_size, int N_latent, int N_input, int cu_count,
                    int* latents_per_workgroup, int* num_splits);
/* Latents per workgroup launch_splitk_kernel uses for num_splits key splits
 * of ceil(N_input / num_splits) keys (64, 32 or 16, by the cost model of
 * xattn_f32_plan; no reference counterpart). */
int xattn_f32_split_latents(int batch_size, int N_latent, int N_input, int num_splits,
                            int cu_count);
/* Launch shape launch_wmma_kernel / launch_wmma_bf16_kernel use (no
 * reference counterpart): latents per workgroup (64 on 8 wavefronts, or 32
 * on 4) and key splits (32-key tiles, whole tiles per split), chosen by a
 * cost model of the 16-bit kernel and the merge fitted to MI355X launches.
 * Writes the latents per workgroup and the number of key splits (the column
 * parts of 64-latent plans: xattn_wmma_plan_ex). */
void xattn_wmma_plan(int batch_size, int N_latent, int N_input, int cu_count,
                     int* latents_per_workgroup, int* num_splits);
/* The same plan with its third coordinate (no reference counterpart):
 * column_parts 2 means each row block of 64 latents runs as two workgroups,
 * one per half of the 768 output columns, both computing the block's scores
 * over all of dim. */
void xattn_wmma_plan_ex(int batch_size, int N_latent, int N_input, int cu_count,
                        int* latents_per_workgroup, int* column_parts,
                        int* num_splits);
/* Latents per workgroup launch_wmma_splitk_kernel and its bf16 twin use for
 * num_splits key splits (64 or 32, by the cost model of xattn_wmma_plan; no
 * reference counterpart). */
int xattn_wmma_split_latents(int batch_size, int N_latent, int N_input, int num_splits,
                             int cu_count);

#ifdef __cplusplus
}
#endif

#endif /* XATTN_H */
