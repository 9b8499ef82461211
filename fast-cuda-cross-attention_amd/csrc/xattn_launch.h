// Internal (non-exported) launch helpers shared between translation units.
#pragma once

#include <hip/hip_runtime.h>

namespace xattn {

int device_cu_count();
int device_max_lds();
int optimized_num_splits(int B, int NL, int NI, int cu);
int plan_splits(int B, int NL, int NI, int cu, int bm, int tile);
bool validate_common(const char* who, const void* Q, const void* K, const void* V,
                     const void* out, int B, int NL, int NI, int dim);
bool validate_dim768(const char* who, int dim);
bool validate_splits(const char* who, const void* po, const void* pm, const void* pl, int B,
                     int NL, int S);

// fp32 MFMA flash kernel.  po == nullptr: normalised output over all keys
// (S must be 1).  Otherwise: unnormalised split partials, split s covering
// keys [s*chunk, min((s+1)*chunk, NI)).  ds = wavefronts per 16-latent block
// (1, 2 or 4; each holds 768/ds columns of Q and O): 64/ds-latent workgroups.
int f32_row_blocks(int NL, int ds);
bool launch_flash_f32(int ds, const float* Q, const float* K, const float* V, float* out, float* po,
                      float* pm, float* pl, int B, int NL, int NI, int S, int chunk,
                      hipStream_t stream);
// The LSE merge of split partials into out; parts <= 0 takes
// lse_combine_parts' column parts (1, 2 or 4 workgroups per row; any choice
// gives bit-identical output).
int lse_combine_parts(int rows, int S, int cu);
bool launch_lse_combine(const float* po, const float* pm, const float* pl, float* out, int rows,
                        int S, hipStream_t stream, int parts = 0);

// fp16 / bf16 MFMA flash kernel; Q/K/V are 16-bit bit patterns, Q pre-scaled
// by 1/sqrt(768).  Same po semantics as launch_flash_f32.  nw = 8: 64-latent
// workgroups of 8 wavefronts; nw = 4: 32-latent workgroups of 4.  cp = 2 (nw
// = 8 only): each row block runs as two workgroups, one per half of the
// output columns (each computes the block's scores over all of D).
bool launch_flash16(bool bf16, int nw, int cp, const void* Q, const void* K, const void* V,
                    float* out, float* po, float* pm, float* pl, int B, int NL, int NI, int S,
                    int chunk, hipStream_t stream);
int h16_row_blocks(int NL, int nw);

// fp32 ladder rungs
bool launch_naive(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                  int NI, int dim, hipStream_t stream);
bool launch_warp(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                 int NI, int dim, hipStream_t stream);
bool launch_tiled(const float* Q, const float* K, const float* V, float* out, int B, int NL,
                  int NI, int dim, hipStream_t stream);

}  // namespace xattn
