/* A kernels.so that exports only what cuda_wrappers.py binds unconditionally:
 * the four fp32 launchers and the xattn_* status/planning helpers, with no
 * bodies worth calling.  The loader tests build it with gcc and check that
 * the wrapper reports every optional entry point (16-bit, split-K) absent,
 * as the reference's wrapper does for a library built without them
 * (cuda_wrappers.py:136-175).  Never launched. */
void launch_naive_kernel(void) {}
void launch_parallel_kernel(void) {}
void launch_tiled_kernel(void) {}
void launch_optimized_kernel(void) {}
int xattn_get_last_error(void) { return 0; }
const char* xattn_get_last_error_string(void) { return ""; }
int xattn_device_info(void) { return 1; }
int xattn_device_arch(void) { return 1; }
int xattn_xcd_remap(int b, int n) { (void)n; return b; }
int xattn_optimized_num_splits(void) { return 1; }
int xattn_plan_splits(void) { return 1; }
void xattn_f32_plan(void) {}
void xattn_wmma_plan(void) {}
void xattn_wmma_plan_ex(void) {}
int xattn_f32_split_latents(void) { return 64; }
int xattn_wmma_split_latents(void) { return 64; }
