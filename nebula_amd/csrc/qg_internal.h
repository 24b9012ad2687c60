// Internal declarations shared by the libqwen_gpu.so translation units.
#pragma once
#include "qg_common.h"
#include "../../include/qwen_gpu.h"

// The calling thread's launch stream (null stream, or the capture stream).
hipStream_t qg_stream(void);

// Grows a library-owned scratch buffer to at least `need` bytes (0 or an
// error code).  Superseded buffers stay allocated until the process ends, so
// a graph captured with the old address never touches freed memory.
int qg_scratch_grow(void **buf, size_t *cap, size_t need);
// Compute units of the current device (persistent grids: one workgroup each).
int qg_cu_count();

// Shapes used by the entry points that take no width (gather, scatter,
// reduce, mtp_moe, shared_add); set by qg_moe_configure.
int qg_cfg_width(void);
int qg_cfg_ff(void);

// Launchers shared between the drop-in entry points and the fused layer.
int qg_launch_matmul_exact(float *out, const uint8_t *w, int type, int rows, int cols, const float *x, int nt,
                           const uint8_t *w_extra_row, hipStream_t s);

// The layer through the generic kernels (any format/width qg_moe_forward
// accepts); used when the decode fast path does not cover the layer.
extern "C" size_t qg_generic_workspace_bytes(int width, int ff, int tokens);
extern "C" int qg_generic_forward(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, const float *x, int nt,
                       const qg_moe_layer *L, void *workspace, size_t ws_bytes);

// Benchmark timing: the events registered by qg_moe_kernel_events for kernel
// `slot` of this thread's calls, if any.
bool qg_kernel_event_pair(int slot, void **begin, void **end);

// The prefill path (18..8192 tokens) of qg_moe_forward(_residual).
bool qg_prefill_ok(const qg_moe_layer *L);
size_t qg_prefill_workspace_bytes(int width, int ff, int tokens);
int qg_prefill_forward(float *out, float *resid, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                       const float *x, float *xn_out, int norm, int nt, const qg_moe_layer *L, void *workspace);
size_t qg_prefill_dispatch_scratch(int nt);
int qg_prefill_dispatch(int *offsets, int *row_token, int *row_slot, int *status, const int *ids, int nt, void *scratch);
