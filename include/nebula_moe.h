/* libnebula_moe.so: C host driver of routed-MoE layers on top of
 * libqwen_gpu.so's C ABI (it calls only qg_* entry points).
 *
 * It plays the role of the reference's moe()/shared_direct() and the
 * per-layer loop of qwen_target (qwen.c:714-735,759-762) for a stack of MoE
 * layers without attention: each layer is h <- h + MoE(RMSNorm(h)) (eps 1e-6,
 * unit weight, the norm of gpu.cu:204-214), one qg_moe_forward_residual call.  The whole stack for a token
 * count is captured once into a graph and replayed, the way qwen.c:726-734
 * captures the shared expert per batch size; unlike the reference no routing
 * decision crosses to the host, so the routed part is captured too.
 *
 * Errors: functions return 0 or a nonzero code / NULL; nm_last_error() gives
 * a thread-local message (the convention of qwen.c:78-83). */
#ifndef NEBULA_MOE_H
#define NEBULA_MOE_H
#include "qwen_gpu.h"
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct nm_stack nm_stack;

/* Copies the layer descriptors (device pointers stay owned by the caller).
 * max_tokens 1..17.  record != 0 keeps per-layer routing and inputs for
 * inspection (nm_stack_record). */
nm_stack *nm_stack_create(const qg_moe_layer *layers, int n_layers, int max_tokens, int record);
void nm_stack_destroy(nm_stack *s);
/* Device hidden state [max_tokens][width]; write the input here. */
float *nm_stack_hidden(nm_stack *s);
/* Runs all layers on the first `tokens` rows of the hidden state, on the
 * calling thread's stream.  use_graph: capture on first use per token count,
 * then replay. */
int nm_stack_forward(nm_stack *s, int tokens, int use_graph);
/* With record != 0: device arrays of layer l: normalised input [tokens][D],
 * ids [tokens][10], weights [tokens][10], MoE output [tokens][D]. */
int nm_stack_record(nm_stack *s, int layer, const float **x, const int **ids, const float **weights, const float **out);
const char *nm_last_error(void);

/* CPU handoff of one layer's flag-2 tokens (the hybrid path of
 * qwen.c:658-678, narrowed from the whole batch to the flagged tokens).
 * cpu_moe computes the routed part (qc_moe of cpu.c:235-261, through
 * qwen.c:615-617) of `tokens` packed rows: out [tokens][D] from x
 * [tokens][D], ids/weights [tokens][10]; it returns 0 on success. */
typedef int (*nm_cpu_moe_fn)(void *ctx, float *out, const float *x, const int *ids, const float *weights, int tokens);
/* Device scratch bytes nm_moe_handoff needs for up to `tokens` tokens. */
size_t nm_handoff_scratch_bytes(int width, int tokens);
/* Allocates the calling thread's host buffers of nm_moe_handoff (packed
 * rows, ids, weights, the CPU MoE's rows and a page-locked count word) for
 * up to `tokens` tokens of `width`, so that later handoffs allocate nothing;
 * nm_moe_handoff grows them itself when it meets a larger batch. */
int nm_handoff_reserve(int width, int tokens);
/* Number of synchronous device-to-host reads (qg_read) this library has
 * issued in the process: the layer paths' host round trips, for tests and
 * statistics. */
uint64_t nm_device_reads(void);
/* After qg_moe_forward(_residual) with flags: packs the flag-2 tokens on the
 * device, waits for their count, which the device stores into a page-locked
 * host word (qg_moe_handoff_notify: no device-to-host copy, so a layer with
 * no flag-2 token makes none), and then reads only their input rows, ids and
 * weights, calls cpu_moe, writes its rows back and adds
 * them to out (and to out2 when not NULL: the residual stream h) at the
 * tokens' rows, where the device left the shared expert's part.  x is the
 * layer input the forward used (xn_out for the residual form).  Synchronous
 * (not capturable), like the reference's handoff.  *handed_off (may be NULL)
 * = number of tokens sent to the host. */
int nm_moe_handoff(float *out, float *out2, const unsigned char *flags, const float *x, const int *ids,
                   const float *weights, int tokens, int width, void *scratch, size_t scratch_bytes,
                   nm_cpu_moe_fn cpu_moe, void *ctx, int *handed_off);

#ifdef __cplusplus
}
#endif
#endif
