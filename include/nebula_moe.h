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

#ifdef __cplusplus
}
#endif
#endif
