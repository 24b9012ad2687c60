/* libqwen_gpu.so: MI355X (gfx950) implementation of the routed-MoE subset of
 * the reference's GPU C ABI.  Names, argument lists, return conventions and
 * semantics follow /root/reference/qwen/gpu.h, so the reference's ctypes
 * caller (test_gpu.py:12-36) and host engine (qwen.c) bind unchanged.
 *
 * Conventions (gpu.h:4-10, gpu.cu:38-46,181-189):
 *  - device arrays are token-major; the caller owns every device buffer;
 *  - int returns are runtime error codes (hipError_t here, cudaError_t in the
 *    reference), 0 = success, text from qg_error(); argument errors return
 *    the "invalid value" code;
 *  - operator wrappers are asynchronous on the calling thread's stream and
 *    return the launch status; qg_write/qg_read are synchronous;
 *  - between qg_graph_begin and qg_graph_end the calling thread's launches
 *    are captured (per-thread capture stream, gpu.cu:10,21-34).
 * Entry points whose reference signature carries no width (gather, scatter,
 * reduce, mtp_moe, shared_add) use the hidden/FFN widths set by
 * qg_moe_configure (default 2560/640, the reference's hard-coded shapes,
 * gpu.cu:508-553). */
#ifndef NEBULA_QWEN_GPU_H
#define NEBULA_QWEN_GPU_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime (gpu.h:11-21,24,30-36; gpu.cu:13-85,114-120) ---- */
void *qg_alloc(size_t bytes);                                   /* gpu.h:11, NULL on failure */
void qg_free(void *p);                                          /* gpu.h:12 */
int qg_write(void *dst, const void *src, size_t bytes);         /* gpu.h:13, synchronous H2D */
int qg_read(void *dst, const void *src, size_t bytes);          /* gpu.h:14, synchronous D2H */
int qg_copy(void *dst, const void *src, size_t bytes);          /* gpu.h:15, async D2D */
int qg_zero(void *dst, size_t bytes);                           /* gpu.h:16, async fill */
int qg_sync(void);                                              /* gpu.h:17 */
int qg_graph_begin(void **graph);                               /* gpu.h:18 */
int qg_graph_end(void *graph);                                  /* gpu.h:19 */
int qg_graph_launch(void *graph);                               /* gpu.h:20 */
void qg_graph_destroy(void *graph);                             /* gpu.h:21 */
int qg_memory(size_t *free_bytes, size_t *total_bytes);         /* gpu.h:24 */
const char *qg_error(int error);                                /* gpu.h:30 */
int qg_tensor_bytes(int type, const uint64_t dims[4], uint64_t *bytes); /* gpu.h:31 */
void *qg_upload_create(size_t expert_bytes);                    /* gpu.h:32 */
void qg_upload_destroy(void *uploader);                         /* gpu.h:33 */
int qg_upload_expert(void *uploader, void *dst, const void *gate, size_t gate_bytes,
                     const void *up, size_t up_bytes, const void *down, size_t down_bytes); /* gpu.h:34-35 */
double qg_upload_seconds(void *uploader);                       /* gpu.h:36 */

/* ---- operators on the MoE path (gpu.h:37-43,62-78) ---- */
/* out[t,r] = sum_c deq(W)[r,c] x[t,c]; types 0,1,30,2,6,7,8,12,13,14,20;
 * tokens 1..8192; the reference's fixed summation order (gpu.cu:154-189,
 * cpu.c:119-148), so results equal cpu.c's qc_matmul bit for bit. */
int qg_matmul(float *out, const void *w, int type, int rows, int cols, const float *x, int tokens); /* gpu.h:37-38 */
int qg_gather(float *out, const void *w, int type, int cols, int row);          /* gpu.h:39 */
int qg_norm(float *out, const float *x, const float *weight, int width,
            int groups, int tokens, int weight_groups, int l2, float eps);      /* gpu.h:40-41 */
int qg_unary(float *out, const float *x, int count, int op, float scale);      /* gpu.h:42 */
int qg_binary(float *out, const float *a, const float *b, int count, int op);  /* gpu.h:43 */
int qg_route(int *ids, float *weights, const float *logits, int tokens);        /* gpu.h:62 */
typedef struct {
    uint64_t token_layers, missing_selections, skipped_selections, avoided_token_handoffs;
    double skipped_mass;
} qg_prune_stats;                                                               /* gpu.h:63-66 */
int qg_prune_routes(int *ids, float *weights, const unsigned char *resident,
                    int tokens, double threshold, qg_prune_stats *stats);       /* gpu.h:67-68 */
int qg_moe_map(int *map, const int *ids, int tokens);                          /* gpu.h:69 */
int qg_moe_gather(float *out, const float *x, const int *token_map, int selected_tokens);   /* gpu.h:70 */
int qg_moe_scatter(float *slots, const float *expert, const float *weights, const int *ids,
                   const int *token_map, int expert_id, int selected_tokens);  /* gpu.h:71-72 */
int qg_moe_reduce(float *out, const float *slots, int tokens);                 /* gpu.h:73 */
int qg_mtp_moe(float *slots, float *mid, const float *x, const int *ids, const float *weights,
               const void *gate, int gate_type, const void *up, int up_type,
               const void *down, int down_type, int tokens);                    /* gpu.h:74-76 */
int qg_dequant(float *out, const void *packed, int type, int rows, int cols);  /* gpu.h:77 */
int qg_shared_add(float *out, const float *shared, const float *gate, int tokens); /* gpu.h:78 */

/* ---- additions (no reference counterpart; the reference hard-codes the
 * shapes and drives the layer from the host, qwen.c:633-735) ---- */

/* Hidden width D and expert FFN width F used by the width-less entry points
 * above: a process-wide setting (initially 2560/640), seen by every thread.
 * D multiple of 256, F multiple of 32, D <= 8192, F <= 4096. */
int qg_moe_configure(int width, int ff);
/* A per-thread override of that setting for the calling thread's width-less
 * calls (a thread driving a model of its own shape); (0, 0) removes it.
 * Added entry point, no counterpart in gpu.h. */
int qg_moe_configure_thread(int width, int ff);

/* Dispatch of routing ids into per-expert contiguous row lists (CSR), the
 * device-side histogram/prefix-sum/permutation replacing qg_moe_map's
 * [512, tokens] map and the host count loop of qwen.c:650-655.  offsets[513];
 * entries offsets[e]..offsets[e+1]-1 list (ascending token) the selections of
 * expert e: row_token = t, row_slot = t*10+k.  Ids in [-513,-2] (pruned) are
 * skipped; any other id outside [0,512), or a token listing an expert twice,
 * makes *status nonzero (the lists are then unspecified). */
int qg_moe_dispatch(int *offsets, int *row_token, int *row_slot, int *status, const int *ids, int tokens);

/* One routed-MoE layer, device-driven (no host read of routing ids), so it
 * can be captured into a graph: router -> top-10 -> [coverage/prune] ->
 * dispatch -> gate/up + SwiGLU -> down + router-rank combine -> shared expert.
 * Replaces moe()/grouped_moe()/shared_direct() of qwen.c:633-735 for one
 * layer.  Arithmetic: router logits in fp32 in the reference's fixed order
 * (ids and weights bit-exact); expert products on fp16 matrix cores with fp32
 * accumulation: each weight enters exactly (Q4_K as the integer s*q, at most
 * 945; IQ4_NL as its table value), each activation as two fp16 planes (hi =
 * fp16(x), lo = fp16(x - hi), about 22 significant bits), superblock and
 * block scales and the Q4_K min term applied in fp32; outputs agree with the
 * reference's fp32 path within max-abs 1e-3 / rel-L2 1e-4 (about 1e-6
 * relative in practice). */
typedef struct {
    int width, ff;                              /* D, F */
    const float *router;                        /* F32 [512, D] (ffn_gate_inp) */
    const void *gate, *up, *down;               /* [512][F][row(D)], [512][F][row(D)], [512][D][row(F)] */
    int gate_type, up_type, down_type;
    const void *sh_gate, *sh_up, *sh_down;      /* shared expert or NULL (ffn_*_shexp) */
    int sh_gate_type, sh_up_type, sh_down_type;
    const float *sh_gate_inp;                   /* F32 [1, D] (ffn_gate_inp_shexp) */
    const unsigned char *resident;              /* 512-byte device mask or NULL */
    double threshold;                           /* omitted-mass threshold (0.10, config.py:9) */
    const float *router_bias;                   /* F32 [512] added to every logit before routing, or NULL
                                                   (synthetic workloads; the reference's router has no bias) */
} qg_moe_layer;

/* Device workspace bytes for qg_moe_forward / qg_moe_forward_residual at up
 * to `tokens` tokens.  The workspace needs no initialisation; one workspace
 * per concurrent caller. */
size_t qg_moe_workspace_bytes(int width, int ff, int tokens);

/* out [tokens, D]; ids/weights [tokens, 10] (after pruning); flags [tokens]
 * or NULL: 0 all selections resident, 1 pruned (omitted mass < threshold),
 * 2 handoff (coverage below 1-threshold), 3 invalid router distribution;
 * stats may be NULL.  With flags==2 the token's routed part is not computed
 * here (it belongs to the host handoff, qwen.c:658-678): its row holds only
 * the sigmoid-gated shared expert (which stays on the device, qwen.c:661-663),
 * or 0 without one; qg_moe_handoff_pack/merge move the routed part through
 * the host.  flags==3 rows are 0.
 * Device pointers to weights, activations, outputs and the workspace must be
 * 16-byte aligned (qg_alloc returns 256-byte aligned memory); otherwise the
 * call returns an invalid-value error and launches nothing.
 * tokens 1..8192: up to 17 the decode kernels (any format qg_matmul takes);
 * above, the prefill grouped GEMMs, which need Q4_K gate/up, Q4_K or IQ4_NL
 * down, D a multiple of 256 and F a multiple of 128 (else an error). */
int qg_moe_forward(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                   const float *x, int tokens, const qg_moe_layer *layer, void *workspace, size_t workspace_bytes);

/* No reference counterpart: for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  qg_moe_forward with the library's own workspace, a static
 * 16 MiB array in device memory per GPU (held until the process ends); no
 * allocation of any kind happens.  Layers whose qg_moe_workspace_bytes at
 * `tokens` exceeds 16 MiB are rejected with the invalid-value code before
 * anything is launched (every decode batch of 1..17 tokens fits up to
 * D=8192/F=4096; at D=2048/F=512 prefill batches up to about 120 tokens
 * fit).  Calls that overlap on one GPU share the workspace and race. */
int qg_moe_forward_noalloc(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                           const float *x, int tokens, const qg_moe_layer *layer);

/* The layer applied to a residual stream, as one layer of qwen_target's loop
 * without attention (qwen.c:759-762): x = RMSNorm(h) (eps 1e-6, unit weight,
 * the norm of gpu.cu:204-214), h += MoE(x).  xn_out [tokens, D] (the
 * normalised input) and out [tokens, D] (the MoE output) may be NULL.  Other
 * arguments as qg_moe_forward. */
int qg_moe_forward_residual(float *h, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                            float *xn_out, float *out, int tokens, const qg_moe_layer *layer,
                            void *workspace, size_t workspace_bytes);

/* CPU handoff of the flag-2 tokens (replaces the whole-batch reads of
 * qwen.c:665-666 and the write of qwen.c:672).  Device arrays; async on the
 * calling thread's stream.  pack: count[0] = number of tokens with
 * flags[t] == 2, rows[i] = the i-th of them (ascending), and row i of x_pack
 * [tokens, width], ids_pack / w_pack [tokens, 10] = that token's input row,
 * ids and weights (only the first count[0] rows are written).  merge:
 * out[rows[i]] += y_pack[i] for i < count[0], y_pack [tokens, width] being
 * the host's routed rows (qc_moe, cpu.c:235-261, of the packed tokens).
 * tokens 1..8192. */
int qg_moe_handoff_pack(int *count, int *rows, float *x_pack, int *ids_pack, float *w_pack,
                        const unsigned char *flags, const float *x, const int *ids, const float *weights,
                        int tokens, int width);
int qg_moe_handoff_merge(float *out, const float *y_pack, const int *count, const int *rows, int tokens, int width);
/* After qg_moe_handoff_pack: count[0] is stored into *host_word, a word of
 * qg_host_alloc memory, by a kernel on the calling thread's stream, so the
 * host learns the number of handed-off tokens by polling the word instead of
 * a device-to-host copy.  Added entry point, no counterpart in gpu.h. */
int qg_moe_handoff_notify(int *host_word, const int *count);
/* Page-locked host memory that device code may access through the same
 * pointer (NULL on failure), and its release.  Added entry points (the
 * reference allocates its pinned staging inside qg_upload_create). */
void *qg_host_alloc(size_t bytes);
void qg_host_free(void *p);

/* Benchmark support: events[2i] and events[2i+1] (qg_event_create handles)
 * are recorded at the start and end of kernel i of this thread's
 * qg_moe_forward calls, timestamped by the dispatch itself
 * (hipExtLaunchKernelGGL).  Decode: 0 router, 1 routing, 2 gate/up, 3 down,
 * 4 combine.
 * Prefill: 0 router, 1 routing, 2 scan, 3 fill, 4 gate/up dense pass,
 * 5 gate/up other experts, 6 down dense pass, 7 down other experts,
 * 8 shared-expert down (when its format differs), 9 combine, 10 chunk
 * histogram.  n <= 32;
 * n = 0 disables. */
int qg_moe_kernel_events(void **events, int n);

/* Benchmark support: record events[i] (qg_event_create handles) on the
 * launch stream at the phase boundaries of this thread's qg_moe_forward
 * calls: 0 start, 1 after the router, 2 after routing/dispatch, 3 after
 * gate/up, 4 after down, 5 after the combine (phases fused into one kernel
 * record adjacent events back to back).  n = 0 disables. */
int qg_moe_phase_events(void **events, int n);

/* Timing helpers for the benchmark (events on the calling thread's stream). */
void *qg_event_create(void);
void qg_event_destroy(void *event);
int qg_event_record(void *event);
int qg_event_elapsed(float *ms, void *begin, void *end);
int qg_device_info(char *name, size_t name_len, int *cus, int *clock_khz, int *mem_clock_khz, int *bus_bits);

/* Synthetic inputs generated on the device (benchmark/test support; not a
 * reference interface).  Value (r,c) of tensor `stream` under `seed` is
 * sigma*N(0,1) from a counter-based hash; encoded to type 0/12/20.  The
 * bytes equal the CPU generator's in oracle/nb_synth.c. */
int qg_synth_matrix(void *out, int type, uint64_t seed, uint64_t stream, int rows, int cols, float sigma);
/* `experts` such matrices in one launch: matrix e uses stream
 * (tensor << 32 | e) and starts e * rows * row_bytes(type, cols) bytes after
 * out, the per-tensor expert layout of a layer. */
int qg_synth_experts(void *out, int type, uint64_t seed, int tensor, int experts, int rows, int cols, float sigma);

/* No reference counterpart: how the calling thread's prefill layers launch
 * gate/up.  mode 0 (the default): one launch over every expert group.
 * mode 1: the dense experts (256 or more rows) in a launch of their own on
 * int8 matrix cores (two int8 activation planes per token row with a row
 * scale, the Q4_K nibbles as int8, per-group int32 -> fp32 scaling), then the
 * rest on fp16.  mode 2: the same split with both launches on fp16 hi/lo
 * planes.  Other values select mode 0.  Returns the previous mode.  A
 * measurement switch for the benchmark's int8-vs-fp16 comparison of the dense
 * experts and its parity test. */
int qg_prefill_int8_dense(int mode);

#ifdef __cplusplus
}
#endif
#endif
