/* The routed-MoE part of the reference's host-engine ABI (qwen/qwen.h),
 * exported by libnebula_moe.so over libqwen_gpu.so's C ABI.
 *
 * A qwen_model here holds the MoE tensors of a COB_QWEN_INDEX_V1 index
 * (qwen.c:108-146): per layer the router (ffn_gate_inp), the routed experts
 * (ffn_{gate,up,down}_exps), the shared expert (ffn_{gate,up,down}_shexp) and
 * its gate vector (ffn_gate_inp_shexp), for target layers blk.0 ..
 * blk.(n-1) (n <= 48) and optionally the MTP layer blk.48.  Attention, the
 * embeddings and the rest of the model are not part of this path; other
 * tensors in the index are parsed, validated and ignored.  Hidden width D
 * and expert width F are read from the tensors (the reference hard-codes
 * 2560/640, qwen.c:20,160-161).
 *
 * Names, struct layouts, argument lists and conventions follow qwen.h:
 * functions return 0 / -1 (or NULL) and qwen_last_error() gives a
 * thread-local message (qwen.c:78-80).  One caller thread per model.
 *
 * Layer execution (qwen_moe, the reference's static moe(), qwen.c:714-735):
 *  - target layer with the fixed hotlist (official mode): the device layer
 *    (qg_moe_forward) with the layer's resident mask and the 0.10 omitted-
 *    mass threshold; tokens whose missing routed weight is not negligible
 *    (coverage flag 2) have their routed part computed on the host by the
 *    registered CPU MoE, one token set per layer (qwen.c:658-678 hands the
 *    whole batch over instead);
 *  - target layer without a hotlist: the reference's grouped_moe
 *    (qwen.c:633-707) over an LRU expert cache of resident_per_layer slots
 *    (cache_slot, qwen.c:558-570) filled through the pinned uploader, driven
 *    through the drop-in qg_* entry points;
 *  - the MTP layer: all experts resident, the device layer without a mask.
 */
#ifndef NEBULA_QWEN_MOE_H
#define NEBULA_QWEN_MOE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct qwen_model qwen_model;
enum { QWEN_MAX_DRAFT = 16, QWEN_VERIFY_ROWS = QWEN_MAX_DRAFT + 1 };   /* qwen.h:10 */

typedef struct {                                                         /* qwen.h:11-18 */
    uint64_t gpu_weight_bytes, gpu_state_bytes, gpu_workspace_bytes, gpu_arena_bytes;
    uint64_t target_tokens, mtp_tokens, expert_handoffs, expert_upload_bytes;
    uint64_t expert_hits, expert_requests, metadata_read_bytes, ple_read_bytes;
    uint64_t host_weight_bytes, host_staging_bytes;
    double target_seconds, mtp_seconds, expert_handoff_host_seconds, expert_dma_seconds, ple_lookup_seconds,
        core_load_seconds, host_load_seconds;
    int target_position, mtp_position, context, resident_per_layer;
} qwen_stats;
typedef struct {                                                         /* qwen.h:19-21 */
    uint64_t layer_calls[48], layer_handoffs[48];
} qwen_handoff_profile;
typedef struct {                                                         /* qwen.h:68-71 */
    uint64_t layer_handoffs, token_layers, missing_selections, activation_bytes;
    double compute_seconds, handoff_seconds;
} qwen_cpu_stats;
typedef struct {                                                         /* qwen.h:80-84 */
    uint64_t token_layers, missing_selections, skipped_selections, avoided_token_handoffs;
    double skipped_mass;
} qwen_prune_stats;

/* Read-only preflight of an index: header, FILE and TENSOR lines, file sizes
 * and the MoE tensors' types and shapes; maps nothing (qwen.h:7-8). */
int qwen_validate_index(const char *index_path);
/* Parses the index, maps its files and uploads the routers, shared experts
 * and (MTP layer) all experts.  context >= 1; resident_per_layer 1..512
 * expert slots per target layer; prefill_capacity 1..8192 tokens per call
 * (qwen.h:22). */
qwen_model *qwen_open(const char *index_path, int context, int resident_per_layer, int prefill_capacity);
void qwen_close(qwen_model *m);
const char *qwen_last_error(void);
int qwen_max_draft(void);                                   /* 16 (qwen.c:746) */
/* Pins count = layers * resident_per_layer expert ids (layer-major) as the
 * fixed device set (validation and mask build of qwen.c:571-602): each id
 * 0..511, no duplicate within a layer, threads 1..28, once per model, and a
 * CPU MoE must be registered first (qwen_set_cpu_moe). */
int qwen_set_hotlist(qwen_model *m, const int *ids, int count, int threads);
int qwen_set_cpu_threads(qwen_model *m, int threads);       /* qwen.c:604-607 */
int qwen_cpu_threads(qwen_model *m);
void qwen_get_cpu_stats(qwen_model *m, qwen_cpu_stats *out);
int qwen_handoff_version(void);                             /* 1 (qwen.c:609) */
/* Device prune counters accumulated since qwen_set_hotlist (qwen.c:610-613). */
int qwen_get_prune_stats(qwen_model *m, qwen_prune_stats *out);
/* Per target layer: executions, and executions with a CPU handoff (hotlist
 * mode) or an expert upload (cache mode) (qwen.h:57-59). */
void qwen_get_handoff_profile(qwen_model *m, qwen_handoff_profile *out);
void qwen_get_stats(qwen_model *m, qwen_stats *out);
/* Route trace (qwen.c:86-94): "QROUTE1\n", then per traced target-layer call
 * uint32 {layer, position, tokens}, int32 ids[tokens*10] and float
 * weights[tokens*10] as routed, before the hotlist's pruning
 * (qwen.c:638-646).  NULL closes the file. */
int qwen_profile_routes(qwen_model *m, const char *path);

/* ---- additions (no reference counterpart) ---- */

/* The host routed MoE used for handed-off tokens: the reference's qc_moe
 * argument list (cpu.h:15) with its workspace as ctx; weights are the host
 * copies of the layer's expert tensors (the mapped index files). */
typedef int (*qwen_cpu_moe_fn)(void *ctx, float *out, const float *x, const int *ids, const float *weights, int tokens,
                               const void *gate, int gate_type, const void *up, int up_type, const void *down,
                               int down_type);
int qwen_set_cpu_moe(qwen_model *m, qwen_cpu_moe_fn fn, void *ctx);
/* Width, expert width and the number of target layers (MTP excluded); *has_mtp
 * = 1 when blk.48's MoE is present.  Pointers may be NULL. */
int qwen_moe_shape(qwen_model *m, int *width, int *ff, int *layers, int *has_mtp);
/* One MoE layer (moe(), qwen.c:714-735): out [tokens][D] = rank-order routed
 * sum + sigmoid-gated shared expert of x [tokens][D]; both device buffers,
 * 16-byte aligned.  layer 0..layers-1 (target) or 48 (MTP).  position is the
 * target position of the first token, recorded in the route trace.
 * Synchronous. */
int qwen_moe(qwen_model *m, int layer, float *out, const float *x, int tokens, int position);

#ifdef __cplusplus
}
#endif
#endif
