/* CPU oracle for the routed-MoE layer: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product (nebula_amd/)
 * never links, loads or calls it.
 *
 * Every function restates the reference's algorithm and cites the file:line
 * it follows (paths are under /root/reference/qwen/).  Shapes are run-time
 * parameters here (the reference hard-codes D=2560, F=640). */
#ifndef NB_ORACLE_H
#define NB_ORACLE_H
#include <stddef.h>
#include <stdint.h>

enum { NBO_EXPERTS = 512, NBO_TOP = 10 };

typedef struct {
    uint64_t token_layers, missing_selections, skipped_selections, avoided_token_handoffs;
    double skipped_mass;
} nbo_prune_stats; /* layout of qg_prune_stats, gpu.h:63-66 */

/* GGML block formats (cpu.c:17-67). */
size_t nbo_row_bytes(int type, int cols);
float nbo_half(const uint8_t *p);
float nbo_weight_at(const void *row, int type, int i);

/* Quantised GEMV/GEMM with the reference's fixed summation order
 * (cpu.c:119-148, cpu_portable.h:326-336, gpu.cu:154-180). */
int nbo_matmul(float *out, const void *w, int type, int rows, int cols, const float *x, int nt);

/* exp as (float)exp((double)x) with the oracle's own double exp. */
double nbo_exp_d(double x);
float nbo_expf(float x);

/* Routing (gpu.cu:456-465), pruning (gpu.cu:467-488), coverage flags. */
void nbo_route(int *ids, float *weights, const float *logits, int nt);
void nbo_prune(int *ids, float *weights, const uint8_t *resident, int nt, double threshold,
               nbo_prune_stats *stats);
void nbo_coverage(uint8_t *flags, double *mass, const int *ids, const float *weights,
                  const uint8_t *resident, int nt);

/* Dispatch: the reference's [512, nt] token map (gpu.cu:489-500) and the
 * CSR form of the same permutation. */
void nbo_moe_map(int *map, int *counts, const int *ids, int nt);
int nbo_dispatch(int *offsets, int *row_token, int *row_slot, const int *ids, int nt);

/* qc_moe (cpu.c:235-261) with D/F as parameters.  Returns -1 on invalid ids. */
int nbo_moe(float *out, const float *x, const int *ids, const float *weights, int nt, int D, int F,
            const void *gate, int gt, const void *up, int ut, const void *down, int dt);

/* Shared expert (qwen.c:708-713, gpu.cu:215-226,552-553). */
int nbo_shared(float *out, const float *x, int nt, int D, int F, const void *gate, int gt,
               const void *up, int ut, const void *down, int dt, const float *gate_inp);

/* One routed-MoE layer as the reference's moe() runs it (qwen.c:714-735).
 * resident may be NULL (no pruning).  shared_* may be NULL (no shared expert).
 * router_bias (synthetic workloads only; the reference's router has none) is
 * added to each logit with one fp32 add before routing.
 * ids/weights/logits/flags outputs may be NULL. */
typedef struct {
    int D, F;
    const float *router;                     /* F32 [512, D] */
    const void *gate, *up, *down; int gt, ut, dt;
    const void *sh_gate, *sh_up, *sh_down; int sgt, sut, sdt;
    const float *sh_inp;                     /* F32 [1, D] */
    const float *router_bias;                /* F32 [512] added to the logits, or NULL */
} nbo_layer_desc;
int nbo_layer(float *out, int *ids, float *weights, float *logits, uint8_t *flags,
              const nbo_layer_desc *L, const float *x, int nt, const uint8_t *resident,
              double threshold, nbo_prune_stats *stats);

void nbo_rmsnorm(float *out, const float *x, int nt, int D, float eps);

/* ---- synthetic input generator (nb_synth.c), CPU mirror of the device one ---- */
uint64_t nbs_hash(uint64_t seed, uint64_t stream, uint64_t index);
double nbs_gauss(uint64_t seed, uint64_t stream, uint64_t index);
uint16_t nbs_f32_to_f16(float f);
float nbs_f16_to_f32(uint16_t h);
void nbs_encode_q4k(uint8_t *block, const float *x);      /* 256 values -> 144 B */
void nbs_encode_iq4nl(uint8_t *block, const float *x);    /* 32 values -> 18 B */
/* rows x cols matrix of sigma*N(0,1) values, value (r,c) = index r*cols+c of
 * (seed, stream); encoded to `type` (0 F32, 12 Q4_K, 20 IQ4_NL). */
int nbs_fill_matrix(void *out, int type, uint64_t seed, uint64_t stream, int rows, int cols, float sigma);
uint64_t nbs_stream(int tensor, int expert);

#endif
