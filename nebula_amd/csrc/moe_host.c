/* Host C driver of stacked routed-MoE layers (declarations and contract in
 * include/nebula_moe.h).  Calls only the qg_* C ABI of libqwen_gpu.so. */
#define _POSIX_C_SOURCE 200809L
#include "nebula_moe.h"
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

enum { NM_MAX_TOKENS = 17, NM_TOP = 10 };

/* Every synchronous device-to-host read this library makes goes through
 * nm_read, which counts them (nm_device_reads). */
static _Atomic uint64_t nm_reads;
int nm_read(void *dst, const void *src, size_t n) {
    nm_reads++;
    return qg_read(dst, src, n);
}
uint64_t nm_device_reads(void) { return nm_reads; }

static _Thread_local char nm_error[256];
static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(nm_error, sizeof nm_error, fmt, ap);
    va_end(ap);
    return -1;
}
const char *nm_last_error(void) { return nm_error; }

struct nm_stack {
    int n_layers, max_tokens, width, record;
    qg_moe_layer *layers;
    float *h, *w;
    int *ids;
    void *ws;
    size_t ws_bytes;
    float *rec_x, *rec_out, *rec_w;
    int *rec_ids;
    void *graphs[NM_MAX_TOKENS + 1];
};

void nm_stack_destroy(nm_stack *s) {
    if (!s) return;
    for (int i = 0; i <= NM_MAX_TOKENS; i++) if (s->graphs[i]) qg_graph_destroy(s->graphs[i]);
    qg_free(s->h); qg_free(s->w); qg_free(s->ids); qg_free(s->ws);
    qg_free(s->rec_x); qg_free(s->rec_out); qg_free(s->rec_w); qg_free(s->rec_ids);
    free(s->layers);
    free(s);
}

nm_stack *nm_stack_create(const qg_moe_layer *layers, int n_layers, int max_tokens, int record) {
    if (!layers || n_layers < 1 || max_tokens < 1 || max_tokens > NM_MAX_TOKENS) { fail("invalid stack arguments"); return NULL; }
    const int D = layers[0].width;
    for (int l = 1; l < n_layers; l++)
        if (layers[l].width != D || layers[l].ff != layers[0].ff) { fail("layer %d shape differs from layer 0", l); return NULL; }
    nm_stack *s = calloc(1, sizeof *s);
    if (!s) { fail("host allocation"); return NULL; }
    s->n_layers = n_layers; s->max_tokens = max_tokens; s->width = D; s->record = record;
    s->layers = malloc(sizeof(qg_moe_layer) * (size_t)n_layers);
    s->ws_bytes = qg_moe_workspace_bytes(D, layers[0].ff, max_tokens);
    const size_t act = (size_t)max_tokens * D * sizeof(float), sel = (size_t)max_tokens * NM_TOP * 4;
    if (!s->layers || !s->ws_bytes) { fail("invalid layer shape"); nm_stack_destroy(s); return NULL; }
    memcpy(s->layers, layers, sizeof(qg_moe_layer) * (size_t)n_layers);
    s->h = qg_alloc(act);
    s->w = qg_alloc(sel); s->ids = qg_alloc(sel); s->ws = qg_alloc(s->ws_bytes);
    if (!s->h || !s->w || !s->ids || !s->ws) { fail("device allocation"); nm_stack_destroy(s); return NULL; }
    if (record) {
        s->rec_x = qg_alloc(act * n_layers); s->rec_out = qg_alloc(act * n_layers);
        s->rec_w = qg_alloc(sel * n_layers); s->rec_ids = qg_alloc(sel * n_layers);
        if (!s->rec_x || !s->rec_out || !s->rec_w || !s->rec_ids) { fail("device allocation (record)"); nm_stack_destroy(s); return NULL; }
    }
    if (qg_zero(s->h, act) || qg_sync()) { fail("initialise hidden state"); nm_stack_destroy(s); return NULL; }
    return s;
}

float *nm_stack_hidden(nm_stack *s) { return s ? s->h : NULL; }

#define GPU(call) do { int rc_ = (call); if (rc_) return fail("%s: %s", #call, qg_error(rc_)); } while (0)

static int run_layers(nm_stack *s, int nt) {
    const size_t act_stride = (size_t)s->max_tokens * s->width, sel_stride = (size_t)s->max_tokens * NM_TOP;
    for (int l = 0; l < s->n_layers; l++) {
        /* h <- h + MoE(RMSNorm(h)); with record on, the normalised input, the
         * routing and the MoE output of the layer are kept */
        float *xn = s->record ? s->rec_x + act_stride * l : NULL;
        float *out = s->record ? s->rec_out + act_stride * l : NULL;
        int *ids = s->record ? s->rec_ids + sel_stride * l : s->ids;
        float *w = s->record ? s->rec_w + sel_stride * l : s->w;
        GPU(qg_moe_forward_residual(s->h, ids, w, NULL, NULL, xn, out, nt, &s->layers[l], s->ws, s->ws_bytes));
    }
    return 0;
}

int nm_stack_forward(nm_stack *s, int nt, int use_graph) {
    if (!s || nt < 1 || nt > s->max_tokens) return fail("invalid token count");
    if (!use_graph) return run_layers(s, nt);
    void **g = &s->graphs[nt];
    if (!*g) {
        GPU(qg_graph_begin(g));
        if (run_layers(s, nt)) { qg_graph_destroy(*g); *g = NULL; return -1; }
        int end = qg_graph_end(*g);
        if (end) { qg_graph_destroy(*g); *g = NULL; return fail("capture MoE stack: %s", qg_error(end)); }
    }
    GPU(qg_graph_launch(*g));
    return 0;
}

int nm_stack_record(nm_stack *s, int layer, const float **x, const int **ids, const float **weights, const float **out) {
    if (!s || !s->record || layer < 0 || layer >= s->n_layers) return fail("no record for this layer");
    const size_t a = (size_t)s->max_tokens * s->width, b = (size_t)s->max_tokens * NM_TOP;
    if (x) *x = s->rec_x + a * layer;
    if (out) *out = s->rec_out + a * layer;
    if (ids) *ids = s->rec_ids + b * layer;
    if (weights) *weights = s->rec_w + b * layer;
    return 0;
}

/* ---- CPU handoff of flag-2 tokens (qwen.c:658-678) ---- */
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

/* scratch: count | rows [T] | x_pack [T][D] | ids [T][10] | weights [T][10] | y [T][D] */
typedef struct { int *count, *rows, *ids; float *x, *w, *y; size_t bytes; } handoff_layout;
static handoff_layout handoff_at(uintptr_t base, int D, int T) {
    handoff_layout L;
    size_t o = 0;
    L.count = (int *)(base + o); o += 256;
    L.rows = (int *)(base + o); o += align256((size_t)T * 4);
    L.x = (float *)(base + o); o += align256((size_t)T * D * 4);
    L.ids = (int *)(base + o); o += align256((size_t)T * NM_TOP * 4);
    L.w = (float *)(base + o); o += align256((size_t)T * NM_TOP * 4);
    L.y = (float *)(base + o); o += align256((size_t)T * D * 4);
    L.bytes = o;
    return L;
}

size_t nm_handoff_scratch_bytes(int width, int tokens) {
    if (width < 1 || tokens < 1 || tokens > 8192) return 0;
    return handoff_at(0, width, tokens).bytes;
}

/* The calling thread's host side of the handoff, allocated once for the
 * largest (width, tokens) reserved or met and kept for later layers: the
 * packed rows, ids and weights read from the device, the CPU MoE's output
 * rows, and the page-locked word the device writes the handed-off count to. */
typedef struct { float *x, *y, *w; int *ids; int *word; size_t rows_cap, width; } handoff_host;
static _Thread_local handoff_host hh;

static void handoff_host_free(void) {
    free(hh.x); free(hh.y); free(hh.w); free(hh.ids);
    qg_host_free(hh.word);
    memset(&hh, 0, sizeof hh);
}

int nm_handoff_reserve(int width, int tokens) {
    if (width < 1 || tokens < 1 || tokens > 8192) return fail("invalid handoff reservation");
    if (hh.word && hh.width == (size_t)width && hh.rows_cap >= (size_t)tokens) return 0;
    const size_t rows = hh.width == (size_t)width && hh.rows_cap > (size_t)tokens ? hh.rows_cap : (size_t)tokens;
    handoff_host_free();
    hh.x = malloc(rows * (size_t)width * sizeof(float));
    hh.y = malloc(rows * (size_t)width * sizeof(float));
    hh.w = malloc(rows * NM_TOP * sizeof(float));
    hh.ids = malloc(rows * NM_TOP * sizeof(int));
    hh.word = qg_host_alloc(sizeof(int));
    if (!hh.x || !hh.y || !hh.w || !hh.ids || !hh.word) { handoff_host_free(); return fail("handoff host allocation"); }
    hh.rows_cap = rows;
    hh.width = (size_t)width;
    return 0;
}

/* Waits for the device's store of the handed-off count into the host word
 * (set to -1 before the notify kernel was queued).  After ~2 ms of polling it
 * synchronises the device instead, so a failed layer reports its error. */
static int handoff_wait_count(int *n) {
    volatile int *word = hh.word;
    const double t_end = 2e-3;
    struct timespec t0, t;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    while (*word < 0) {
        clock_gettime(CLOCK_MONOTONIC, &t);
        if ((t.tv_sec - t0.tv_sec) + (t.tv_nsec - t0.tv_nsec) * 1e-9 > t_end) {
            const int rc = qg_sync();
            if (rc) return fail("handoff count: %s", qg_error(rc));
            if (*word < 0) return fail("handoff count not delivered");
            break;
        }
    }
    __atomic_thread_fence(__ATOMIC_ACQUIRE);
    *n = *word;
    return 0;
}

int nm_moe_handoff(float *out, float *out2, const unsigned char *flags, const float *x, const int *ids,
                   const float *weights, int nt, int D, void *scratch, size_t scratch_bytes,
                   nm_cpu_moe_fn cpu_moe, void *ctx, int *handed_off) {
    if (handed_off) *handed_off = 0;
    if (!out || !flags || !x || !ids || !weights || !scratch || !cpu_moe || nt < 1 || nt > 8192 || D < 1)
        return fail("invalid handoff arguments");
    const handoff_layout L = handoff_at((uintptr_t)scratch, D, nt);
    if (scratch_bytes < L.bytes) return fail("handoff scratch of %zu bytes, %zu needed", scratch_bytes, L.bytes);
    if (nm_handoff_reserve(D, nt)) return -1;
    *(volatile int *)hh.word = -1;
    int rc = qg_moe_handoff_pack(L.count, L.rows, L.x, L.ids, L.w, flags, x, ids, weights, nt, D);
    if (!rc) rc = qg_moe_handoff_notify(hh.word, L.count);
    if (rc) return fail("handoff pack: %s", qg_error(rc));
    int n = 0;
    if (handoff_wait_count(&n)) return -1;
    if (n < 0 || n > nt) return fail("handoff count %d out of range", n);
    if (!n) return 0;
    const size_t xb = (size_t)n * D * sizeof(float), sb = (size_t)n * NM_TOP * 4;
    if ((rc = nm_read(hh.x, L.x, xb)) || (rc = nm_read(hh.ids, L.ids, sb)) || (rc = nm_read(hh.w, L.w, sb)))
        return fail("handoff read: %s", qg_error(rc));
    if (cpu_moe(ctx, hh.y, hh.x, hh.ids, hh.w, n)) return fail("CPU MoE of %d handed-off tokens failed", n);
    if ((rc = qg_write(L.y, hh.y, xb)) || (rc = qg_moe_handoff_merge(out, L.y, L.count, L.rows, nt, D)) ||
        (out2 && (rc = qg_moe_handoff_merge(out2, L.y, L.count, L.rows, nt, D))))
        return fail("handoff merge: %s", qg_error(rc));
    if (handed_off) *handed_off = n;
    return 0;
}
