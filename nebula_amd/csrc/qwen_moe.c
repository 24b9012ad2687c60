/* MoE part of the reference's host engine (declarations and contract in
 * include/qwen_moe.h): COB_QWEN_INDEX_V1 loading, the expert cache, the
 * fixed hotlist and its statistics, the route trace and moe() for one layer.
 * Device work goes through libqwen_gpu.so's qg_* C ABI only; the CPU handoff
 * through nm_moe_handoff (moe_host.c). */
#define _POSIX_C_SOURCE 200809L
#include "qwen_moe.h"
#include "nebula_moe.h"
#include <errno.h>
#include <fcntl.h>
#include <inttypes.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

enum { QM_LAYERS = 48, QM_MTP = 48, QM_EXPERTS = 512, QM_TOP = 10, QM_MAX_FILES = 16, QM_MAX_TENSORS = 1600,
       QM_MAX_TOKENS = 8192 };

typedef struct {
    char name[128];
    int file, type;
    uint64_t offset, bytes, dim[4];
    const unsigned char *host;
} qm_tensor;

typedef struct {
    int fd;
    unsigned char *data;
    uint64_t bytes;
} qm_file;

typedef struct {
    const qm_tensor *router, *eg, *eu, *ed, *sg, *su, *sd, *sr;
    uint64_t gate_bytes, up_bytes, down_bytes, expert_bytes;  /* per expert */
    void *d_router, *d_sg, *d_su, *d_sd, *d_sr;               /* always on the device */
    unsigned char *d_gate, *d_up, *d_down;                    /* per-tensor [512] layout (hotlist and MTP layers) */
    unsigned char *slots;                                     /* cache mode: resident slots, gate|up|down each */
    int *cache_ids;                                           /* slot -> expert or -1 */
    uint64_t *cache_age, clock;
    unsigned char pinned[512];                                /* hotlist mode: the layer's resident experts */
    qg_moe_layer desc;
} qm_layer;

struct qwen_model {
    qm_file files[QM_MAX_FILES];
    int n_files;
    qm_tensor *tensors;
    int n_tensors;
    uint64_t multiplier[3], head_offset[16], head_vocab[16];
    int ple_eos;
    int D, F, n_layers, has_mtp, context, resident, capacity;
    qm_layer layers[QM_LAYERS + 1];
    void *uploader;
    /* device buffers sized for `capacity` tokens */
    float *logits, *route_w, *slots, *expert_x, *ffg, *ffu, *ffmid, *ffout, *shared, *shared_gate;
    int *route_ids, *route_map;
    unsigned char *flags, *masks;
    void *ws, *handoff;
    size_t ws_bytes, handoff_bytes;
    qg_prune_stats *prune_device;
    /* host state */
    int *h_ids;
    float *h_w;
    int fixed_hotlist, hotlist_tried, ran_target, cpu_threads;
    qwen_cpu_moe_fn cpu_moe;
    void *cpu_ctx;
    qwen_stats stats;
    qwen_handoff_profile profile;
    qwen_cpu_stats cpu_stats;
    FILE *route_profile;
};

static _Thread_local char qm_error[512];
static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(qm_error, sizeof qm_error, fmt, ap);
    va_end(ap);
    return -1;
}
const char *qwen_last_error(void) { return qm_error; }
int qwen_max_draft(void) { return QWEN_MAX_DRAFT; }
int qwen_handoff_version(void) { return 1; }

static double seconds_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

#define GPU(call) do { int rc_ = (call); if (rc_) return fail("%s: %s", #call, qg_error(rc_)); } while (0)

int nm_read(void *dst, const void *src, size_t n);  /* moe_host.c: qg_read, counted */

/* ---------------- index (qwen.c:108-146) ---------------- */

static const qm_tensor *find_tensor(const qwen_model *m, const char *name) {
    for (int i = 0; i < m->n_tensors; i++)
        if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
    return NULL;
}

static const qm_tensor *layer_tensor(const qwen_model *m, int il, const char *suffix) {
    char name[128];
    snprintf(name, sizeof name, "blk.%d.%s", il, suffix);
    return find_tensor(m, name);
}

static void unmap_files(qwen_model *m) {
    for (int i = 0; i < QM_MAX_FILES; i++) {
        qm_file *f = &m->files[i];
        if (f->data) munmap(f->data, f->bytes);
        if (f->fd >= 0) close(f->fd);
        f->data = NULL;
        f->fd = -1;
    }
}

/* Parses the index.  With map = 0 the files are only checked to exist with
 * the stated size (the preflight); with map = 1 they are mapped read-only
 * and each tensor points at its bytes. */
static int read_index(qwen_model *m, const char *path, int map) {
    FILE *f = fopen(path, "r");
    if (!f) return fail("open index: %s", strerror(errno));
    char *line = NULL;
    size_t cap = 0;
    int ret = -1;
    if (getline(&line, &cap, f) < 0 || strcmp(line, "COB_QWEN_INDEX_V1\n")) { fail("invalid Qwen index version"); goto out; }
    if (getline(&line, &cap, f) < 0 || strcmp(line, "VERIFIED 1\n")) {
        fail("weights must pass SHA256 verification before loading");
        goto out;
    }
    /* 3 id multipliers, 16 head offsets, 16 nonzero head vocab sizes, the PLE
     * end-of-sequence id: whitespace-separated integers */
    for (int j = 0; j < 3; j++) if (fscanf(f, "%" SCNu64, &m->multiplier[j]) != 1) goto bad;
    for (int j = 0; j < 16; j++) if (fscanf(f, "%" SCNu64, &m->head_offset[j]) != 1) goto bad;
    for (int j = 0; j < 16; j++) if (fscanf(f, "%" SCNu64, &m->head_vocab[j]) != 1 || !m->head_vocab[j]) goto bad;
    if (fscanf(f, "%d", &m->ple_eos) != 1) goto bad;
    ssize_t n;
    while ((n = getline(&line, &cap, f)) >= 0) {
        if (!strncmp(line, "FILE\t", 5)) {
            int id, used = 0;
            uint64_t bytes;
            if (sscanf(line, "FILE\t%d\t%" SCNu64 "\t%n", &id, &bytes, &used) != 2 || !used || id < 0 || id >= QM_MAX_FILES ||
                m->files[id].bytes)
                goto bad;
            char *p = line + used;
            p[strcspn(p, "\r\n")] = 0;
            qm_file *mf = &m->files[id];
            struct stat st;
            int fd = open(p, O_RDONLY);
            if (fd < 0 || fstat(fd, &st) || (uint64_t)st.st_size != bytes || !bytes) {
                if (fd >= 0) close(fd);
                fail("weights missing/incomplete: %s", p);
                goto out;
            }
            mf->bytes = bytes;
            if (map) {
                mf->fd = fd;
                mf->data = mmap(NULL, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
                if (mf->data == MAP_FAILED) { mf->data = NULL; fail("mmap: %s", strerror(errno)); goto out; }
            } else {
                close(fd);
            }
            if (id >= m->n_files) m->n_files = id + 1;
        } else if (!strncmp(line, "TENSOR\t", 7)) {
            if (m->n_tensors >= QM_MAX_TENSORS) goto bad;
            qm_tensor *t = &m->tensors[m->n_tensors];
            memset(t, 0, sizeof *t);
            if (sscanf(line, "TENSOR\t%127[^\t]\t%d\t%" SCNu64 "\t%" SCNu64 "\t%d\t%" SCNu64 "\t%" SCNu64 "\t%" SCNu64 "\t%" SCNu64,
                       t->name, &t->file, &t->offset, &t->bytes, &t->type, &t->dim[0], &t->dim[1], &t->dim[2], &t->dim[3]) != 9)
                goto bad;
            if (t->file < 0 || t->file >= m->n_files || !m->files[t->file].bytes || !t->bytes ||
                t->offset > m->files[t->file].bytes || t->bytes > m->files[t->file].bytes - t->offset || find_tensor(m, t->name))
                goto bad;
            uint64_t expected = 0;
            if (qg_tensor_bytes(t->type, t->dim, &expected) || expected != t->bytes) goto bad;
            t->host = map ? m->files[t->file].data + t->offset : NULL;
            m->n_tensors++;
        } else if (line[0] != '\n' && line[0] != '\r') {
            goto bad;
        }
    }
    ret = 0;
    goto out;
bad:
    fail("malformed or unsupported Qwen index");
out:
    free(line);
    fclose(f);
    return ret;
}

static int dims_are(const qm_tensor *t, uint64_t d0, uint64_t d1, uint64_t d2) {
    return t && t->dim[0] == d0 && t->dim[1] == d1 && t->dim[2] == d2 && t->dim[3] == 1;
}

/* Binds the MoE tensors of layer il (qwen.c:157-163 with D and F taken from
 * the tensors). */
static int bind_layer(qwen_model *m, int il) {
    qm_layer *l = &m->layers[il];
    l->router = layer_tensor(m, il, "ffn_gate_inp.weight");
    l->eg = layer_tensor(m, il, "ffn_gate_exps.weight");
    l->eu = layer_tensor(m, il, "ffn_up_exps.weight");
    l->ed = layer_tensor(m, il, "ffn_down_exps.weight");
    l->sg = layer_tensor(m, il, "ffn_gate_shexp.weight");
    l->su = layer_tensor(m, il, "ffn_up_shexp.weight");
    l->sd = layer_tensor(m, il, "ffn_down_shexp.weight");
    l->sr = layer_tensor(m, il, "ffn_gate_inp_shexp.weight");
    const uint64_t D = (uint64_t)m->D, F = (uint64_t)m->F;
    if (!dims_are(l->router, D, QM_EXPERTS, 1) || l->router->type != 0 || !dims_are(l->eg, D, F, QM_EXPERTS) ||
        !dims_are(l->eu, D, F, QM_EXPERTS) || !dims_are(l->ed, F, D, QM_EXPERTS) || !dims_are(l->sg, D, F, 1) ||
        !dims_are(l->su, D, F, 1) || !dims_are(l->sd, F, D, 1) || !dims_are(l->sr, D, 1, 1) || l->sr->type != 0)
        return fail("invalid MoE layer %d", il);
    l->gate_bytes = l->eg->bytes / QM_EXPERTS;
    l->up_bytes = l->eu->bytes / QM_EXPERTS;
    l->down_bytes = l->ed->bytes / QM_EXPERTS;
    l->expert_bytes = l->gate_bytes + l->up_bytes + l->down_bytes;
    return 0;
}

/* Whether the device layer's batch kernels (above 17 tokens) take layer il:
 * Q4_K gate/up (routed and shared), Q4_K (F a multiple of 256) or IQ4_NL
 * down, D a multiple of 256 and F of 128.  Batches above 17 tokens of the
 * hotlist target layers and of the MTP layer run there; the cache mode's
 * grouped qg_* path takes any format. */
static int batch_formats_ok(const qwen_model *m, int il) {
    const qm_layer *l = &m->layers[il];
    const int F = m->F;
    if (m->D % 256 || F % 128) return 0;
#define QM_DOWN_OK(t) ((t) == 20 || ((t) == 12 && F % 256 == 0))
    return l->eg->type == 12 && l->eu->type == 12 && QM_DOWN_OK(l->ed->type) && l->sg->type == 12 && l->su->type == 12 &&
           QM_DOWN_OK(l->sd->type);
#undef QM_DOWN_OK
}

/* Layers present: blk.0 .. blk.(n-1) (n <= 48) and optionally blk.48. */
static int bind_model(qwen_model *m) {
    const qm_tensor *g0 = layer_tensor(m, 0, "ffn_gate_exps.weight");
    if (!g0) return fail("index holds no MoE layer 0");
    m->D = (int)g0->dim[0];
    m->F = (int)g0->dim[1];
    if (m->D < 256 || m->D > 8192 || m->D % 256 || m->F < 32 || m->F > 4096 || m->F % 32)
        return fail("unsupported MoE widths %d/%d", m->D, m->F);
    m->n_layers = 0;
    while (m->n_layers < QM_LAYERS && layer_tensor(m, m->n_layers, "ffn_gate_exps.weight")) {
        if (bind_layer(m, m->n_layers)) return -1;
        m->n_layers++;
    }
    m->has_mtp = layer_tensor(m, QM_MTP, "ffn_gate_exps.weight") != NULL;
    if (m->has_mtp && bind_layer(m, QM_MTP)) return -1;
    return 0;
}

int qwen_validate_index(const char *path) {
    if (!path) return fail("index path required");
    qwen_model *m = calloc(1, sizeof *m);
    if (!m) return fail("host allocation");
    m->tensors = calloc(QM_MAX_TENSORS, sizeof *m->tensors);
    for (int i = 0; i < QM_MAX_FILES; i++) m->files[i].fd = -1;
    int rc = !m->tensors ? fail("host allocation") : read_index(m, path, 0);
    if (!rc) rc = bind_model(m);
    free(m->tensors);
    free(m);
    return rc;
}

/* ---------------- open / close ---------------- */

static void *dev_alloc(qwen_model *m, size_t bytes) {
    void *p = qg_alloc(bytes);
    if (p) m->stats.gpu_arena_bytes += bytes;
    return p;
}

static int upload_tensor(qwen_model *m, void **dst, const qm_tensor *t) {
    *dst = dev_alloc(m, t->bytes);
    if (!*dst) return fail("device allocation for %s", t->name);
    GPU(qg_write(*dst, t->host, t->bytes));
    m->stats.gpu_weight_bytes += t->bytes;
    return 0;
}

void qwen_close(qwen_model *m) {
    if (!m) return;
    if (m->route_profile) fclose(m->route_profile);
    for (int il = 0; il <= QM_LAYERS; il++) {
        qm_layer *l = &m->layers[il];
        qg_free(l->d_router); qg_free(l->d_sg); qg_free(l->d_su); qg_free(l->d_sd); qg_free(l->d_sr);
        qg_free(l->d_gate); qg_free(l->d_up); qg_free(l->d_down); qg_free(l->slots);
        free(l->cache_ids);
        free(l->cache_age);
    }
    void *bufs[] = {m->logits, m->route_w, m->slots, m->expert_x, m->ffg, m->ffu, m->ffmid, m->ffout, m->shared,
                    m->shared_gate, m->route_ids, m->route_map, m->flags, m->masks, m->ws, m->handoff, m->prune_device};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) qg_free(bufs[i]);
    if (m->uploader) qg_upload_destroy(m->uploader);
    free(m->h_ids);
    free(m->h_w);
    unmap_files(m);
    free(m->tensors);
    free(m);
}

static int open_device(qwen_model *m) {
    const int D = m->D, F = m->F, T = m->capacity;
    for (int il = 0; il <= QM_LAYERS; il++) {
        if (il >= m->n_layers && !(il == QM_MTP && m->has_mtp)) continue;
        qm_layer *l = &m->layers[il];
        if (upload_tensor(m, &l->d_router, l->router) || upload_tensor(m, &l->d_sg, l->sg) ||
            upload_tensor(m, &l->d_su, l->su) || upload_tensor(m, &l->d_sd, l->sd) || upload_tensor(m, &l->d_sr, l->sr))
            return -1;
        if (il == QM_MTP) {
            /* the MTP layer keeps every expert on the device (qwen.c:690) */
            if (upload_tensor(m, (void **)&l->d_gate, l->eg) || upload_tensor(m, (void **)&l->d_up, l->eu) ||
                upload_tensor(m, (void **)&l->d_down, l->ed))
                return -1;
        } else {
            l->cache_ids = malloc(sizeof(int) * (size_t)m->resident);
            l->cache_age = calloc((size_t)m->resident, sizeof(uint64_t));
            if (!l->cache_ids || !l->cache_age) return fail("host allocation");
            for (int j = 0; j < m->resident; j++) l->cache_ids[j] = -1;
        }
        qg_moe_layer *d = &l->desc;
        memset(d, 0, sizeof *d);
        d->width = D; d->ff = F;
        d->router = l->d_router;
        d->gate = l->d_gate; d->up = l->d_up; d->down = l->d_down;
        d->gate_type = l->eg->type; d->up_type = l->eu->type; d->down_type = l->ed->type;
        d->sh_gate = l->d_sg; d->sh_up = l->d_su; d->sh_down = l->d_sd;
        d->sh_gate_type = l->sg->type; d->sh_up_type = l->su->type; d->sh_down_type = l->sd->type;
        d->sh_gate_inp = l->d_sr;
    }
    const size_t act = (size_t)T * D * 4, sel = (size_t)T * QM_TOP * 4;
    m->ws_bytes = qg_moe_workspace_bytes(D, F, T);
    m->handoff_bytes = nm_handoff_scratch_bytes(D, T);
    if (!m->ws_bytes || !m->handoff_bytes) return fail("unsupported MoE shape for %d tokens", T);
    if (nm_handoff_reserve(D, T)) return fail("handoff host buffers: %s", nm_last_error());
    if (!(m->logits = dev_alloc(m, (size_t)T * QM_EXPERTS * 4)) || !(m->route_w = dev_alloc(m, sel)) ||
        !(m->route_ids = dev_alloc(m, sel)) || !(m->route_map = dev_alloc(m, (size_t)QM_EXPERTS * T * 4)) ||
        !(m->slots = dev_alloc(m, act * QM_TOP)) || !(m->expert_x = dev_alloc(m, act)) ||
        !(m->ffg = dev_alloc(m, (size_t)T * F * 4)) || !(m->ffu = dev_alloc(m, (size_t)T * F * 4)) ||
        !(m->ffmid = dev_alloc(m, (size_t)T * F * 4)) || !(m->ffout = dev_alloc(m, act)) || !(m->shared = dev_alloc(m, act)) ||
        !(m->shared_gate = dev_alloc(m, (size_t)T * 4)) || !(m->flags = dev_alloc(m, (size_t)T)) ||
        !(m->masks = dev_alloc(m, (size_t)QM_LAYERS * QM_EXPERTS)) || !(m->ws = dev_alloc(m, m->ws_bytes)) ||
        !(m->handoff = dev_alloc(m, m->handoff_bytes)))
        return fail("device workspace allocation");
    m->stats.gpu_workspace_bytes = m->stats.gpu_arena_bytes - m->stats.gpu_weight_bytes;
    /* the staging buffers hold the largest expert of any target layer, whose
     * formats may differ from layer to layer (qwen.c:365-367) */
    size_t largest = 0;
    for (int il = 0; il < m->n_layers; il++)
        if (m->layers[il].expert_bytes > largest) largest = m->layers[il].expert_bytes;
    m->uploader = qg_upload_create(largest);
    m->stats.host_staging_bytes = 2 * (uint64_t)largest;
    m->h_ids = malloc(sel);
    m->h_w = malloc(sel);
    if (!m->uploader || !m->h_ids || !m->h_w) return fail("expert uploader allocation");
    GPU(qg_sync());
    return 0;
}

qwen_model *qwen_open(const char *path, int context, int resident, int capacity) {
    if (!path || context < 1 || resident < 1 || resident > QM_EXPERTS || capacity < 1 || capacity > QM_MAX_TOKENS) {
        fail("invalid open arguments");
        return NULL;
    }
    double begin = seconds_now();
    qwen_model *m = calloc(1, sizeof *m);
    if (!m) { fail("host allocation"); return NULL; }
    for (int i = 0; i < QM_MAX_FILES; i++) m->files[i].fd = -1;
    m->tensors = calloc(QM_MAX_TENSORS, sizeof *m->tensors);
    m->context = context; m->resident = resident; m->capacity = capacity;
    if (!m->tensors) { fail("host allocation"); free(m); return NULL; }
    if (read_index(m, path, 1) || bind_model(m)) { unmap_files(m); free(m->tensors); free(m); return NULL; }
    if (capacity > QWEN_MAX_DRAFT + 1 && m->has_mtp && !batch_formats_ok(m, QM_MTP)) {
        fail("batch capacity %d above %d needs Q4_K gate/up and Q4_K or IQ4_NL down in the MTP layer", capacity,
             QWEN_MAX_DRAFT + 1);
        unmap_files(m); free(m->tensors); free(m);
        return NULL;
    }
    /* width-less drop-in entry points of this thread use this model's shape */
    int rc = qg_moe_configure_thread(m->D, m->F);
    if (rc) { fail("qg_moe_configure_thread: %s", qg_error(rc)); qwen_close(m); return NULL; }
    if (open_device(m)) { qwen_close(m); return NULL; }
    for (int il = 0; il < m->n_layers; il++)
        m->stats.host_weight_bytes += m->layers[il].eg->bytes + m->layers[il].eu->bytes + m->layers[il].ed->bytes;
    m->stats.context = context;
    m->stats.resident_per_layer = resident;
    m->stats.core_load_seconds = seconds_now() - begin;
    return m;
}

int qwen_moe_shape(qwen_model *m, int *width, int *ff, int *layers, int *has_mtp) {
    if (!m) return fail("model required");
    if (width) *width = m->D;
    if (ff) *ff = m->F;
    if (layers) *layers = m->n_layers;
    if (has_mtp) *has_mtp = m->has_mtp;
    return 0;
}

int qwen_set_cpu_moe(qwen_model *m, qwen_cpu_moe_fn fn, void *ctx) {
    if (!m || !fn) return fail("CPU MoE function required");
    m->cpu_moe = fn;
    m->cpu_ctx = ctx;
    return 0;
}

/* ---------------- expert cache (qwen.c:558-570) ---------------- */

/* Device destination of expert e: its place in the per-tensor layout once a
 * hotlist is being pinned (the layout the device layer reads), else cache
 * slot `slot` (gate|up|down, the reference's expert_cache layout). */
static int upload_expert(qwen_model *m, qm_layer *l, int e, int slot, int pinned) {
    const unsigned char *g = l->eg->host + (size_t)e * l->gate_bytes, *u = l->eu->host + (size_t)e * l->up_bytes,
                        *d = l->ed->host + (size_t)e * l->down_bytes;
    int rc;
    if (pinned) {
        if ((rc = qg_upload_expert(m->uploader, l->d_gate + (size_t)e * l->gate_bytes, g, l->gate_bytes, u, 0, d, 0)) ||
            (rc = qg_upload_expert(m->uploader, l->d_up + (size_t)e * l->up_bytes, u, l->up_bytes, g, 0, d, 0)) ||
            (rc = qg_upload_expert(m->uploader, l->d_down + (size_t)e * l->down_bytes, d, l->down_bytes, g, 0, u, 0)))
            return fail("expert handoff upload: %s", qg_error(rc));
    } else if ((rc = qg_upload_expert(m->uploader, l->slots + (size_t)slot * l->expert_bytes, g, l->gate_bytes, u, l->up_bytes,
                                      d, l->down_bytes))) {
        return fail("expert handoff upload: %s", qg_error(rc));
    }
    return 0;
}

/* The slot holding expert e, uploading it first when absent: a free slot,
 * else the least recently used slot whose expert is not protected.  With a
 * fixed hotlist a missing expert is an error (it belongs to the CPU). */
static int cache_slot(qwen_model *m, qm_layer *l, int e, const unsigned char *protected_ids, int pinned) {
    for (int j = 0; j < m->resident; j++)
        if (l->cache_ids[j] == e) { l->cache_age[j] = ++l->clock; return j; }
    if (m->fixed_hotlist) return fail("fixed hotlist must never upload a missing expert");
    int slot = -1;
    uint64_t oldest = UINT64_MAX;
    for (int j = 0; j < m->resident; j++) {
        if (l->cache_ids[j] < 0) { slot = j; break; }
        if (!protected_ids[l->cache_ids[j]] && l->cache_age[j] < oldest) { oldest = l->cache_age[j]; slot = j; }
    }
    if (slot < 0) return fail("expert cache has no evictable slot");
    double begin = seconds_now();
    if (upload_expert(m, l, e, slot, pinned)) return -1;
    l->cache_ids[slot] = e;
    l->cache_age[slot] = ++l->clock;
    m->stats.expert_handoffs++;
    m->stats.expert_upload_bytes += l->expert_bytes;
    m->stats.expert_handoff_host_seconds += seconds_now() - begin;
    return slot;
}

/* ---------------- hotlist (qwen.c:571-613) ---------------- */

int qwen_set_hotlist(qwen_model *m, const int *ids, int count, int threads) {
    if (!m || !ids || count != m->n_layers * m->resident || threads < 1 || threads > 28 || m->ran_target ||
        m->fixed_hotlist)
        return fail("hotlist requires a fresh target and matching capacity");
    for (int il = 0; il < m->n_layers; il++) {
        unsigned char seen[QM_EXPERTS] = {0};
        for (int j = 0; j < m->resident; j++) {
            const int e = ids[il * m->resident + j];
            if (e < 0 || e >= QM_EXPERTS || seen[e]) return fail("invalid or duplicate hotlist expert in layer %d", il);
            seen[e] = 1;
        }
    }
    if (m->capacity > QWEN_MAX_DRAFT + 1)
        for (int il = 0; il < m->n_layers; il++)
            if (!batch_formats_ok(m, il))
                return fail("hotlist with batch capacity %d above %d needs Q4_K gate/up and Q4_K or IQ4_NL down (layer %d)",
                            m->capacity, QWEN_MAX_DRAFT + 1, il);
    if (m->hotlist_tried) return fail("CPU hotlist initialization already attempted; reopen the model");
    m->hotlist_tried = 1;
    if (!m->cpu_moe) return fail("register the CPU MoE (qwen_set_cpu_moe) before the hotlist");
    if (!m->prune_device && !(m->prune_device = dev_alloc(m, sizeof(qg_prune_stats))))
        return fail("hotlist routing allocation");
    unsigned char *masks = calloc((size_t)QM_LAYERS * QM_EXPERTS, 1);
    if (!masks) return fail("host allocation");
    for (int il = 0; il < m->n_layers; il++) {
        qm_layer *l = &m->layers[il];
        if (!l->d_gate && (!(l->d_gate = dev_alloc(m, l->eg->bytes)) || !(l->d_up = dev_alloc(m, l->eu->bytes)) ||
                           !(l->d_down = dev_alloc(m, l->ed->bytes)))) {
            free(masks);
            return fail("device allocation for the layer %d experts", il);
        }
        unsigned char keep[QM_EXPERTS] = {0};
        for (int j = 0; j < m->resident; j++) keep[ids[il * m->resident + j]] = 1;
        /* the cache is empty here: every pinned expert takes a free slot */
        for (int j = 0; j < m->resident; j++)
            if (cache_slot(m, l, ids[il * m->resident + j], keep, 1) < 0) { free(masks); return -1; }
        for (int j = 0; j < m->resident; j++) {
            masks[(size_t)il * QM_EXPERTS + ids[il * m->resident + j]] = 1;
            l->pinned[ids[il * m->resident + j]] = 1;
        }
        l->desc.gate = l->d_gate; l->desc.up = l->d_up; l->desc.down = l->d_down;
        l->desc.resident = m->masks + (size_t)il * QM_EXPERTS;
        l->desc.threshold = 0.10;   /* omitted-mass threshold (config.py:9) */
    }
    int rc = qg_write(m->masks, masks, (size_t)QM_LAYERS * QM_EXPERTS);
    free(masks);
    if (rc) return fail("qg_write masks: %s", qg_error(rc));
    GPU(qg_zero(m->prune_device, sizeof(qg_prune_stats)));
    GPU(qg_sync());
    m->cpu_threads = threads;
    m->fixed_hotlist = 1;
    return 0;
}

int qwen_set_cpu_threads(qwen_model *m, int threads) {
    if (!m || !m->fixed_hotlist || threads < 1 || threads > 28)
        return fail("CPU thread count must be 1..28 on an initialized idle model");
    m->cpu_threads = threads;
    return 0;
}
int qwen_cpu_threads(qwen_model *m) { return m ? m->cpu_threads : 0; }
void qwen_get_cpu_stats(qwen_model *m, qwen_cpu_stats *out) { if (m && out) *out = m->cpu_stats; }
void qwen_get_handoff_profile(qwen_model *m, qwen_handoff_profile *out) { if (m && out) *out = m->profile; }
/* In hotlist mode the selections are counted on the device (the prune
 * counters of qg_moe_forward) instead of reading every layer's ids back
 * (qwen.c:649-657): a token with a valid routing has 10 - missing resident
 * selections, so the layers' hits are 10 token_layers - missing_selections. */
void qwen_get_stats(qwen_model *m, qwen_stats *out) {
    if (!m || !out) return;
    *out = m->stats;
    qg_prune_stats p;
    if (m->fixed_hotlist && m->prune_device && !nm_read(&p, m->prune_device, sizeof p))
        out->expert_hits += QM_TOP * p.token_layers - p.missing_selections;
}

int qwen_get_prune_stats(qwen_model *m, qwen_prune_stats *out) {
    if (!m || !out || !m->prune_device) return fail("hotlist statistics unavailable");
    GPU(nm_read(out, m->prune_device, sizeof *out));
    return 0;
}

/* ---------------- route trace (qwen.c:86-94,638-646) ---------------- */

int qwen_profile_routes(qwen_model *m, const char *path) {
    if (!m) return fail("route profile requires an open model");
    if (m->route_profile) {
        FILE *old = m->route_profile;
        m->route_profile = NULL;
        if (fclose(old)) return fail("close route profile: %s", strerror(errno));
    }
    if (!path) return 0;
    FILE *f = fopen(path, "wb");
    if (!f) return fail("open route profile: %s", strerror(errno));
    if (fwrite("QROUTE1\n", 1, 8, f) != 8) { fclose(f); return fail("write route profile header"); }
    m->route_profile = f;
    return 0;
}

/* Router logits and top-10 (ids/weights before any pruning) into route_ids /
 * route_w, copied to h_ids / h_w; the same arithmetic the device layer uses. */
static int route_to_host(qwen_model *m, qm_layer *l, const float *x, int nt) {
    GPU(qg_matmul(m->logits, l->d_router, 0, QM_EXPERTS, m->D, x, nt));
    GPU(qg_route(m->route_ids, m->route_w, m->logits, nt));
    GPU(nm_read(m->h_ids, m->route_ids, (size_t)nt * QM_TOP * 4));
    GPU(nm_read(m->h_w, m->route_w, (size_t)nt * QM_TOP * 4));
    m->stats.metadata_read_bytes += (uint64_t)nt * QM_TOP * 4;
    return 0;
}

static int trace_routes(qwen_model *m, int il, int position, int nt) {
    const uint32_t header[3] = {(uint32_t)il, (uint32_t)position, (uint32_t)nt};
    const size_t n = (size_t)nt * QM_TOP;
    if (fwrite(header, sizeof(uint32_t), 3, m->route_profile) != 3 || fwrite(m->h_ids, sizeof(int), n, m->route_profile) != n ||
        fwrite(m->h_w, sizeof(float), n, m->route_profile) != n)
        return fail("write route profile");
    return 0;
}

/* ---------------- moe() (qwen.c:714-735) ---------------- */

typedef struct { qwen_model *m; qm_layer *l; uint64_t missing; } cpu_call;

/* The registered CPU MoE on the handed-off rows; compute_seconds counts this
 * call alone, without the device reads and writes around it (qwen.c:663-668). */
static int cpu_moe_tokens(void *ctx, float *out, const float *x, const int *ids, const float *weights, int nt) {
    cpu_call *c = ctx;
    /* the handed-off tokens' selections of experts not on the device (the
     * batch's other missing selections were pruned, qwen.c:656) */
    for (int j = 0; j < nt * QM_TOP; j++)
        if (ids[j] >= 0 && ids[j] < QM_EXPERTS && !c->l->pinned[ids[j]]) c->missing++;
    const double begin = seconds_now();
    const int rc = c->m->cpu_moe(c->m->cpu_ctx, out, x, ids, weights, nt, c->l->eg->host, c->l->eg->type, c->l->eu->host,
                                 c->l->eu->type, c->l->ed->host, c->l->ed->type);
    c->m->cpu_stats.compute_seconds += seconds_now() - begin;
    return rc;
}

/* Fixed hotlist: the device layer with the resident mask; flag-2 tokens'
 * routed parts come from the host's CPU MoE.  Nothing is read back for a
 * layer without a flag-2 token (the handoff learns the count from a host
 * word the device writes); hits are counted on the device. */
static int moe_hotlist(qwen_model *m, int il, float *out, const float *x, int nt) {
    qm_layer *l = &m->layers[il];
    GPU(qg_moe_forward(out, m->route_ids, m->route_w, m->flags, m->prune_device, x, nt, &l->desc, m->ws, m->ws_bytes));
    m->stats.expert_requests += (uint64_t)nt * QM_TOP;
    const double begin = seconds_now();
    cpu_call c = {m, l, 0};
    int handed = 0;
    if (nm_moe_handoff(out, NULL, m->flags, x, m->route_ids, m->route_w, nt, m->D, m->handoff, m->handoff_bytes,
                       cpu_moe_tokens, &c, &handed))
        return fail("CPU MoE handoff: %s", nm_last_error());
    m->profile.layer_calls[il]++;
    if (handed) {
        m->cpu_stats.handoff_seconds += seconds_now() - begin;
        m->cpu_stats.layer_handoffs++;
        m->cpu_stats.token_layers += (uint64_t)handed;
        m->cpu_stats.missing_selections += c.missing;
        m->cpu_stats.activation_bytes += (uint64_t)handed * ((uint64_t)m->D * 8 + QM_TOP * 4);
        m->profile.layer_handoffs[il]++;
    }
    return 0;
}

/* No hotlist: grouped_moe (qwen.c:633-707) over the LRU expert cache, then
 * the rank-order reduce and shared_direct (qwen.c:708-713). */
static int moe_cached(qwen_model *m, int il, float *out, const float *x, int nt) {
    qm_layer *l = &m->layers[il];
    const int D = m->D, F = m->F;
    if (!l->slots && !(l->slots = dev_alloc(m, (size_t)m->resident * l->expert_bytes)))
        return fail("device allocation for the layer %d expert cache", il);
    const uint64_t uploads_before = m->stats.expert_handoffs;
    unsigned char needed[QM_EXPERTS] = {0}, resident[QM_EXPERTS] = {0};
    int counts[QM_EXPERTS] = {0}, order[QM_EXPERTS], n_order = 0;
    for (int j = 0; j < nt * QM_TOP; j++) {
        const int e = m->h_ids[j];
        if (e < 0 || e >= QM_EXPERTS) return fail("non-finite router distribution");
        needed[e] = 1;
        counts[e]++;
    }
    for (int j = 0; j < m->resident; j++) if (l->cache_ids[j] >= 0) resident[l->cache_ids[j]] = 1;
    for (int j = 0; j < nt * QM_TOP; j++) { m->stats.expert_requests++; m->stats.expert_hits += resident[m->h_ids[j]]; }
    if (nt > 1) GPU(qg_moe_map(m->route_map, m->route_ids, nt));
    /* resident experts first, releasing their slots before cold ones arrive */
    for (int phase = 0; phase < 2; phase++)
        for (int e = 0; e < QM_EXPERTS; e++) if (needed[e] && (resident[e] ? 0 : 1) == phase) order[n_order++] = e;
    GPU(qg_zero(m->slots, (size_t)nt * QM_TOP * D * 4));
    for (int j = 0; j < n_order; j++) {
        const int e = order[j], ne = counts[e];
        const float *input = x;
        const int *token_map = NULL;
        if (ne < nt) {
            token_map = m->route_map + (size_t)e * nt;
            GPU(qg_moe_gather(m->expert_x, x, token_map, ne));
            input = m->expert_x;
        }
        const int slot = cache_slot(m, l, e, needed, 0);
        if (slot < 0) return -1;
        const unsigned char *wg = l->slots + (size_t)slot * l->expert_bytes, *wu = wg + l->gate_bytes, *wd = wu + l->up_bytes;
        GPU(qg_matmul(m->ffg, wg, l->eg->type, F, D, input, ne));
        GPU(qg_matmul(m->ffu, wu, l->eu->type, F, D, input, ne));
        GPU(qg_unary(m->ffmid, m->ffg, ne * F, 0, 1.0f));
        GPU(qg_binary(m->ffmid, m->ffmid, m->ffu, ne * F, 1));
        GPU(qg_matmul(m->ffout, wd, l->ed->type, D, F, m->ffmid, ne));
        GPU(qg_moe_scatter(m->slots, m->ffout, m->route_w, m->route_ids, token_map, e, ne));
        needed[e] = 0;
    }
    m->profile.layer_calls[il]++;
    m->profile.layer_handoffs[il] += m->stats.expert_handoffs != uploads_before;
    GPU(qg_moe_reduce(out, m->slots, nt));
    GPU(qg_matmul(m->ffg, l->d_sg, l->sg->type, F, D, x, nt));
    GPU(qg_matmul(m->ffu, l->d_su, l->su->type, F, D, x, nt));
    GPU(qg_unary(m->ffmid, m->ffg, nt * F, 0, 1.0f));
    GPU(qg_binary(m->ffmid, m->ffmid, m->ffu, nt * F, 1));
    GPU(qg_matmul(m->shared, l->d_sd, l->sd->type, D, F, m->ffmid, nt));
    GPU(qg_matmul(m->shared_gate, l->d_sr, 0, 1, D, x, nt));
    GPU(qg_shared_add(out, m->shared, m->shared_gate, nt));
    return 0;
}

int qwen_moe(qwen_model *m, int il, float *out, const float *x, int nt, int position) {
    if (!m || !out || !x || nt < 1 || nt > m->capacity || position < 0) return fail("invalid MoE call");
    const int mtp = il == QM_MTP;
    if (mtp ? !m->has_mtp : (il < 0 || il >= m->n_layers)) return fail("no MoE layer %d", il);
    if (!mtp && position + nt > m->context) return fail("target batch exceeds context");
    GPU(qg_moe_configure_thread(m->D, m->F));
    const double begin = seconds_now();
    int rc;
    if (mtp) {
        GPU(qg_moe_forward(out, m->route_ids, m->route_w, NULL, NULL, x, nt, &m->layers[il].desc, m->ws, m->ws_bytes));
        rc = 0;
    } else {
        m->ran_target = 1;
        /* the routes as selected, before pruning, when tracing or when the
         * host drives the expert loop */
        if ((m->route_profile || !m->fixed_hotlist) && route_to_host(m, &m->layers[il], x, nt)) return -1;
        if (m->route_profile && trace_routes(m, il, position, nt)) return -1;
        rc = m->fixed_hotlist ? moe_hotlist(m, il, out, x, nt) : moe_cached(m, il, out, x, nt);
    }
    if (rc) return rc;
    /* no synchronisation: the layer's device work is ordered on the calling
     * thread's stream, like the reference's moe(); a hotlist layer has
     * already waited for its handoff decision */
    if (mtp) {
        m->stats.mtp_tokens += (uint64_t)nt;
        m->stats.mtp_seconds += seconds_now() - begin;
        m->stats.mtp_position = position + nt;
    } else {
        if (il == 0) m->stats.target_tokens += (uint64_t)nt;
        m->stats.target_seconds += seconds_now() - begin;
        m->stats.target_position = position + nt;
    }
    return 0;
}
