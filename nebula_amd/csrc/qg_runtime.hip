// Runtime half of libqwen_gpu.so: memory, copies, streams, graphs, the
// pinned expert uploader and event timing, behind the reference's C ABI
// (gpu.h:11-36).  Return codes are hipError_t values (0 = success) and the
// text comes from qg_error, as gpu.cu:38-46 does with cudaError_t.
#include "qg_internal.h"
#include <stdlib.h>
#include <string.h>
#include <mutex>
#include <vector>

// Kernels launch on the calling thread's stream: the null stream, or the
// capture stream between qg_graph_begin and qg_graph_end (gpu.cu:10,21-34).
static thread_local hipStream_t tl_stream = nullptr;
hipStream_t qg_stream(void) { return tl_stream; }

namespace {
__global__ void fill_zero_kernel(uint32_t *p, size_t words) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, step = (size_t)gridDim.x * blockDim.x;
    for (; i < words; i += step) p[i] = 0u;
}
__global__ void fill_zero_bytes_kernel(uint8_t *p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}
__global__ void copy_kernel(uint4 *dst, const uint4 *src, size_t n16) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, step = (size_t)gridDim.x * blockDim.x;
    for (; i < n16; i += step) dst[i] = src[i];
}
__global__ void copy_bytes_kernel(uint8_t *dst, const uint8_t *src, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}
}  // namespace

extern "C" {

void *qg_alloc(size_t n) {  // gpu.cu:38: NULL on failure
    void *p = nullptr;
    return hipMalloc(&p, n ? n : 1) == hipSuccess ? p : nullptr;
}
void qg_free(void *p) { if (p) (void)hipFree(p); }
int qg_write(void *d, const void *s, size_t n) { return hipMemcpy(d, s, n, hipMemcpyHostToDevice); }
int qg_read(void *d, const void *s, size_t n) { return hipMemcpy(d, s, n, hipMemcpyDeviceToHost); }

// Device-to-device copy on the calling thread's stream.  A kernel, not
// hipMemcpyAsync, so that it records as a plain kernel node under capture.
int qg_copy(void *d, const void *s, size_t n) {
    if (!n) return hipSuccess;
    if (!d || !s) return hipErrorInvalidValue;
    if ((((uintptr_t)d | (uintptr_t)s | n) & 15) == 0) {
        size_t n16 = n / 16;
        unsigned blocks = (unsigned)((n16 + 255) / 256 < 4096 ? (n16 + 255) / 256 : 4096);
        copy_kernel<<<blocks, 256, 0, tl_stream>>>((uint4 *)d, (const uint4 *)s, n16);
    } else {
        copy_bytes_kernel<<<(unsigned)((n + 255) / 256), 256, 0, tl_stream>>>((uint8_t *)d, (const uint8_t *)s, n);
    }
    return hipGetLastError();
}

// Zero fill with a kernel (gpu.cu:43 uses cudaMemsetAsync; memset nodes are
// avoided here because this call is legal inside a capture).
int qg_zero(void *d, size_t n) {
    if (!n) return hipSuccess;
    if (!d) return hipErrorInvalidValue;
    if ((((uintptr_t)d | n) & 3) == 0) {
        size_t words = n / 4;
        unsigned blocks = (unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
        fill_zero_kernel<<<blocks, 256, 0, tl_stream>>>((uint32_t *)d, words);
    } else {
        fill_zero_bytes_kernel<<<(unsigned)((n + 255) / 256), 256, 0, tl_stream>>>((uint8_t *)d, n);
    }
    return hipGetLastError();
}
int qg_sync(void) { return hipDeviceSynchronize(); }

// Page-locked host memory that kernels may read and write through the same
// address (a mailbox the host polls without a device-to-host copy).
void *qg_host_alloc(size_t n) {
    void *p = nullptr;
    return hipHostMalloc(&p, n ? n : 1, hipHostMallocDefault) == hipSuccess ? p : nullptr;
}
void qg_host_free(void *p) { if (p) (void)hipHostFree(p); }

}  // extern "C"

// Library-owned scratch that grows on demand.  A graph captured earlier may
// still hold the old buffer's address, so a superseded buffer is never freed:
// it is kept on a retired list until the process ends.  Growth is at least
// twofold, so the retired buffers together stay below the live one's size.
// Growing is refused inside a capture (the allocation would not be replayed).
namespace {
std::mutex g_retired_mu;
std::vector<void *> *g_retired = nullptr;
}
int qg_scratch_grow(void **buf, size_t *cap, size_t need) {
    if (*cap >= need) return hipSuccess;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (tl_stream && hipStreamIsCapturing(tl_stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone)
        return hipErrorInvalidValue;
    size_t bytes = need > 2 * *cap ? need : 2 * *cap;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return hipErrorOutOfMemory;
    if (*buf) {
        std::lock_guard<std::mutex> lock(g_retired_mu);
        if (!g_retired) g_retired = new std::vector<void *>();
        g_retired->push_back(*buf);
    }
    *buf = p;
    *cap = bytes;
    return hipSuccess;
}

extern "C" {
int qg_memory(size_t *f, size_t *t) { return hipMemGetInfo(f, t); }
const char *qg_error(int e) { return hipGetErrorString((hipError_t)e); }

// Bytes of a GGML tensor with dims[0] columns (gpu.cu:114-120).
int qg_tensor_bytes(int type, const uint64_t dims[4], uint64_t *bytes) {
    if (!dims || !bytes || dims[0] < 1 || dims[0] > 2147483647ULL) return hipErrorInvalidValue;
    int block = (type == QT_Q4_K || type == QT_Q5_K || type == QT_Q6_K) ? 256
              : (type == QT_Q4_0 || type == QT_Q5_0 || type == QT_Q4_1 || type == QT_Q8_0 || type == QT_IQ4_NL) ? 32 : 1;
    uint64_t n = qg_row_bytes_host(type, (int)dims[0]);
    if (!n || dims[0] % block) return hipErrorInvalidValue;
    for (int i = 1; i < 4; i++) {
        if (!dims[i] || dims[i] > UINT64_MAX / n) return hipErrorInvalidValue;
        n *= dims[i];
    }
    *bytes = n;
    return hipSuccess;
}

// ---- graphs (gpu.cu:12-37): thread-local capture into a private stream ----
struct qg_graph {
    hipStream_t stream;
    hipGraph_t graph;
    hipGraphExec_t exec;
    int active;
};

void qg_graph_destroy(void *ptr) {
    qg_graph *g = (qg_graph *)ptr;
    if (!g) return;
    if (g->active) {
        hipGraph_t dropped = nullptr;
        (void)hipStreamEndCapture(g->stream, &dropped);
        if (dropped) (void)hipGraphDestroy(dropped);
        tl_stream = nullptr;
    }
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->stream) (void)hipStreamDestroy(g->stream);
    free(g);
}

int qg_graph_begin(void **out) {
    if (!out || *out || tl_stream) return hipErrorInvalidValue;
    qg_graph *g = (qg_graph *)calloc(1, sizeof(*g));
    if (!g) return hipErrorOutOfMemory;
    int rc = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
    if (!rc) rc = hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal);
    if (rc) { qg_graph_destroy(g); return rc; }
    g->active = 1;
    tl_stream = g->stream;
    *out = g;
    return hipSuccess;
}

int qg_graph_end(void *ptr) {
    qg_graph *g = (qg_graph *)ptr;
    if (!g || !g->active) return hipErrorInvalidValue;
    int rc = hipStreamEndCapture(g->stream, &g->graph);
    g->active = 0;
    tl_stream = nullptr;
    if (!rc) rc = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    return rc;
}

int qg_graph_launch(void *ptr) {
    qg_graph *g = (qg_graph *)ptr;
    return g && g->exec ? hipGraphLaunch(g->exec, tl_stream) : hipErrorInvalidValue;
}

// ---- pinned double-buffered expert uploader (gpu.cu:48-85) ----
struct qg_uploader {
    unsigned char *stage[2];
    hipEvent_t begin[2], end[2];
    int next, pending[2];
    size_t capacity;
    double seconds;
};

void qg_upload_destroy(void *ptr) {
    qg_uploader *u = (qg_uploader *)ptr;
    if (!u) return;
    (void)hipDeviceSynchronize();
    for (int i = 0; i < 2; i++) {
        if (u->stage[i]) (void)hipHostFree(u->stage[i]);
        if (u->begin[i]) (void)hipEventDestroy(u->begin[i]);
        if (u->end[i]) (void)hipEventDestroy(u->end[i]);
    }
    free(u);
}

void *qg_upload_create(size_t bytes) {
    qg_uploader *u = (qg_uploader *)calloc(1, sizeof(*u));
    if (!u) return nullptr;
    u->capacity = bytes;
    for (int i = 0; i < 2; i++)
        if (hipHostMalloc((void **)&u->stage[i], bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess ||
            hipEventCreate(&u->begin[i]) != hipSuccess || hipEventCreate(&u->end[i]) != hipSuccess) {
            qg_upload_destroy(u);
            return nullptr;
        }
    return u;
}

static int upload_finish(qg_uploader *u, int i, int wait) {
    if (!u->pending[i]) return hipSuccess;
    hipError_t rc = wait ? hipEventSynchronize(u->end[i]) : hipEventQuery(u->end[i]);
    if (rc == hipErrorNotReady) return hipSuccess;
    if (rc != hipSuccess) return rc;
    float ms = 0;
    rc = hipEventElapsedTime(&ms, u->begin[i], u->end[i]);
    if (rc != hipSuccess) return rc;
    u->seconds += ms / 1000.0;
    u->pending[i] = 0;
    return hipSuccess;
}

int qg_upload_expert(void *ptr, void *dst, const void *g, size_t ng, const void *up, size_t nu, const void *down, size_t nd) {
    qg_uploader *u = (qg_uploader *)ptr;
    if (!u || ng > u->capacity || nu > u->capacity - ng || nd > u->capacity - ng - nu) return hipErrorInvalidValue;
    int i = u->next, rc = upload_finish(u, i, 1);
    if (rc) return rc;
    memcpy(u->stage[i], g, ng);
    memcpy(u->stage[i] + ng, up, nu);
    memcpy(u->stage[i] + ng + nu, down, nd);
    if ((rc = hipEventRecord(u->begin[i], tl_stream))) return rc;
    if ((rc = hipMemcpyAsync(dst, u->stage[i], ng + nu + nd, hipMemcpyHostToDevice, tl_stream))) return rc;
    if ((rc = hipEventRecord(u->end[i], tl_stream))) return rc;
    u->pending[i] = 1;
    u->next = 1 - i;
    return hipSuccess;
}

double qg_upload_seconds(void *ptr) {
    qg_uploader *u = (qg_uploader *)ptr;
    if (!u) return 0;
    for (int i = 0; i < 2; i++) if (upload_finish(u, i, 0)) return -1;
    return u->seconds;
}

// ---- event timing on the calling thread's stream (no reference counterpart;
// used by the benchmark to time kernels on the stream they run on) ----
void *qg_event_create(void) {
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? (void *)e : nullptr;
}
void qg_event_destroy(void *e) { if (e) (void)hipEventDestroy((hipEvent_t)e); }
int qg_event_record(void *e) { return e ? hipEventRecord((hipEvent_t)e, tl_stream) : hipErrorInvalidValue; }
int qg_event_elapsed(float *ms, void *begin, void *end) {
    if (!ms || !begin || !end) return hipErrorInvalidValue;
    int rc = hipEventSynchronize((hipEvent_t)end);
    if (!rc) rc = hipEventElapsedTime(ms, (hipEvent_t)begin, (hipEvent_t)end);
    // an event that was never recorded is reported here only: clear the
    // runtime's sticky last error so the next launch check does not see it
    if (rc) (void)hipGetLastError();
    return rc;
}

// Device description for roofline bookkeeping.
int qg_device_info(char *name, size_t name_len, int *cus, int *clock_khz, int *mem_clock_khz, int *bus_bits) {
    int dev = 0, rc = hipGetDevice(&dev);
    if (rc) return rc;
    hipDeviceProp_t p;
    if ((rc = hipGetDeviceProperties(&p, dev))) return rc;
    if (name && name_len) { strncpy(name, p.gcnArchName, name_len - 1); name[name_len - 1] = 0; }
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (mem_clock_khz) *mem_clock_khz = p.memoryClockRate;
    if (bus_bits) *bus_bits = p.memoryBusWidth;
    return hipSuccess;
}

}  // extern "C"

int qg_cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            v <= 0)
            return 256;
        n = v;
    }
    return n;
}
