// Routed-MoE layer for prefill batches (18..8192 tokens): the path of
// qg_moe_forward / qg_moe_forward_residual above the decode sizes, for Q4_K
// gate/up and Q4_K or IQ4_NL down.  It replaces the per-expert loop of
// qwen.c:680-700 (qg_moe_map, then qg_matmul x3 and qg_moe_scatter per expert,
// or qc_moe of cpu.c:235-261 on the CPU handoff) with grouped GEMMs over
// per-expert row lists built on the device.
//
// Kernels per layer:
//   P1 router   : exact-order router GEMM (the summation order of
//                 cpu.c:122-139, so logits and routing are bit-exact), rows
//                 0..511 plus the shared gate vector, + optional bias.
//   P2 route    : a wave per token: top-10, coverage/prune, flags, and the
//                 token's fp16 activation planes.
//   P2b count   : per 32-token chunk, the per-expert token masks, whose
//                 popcounts are the chunk's histogram counts[chunk][e].
//   P3 scan     : per-expert totals, CSR offsets, per-chunk bases (exclusive
//                 prefix over chunks), and the table of 64-row tiles per group.
//   P4 fill     : the stable permutation: a selection's row is its chunk's base
//                 plus the rank of its token in the chunk's mask, so each
//                 expert's rows are in ascending token order (the order of
//                 moe_map_kernel, gpu.cu:489-500).
//   P5 gate/up  : persistent grouped GEMM, one launch over every group
//                 (the int8 variant: the dense experts in a launch of their
//                 own); item = (group, 64-row tile, 128 F rows); SwiGLU; mid
//                 rows as fp16 hi/lo planes.
//   P6 down     : persistent grouped GEMM, one launch (three when the shared
//                 expert's down format differs); item = (group, 64-row tile,
//                 256 D rows); y rows written to the selection's slot.
//   P7 combine  : out[t] = sum over ranks k of w[t,k]*y[t,k] in rank order,
//                 + sigmoid-gated shared expert, + optional residual.
// Groups are the 512 experts plus the shared expert (group 512, every token).
//
// GEMM tiles (operand conventions of qg_frag.h): a workgroup is 8 waves, one
// per CU; each workgroup streams the (item, K step) steps of its items, the
// items cut between XCDs by estimated cost (balanced_items).  The tile's
// activation rows (64 rows x 2 planes x one K step) are staged in shared
// memory by direct global->shared copies, double-buffered over steps; each
// wave owns 32 weight rows (gate/up: 16 gate + 16 up) whose quantised bytes
// it copies, two steps ahead, into a ring of its own in shared memory (the
// Q4_K down launch keeps them in registers instead).  A
// 16x16x32 MFMA pair (hi and lo plane) per (row tile, column tile, 32-element
// group); row tiles past the group's last row are skipped.  16-byte chunk c of
// a staged row r sits at chunk c ^ (r & 15), so the 16 rows one MFMA reads
// hit 16 different bank groups.
#include "qg_internal.h"
#include "qg_frag.h"
#include <hip/hip_ext.h>
#include <type_traits>

namespace {

constexpr int PF_MIN = QG_MAX_DECODE + 1;   // smallest batch on this path
constexpr int PF_CHUNK = 32;                 // tokens per routing chunk (one 32-bit mask per expert)
constexpr int PT = 64;                       // rows per GEMM tile
constexpr int KC = 256;                      // K elements per staged chunk
constexpr int GU_FB = 128;                   // F rows per gate/up item (16 per wave)
constexpr int DN_DB = 256;                   // D rows per down item (32 per wave)
constexpr int NG = QG_EXPERTS + 1;           // groups: experts + shared expert
constexpr int DENSE_MIN = 256;               // rows from which an expert is dense (pass order; the int8 variant)
constexpr int STAGE_BYTES = PT * 2 * KC * 2; // [64 rows][2 planes][256] fp16
constexpr int SUMS_BYTES = PT * 2 * 16;      // [64 rows][2 planes][8 group sums] fp16
constexpr int PF_LDS = 2 * (STAGE_BYTES + SUMS_BYTES);

// Groups in pass order: the dense experts (>= DENSE_MIN rows), the shared
// expert, the other experts; experts by row count, largest first (ties by
// expert id), so a pass's big tiles come first.  Order position p holds
// group gorder[p], whose tiles start at tbase[p]; tiles bounds[s] ..
// bounds[s+1]-1 form segment s (0 dense, 1 shared, 2 the others).  mbase /
// mbounds: the same prefixes of the row-tile counts M (a group of n rows has
// ceil(n / 16) of them over its tiles).
struct TileTable { int bounds[4]; int tbase[NG + 1]; int gorder[NG]; int mbase[NG + 1]; int mbounds[4]; };

struct PfLayout {
    size_t logits, flag, missing, mass, xp, xsp, counts, offsets, tbase, row_token, row_slot, midp, msp, slots, xn, xi8, xsc,
        row_sx, total;
};
PfLayout pf_layout(int D, int F, int nt) {
    PfLayout L;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += (n + 255) & ~(size_t)255; return o; };
    const size_t nch = (nt + PF_CHUNK - 1) / PF_CHUNK, rows = (size_t)nt * (QG_TOP + 1);
    L.logits = take((size_t)nt * (QG_EXPERTS + 1) * 4);
    L.flag = take((size_t)nt * 4);
    L.missing = take((size_t)nt * 4);
    L.mass = take((size_t)nt * 8);
    L.xp = take((size_t)nt * 2 * D * 2);
    L.xsp = take((size_t)nt * 2 * (D / 32) * 2);
    L.counts = take(nch * QG_EXPERTS * 4);
    L.offsets = take((QG_EXPERTS + 1) * 4);
    L.tbase = take(sizeof(TileTable));
    L.row_token = take((size_t)nt * QG_TOP * 4);
    L.row_slot = take((size_t)nt * QG_TOP * 4);
    L.midp = take(rows * 2 * F * 2);
    L.msp = take(rows * 2 * (F / 32) * 2);
    L.slots = take(rows * D * 4);
    L.xn = take((size_t)nt * D * 4);
    L.xi8 = take((size_t)nt * 2 * D);
    L.xsc = take((size_t)nt * 4);
    L.row_sx = take((size_t)nt * QG_TOP * 4);
    L.total = off;
    return L;
}


template <typename K, typename... Args>
void pf_launch(int slot, K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    hipEvent_t b = nullptr, e = nullptr;
    if (qg_kernel_event_pair(slot, (void **)&b, (void **)&e))
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, b, e, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}

QG_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------- input normalisation (residual form) ----------------
// xn = x / sqrt(mean(x^2) + eps), one wave per row, with the decode path's
// row_rms_scale so both paths normalise bit-identically.
__global__ __launch_bounds__(256) void pf_norm_kernel(float *xn, const float *x, int nt, int D, float eps) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = blockIdx.x * 4 + wave;
    if (t >= nt) return;
    const float *xr = x + (size_t)t * D;
    const float sc = row_rms_scale(xr, D, eps, lane);
    for (int i = lane; i < D; i += 64) xn[(size_t)t * D + i] = xr[i] * sc;
}

// ---------------- P1: router logits ----------------
// logits[t][r] = sum_k R[r][k] x[t][k] in the order of cpu.c:122-139: chain j
// (0..31) accumulates k = j, j+32, ... ascending with fused multiply-add,
// then the tree 16/8/4/2/1 of gpu.cu:154-180 (qg_tree32).  Block = 16 waves
// = 64 tokens x 32 rows; half-wave h of wave w owns 8 tokens (w % 8) x 8 rows
// ((w / 8) * 2 + h), lane j of the half-wave owns chain j of all 64 of its
// outputs (112 registers: four waves per SIMD hide the shared-memory reads).
// K chunks of 128 columns of both operands are staged in shared memory
// (direct global->shared copies, double-buffered); the two half-waves of a
// wave read the same token rows (broadcast) and different router rows.  The
// final tree runs as an exchange butterfly: at offset s the lanes with bit s
// clear keep the lower half of their outputs, the others the upper half, and
// each adds its partner's value; float addition is commutative, so every
// output is the same sum, paired the same way, as lane 0's of qg_tree32.
// Lane j ends with outputs 2j, 2j+1 = token j/4, rows 2(j&3), 2(j&3)+1.
constexpr int RT_TOK = 64, RT_ROWS = 32, RT_KC = 128;
constexpr int RT_TT = 8;                          // tokens per half-wave (x 8 rows: RT_TT * 8 chains per lane)
constexpr int RT_WAVES = (RT_TOK / RT_TT) * (RT_ROWS / 8) / 2;
constexpr int RT_LDS = 2 * (RT_ROWS + RT_TOK) * RT_KC * 4;

struct RouterArgs {
    const float *x; int nt, D, rows;
    const float *router, *sh_row;    // rows 0..511, row 512 (the shared gate vector) when rows == 513
    const float *bias;               // added to rows 0..511, or null
    float *logits;                   // [nt][rows]
};

__global__ __launch_bounds__(64 * RT_WAVES) void pf_router_kernel(RouterArgs A) {
    constexpr int NTG = RT_TOK / RT_TT, V = RT_TT / 4;  // token groups; outputs per lane after the tree
    extern __shared__ uint4 s_dyn[];
    float *sw = (float *)s_dyn;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, j = lane & 31;
    const int tg = wave % NTG, rg = (wave / NTG) * 2 + h;
    const int t0 = blockIdx.x * RT_TOK, r0 = blockIdx.y * RT_ROWS, nch = A.D / RT_KC;
    auto stage = [&](int c, int b) {
        // 32 router rows then 64 token rows, 512 B each: 48 copies of two rows
        for (int q = wave; q < (RT_ROWS + RT_TOK) / 2; q += RT_WAVES) {
            const int R = 2 * q + h;
            const float *src;
            if (R < RT_ROWS) {
                const int r = min(r0 + R, A.rows - 1);
                src = r == QG_EXPERTS ? A.sh_row : A.router + (size_t)r * A.D;
            } else {
                src = A.x + (size_t)min(t0 + R - RT_ROWS, A.nt - 1) * A.D;
            }
            dma16(src + (size_t)c * RT_KC + 4 * j, sw + (size_t)b * (RT_ROWS + RT_TOK) * RT_KC + q * 2 * RT_KC);
        }
    };
    float acc[RT_TT][8];
#pragma unroll
    for (int t = 0; t < RT_TT; t++)
#pragma unroll
        for (int r = 0; r < 8; r++) acc[t][r] = 0.0f;
    stage(0, 0);
    for (int c = 0; c < nch; c++) {
        wait_vmem();
        __syncthreads();
        if (c + 1 < nch) stage(c + 1, (c + 1) & 1);
        const float *W = sw + (size_t)(c & 1) * (RT_ROWS + RT_TOK) * RT_KC + rg * 8 * RT_KC;
        const float *X = sw + (size_t)(c & 1) * (RT_ROWS + RT_TOK) * RT_KC + (RT_ROWS + tg * RT_TT) * RT_KC;
#pragma unroll
        for (int i = 0; i < RT_KC / 32; i++) {
            float wv[8], xv[RT_TT];
#pragma unroll
            for (int r = 0; r < 8; r++) wv[r] = W[r * RT_KC + 32 * i + j];
#pragma unroll
            for (int t = 0; t < RT_TT; t++) xv[t] = X[t * RT_KC + 32 * i + j];
#pragma unroll
            for (int t = 0; t < RT_TT; t++)
#pragma unroll
                for (int r = 0; r < 8; r++) acc[t][r] = __builtin_fmaf(wv[r], xv[t], acc[t][r]);
        }
    }
    // exchange butterfly over the 32 lanes of the half-wave; v[o], o = 8t + r
    float *v = &acc[0][0];
#pragma unroll
    for (int s = 16, n = 8 * RT_TT; s >= 1; s >>= 1, n >>= 1) {
        const bool up = (j & s) != 0;
#pragma unroll
        for (int q = 0; q < n / 2; q++) {
            const float send = up ? v[q] : v[q + n / 2];
            const float recv = __shfl_xor(send, s, 32);
            v[q] = (up ? v[q + n / 2] : v[q]) + recv;
        }
    }
    // lane j holds outputs o = V j .. V j + V - 1
    const int t = t0 + tg * RT_TT + (V * j) / 8;
    if (t < A.nt) {
#pragma unroll
        for (int q = 0; q < V; q++) {
            const int r = r0 + rg * 8 + (V * j) % 8 + q;
            if (r < A.rows) A.logits[(size_t)t * A.rows + r] = A.bias && r < QG_EXPERTS ? v[q] + A.bias[r] : v[q];
        }
    }
}

// ---------------- P2: routing and activation planes ----------------
struct RouteArgs {
    int nt; const float *logits; int ld;
    const uint8_t *resident; double thr;
    int *ids; float *w; uint8_t *flags_out; int *flag; int *missing; double *mass;
    const float *x; int D; _Float16 *xp, *xsp;
    int8_t *xi8; float *xsc;          // int8 planes and row scales (the int8 dense pass), or null
};

// The int8 planes of one token row (natural K order): x ~= sx * (256 hi + lo)
// with q = rint(x / sx) in [-32639, 32639], sx = max|x| / 32639, hi =
// floor((q + 128) / 256) in [-127, 127], lo = q - 256 hi in [-128, 127].
QG_DEV void token_planes_i8(const float *xr, int D, int lane, int8_t *hi, int8_t *lo, float *sx_out) {
    float mx = 0.0f;
    for (int k = lane; k < D; k += 64) mx = fmaxf(mx, fabsf(xr[k]));
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float sx = mx > 0.0f ? mx / 32639.0f : 1.0f, inv = 1.0f / sx;
    if (lane == 0) *sx_out = sx;
    for (int k = 4 * lane; k < D; k += 256) {
        const float4 v = *(const float4 *)(xr + k);
        const float xv[4] = {v.x, v.y, v.z, v.w};
        uint32_t ph = 0, pl = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = max(-32639, min(32639, (int)rintf(xv[i] * inv)));
            const int h = (q + 128) >> 8, l = q - 256 * h;
            ph |= (uint32_t)(h & 0xff) << (8 * i);
            pl |= (uint32_t)(l & 0xff) << (8 * i);
        }
        *(uint32_t *)(hi + k) = ph;
        *(uint32_t *)(lo + k) = pl;
    }
}

// Two waves per token (block = 4 tokens): wave w < 4 routes token 4b + w
// (top-10 of the (biased) logits, coverage/prune, flags) while wave w + 4
// writes its fp16 hi/lo planes and 32-group sum planes.
__global__ __launch_bounds__(512) void pf_route_kernel(RouteArgs A) {
    __shared__ __align__(16) float s_rv[4][QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_ri[4][QG_ROUTE_SCRATCH];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = blockIdx.x * 4 + (wave & 3);
    if (t >= A.nt) return;  // whole wave; no block barrier in this kernel
    if (wave >= 4) {  // the token's activation planes, beside its routing
        _Float16 *hi = A.xp + (size_t)t * 2 * A.D, *shi = A.xsp + (size_t)t * 2 * (A.D / 32);
        token_planes(A.x + (size_t)t * A.D, A.D, false, 1.0f, lane, hi, hi + A.D, shi, shi + A.D / 32, nullptr);
        if (A.xi8) token_planes_i8(A.x + (size_t)t * A.D, A.D, lane, A.xi8 + (size_t)t * 2 * A.D, A.xi8 + (size_t)t * 2 * A.D + A.D, A.xsc + t);
        return;
    }
    int id, missing;
    float wv;
    double mass;
    qg_route_fast(A.logits + (size_t)t * A.ld, lane, id, wv, s_rv[wave], s_ri[wave]);
    const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
    if (lane < QG_TOP) {
        A.ids[(size_t)t * QG_TOP + lane] = id;
        A.w[(size_t)t * QG_TOP + lane] = wv;
    }
    if (lane == 0) {
        A.flag[t] = flag;
        A.missing[t] = missing;
        A.mass[t] = mass;
        if (A.flags_out) A.flags_out[t] = (uint8_t)flag;
    }
}

// ---------------- P3: offsets, chunk bases, tile table ----------------
// Inclusive scan of one int per thread over a 512-thread block.
QG_DEV int scan512(int v, int *s_tmp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    if (lane == 63) s_tmp[wave] = v;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; w++) base += s_tmp[w];
    __syncthreads();
    return v + base;
}

// tt may be null (dispatch only); with `status`, *status = OR of bad[0..nch).
__global__ __launch_bounds__(512) void pf_scan_kernel(int *counts, int nch, int *offsets, TileTable *tt, int shared_rows,
                                                      const int *bad, int *status) {
    __shared__ int s_tmp[8];
    __shared__ int s_tiles[NG], s_m16[NG];
    __shared__ int s_wh[8][64], s_above[64];
    const int e = threadIdx.x;
    if (status) {
        int b = 0;
        for (int c = e; c < nch; c += QG_EXPERTS) b |= bad[c];
        b = __syncthreads_or(b);
        if (e == 0) *status = b ? 1 : 0;
    }
    constexpr int U = 16;  // loads in flight per thread
    int n = 0;
    for (int c0 = 0; c0 < nch; c0 += U) {
        int v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = c0 + u < nch ? counts[(size_t)(c0 + u) * QG_EXPERTS + e] : 0;
#pragma unroll
        for (int u = 0; u < U; u++) n += v[u];
    }
    const int incl = scan512(n, s_tmp), off = incl - n;
    offsets[e] = off;
    if (e == QG_EXPERTS - 1) offsets[QG_EXPERTS] = incl;
    // counts[c][e] -> first CSR position of chunk c's rows of expert e
    int run = off;
    for (int c0 = 0; c0 < nch; c0 += U) {
        int v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = c0 + u < nch ? counts[(size_t)(c0 + u) * QG_EXPERTS + e] : 0;
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (c0 + u < nch) counts[(size_t)(c0 + u) * QG_EXPERTS + e] = run;
            run += v[u];
        }
    }
    if (!tt) return;  // block-uniform
    // pass order: experts by row-count bucket, largest first, ties by id (a
    // counting sort); buckets 0..16 hold ceil(n / 16) of the others, 17..63
    // the dense experts by 32-row steps, so the dense ones lead; the shared
    // expert follows them
    const int lane = e & 63, wave = e >> 6;
    const int bk = n >= DENSE_MIN ? 17 + min((n - DENSE_MIN) >> 5, 46) : (n + 15) >> 4;
    unsigned long long same = ~0ull;  // lanes of this wave in the same bucket
#pragma unroll
    for (int bit = 0; bit < 6; bit++) {
        const unsigned long long m = __ballot((bk >> bit) & 1);
        same &= ((bk >> bit) & 1) ? m : ~m;
    }
    const int below = __popcll(same & ((1ull << lane) - 1ull));
    s_wh[wave][lane] = 0;
    const int nd = __syncthreads_count(n >= DENSE_MIN);
    if (below == 0) s_wh[wave][bk] = __popcll(same);
    __syncthreads();
    if (wave == 0) {  // experts in buckets above each bucket
        int t = 0;
        for (int w = 0; w < 8; w++) t += s_wh[w][63 - lane];
        int incl = t;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        s_above[63 - lane] = incl - t;
    }
    __syncthreads();
    int rank = s_above[bk] + below;
    for (int w = 0; w < wave; w++) rank += s_wh[w][bk];
    const int pos = rank < nd ? rank : rank + 1;
    s_tiles[pos] = (n + PT - 1) / PT;
    s_m16[pos] = (n + 15) / 16;
    tt->gorder[pos] = e;
    if (e == 0) {
        s_tiles[nd] = (shared_rows + PT - 1) / PT;
        s_m16[nd] = (shared_rows + 15) / 16;
        tt->gorder[nd] = QG_EXPERTS;
    }
    __syncthreads();
    // prefixes over positions 0..511 (thread e: position e), then position 512
    const int v = s_tiles[e], tincl = scan512(v, s_tmp);
    const int m = s_m16[e], mincl = scan512(m, s_tmp);
    tt->tbase[e] = tincl - v;
    tt->mbase[e] = mincl - m;
    if (e == nd) {
        tt->bounds[1] = tincl - v;
        tt->mbounds[1] = mincl - m;
    }
    if (e == nd + 1) {
        tt->bounds[2] = tincl - v;
        tt->mbounds[2] = mincl - m;
    }
    if (e == QG_EXPERTS - 1) {
        const int all = tincl + s_tiles[QG_EXPERTS], mall = mincl + s_m16[QG_EXPERTS];
        tt->tbase[QG_EXPERTS] = tincl;
        tt->mbase[QG_EXPERTS] = mincl;
        tt->tbase[NG] = all;
        tt->mbase[NG] = mall;
        tt->bounds[0] = 0;
        tt->mbounds[0] = 0;
        if (nd == QG_EXPERTS) {  // position 512 (the shared expert) starts segment 1
            tt->bounds[1] = tincl;
            tt->mbounds[1] = mincl;
        }
        if (nd + 1 == QG_EXPERTS) {
            tt->bounds[2] = tincl;
            tt->mbounds[2] = mincl;
        } else if (nd == QG_EXPERTS) {
            tt->bounds[2] = all;
            tt->mbounds[2] = mall;
        }
        tt->bounds[3] = all;
        tt->mbounds[3] = mall;
    }
}

// Histogram of an ids array alone (qg_moe_dispatch): chunk masks as in
// pf_route_kernel; bad[chunk] = 1 if an id is neither in [0,512) nor a pruned
// encoding in [-513,-2], or a token lists an expert twice (the validation of
// cpu.c:242-244).
__global__ __launch_bounds__(512) void pf_count_kernel(int *counts, int *bad, const int *ids, const int *flag, int nt) {
    __shared__ uint32_t s_mask[QG_EXPERTS];
    __shared__ int s_bad;
    const int tid = threadIdx.x, t0 = blockIdx.x * PF_CHUNK;
    s_mask[tid] = 0u;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    if (tid < PF_CHUNK * QG_TOP) {
        const int tl = tid / QG_TOP, t = t0 + tl;
        if (t < nt && (!flag || flag[t] < 2)) {
            const int id = ids[(size_t)t * QG_TOP + tid - tl * QG_TOP];
            if (id >= 0 && id < QG_EXPERTS) {
                if (atomicOr(&s_mask[id], 1u << tl) & (1u << tl)) s_bad = 1;
            } else if (!(id <= -2 && id >= -QG_EXPERTS - 1)) {
                s_bad = 1;
            }
        }
    }
    __syncthreads();
    counts[(size_t)blockIdx.x * QG_EXPERTS + tid] = __popc(s_mask[tid]);
    if (tid == 0 && bad) bad[blockIdx.x] = s_bad;
}

// ---------------- P4: stable fill ----------------
__global__ __launch_bounds__(512) void pf_fill_kernel(int *row_token, int *row_slot, const int *bases, const int *ids,
                                                      const int *flag, int nt, float *row_sx, const float *xsc) {
    __shared__ uint32_t s_mask[QG_EXPERTS];
    const int tid = threadIdx.x, t0 = blockIdx.x * PF_CHUNK;
    s_mask[tid] = 0u;
    __syncthreads();
    int e = -1, tl = 0, k = 0;
    if (tid < PF_CHUNK * QG_TOP) {
        tl = tid / QG_TOP;
        k = tid - tl * QG_TOP;
        const int t = t0 + tl;
        if (t < nt) {
            const int id = ids[(size_t)t * QG_TOP + k];
            if ((!flag || flag[t] < 2) && id >= 0 && id < QG_EXPERTS) {
                e = id;
                atomicOr(&s_mask[e], 1u << tl);
            }
        }
    }
    __syncthreads();
    if (e >= 0) {
        const int pos = bases[(size_t)blockIdx.x * QG_EXPERTS + e] + __popc(s_mask[e] & ((1u << tl) - 1u));
        row_token[pos] = t0 + tl;
        row_slot[pos] = (t0 + tl) * QG_TOP + k;
        if (row_sx) row_sx[pos] = xsc[t0 + tl];
    }
}

// ---------------- GEMM building blocks ----------------

constexpr int PF_WAVES = 8;                  // waves per GEMM workgroup
constexpr int NCT = 2;                       // column tiles of 16 weight rows per wave

// Stage K chunk `chunk` of the tile's first nrows rows (a multiple of 16):
// plane rows of `planes` (row stride `stride` elements per plane, 2 planes
// per source row; source row of tile row r = src[r]) into `stage`, swizzled;
// nck = 16-byte chunks per plane row in this K chunk.  With `sums`, the 2 x 8
// group sums of the chunk ([tile row][plane][8]).
QG_DEV void stage_rows(uint8_t *stage, uint8_t *sums, const _Float16 *planes, int stride, const _Float16 *sum_planes,
                       int sum_stride, const int *src, int chunk, int nck, int nrows, int wave, int lane) {
    for (int q = wave; q < nrows; q += PF_WAVES) {
        const int R = 2 * q + (lane >> 5), tr = R >> 1, p = R & 1;
        int c = (lane & 31) ^ (tr & 15);
        if (c >= nck) c = 0;  // positions no reader uses
        dma16_ordered(planes + ((size_t)src[tr] * 2 + p) * stride + (size_t)chunk * KC + c * 8, stage + q * 1024);
    }
    if (sums && wave * 32 < nrows) {
        const int C = wave * 64 + lane, tr = C >> 1, p = C & 1;
        dma16_ordered(sum_planes + ((size_t)src[tr] * 2 + p) * sum_stride + (size_t)chunk * 8, sums + wave * 1024);
    }
}

// A fragment of tile row r (within the stage), plane p, 16-byte chunk c.
QG_DEV qg_half8 stage_frag(const uint8_t *st, int r, int p, int c) {
    return ld_frag((const _Float16 *)(st + (r * 2 + p) * 512 + 16 * (c ^ (r & 15))));
}

// Q4_K operands of one superblock for the wave's column tiles: 3 loads per
// tile (header, qs chunks kq and kq + 4).
constexpr int Q4_LOADS = 3 * NCT;
struct Q4Ops { uint4 hd[NCT], c0[NCT], c1[NCT]; };
QG_DEV void q4_load(Q4Ops &o, const uint8_t *const *wrow, int sb, int kq) {
#pragma unroll
    for (int n = 0; n < NCT; n++) {
        const uint8_t *p = wrow[n] + (size_t)sb * 144;
        o.hd[n] = qg_ld16(p);
        o.c0[n] = qg_ld16(p + 16 + 16 * kq);
        o.c1[n] = qg_ld16(p + 16 + 16 * (kq + 4));
    }
}

// y[m][n] += d * (s*q . x) - dmin * (m . X) over one Q4_K superblock, for the
// first M row tiles (A fragments read from shared memory per K step; the
// other wave on the SIMD hides their latency).
QG_DEV void q4_chunk(qg_f4 (&y)[4][NCT], const Q4Ops &o, const uint8_t *st, const uint8_t *ss, int j, int kq, int M) {
    Q4kHeader h[NCT];
#pragma unroll
    for (int n = 0; n < NCT; n++) h[n] = q4k_header(o.hd[n]);
    qg_f4 acc[4][NCT];
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int n = 0; n < NCT; n++) acc[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int gA = 2 * (kq >> 1);
#pragma unroll
    for (int f = 0; f < 8; f++) {
        qg_half8 b[NCT];
#pragma unroll
        for (int n = 0; n < NCT; n++) {
            const uint4 c = f < 4 ? o.c0[n] : o.c1[n];
            const int g = (f < 4 ? gA : gA + 4) + ((f & 3) >> 1);
            b[n] = q4k_chunk_frag(c, f & 3, (_Float16)q4k_s(h[n], g));
        }
#pragma unroll
        for (int m = 0; m < 4; m++) {
            if (m < M) {  // uniform
                const qg_half8 a0 = stage_frag(st, m * 16 + j, 0, 4 * f + kq), a1 = stage_frag(st, m * 16 + j, 1, 4 * f + kq);
#pragma unroll
                for (int n = 0; n < NCT; n++) {
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[n], acc[m][n], 0, 0, 0);
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[n], acc[m][n], 0, 0, 0);
                }
            }
        }
    }
    // min term: lanes kq = 0 / 1 carry the hi / lo plane of the 8 group sums
    const qg_half8 z8 = qg_half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int n = 0; n < NCT; n++) {
        qg_half8 bm;
#pragma unroll
        for (int g = 0; g < 8; g++) bm[g] = kq < 2 ? (_Float16)q4k_m(h[n], g) : (_Float16)0.0f;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            if (m < M) {
                const qg_half8 as = kq < 2 ? ld_frag((const _Float16 *)(ss + ((m * 16 + j) * 2 + kq) * 16)) : z8;
                const qg_f4 mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bm, qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    y[m][n][i] = __builtin_fmaf(h[n].d, acc[m][n][i], __builtin_fmaf(-h[n].dmin, mm[i], y[m][n][i]));
            }
        }
    }
}

// Items of a persistent launch, XCD-aware: workgroup b runs on XCD b % 8
// (round-robin dispatch) and takes its XCD's share xs .. xe-1 of the items
// in rounds of nx (the XCD's workgroups), position slot of each round, so
// neighbouring items (the row blocks of one tile, the tiles of one expert)
// run at the same time on one XCD and share its L2.
struct ItemRange { int xs, xe, nx, slot; };
QG_DEV int range_count(const ItemRange &r) { return r.xe - r.xs > r.slot ? (r.xe - r.xs - r.slot + r.nx - 1) / r.nx : 0; }

// The XCDs' shares of a pass, of equal estimated cost.  An item of a tile
// with M row tiles is priced CA + CB M (its fixed per-step costs plus its
// products, fitted to per-workgroup durations on config 3); the pass's items
// are cut at item granularity into 8 parts of equal total price.  The pass
// order lists groups by row count, largest first, so the cut gives each XCD
// items of like size, which its workgroups share evenly.  All threads of the
// block call it (s_tb: the tile table's tbase, filled before the call).
template <int CA, int CB>
QG_DEV ItemRange balanced_items(const TileTable *tt, const int *s_tb, int seg_lo, int seg_hi, int nblk) {
    __shared__ int s_res[2];
    const int t_lo = tt->bounds[seg_lo], t_hi = tt->bounds[seg_hi], m_lo = tt->mbounds[seg_lo];
    const long long total_cost = (long long)nblk * (CA * (long long)(t_hi - t_lo) + CB * (long long)(tt->mbounds[seg_hi] - m_lo));
    // one part per XCD (a grid of fewer than 8 workgroups: one per workgroup)
    const int parts = min(8, (int)gridDim.x);
    const int x = blockIdx.x % parts, slot = blockIdx.x / parts, n_x = (gridDim.x - x + parts - 1) / parts;
    // first item of parts x and x + 1: the first item whose price prefix
    // reaches ceil(total_cost * q / parts)
    long long Q[2];
#pragma unroll
    for (int k = 0; k < 2; k++) Q[k] = (total_cost * (x + k) + parts - 1) / parts;
    if (threadIdx.x < 2) s_res[threadIdx.x] = Q[threadIdx.x] >= total_cost ? (t_hi - t_lo) * nblk : 0;
    __syncthreads();
    for (int e = threadIdx.x; e < NG; e += blockDim.x) {
        const int tb0 = s_tb[e], tb1 = s_tb[e + 1];
        if (tb1 == tb0 || tb0 < t_lo || tb1 > t_hi) continue;
        const int mb0 = tt->mbase[e], mb1 = tt->mbase[e + 1];
        const long long g0 = (long long)nblk * (CA * (long long)(tb0 - t_lo) + CB * (long long)(mb0 - m_lo));
        const long long g1 = (long long)nblk * (CA * (long long)(tb1 - t_lo) + CB * (long long)(mb1 - m_lo));
        const int T = tb1 - tb0, m_last = mb1 - mb0 - 4 * (T - 1);
        const long long full = (long long)nblk * (CA + 4 * CB);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if (!(g0 < Q[k] && Q[k] <= g1) || Q[k] >= total_cost) continue;
            const int j = (int)min((long long)(T - 1), (Q[k] - g0 - 1) / full);
            const long long ct = g0 + j * full;
            const int w = CA + CB * (j < T - 1 ? 4 : m_last);
            const int blk = (int)((Q[k] - ct + w - 1) / w);
            s_res[k] = (tb0 + j - t_lo) * nblk + blk;
        }
    }
    __syncthreads();
    const int n_items = (t_hi - t_lo) * nblk, i0 = min(max(s_res[0], 0), n_items), i1 = min(max(s_res[1], i0), n_items);
    __syncthreads();
    return ItemRange{i0, i1, n_x, slot};
}

// Tile -> order position (block-uniform): the largest p with tb[p] <= tile_idx
// (empty groups share their successor's start).
QG_DEV int find_group(const int *tb, int tile_idx) {
    int lo = 0, hi = NG;  // tb[0] = 0 <= tile_idx < tb[NG]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (tb[mid] <= tile_idx) lo = mid;
        else hi = mid;
    }
    return lo;
}

// The GEMM workgroups stream (item, K chunk) steps: while step s computes,
// the activation stage of step s + 1 and the weights of step s + 2 are in
// flight.  Only the newest weight loads (those of step s + 2) may be
// outstanding when step s + 1 starts: loads complete in issue order, so
// waiting for at most that many outstanding operations leaves every older
// load done, whatever the epilogue's stores (issued in between) do.
//
// An item of a workgroup's range: group g (QG_EXPERTS: the shared expert),
// block blk of its output rows, nv valid rows (1..64) from `base` (the CSR
// position of the tile's first row; the shared expert: its first token).
struct PfItem { int g, blk, nv, M, base; bool shared; };
QG_DEV int2 pf_item_packed(const int *s_tb, const int *s_go, const int *s_off, int nt, int t_lo, int nblk, int item) {
    const int tile_idx = t_lo + item / nblk, blk = item % nblk;
    const int gp = find_group(s_tb, tile_idx);
    const int g = s_go[gp], r0 = (tile_idx - s_tb[gp]) * PT;
    const bool shared = g == QG_EXPERTS;
    const int off = shared ? 0 : s_off[g], n_g = shared ? nt : s_off[g + 1] - off;
    return make_int2(g | blk << 10 | min(PT, n_g - r0) << 17, off + r0);
}
QG_DEV PfItem pf_unpack(int2 v) {
    PfItem it;
    it.g = v.x & 1023;
    it.blk = (v.x >> 10) & 127;
    it.nv = v.x >> 17;
    it.M = (it.nv + 15) >> 4;
    it.base = v.y;
    it.shared = it.g == QG_EXPERTS;
    return it;
}

// The workgroup's items, decoded ahead into a ring in shared memory (the
// search over the tile table stays out of the step stream): items k .. k+63
// are written when item k - 64 starts (k a multiple of 64), into the slots of
// items k - 128 .. k - 65, all finished by then; the next reader of the new
// slots is two steps or more (and a barrier) away.
constexpr int IT_RING = 128, IT_BATCH = 64;
struct ItemRing {
    int2 *ring; const int *tb, *go, *off; int nt, t_lo, nblk, nitems; ItemRange ir;
    __device__ __forceinline__ void fill(int k0, int n, int tid) const {
        const int k = k0 + tid;
        if (tid < n && k < nitems) ring[k & (IT_RING - 1)] = pf_item_packed(tb, go, off, nt, t_lo, nblk, ir.xs + ir.slot + k * ir.nx);
    }
    __device__ __forceinline__ PfItem at(int k) const { return pf_unpack(ring[k & (IT_RING - 1)]); }
};

// Tile row r (< 64, past the item's rows: its last row) of a routed item as
// per-row indices into shared memory by a 4-byte direct copy per lane of
// wave 0 (tracked like the stage copies); shared-expert rows are computed.
// `list` is the CSR array to index (row_token or row_slot), `shared_base`
// the index of shared row 0.
QG_DEV void item_rows(int *dst, const PfItem &it, const int *list, int shared_base, int wave, int lane) {
    if (wave != 0) return;
    const int r = it.base + min(lane, it.nv - 1);
    if (it.shared) dst[lane] = shared_base + r;
    else dma4_ordered(list + r, dst);
}

// Position (item k, chunk c) of a step, advanced without division.
struct StepPos { int k, c; };
QG_DEV StepPos next_pos(StepPos p, int nc) { return ++p.c == nc ? StepPos{p.k + 1, 0} : p; }

// ---------------- P5: gate/up + SwiGLU ----------------
struct GuArgs {
    int nt, D, F;
    const int *offsets; const TileTable *tt; int seg_lo, seg_hi;   // tiles of segments seg_lo .. seg_hi-1
    const int *row_token;
    const uint8_t *gate, *up, *sh_gate, *sh_up; size_t rb;   // Q4_K rows of D
    const _Float16 *xp, *xsp;
    _Float16 *midp, *msp;            // [rows][2][F] (down format order), [rows][2][F/32]
    int down_fmt, sh_down_fmt;
    const int8_t *xi8; const float *xsc, *row_sx;   // the int8 variant: planes [nt][2][D], scale per token and per CSR row
};

// (the kernel follows the down kernels: it shares their 128-element stage)

// ---------------- P6: down ----------------
struct DnArgs {
    int nt, D, F;
    const int *offsets; const TileTable *tt; int seg_lo, seg_hi;   // tiles of segments seg_lo .. seg_hi-1
    const int *row_slot;
    const uint8_t *down, *sh_down; size_t rb, sh_rb;   // every group in the launch has format FMT
    const _Float16 *midp, *msp;
    float *slots;                    // [rows][D]: slot t*10+k, shared rows at nt*10+t
};

// Q4_K down.  Item = (group, 64-row tile, 256 D rows); wave w: D rows 32 w ..
// +31 of the block as two column tiles, their weights in registers loaded two
// steps ahead.  Steps are the item's K chunks of 256 (F / 256 superblocks).
__global__ __launch_bounds__(512, 1) void pf_down_kernel(DnArgs A) {
    extern __shared__ uint4 s_dyn[];
    uint8_t *lds = (uint8_t *)s_dyn;
    __shared__ int s_tb[NG + 1], s_go[NG], s_off[QG_EXPERTS + 1];
    __shared__ int2 s_it[IT_RING];
    __shared__ int s_src[2][PT], s_slot[2][PT];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    for (int i = tid; i <= NG; i += 512) {
        s_tb[i] = A.tt->tbase[i];
        if (i < NG) s_go[i] = A.tt->gorder[i];
        if (i <= QG_EXPERTS) s_off[i] = A.offsets[i];
    }
    const int ndb = A.D / DN_DB, F = A.F, F32 = A.F / 32, nkc = (F + KC - 1) / KC;
    const int t_lo = A.tt->bounds[A.seg_lo], total = (A.tt->bounds[A.seg_hi] - t_lo) * ndb;
    const ItemRange ir = balanced_items<10, 3>(A.tt, s_tb, A.seg_lo, A.seg_hi, ndb);
    const int nitems = range_count(ir), steps = nitems * nkc;
    if (steps == 0) return;  // block-uniform
    const ItemRing R{s_it, s_tb, s_go, s_off, A.nt, t_lo, ndb, nitems, ir};
    __syncthreads();
    R.fill(0, IT_RING, tid);
    __syncthreads();
    // the item's mid rows (computed) and output slots (copied from row_slot)
    auto set_rows = [&](const PfItem &it, int buf) {
        if (wave == 0) s_src[buf][lane] = (it.shared ? A.nt * QG_TOP : 0) + it.base + min(lane, it.nv - 1);
        item_rows(s_slot[buf], it, A.row_slot, A.nt * QG_TOP, wave, lane);
    };
    auto weight_rows = [&](const PfItem &it, const uint8_t **wrow) {
        const uint8_t *bw = it.shared ? A.sh_down : A.down + (size_t)it.g * A.D * A.rb;
        const size_t rb = it.shared ? A.sh_rb : A.rb;
        const int d = it.blk * DN_DB + wave * 32 + j;
#pragma unroll
        for (int n = 0; n < NCT; n++) wrow[n] = bw + (size_t)(d + 16 * n) * rb;
    };
    auto stage = [&](const PfItem &it, int buf, int kc, int b) {
        stage_rows(lds + b * STAGE_BYTES, lds + 2 * STAGE_BYTES + b * SUMS_BYTES, A.midp, F, A.msp, F32, s_src[buf], kc, 32,
                   16 * it.M, wave, lane);
    };
    using Ops = Q4Ops;
    const uint8_t *wrow[NCT];
    auto load_step = [&](Ops &o, StepPos p) {
        weight_rows(R.at(p.k), wrow);
        q4_load(o, wrow, p.c, kq);
    };
    PfItem cur = R.at(0);
    set_rows(cur, 0);
    wait_vmem();
    __syncthreads();
    stage(cur, 0, 0, 0);
    Ops w0, w1, w2;   // weights of step s in w[s % 3], loaded two steps ahead, never copied
    StepPos pos{0, 0};
    load_step(w0, pos);
    if (1 < steps) load_step(w1, next_pos(pos, nkc));
    qg_f4 y[4][NCT];
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int n = 0; n < NCT; n++) y[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](int s, const Ops &wc, Ops &wn) {
        const int k = pos.k, kc = pos.c;
        const StepPos p1 = next_pos(pos, nkc), p2 = next_pos(p1, nkc);
        if (s + 1 < steps) wait_vmem_but<Q4_LOADS>();
        else wait_vmem();
        __syncthreads();
        if (kc == 0) {
            if (k > 0 && (k & (IT_BATCH - 1)) == 0) R.fill(k + IT_BATCH, IT_BATCH, tid);
            // the next item's rows, copied while this item streams
            if (k + 1 < nitems) set_rows(R.at(k + 1), (k + 1) & 1);
        }
        if (s + 1 < steps) {
            if (p1.k != k) {
                if (nkc == 1) {  // the rows were copied just above
                    wait_vmem();
                    __syncthreads();
                }
                stage(R.at(p1.k), p1.k & 1, p1.c, (s + 1) & 1);
            } else {
                stage(cur, k & 1, p1.c, (s + 1) & 1);
            }
        }
        if (s + 2 < steps) load_step(wn, p2);
        const uint8_t *st = lds + (s & 1) * STAGE_BYTES, *ss = lds + 2 * STAGE_BYTES + (s & 1) * SUMS_BYTES;
        q4_chunk(y, wc, st, ss, j, kq, cur.M);
        if (kc == nkc - 1) {
            const int d0 = cur.blk * DN_DB + wave * 32;
#pragma unroll
            for (int m = 0; m < 4; m++) {
                if (m >= cur.M) break;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int tr = m * 16 + 4 * kq + i;
                    if (tr < cur.nv) {
                        float *o = A.slots + (size_t)s_slot[k & 1][tr] * A.D + d0 + j;
#pragma unroll
                        for (int n = 0; n < NCT; n++) o[16 * n] = y[m][n][i];
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int n = 0; n < NCT; n++) y[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
            if (s + 1 < steps) cur = R.at(k + 1);
        }
        pos = p1;
    };
    for (int s = 0; s < steps; s += 3) {
        step(s, w0, w2);
        if (s + 1 < steps) step(s + 1, w1, w0);
        if (s + 2 < steps) step(s + 2, w2, w1);
    }
}

// ---- IQ4_NL down: the weights through each wave's own shared-memory ring ----
// IQ4_NL rows are 18-byte blocks, so a lane's bytes of a block (its scale and
// 4 qs bytes) are two or three narrow loads.  Here each wave instead copies
// its 32 weight rows' bytes of a step as whole 16-byte pieces (three direct
// copies of 64 lanes) into one of three slots of its own ring and reads them
// back from shared memory.  A step is 128 K elements (4 blocks); a row's
// 72 bytes of it start at byte offset delta = address % 16 of its first
// piece, and delta is 0 or 8 (rows are 72 k bytes for F = 128 k, the tensors
// 16-byte aligned), so 5 pieces hold them.
constexpr int IQ_KC = 128;                          // K elements per step
constexpr int IQ_PIECES = 5;                        // 16-byte pieces per weight row and step (72 bytes from offset 0 or 8)
constexpr int IQ_ROWB = IQ_PIECES * 16;             // 20 dwords: the 16 rows of a fragment read hit distinct banks
constexpr int IQ_COPIES = 3;                        // direct copies per wave and step
constexpr int IQ_SLOT = IQ_COPIES * 64 * 16;        // bytes per wave and slot (rows use 32 x 80)
constexpr int IQ_STAGE = PT * 2 * IQ_KC * 2;        // [64 rows][2 planes][128] fp16
constexpr int PF_IQ_LDS = 2 * IQ_STAGE + PF_WAVES * 3 * IQ_SLOT;
static_assert(32 * IQ_PIECES <= IQ_COPIES * 64, "the copies cover the slot");

// Activation stage of one 128-element K chunk: [row][plane][16 chunks of 16
// bytes], chunk position c ^ (row & 15); one copy covers two rows.
QG_DEV void stage_rows128(uint8_t *stage, const _Float16 *planes, int stride, const int *src, int chunk, int nck, int nrows,
                          int wave, int lane) {
    for (int q = wave; 2 * q < nrows; q += PF_WAVES) {
        const int tr = 2 * q + (lane >> 5), p = (lane >> 4) & 1;
        int c = (lane & 15) ^ (tr & 15);
        if (c >= nck) c = 0;  // positions no reader uses
        dma16_ordered(planes + ((size_t)src[tr] * 2 + p) * stride + (size_t)chunk * IQ_KC + c * 8, stage + q * 1024);
    }
}
QG_DEV qg_half8 stage_frag128(const uint8_t *st, int r, int p, int c) {
    return ld_frag((const _Float16 *)(st + (r * 2 + p) * 256 + 16 * (c ^ (r & 15))));
}

struct NoIssue {
    __device__ __forceinline__ void operator()(int) const {}
};
// y[m][n] += d_b * (lut[q] . x) for the 4 blocks of a step, weights from the
// slot (row 16 n + j of the wave's 32: its step's bytes start at byte del[n]
// of its slot row), activations from the stage; issue(b) runs after block
// b's products (the caller's copies for later steps go out while the matrix
// cores work).
template <int M, int MY, typename Issue = NoIssue>
QG_DEV void iq_chunk_lds(qg_f4 (&y)[MY][NCT], const uint8_t *slot, const int (&del)[NCT], const uint8_t *st, int j, int kq,
                         Issue issue = Issue{}) {
    static_assert(M <= MY, "row tiles");
    const uint8_t *rowp[NCT];
#pragma unroll
    for (int n = 0; n < NCT; n++) rowp[n] = slot + (16 * n + j) * IQ_ROWB + del[n];
#pragma unroll
    for (int b = 0; b < IQ_KC / 32; b++) {  // F is a multiple of 128 (checked at launch): 4 blocks per step
        qg_half8 bf[NCT];
        float d[NCT];
#pragma unroll
        for (int n = 0; n < NCT; n++) {
            const uint16_t *p16 = (const uint16_t *)(rowp[n] + 18 * b);
            d[n] = qg_half_u16(p16[0]);
            bf[n] = iq4_frag4((uint32_t)p16[1 + 2 * kq] | ((uint32_t)p16[2 + 2 * kq] << 16));
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const qg_half8 a0 = stage_frag128(st, m * 16 + j, 0, 4 * b + kq), a1 = stage_frag128(st, m * 16 + j, 1, 4 * b + kq);
#pragma unroll
            for (int n = 0; n < NCT; n++) {
                qg_f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bf[n], qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bf[n], acc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) y[m][n][i] = __builtin_fmaf(d[n], acc[i], y[m][n][i]);
            }
        }
        issue(b);
    }
}

// Item = (group, 64-row tile, 256 D rows); wave w: D rows 32 w .. +31 of the
// block as two column tiles.  Steps are the item's K chunks of 128.  As in
// the gate/up kernel, the step loop runs inside one instantiation per row-tile
// count, and the per-lane copy addresses are formed once per item.
__global__ __launch_bounds__(512, 1) void pf_down_iq_kernel(DnArgs A) {
    extern __shared__ uint4 s_dyn[];
    uint8_t *lds = (uint8_t *)s_dyn;
    __shared__ int s_tb[NG + 1], s_go[NG], s_off[QG_EXPERTS + 1];
    __shared__ int2 s_it[IT_RING];
    __shared__ int s_src[2][PT], s_slot[2][PT];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    for (int i = tid; i <= NG; i += 512) {
        s_tb[i] = A.tt->tbase[i];
        if (i < NG) s_go[i] = A.tt->gorder[i];
        if (i <= QG_EXPERTS) s_off[i] = A.offsets[i];
    }
    const int ndb = A.D / DN_DB, F = A.F, nkc = (F + IQ_KC - 1) / IQ_KC;
    const int t_lo = A.tt->bounds[A.seg_lo], total = (A.tt->bounds[A.seg_hi] - t_lo) * ndb;
    const ItemRange ir = balanced_items<7, 3>(A.tt, s_tb, A.seg_lo, A.seg_hi, ndb);
    const int nitems = range_count(ir), steps = nitems * nkc;
    if (steps == 0) return;  // block-uniform
    const ItemRing R{s_it, s_tb, s_go, s_off, A.nt, t_lo, ndb, nitems, ir};
    __syncthreads();
    R.fill(0, IT_RING, tid);
    __syncthreads();
    uint8_t *ring = lds + 2 * IQ_STAGE + (size_t)wave * 3 * IQ_SLOT;   // this wave's three slots
    auto set_rows = [&](const PfItem &it, int buf) {
        if (wave == 0) s_src[buf][lane] = (it.shared ? A.nt * QG_TOP : 0) + it.base + min(lane, it.nv - 1);
        item_rows(s_slot[buf], it, A.row_slot, A.nt * QG_TOP, wave, lane);
    };
    // the wave's first weight row of an item, and the row stride
    auto wave_rows = [&](const PfItem &it, size_t &rb) {
        rb = it.shared ? A.sh_rb : A.rb;
        const uint8_t *bw = it.shared ? A.sh_down : A.down + (size_t)it.g * A.D * A.rb;
        return bw + (size_t)(it.blk * DN_DB + wave * 32) * rb;
    };
    // F is a multiple of 128 (checked at launch), so every 128-wide step holds
    // 4 blocks; a constant count lets the block loops unroll without exits
    constexpr int NB = IQ_KC / 32;
    auto nblocks = [&](int) { return NB; };
    // Weight copies: piece i = 64 t + lane of a slot is piece p of the wave's
    // row r; wrow[t] is that row in the item being copied.
    int w_p[IQ_COPIES];
    const uint8_t *wrow[IQ_COPIES];
#pragma unroll
    for (int t = 0; t < IQ_COPIES; t++) w_p[t] = min(t * 64 + lane, 32 * IQ_PIECES - 1) % IQ_PIECES;
    auto set_wc = [&](const PfItem &it) {
        size_t rb;
        const uint8_t *w = wave_rows(it, rb);
#pragma unroll
        for (int t = 0; t < IQ_COPIES; t++) wrow[t] = w + (size_t)(min(t * 64 + lane, 32 * IQ_PIECES - 1) / IQ_PIECES) * rb;
    };
    // step kc of the item being copied into slot q: piece p of a row is the
    // p-th 16-byte piece from the row's first aligned one; pieces past its
    // last needed one copy that one again into a position no reader uses
    auto copy_w = [&](int q, int kc) {
        const int nb = nblocks(kc);
        const uint8_t *g[IQ_COPIES];
#pragma unroll
        for (int t = 0; t < IQ_COPIES; t++) {
            const uintptr_t a = (uintptr_t)wrow[t] + (uintptr_t)kc * 72;
            const int delta = (int)(a & 15), np = (delta + 18 * nb + 15) >> 4;
            g[t] = (const uint8_t *)((a & ~(uintptr_t)15) + 16 * (uintptr_t)min(w_p[t], np - 1));
        }
        static_assert(IQ_COPIES == 3, "three copies under one M0 value");
        dma16x3_ordered(g[0], g[1], g[2], ring + q * IQ_SLOT);
    };
    // Mid-plane copies of the item being staged: copy i of this wave covers
    // tile rows 2 q, 2 q + 1 (q = wave + 8 i); the lane's 16-byte chunk c16 is
    // the same for every i.
    const uint8_t *sp[4] = {nullptr, nullptr, nullptr, nullptr};
    int s_nc = 0;
    const int c16 = (lane & 15) ^ ((2 * wave + (lane >> 5)) & 15);
    auto set_sp = [&](const PfItem &it, int buf) {
        s_nc = it.M;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tr = 2 * (wave + PF_WAVES * i) + (lane >> 5), p = (lane >> 4) & 1;
            if (i < it.M) sp[i] = (const uint8_t *)(A.midp + ((size_t)s_src[buf][tr] * 2 + p) * F);
        }
    };
    auto stage_at = [&](int s, int kc) {
        uint8_t *st = lds + (s & 1) * IQ_STAGE;
        const int c = c16 < 4 * nblocks(kc) ? c16 : 0;  // positions past the chunk: no reader uses them
        const size_t co = ((size_t)kc * IQ_KC + c * 8) * 2;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < s_nc) dma16_ordered(sp[i] + co, st + (wave + PF_WAVES * i) * 1024);
    };
    PfItem cur = R.at(0);
    set_rows(cur, 0);
    wait_vmem();
    __syncthreads();
    set_sp(cur, 0);
    stage_at(0, 0);
    set_wc(cur);
    copy_w(0, 0);
    if (1 < steps) {
        if (nkc == 1) set_wc(R.at(1));
        copy_w(1, nkc == 1 ? 0 : 1);
    }
    // step s reads slot s % 3; the copies of step s + 2 go to slot (s + 2) % 3,
    // whose reads (step s - 1) are done
    int s = 0, qc = 0;
    auto run_item = [&](const int k, auto MC) {
        constexpr int M = decltype(MC)::value;
        const PfItem it = R.at(k);
        // the lane's compute rows 16 n + j: low address bits, for the slot offsets
        uint32_t rlo[NCT];
        {
            size_t rb;
            const uint8_t *w = wave_rows(it, rb);
#pragma unroll
            for (int n = 0; n < NCT; n++) rlo[n] = (uint32_t)(uintptr_t)(w + (size_t)(16 * n + j) * rb);
        }
        qg_f4 y[M][NCT];
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int n = 0; n < NCT; n++) y[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int kc = 0; kc < nkc; kc++, s++) {
            const int qn = qc == 0 ? 2 : qc - 1;
            if (s + 1 < steps) wait_vmem_but<IQ_COPIES>();
            else wait_vmem();
            __syncthreads();
            if (kc == 0) {
                if (k > 0 && (k & (IT_BATCH - 1)) == 0) R.fill(k + IT_BATCH, IT_BATCH, tid);
                // the next item's rows, copied while this item streams
                if (k + 1 < nitems) set_rows(R.at(k + 1), (k + 1) & 1);
            }
            // the next step's stage after block 0's products, then the weights
            // of step s + 2 after block 1's (in this order: the wait above
            // relies on it)
            auto issue = [&](int b) {
                if (b == 0 && s + 1 < steps) {
                    if (kc == nkc - 1) {
                        if (nkc == 1) {  // the rows were copied at the top of the step
                            wait_vmem();
                            __syncthreads();
                        }
                        set_sp(R.at(k + 1), (k + 1) & 1);
                    }
                    stage_at(s + 1, kc + 1 < nkc ? kc + 1 : 0);
                }
                if (b == 1 && s + 2 < steps) {
                    // step s + 2 is step kc + 2 of this item or of the next one(s)
                    const int kr = kc + 2 - nkc, kc2 = kr < 0 ? kc + 2 : nkc == 1 ? 0 : kr;
                    if (kc2 == 0) set_wc(R.at(k + (kr < 0 ? 0 : nkc == 1 ? 2 : 1)));  // it starts a later item
                    copy_w(qn, kc2);
                }
            };
            int del[NCT];
#pragma unroll
            for (int n = 0; n < NCT; n++) del[n] = (int)((rlo[n] + (uint32_t)kc * 72u) & 15u);
            const uint8_t *slot = ring + qc * IQ_SLOT, *st = lds + (s & 1) * IQ_STAGE;
            iq_chunk_lds<M>(y, slot, del, st, j, kq, issue);
            qc = qc == 2 ? 0 : qc + 1;
        }
        const int d0 = it.blk * DN_DB + wave * 32;
#pragma unroll
        for (int m = 0; m < M; m++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tr = m * 16 + 4 * kq + i;
                if (tr < it.nv) {
                    float *o = A.slots + (size_t)s_slot[k & 1][tr] * A.D + d0 + j;
#pragma unroll
                    for (int n = 0; n < NCT; n++) o[16 * n] = y[m][n][i];
                }
            }
        }
    };
    for (int k = 0; k < nitems; k++) {
        switch (R.at(k).M) {  // block-uniform
        case 1: run_item(k, std::integral_constant<int, 1>{}); break;
        case 2: run_item(k, std::integral_constant<int, 2>{}); break;
        case 3: run_item(k, std::integral_constant<int, 3>{}); break;
        default: run_item(k, std::integral_constant<int, 4>{}); break;
        }
    }
}

// ---- gate/up: the Q4_K weights through each wave's own shared-memory ring ----
// A step is half a superblock (128 K elements, groups 4h .. 4h+3): per weight
// row the superblock's 16-byte header (piece 0) and the half's 64 qs bytes
// (pieces 1..4).  A slot is row-major (row r's pieces at 80 r, 160 pieces in
// 3 copies, so each copy's lanes read whole runs of few rows; lanes past them
// copy the last piece again into the slot's padding).  The 8 group sums of a
// superblock are staged with its first half, into their own double buffer.
constexpr int GQ_PIECES = 5;
constexpr int GQ_ROWB = GQ_PIECES * 16;
constexpr int GQ_COPIES = 3;
constexpr int GQ_SLOT = GQ_COPIES * 64 * 16;
constexpr int GQ_SUMS = PT * 2 * 16;                 // [64 rows][2 planes][8 group sums] fp16
constexpr int PF_GQ_LDS = 2 * IQ_STAGE + 2 * GQ_SUMS + PF_WAVES * 3 * GQ_SLOT;
static_assert(32 * GQ_PIECES <= GQ_COPIES * 64, "the copies cover the slot");

// The int8 variant's stage of one 128-element K chunk: [row][plane][8 chunks
// of 16 bytes] (natural K order), chunk position c ^ (row & 7); one copy
// covers four rows.
QG_DEV void stage_rows128_i8(uint8_t *stage, const int8_t *planes, int D, const int *src, int chunk, int nrows, int wave,
                             int lane) {
    for (int q = wave; 4 * q < nrows; q += PF_WAVES) {
        const int tr = 4 * q + (lane >> 4), p = (lane >> 3) & 1, c = (lane & 7) ^ (tr & 7);
        dma16_ordered(planes + ((size_t)src[tr] * 2 + p) * D + (size_t)chunk * 128 + c * 16, stage + q * 1024);
    }
}
// 8 int8 activations of row r, plane p: elements 8 kq .. 8 kq + 7 of group f
// of the chunk.
QG_DEV long stage_frag128_i8(const uint8_t *st, int r, int p, int f, int kq) {
    return *(const long *)(st + r * 256 + p * 128 + 16 * ((2 * f + (kq >> 1)) ^ (r & 7)) + 8 * (kq & 1));
}

// The int8 variant of gq_chunk: one v_mfma_i32_16x16x32_i8 per group and
// activation plane, the weights as their nibbles q (0..15); per group the
// int32 pair is joined (256 hi + lo, exact) and scaled by s_g in fp32, then
// d and the row scale sx are applied per half.  The min term is gq_chunk's.
template <int M, int MY>
QG_DEV void gq_chunk_i8(qg_f4 (&y)[MY][NCT], const uint8_t *slot, const uint8_t *st, const uint8_t *ss, const float (&sx)[4][4],
                        int h, int j, int kq) {
    static_assert(M <= MY, "row tiles");
    Q4kHeader hd[NCT];
    const uint8_t *rowp[NCT];
    uint32_t S[NCT];
#pragma unroll
    for (int n = 0; n < NCT; n++) {
        rowp[n] = slot + (16 * n + j) * GQ_ROWB;
        hd[n] = q4k_header(*(const uint4 *)rowp[n]);
        S[n] = h ? hd[n].S[1] : hd[n].S[0];  // group 4h + f scale in byte f
    }
    qg_f4 ys[M][NCT];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int n = 0; n < NCT; n++) ys[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int f = 0; f < 4; f++) {
        long w[NCT];
        float sg[NCT];
#pragma unroll
        for (int n = 0; n < NCT; n++) {
            // group 4h + f: pair f / 2 of the half, nibble f % 2; the lane's 8 elements
            const uint2 q = *(const uint2 *)(rowp[n] + 16 + 32 * (f >> 1) + 8 * kq);
            const int sh = 4 * (f & 1);
            w[n] = (long)(((uint64_t)((q.y >> sh) & 0x0F0F0F0Fu) << 32) | ((q.x >> sh) & 0x0F0F0F0Fu));
            sg[n] = (float)((S[n] >> (8 * f)) & 0xffu);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const long ah = stage_frag128_i8(st, m * 16 + j, 0, f, kq), al = stage_frag128_i8(st, m * 16 + j, 1, f, kq);
#pragma unroll
            for (int n = 0; n < NCT; n++) {
                const qg_i4 ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, w[n], qg_i4{0, 0, 0, 0}, 0, 0, 0);
                const qg_i4 cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, w[n], qg_i4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) ys[m][n][i] = __builtin_fmaf(sg[n], (float)(ch[i] * 256 + cl[i]), ys[m][n][i]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int n = 0; n < NCT; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) y[m][n][i] = __builtin_fmaf(hd[n].d * sx[m][i], ys[m][n][i], y[m][n][i]);
    if (ss) {
        const qg_half8 z8 = qg_half8{0, 0, 0, 0, 0, 0, 0, 0};
        qg_half8 bm[NCT];  // lanes kq >= 2 multiply zero sums
#pragma unroll
        for (int n = 0; n < NCT; n++) bm[n] = q4k_min_frag(hd[n]);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const qg_half8 as = kq < 2 ? ld_frag((const _Float16 *)(ss + ((m * 16 + j) * 2 + kq) * 16)) : z8;
#pragma unroll
            for (int n = 0; n < NCT; n++) {
                const qg_f4 mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bm[n], qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) y[m][n][i] = __builtin_fmaf(-hd[n].dmin, mm[i], y[m][n][i]);
            }
        }
    }
}

// One half superblock for the first M row tiles: per K step f (4 of them)
// the two weight fragments, then every row tile's products (fragment f + 1
// is built while step f's products run); y += d * acc per half, and with the
// sums (first half) the min term -dmin * (m . X) over the superblock's 8
// groups.  issue(f) runs after K step f's products are issued: the caller's
// copies for later steps go out while the matrix cores work.  Row r of the
// slot starts at RS r, its piece p at PS p from there; column tile n is rows
// 16 n .. 16 n + 15.
template <int M, int NC, int RS, int PS, int MY, typename Issue = NoIssue>
QG_DEV void gq_chunk(qg_f4 (&y)[MY][NC], const uint8_t *slot, const uint8_t *st, const uint8_t *ss, int h, int j, int kq,
                     Issue issue = Issue{}) {
    static_assert(M <= MY, "row tiles");
    Q4kHeader hd[NC];
    uint4 qc[NC];
    qg_half2 sc[NC], of[NC];
#pragma unroll
    for (int n = 0; n < NC; n++) {
        const uint8_t *row = slot + (16 * n + j) * RS;
        hd[n] = q4k_header(*(const uint4 *)row);
        qc[n] = *(const uint4 *)(row + (1 + kq) * PS);
        gq_scales(h ? hd[n].S[1] : hd[n].S[0], kq, sc[n], of[n]);  // a select: h is a runtime value
    }
    qg_f4 acc[M][NC];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int f = 0; f < 4; f++) {
        qg_half8 b[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) b[n] = gq_frag(qc[n], f, sc[n][f >> 1], of[n][f >> 1]);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const qg_half8 a0 = stage_frag128(st, m * 16 + j, 0, 4 * f + kq), a1 = stage_frag128(st, m * 16 + j, 1, 4 * f + kq);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[n], acc[m][n], 0, 0, 0);
                acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[n], acc[m][n], 0, 0, 0);
            }
        }
        issue(f);
        if (M > 2) __builtin_amdgcn_sched_barrier(0);  // one K step's fragments live at a time
    }
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int n = 0; n < NC; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) y[m][n][i] = __builtin_fmaf(hd[n].d, acc[m][n][i], y[m][n][i]);
    if (ss) {
        // min term: lanes kq = 0 / 1 carry the hi / lo plane of the 8 group
        // sums, the other lanes zeros (their mins multiply zero)
        const qg_half8 z8 = qg_half8{0, 0, 0, 0, 0, 0, 0, 0};
        qg_half8 bm[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) bm[n] = q4k_min_frag(hd[n]);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const qg_half8 as = kq < 2 ? ld_frag((const _Float16 *)(ss + ((m * 16 + j) * 2 + kq) * 16)) : z8;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const qg_f4 mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bm[n], qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) y[m][n][i] = __builtin_fmaf(-hd[n].dmin, mm[i], y[m][n][i]);
            }
        }
    }
}

// Item = (group, 64-row tile, 128 F rows); wave w: F rows f0 = 16 w .. +15 of
// the block, column tile 0 their gate rows, tile 1 their up rows.  Steps are
// the item's D/128 half superblocks.  The step loop runs inside one
// instantiation per row-tile count M, entered once per item, so the
// accumulators stay in place for the item's steps; the per-lane addresses of
// the copies are formed once per item and advanced per step.
template <bool I8>
__global__ __launch_bounds__(512, 1) void pf_gateup_kernel(GuArgs A) {
    extern __shared__ uint4 s_dyn[];
    uint8_t *lds = (uint8_t *)s_dyn;
    __shared__ int s_tb[NG + 1], s_go[NG], s_off[QG_EXPERTS + 1];
    __shared__ int2 s_it[IT_RING];
    __shared__ int s_src[2][PT];
    __shared__ float s_sx[2][PT];            // the int8 variant: row scales of the item's rows
    __shared__ float s_gs[PF_WAVES][PT];     // 16-row partial sums of the 32-row groups (Q4_K down format)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    for (int i = tid; i <= NG; i += 512) {
        s_tb[i] = A.tt->tbase[i];
        if (i < NG) s_go[i] = A.tt->gorder[i];
        if (i <= QG_EXPERTS) s_off[i] = A.offsets[i];
    }
    const int nfb = A.F / GU_FB, NH = A.D / 128, D32 = A.D / 32, F = A.F;   // NH steps per item (even)
    const int t_lo = A.tt->bounds[A.seg_lo], total = (A.tt->bounds[A.seg_hi] - t_lo) * nfb;
    const ItemRange ir = balanced_items<7, 3>(A.tt, s_tb, A.seg_lo, A.seg_hi, nfb);
    const int nitems = range_count(ir), steps = nitems * NH;
    if (steps == 0) return;  // block-uniform
    const ItemRing R{s_it, s_tb, s_go, s_off, A.nt, t_lo, nfb, nitems, ir};
    __syncthreads();
    R.fill(0, IT_RING, tid);
    __syncthreads();
    uint8_t *sums = lds + 2 * IQ_STAGE;                                       // two superblock sum buffers
    uint8_t *ring = lds + 2 * IQ_STAGE + 2 * GQ_SUMS + (size_t)wave * 3 * GQ_SLOT;  // this wave's three slots
    // mid row of tile row tr (< nv): the CSR position, shared rows after the 10 nt selections
    auto mrow = [&](const PfItem &it, int tr) { return it.shared ? A.nt * QG_TOP + it.base + tr : it.base + tr; };
    // tile rows: their tokens (and with the int8 variant their row scales)
    auto set_rows = [&](const PfItem &it, int buf) {
        item_rows(s_src[buf], it, A.row_token, 0, wave, lane);
        if (I8 && wave == 1) dma4_ordered((it.shared ? A.xsc : A.row_sx) + it.base + min(lane, it.nv - 1), s_sx[buf]);
    };
    // Weight copies: piece i = 64 t + lane of a slot is piece p of row r (r <
    // 16 the gate row f0 + r, else the up row f0 + r - 16): the superblock's
    // header (p = 0) or 16-byte piece p - 1 of the half's 64 qs bytes, at
    // 16 p + 64 h from the superblock.
    uint32_t w_off[GQ_COPIES], w_h[GQ_COPIES];
    bool w_up[GQ_COPIES];
#pragma unroll
    for (int t = 0; t < GQ_COPIES; t++) {
        const int i = min(t * 64 + lane, 32 * GQ_PIECES - 1), r = i / GQ_PIECES, p = i - GQ_PIECES * r;
        w_off[t] = (uint32_t)((r & 15) * A.rb) + (uint32_t)(16 * p);
        w_h[t] = p == 0 ? 0u : 64u;
        w_up[t] = r >= 16;
    }
    const uint8_t *wp[GQ_COPIES];  // the lane's rows of the item being copied
    auto set_wp = [&](const PfItem &it) {
        const uint8_t *bg = it.shared ? A.sh_gate : A.gate + (size_t)it.g * F * A.rb;
        const uint8_t *bu = it.shared ? A.sh_up : A.up + (size_t)it.g * F * A.rb;
        const size_t f0 = (size_t)(it.blk * GU_FB + wave * 16) * A.rb;
#pragma unroll
        for (int t = 0; t < GQ_COPIES; t++) wp[t] = (w_up[t] ? bu : bg) + f0 + w_off[t];
    };
    auto copy_w = [&](int q, int c) {  // step c of the item being copied into slot q
        const uint32_t sb = (uint32_t)(c >> 1) * 144u;
        const bool h = c & 1;
        static_assert(GQ_COPIES == 3, "three copies under one M0 value");
        dma16x3_ordered(wp[0] + sb + (h ? w_h[0] : 0u), wp[1] + sb + (h ? w_h[1] : 0u), wp[2] + sb + (h ? w_h[2] : 0u),
                        ring + q * GQ_SLOT);
    };
    // Activation copies of the item being staged: copy i of this wave (tile
    // rows of copy number q = wave + 8 i) and, for the waves that copy them,
    // the rows' group sums; step c adds its chunk offset.
    const uint8_t *sp[4] = {nullptr, nullptr, nullptr, nullptr}, *sump = nullptr;
    int s_nc = 0;      // this wave's activation copies per step of the item being staged
    bool s_sum = false; // and whether it copies group sums
    auto set_sp = [&](const PfItem &it, int buf) {
        s_nc = I8 ? (4 * it.M - wave + 7) / 8 : it.M;   // copy numbers q = wave + 8 i below 4 M (int8) or 8 M
        s_sum = wave * 32 < 16 * it.M;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = wave + PF_WAVES * i;
            if (I8 && 4 * q < 16 * it.M) {
                const int tr = 4 * q + (lane >> 4), p = (lane >> 3) & 1, c8 = (lane & 7) ^ (tr & 7);
                sp[i] = (const uint8_t *)A.xi8 + ((size_t)s_src[buf][tr] * 2 + p) * A.D + c8 * 16;
            } else if (!I8 && 2 * q < 16 * it.M) {
                const int tr = 2 * q + (lane >> 5), p = (lane >> 4) & 1, c16 = (lane & 15) ^ (tr & 15);
                sp[i] = (const uint8_t *)(A.xp + ((size_t)s_src[buf][tr] * 2 + p) * A.D + c16 * 8);
            }
        }
        if (s_sum) {
            const int C = wave * 64 + lane, tr = C >> 1, p = C & 1;
            sump = (const uint8_t *)(A.xsp + ((size_t)s_src[buf][tr] * 2 + p) * D32);
        }
    };
    // the stage of step s (chunk c of the item being staged)
    auto stage_at = [&](int s, int c) {
        uint8_t *st = lds + (s & 1) * IQ_STAGE;
        const size_t co = (size_t)c * (I8 ? 128 : 256);
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < s_nc) dma16_ordered(sp[i] + co, st + (wave + PF_WAVES * i) * 1024);
        if ((c & 1) == 0 && s_sum) dma16_ordered(sump + (size_t)(c >> 1) * 16, sums + ((s >> 1) & 1) * GQ_SUMS + wave * 1024);
    };
    // prologue: item 0's rows, its first stage, the weights of steps 0 and 1
    PfItem cur = R.at(0);
    set_rows(cur, 0);
    wait_vmem();
    __syncthreads();
    set_sp(cur, 0);
    stage_at(0, 0);
    set_wp(cur);
    copy_w(0, 0);
    if (1 < steps) copy_w(1, 1);  // NH >= 2: step 1 is item 0's
    int s = 0, qc = 0;  // step s reads slot s % 3; the copies of step s + 2 go to slot (s + 2) % 3 (read by step s - 1)
    auto run_item = [&](const int k, auto MC) {
        constexpr int M = decltype(MC)::value;
        qg_f4 y[M][NCT];
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int n = 0; n < NCT; n++) y[m][n] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = 0; c < NH; c++, s++) {
            const int qn = qc == 0 ? 2 : qc - 1;
            if (s + 1 < steps) wait_vmem_but<GQ_COPIES>();
            else wait_vmem();
            __syncthreads();
            if (c == 0) {
                if (k > 0 && (k & (IT_BATCH - 1)) == 0) R.fill(k + IT_BATCH, IT_BATCH, tid);
                // the next item's rows, copied while this item streams (its buffer
                // held item k - 1's rows, staged long ago)
                if (k + 1 < nitems) set_rows(R.at(k + 1), (k + 1) & 1);
            }
            // the next step's stage, then the weights of step s + 2 (in this
            // order: the wait above relies on it); the fp16 pass issues them
            // between its first K steps' products
            auto issue = [&](int f) {
                if (f == 0 && s + 1 < steps) {
                    if (c == NH - 1) set_sp(R.at(k + 1), (k + 1) & 1);
                    stage_at(s + 1, c == NH - 1 ? 0 : c + 1);
                }
                if (f == 1 && s + 2 < steps) {
                    if (c == NH - 2) set_wp(R.at(k + 1));
                    copy_w(qn, c + 2 < NH ? c + 2 : c + 2 - NH);
                }
            };
            const uint8_t *st = lds + (s & 1) * IQ_STAGE, *slot = ring + qc * GQ_SLOT;
            const uint8_t *ss = (c & 1) == 0 ? sums + ((s >> 1) & 1) * GQ_SUMS : nullptr;
            if constexpr (I8) {
                issue(0);
                issue(1);
                float sxv[4][4];  // the scales of the lane's rows m 16 + 4 kq + i
#pragma unroll
                for (int m = 0; m < 4; m++)
#pragma unroll
                    for (int i = 0; i < 4; i++) sxv[m][i] = s_sx[k & 1][m * 16 + 4 * kq + i];
                gq_chunk_i8<M>(y, slot, st, ss, sxv, c & 1, j, kq);
            } else {
                gq_chunk<M, NCT, GQ_ROWB, 16>(y, slot, st, ss, c & 1, j, kq, issue);
            }
            qc = qc == 2 ? 0 : qc + 1;
        }
        // SwiGLU of the item: tile 0 the gate rows, tile 1 the up rows of F row f
        const PfItem it = R.at(k);
        const int fmt = it.shared ? A.sh_down_fmt : A.down_fmt;
        const int f = it.blk * GU_FB + wave * 16 + j, pa = plane_pos(fmt, f);
#pragma unroll
        for (int m = 0; m < M; m++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tr = m * 16 + 4 * kq + i;
                const float ma = qg_swiglu_fast(y[m][0][i], y[m][1][i]);
                if (tr < it.nv) {
                    _Float16 *hp = A.midp + (size_t)mrow(it, tr) * 2 * F;
                    const _Float16 ha = (_Float16)ma;
                    hp[pa] = ha;
                    hp[F + pa] = (_Float16)(ma - (float)ha);
                }
                if (fmt == QT_Q4_K) {
                    // this wave's 16 rows of the 32-row group (lanes of one kq hold all 16 j)
                    float sp2 = ma;
                    sp2 += __shfl_xor(sp2, 1);
                    sp2 += __shfl_xor(sp2, 2);
                    sp2 += __shfl_xor(sp2, 4);
                    sp2 += __shfl_xor(sp2, 8);
                    if (j == 0) s_gs[wave][tr] = sp2;
                }
            }
        }
        if (fmt == QT_Q4_K) {  // block-uniform
            __syncthreads();
            // waves 2i and 2i+1 hold the two halves of 32-row group i of the block
            if ((wave & 1) == 0 && lane < it.nv) {
                const float sum = s_gs[wave][lane] + s_gs[wave + 1][lane];
                _Float16 *gp = A.msp + (size_t)mrow(it, lane) * 2 * (F / 32) + (it.blk * GU_FB + wave * 16) / 32;
                const _Float16 hs = (_Float16)sum;
                gp[0] = hs;
                gp[F / 32] = (_Float16)(sum - (float)hs);
            }
        }
    };
    for (int k = 0; k < nitems; k++) {
        switch (R.at(k).M) {  // block-uniform
        case 1: run_item(k, std::integral_constant<int, 1>{}); break;
        case 2: run_item(k, std::integral_constant<int, 2>{}); break;
        case 3: run_item(k, std::integral_constant<int, 3>{}); break;
        default: run_item(k, std::integral_constant<int, 4>{}); break;
        }
    }
}

// ---------------- P7: combine ----------------
struct CombArgs {
    int nt, D;
    const int *ids; const float *w; const int *flag;
    const float *slots;
    const float *sh_logit; int ld;   // shared gate logit of token t at sh_logit[t*ld], or null
    float *out, *resid;
};

// out[t] = sum_k (w[t,k] * y[t,k]) in rank order (each product rounded, as
// the slot products of cpu.c:253-259), then + y_sh * sigmoid(logit)
// (gpu.cu:552-553).  Flag 2 rows (host handoff) get the shared part only,
// flag 3 rows 0.
__global__ __launch_bounds__(256) void pf_combine_kernel(CombArgs A) {
    const int t = blockIdx.y, d = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (d >= A.D) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (A.flag[t] < 2) {
#pragma unroll
        for (int k = 0; k < QG_TOP; k++) {
            const int e = A.ids[(size_t)t * QG_TOP + k];
            if (e < 0 || e >= QG_EXPERTS) continue;
            const float wk = A.w[(size_t)t * QG_TOP + k];
            const float4 v = *(const float4 *)(A.slots + ((size_t)t * QG_TOP + k) * A.D + d);
            acc.x += __fmul_rn(v.x, wk);
            acc.y += __fmul_rn(v.y, wk);
            acc.z += __fmul_rn(v.z, wk);
            acc.w += __fmul_rn(v.w, wk);
        }
    }
    if (A.sh_logit && A.flag[t] != 3) {
        const float sg = qg_sig(A.sh_logit[(size_t)t * A.ld]);
        const float4 v = *(const float4 *)(A.slots + ((size_t)A.nt * QG_TOP + t) * A.D + d);
        acc.x = __builtin_fmaf(v.x, sg, acc.x);
        acc.y = __builtin_fmaf(v.y, sg, acc.y);
        acc.z = __builtin_fmaf(v.z, sg, acc.z);
        acc.w = __builtin_fmaf(v.w, sg, acc.w);
    }
    const size_t o = (size_t)t * A.D + d;
    if (A.out) *(float4 *)(A.out + o) = acc;
    if (A.resid) {
        float4 h = *(float4 *)(A.resid + o);
        h.x += acc.x; h.y += acc.y; h.z += acc.z; h.w += acc.w;
        *(float4 *)(A.resid + o) = h;
    }
}

// Pruning counters (gpu.cu:484-487 semantics) over the batch, in a fixed
// reduction order, added to *stats by one block.
__global__ __launch_bounds__(1024) void pf_stats_kernel(qg_prune_stats *stats, const int *flag, const int *missing,
                                                        const double *mass, int nt) {
    __shared__ unsigned long long s_c[4][1024];
    __shared__ double s_m[1024];
    const int tid = threadIdx.x;
    unsigned long long tl = 0, ms = 0, sk = 0, av = 0;
    double sm = 0.0;
    for (int t = tid; t < nt; t += 1024) {
        const int f = flag[t];
        if (f == 3) continue;
        tl += 1;
        ms += (unsigned long long)missing[t];
        if (f == 1) { sk += (unsigned long long)missing[t]; av += 1; sm += mass[t]; }
    }
    s_c[0][tid] = tl; s_c[1][tid] = ms; s_c[2][tid] = sk; s_c[3][tid] = av;
    s_m[tid] = sm;
    __syncthreads();
    for (int h = 512; h > 0; h >>= 1) {
        if (tid < h) {
#pragma unroll
            for (int c = 0; c < 4; c++) s_c[c][tid] += s_c[c][tid + h];
            s_m[tid] += s_m[tid + h];
        }
        __syncthreads();
    }
    if (tid == 0) {
        stats->token_layers += s_c[0][0];
        stats->missing_selections += s_c[1][0];
        stats->skipped_selections += s_c[2][0];
        stats->avoided_token_handoffs += s_c[3][0];
        stats->skipped_mass += s_m[0];
    }
}

}  // namespace

// Gate/up launches of the calling thread's prefill layers: 0 one launch over
// every group; 1 the dense experts in a launch of their own in int8 (two int8
// activation planes, per-group int32 -> fp32 scaling), then the rest; 2 the
// same split with both launches in fp16 (the like-for-like timing of the
// dense experts).  Other values are taken as 0.
static thread_local int tl_pf_split = 0;
extern "C" int qg_prefill_int8_dense(int mode) {
    const int prev = tl_pf_split;
    tl_pf_split = mode == 1 || mode == 2 ? mode : 0;
    return prev;
}

bool qg_prefill_ok(const qg_moe_layer *L) {
    const int D = L->width, F = L->ff;
    if (D % DN_DB || F % GU_FB) return false;
    auto down_ok = [&](int t) { return t == QT_IQ4_NL || (t == QT_Q4_K && F % 256 == 0); };
    if (L->gate_type != QT_Q4_K || L->up_type != QT_Q4_K || !down_ok(L->down_type)) return false;
    if (L->sh_gate && (L->sh_gate_type != QT_Q4_K || L->sh_up_type != QT_Q4_K || !down_ok(L->sh_down_type))) return false;
    return true;
}

size_t qg_prefill_workspace_bytes(int width, int ff, int tokens) {
    if (width < 256 || width % DN_DB || width > 8192 || ff < GU_FB || ff % GU_FB || ff > 4096 || tokens < PF_MIN ||
        tokens > QG_MAX_TOKENS)
        return 0;
    return pf_layout(width, ff, tokens).total;
}

int qg_prefill_forward(float *out, float *resid, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                       const float *x, float *xn_out, int norm, int nt, const qg_moe_layer *L, void *workspace) {
    if (nt < PF_MIN || nt > QG_MAX_TOKENS || !qg_prefill_ok(L)) return hipErrorInvalidValue;
    const int D = L->width, F = L->ff;
    const PfLayout lay = pf_layout(D, F, nt);
    uint8_t *ws = (uint8_t *)workspace;
    hipStream_t s = qg_stream();
    const bool sh = L->sh_gate != nullptr;
    const int rows = QG_EXPERTS + (sh ? 1 : 0), nch = (nt + PF_CHUNK - 1) / PF_CHUNK;
    float *logits = (float *)(ws + lay.logits);
    int *flag = (int *)(ws + lay.flag), *counts = (int *)(ws + lay.counts), *offsets = (int *)(ws + lay.offsets);
    TileTable *tt = (TileTable *)(ws + lay.tbase);
    int *row_token = (int *)(ws + lay.row_token), *row_slot = (int *)(ws + lay.row_slot);
    _Float16 *xp = (_Float16 *)(ws + lay.xp), *xsp = (_Float16 *)(ws + lay.xsp);
    _Float16 *midp = (_Float16 *)(ws + lay.midp), *msp = (_Float16 *)(ws + lay.msp);
    float *slots = (float *)(ws + lay.slots);
    int rc;
    if (norm) {
        float *xn = xn_out ? xn_out : (float *)(ws + lay.xn);
        pf_norm_kernel<<<(nt + 3) / 4, 256, 0, s>>>(xn, x, nt, D, 1e-6f);
        if ((rc = hipGetLastError())) return rc;
        x = xn;
    }
    // P1: router logits in the reference's order (+ shared gate row, + bias)
    RouterArgs R{x, nt, D, rows, L->router, sh ? L->sh_gate_inp : nullptr, L->router_bias, logits};
    pf_launch(0, pf_router_kernel, dim3((nt + RT_TOK - 1) / RT_TOK, (rows + RT_ROWS - 1) / RT_ROWS), dim3(64 * RT_WAVES), RT_LDS, s, R);
    if ((rc = hipGetLastError())) return rc;
    const int split = tl_pf_split;
    const bool i8 = split == 1;
    int8_t *xi8 = i8 ? (int8_t *)(ws + lay.xi8) : nullptr;
    float *xsc = i8 ? (float *)(ws + lay.xsc) : nullptr, *row_sx = i8 ? (float *)(ws + lay.row_sx) : nullptr;
    RouteArgs RA{nt, logits, rows, L->resident, L->threshold, ids, weights, flags, flag,
                 (int *)(ws + lay.missing), (double *)(ws + lay.mass), x, D, xp, xsp, xi8, xsc};
    pf_launch(1, pf_route_kernel, dim3((nt + 3) / 4), dim3(512), 0, s, RA);
    if ((rc = hipGetLastError())) return rc;
    pf_launch(10, pf_count_kernel, dim3(nch), dim3(512), 0, s, counts, (int *)nullptr, (const int *)ids, (const int *)flag, nt);
    if ((rc = hipGetLastError())) return rc;
    pf_launch(2, pf_scan_kernel, dim3(1), dim3(512), 0, s, counts, nch, offsets, tt, sh ? nt : 0, (const int *)nullptr,
              (int *)nullptr);
    if ((rc = hipGetLastError())) return rc;
    pf_launch(3, pf_fill_kernel, dim3(nch), dim3(512), 0, s, row_token, row_slot, (const int *)counts, (const int *)ids,
              (const int *)flag, nt, row_sx, (const float *)xsc);
    if ((rc = hipGetLastError())) return rc;
    // grouped GEMMs: one launch over every group (dense experts, the shared
    // expert, the others); qg_prefill_int8_dense splits the dense experts off
    const int grid = qg_cu_count();
    auto gate_up = [&](int seg_lo, int seg_hi, bool int8, int slot) {
        GuArgs G{nt, D, F, offsets, tt, seg_lo, seg_hi, row_token, (const uint8_t *)L->gate, (const uint8_t *)L->up,
                 sh ? (const uint8_t *)L->sh_gate : nullptr, sh ? (const uint8_t *)L->sh_up : nullptr, qg_row_bytes_host(QT_Q4_K, D),
                 xp, xsp, midp, msp, L->down_type, sh ? L->sh_down_type : L->down_type, xi8, xsc, row_sx};
        if (int8) pf_launch(slot, pf_gateup_kernel<true>, dim3(grid), dim3(512), PF_GQ_LDS, s, G);
        else pf_launch(slot, pf_gateup_kernel<false>, dim3(grid), dim3(512), PF_GQ_LDS, s, G);
        return hipGetLastError();
    };
    if (split) {
        if ((rc = gate_up(0, 1, i8, 4))) return rc;
        if ((rc = gate_up(1, 3, false, 5))) return rc;
    } else if ((rc = gate_up(0, 3, false, 5))) {
        return rc;
    }
    auto down = [&](int seg_lo, int seg_hi, int fmt, int slot) {
        DnArgs DA{nt, D, F, offsets, tt, seg_lo, seg_hi, row_slot, (const uint8_t *)L->down, sh ? (const uint8_t *)L->sh_down : nullptr,
                  qg_row_bytes_host(L->down_type, F), sh ? qg_row_bytes_host(L->sh_down_type, F) : 0, midp, msp, slots};
        if (fmt == QT_Q4_K) pf_launch(slot, pf_down_kernel, dim3(grid), dim3(512), PF_LDS, s, DA);
        else pf_launch(slot, pf_down_iq_kernel, dim3(grid), dim3(512), PF_IQ_LDS, s, DA);
        return hipGetLastError();
    };
    if (!sh || L->sh_down_type == L->down_type) {
        if ((rc = down(0, 3, L->down_type, 7))) return rc;
    } else {  // the shared expert's down in its own format
        if ((rc = down(0, 1, L->down_type, 6))) return rc;
        if ((rc = down(2, 3, L->down_type, 7))) return rc;
        if ((rc = down(1, 2, L->sh_down_type, 8))) return rc;
    }
    CombArgs CA{nt, D, ids, weights, flag, slots, sh ? logits + QG_EXPERTS : nullptr, rows, out, resid};
    pf_launch(9, pf_combine_kernel, dim3((D / 4 + 255) / 256, nt), dim3(256), 0, s, CA);
    if ((rc = hipGetLastError())) return rc;
    if (stats && L->resident) {  // counters exist only with a resident mask (gpu.cu:484-488)
        pf_stats_kernel<<<1, 1024, 0, s>>>(stats, flag, (const int *)(ws + lay.missing), (const double *)(ws + lay.mass), nt);
        if ((rc = hipGetLastError())) return rc;
    }
    return hipSuccess;
}

// CSR dispatch of an ids array (qg_moe_dispatch): histogram per 32-token
// chunk, prefix sums, stable fill.  scratch: qg_prefill_dispatch_scratch(nt) bytes.
size_t qg_prefill_dispatch_scratch(int nt) {
    const size_t nch = (nt + PF_CHUNK - 1) / PF_CHUNK;
    return nch * QG_EXPERTS * 4 + nch * 4;
}

int qg_prefill_dispatch(int *offsets, int *row_token, int *row_slot, int *status, const int *ids, int nt, void *scratch) {
    const int nch = (nt + PF_CHUNK - 1) / PF_CHUNK;
    int *counts = (int *)scratch, *bad = counts + (size_t)nch * QG_EXPERTS;
    hipStream_t s = qg_stream();
    pf_count_kernel<<<nch, 512, 0, s>>>(counts, bad, ids, nullptr, nt);
    int rc = hipGetLastError();
    if (rc) return rc;
    pf_scan_kernel<<<1, 512, 0, s>>>(counts, nch, offsets, nullptr, 0, bad, status);
    if ((rc = hipGetLastError())) return rc;
    pf_fill_kernel<<<nch, 512, 0, s>>>(row_token, row_slot, counts, ids, nullptr, nt, nullptr, nullptr);
    return hipGetLastError();
}
