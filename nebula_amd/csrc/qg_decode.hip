// Device-driven routed-MoE layer for decode batches (1..17 tokens): the fast
// path of qg_moe_forward (and qg_moe_forward_residual) for Q4_K gate/up and
// Q4_K or IQ4_NL down.  It replaces moe()/grouped_moe()/shared_direct() of
// qwen.c:633-735 for one layer without any host round trip.
//
// Kernels per layer (3 for B = 1, 5 above).  No kernel waits on another block
// of its own grid: on MI355X a grid-wide ticket costs ~12 ns per block of
// serialised atomics and a device-scope fence ~17 us per 1000 waves, more than
// a kernel boundary (~1.7-2.4 us).
//   K1 router  : the 512 router rows (plus the shared-expert gate vector as
//                row 512) for every token in the reference's fixed summation
//                order, so logits, ids and weights are bit-exact.  Extra
//                blocks write the fp16 hi/lo activation planes and per-32
//                sums; optionally the input is RMS-normalised first.
//   KR route   : B > 1 only; a block per token (top-10, coverage/prune,
//                flags), setting the token's bit in each eligible expert's
//                token mask (cleared by the router's first plane block); the
//                gate/up workgroups build the plan from the masks (D = 2048)
//                or from the ids (D = 2560).
//   K2 gate/up : B > 1 at D = 2048: one workgroup per CU, each on one
//                expert's run of 16-row F blocks for all of the expert's
//                tiles, so every weight row is read once (dec_gateup3).
//                B = 1: persistent over (tile, 16 F rows) items, routing the
//                token inline (every workgroup routes it; workgroup 0
//                publishes the plan) (dec_gateup2).  D = 2560: the
//                register-weight kernel (dec_gateup).  Products on the
//                matrix cores (v_mfma_f32_16x16x32_f16) with exact integer
//                weights; SwiGLU; mid rows written as fp16 hi/lo planes with
//                their 8-row sums.
//   K3 down    : persistent; item = (tile, 64 output rows): weight slab and
//                the tile's mid planes staged in shared memory, products on
//                the matrix cores, weighted results to per-selection slots
//                (B = 1: down and combine in one kernel, dec_down1).
//   K4 combine : router-rank sum of the 10 slots, the sigmoid-gated shared
//                expert and the optional residual add.
//
// Operand conventions and the K order of the weight formats are those of
// qg_frag.h; here A row j = (token j/2, plane j%2), so a lane's D rows
// 4kq..4kq+3 are tokens 2kq, 2kq+1 (hi, lo) of weight row j.
#include "qg_internal.h"
#include "qg_frag.h"
#include <hip/hip_ext.h>
#include <mutex>
#include <type_traits>

namespace {

constexpr int MB = QG_MAX_DECODE;         // 17 tokens
constexpr int MS = MB * QG_TOP;           // 170 selections
constexpr int ME = MS + MB;               // selection rows + shared-expert rows
constexpr int INLINE_MAX = 1;             // tokens routed inside the gate/up kernel
constexpr int GU_WGS = 512;               // gate/up grid cap (workgroups)
constexpr int GU_NI = 8;                  // items per gate/up workgroup at most
constexpr int DN_WGS = 1024;              // down grid cap (workgroups)

// Routing results of the batch and its tile plan, written once per layer by
// the routing step (the routing kernel, or gate/up workgroup 0 at one token)
// and read by gate/up, down and combine.  A selection q = t*10 + rank is
// eligible when its id is an expert (pruned selections carry -id-2) and its
// token is computed here (flag 0 or 1).  Each expert with eligible selections
// (in order of its first one) contributes tiles of up to 8 of them in token
// order (a token lists an expert at most once).  The shared expert's tiles
// (tokens 8i..8i+7) come first and are implicit.
constexpr int TILE_TOK = 8;
constexpr int MAX_TILES = MS;                // at most one tile per selection
struct DecTile { int e, n, q[TILE_TOK]; };
struct DecPlan {
    int flag[MB]; int missing[MB]; double mass[MB];
    int n_tiles;                             // routed tiles
    uint32_t emask[QG_EXPERTS];              // B > 1: bit t set when token t has an eligible selection of the expert
    DecTile tile[MAX_TILES];
};

struct DecLayout { size_t tok, logits, xp, xsum, midp, msum, slots, total; };
DecLayout dec_layout(int D, int F) {
    DecLayout L;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += (n + 255) & ~(size_t)255; return o; };
    L.tok = take(sizeof(DecPlan));
    L.logits = take((size_t)MB * (QG_EXPERTS + 1) * 4);
    L.xp = take((size_t)MB * 2 * D * 2);
    L.xsum = take((size_t)MB * 2 * (D / 32) * 2);
    L.midp = take((size_t)ME * 2 * F * 2);
    L.msum = take((size_t)ME * (F / 8) * 4);
    L.slots = take((size_t)ME * D * 4);
    L.total = off;
    return L;
}

// Optional kernel timing (benchmark support): events[2i], events[2i+1] are
// recorded at the start and end of kernel i (0 router, 1 route, 2 gate/up,
// 3 down) by hipExtLaunchKernelGGL on the launch stream.
thread_local void *tl_kev[32] = {nullptr};
thread_local int tl_kev_n = 0;

template <typename K, typename... Args>
void dec_launch(int slot, K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    if (2 * slot + 1 < tl_kev_n && tl_kev[2 * slot] && tl_kev[2 * slot + 1])
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, (hipEvent_t)tl_kev[2 * slot],
                              (hipEvent_t)tl_kev[2 * slot + 1], 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}


// ---------------- K1: router + activation planes ----------------
struct RouterArgs {
    const float *x;
    int nt, D, rows;                // rows = 512, or 513 with the shared gate vector
    const float *router, *sh_row;
    float *logits;                  // [nt][rows]
    int norm; float eps; float *xn; // RMS-normalise the input; normalised rows to xn
    _Float16 *xp, *xsp;             // planes [nt][2][D] (Q4_K order); planes of 32-group sums [nt][2][D/32]
    int plane_blocks;               // blockIdx.x < plane_blocks: planes; above: router rows
    const float *bias;              // F32 [512] added to the expert logits, or null
    uint32_t *emask;                // the plan's per-expert token masks, cleared by the first plane block, or null
};


// The exact-order dot product of one router row with one token row: lane j of
// each 32-lane half accumulates columns k = j (mod 32) in ascending k with fma,
// then the 16/8/4/2/1 tree (cpu.c:122-139).  Used by the plane blocks for the
// shared-expert gate vector.
template <int KS>
QG_DEV float exact_row_dot(const float *w, const float *x, bool norm, float sc, int j) {
    float wv[KS], xv[KS], acc = 0.0f;  // every load in flight at once
#pragma unroll
    for (int i = 0; i < KS; i++) { wv[i] = w[32 * i + j]; xv[i] = x[32 * i + j]; }
#pragma unroll
    for (int i = 0; i < KS; i++) acc = __builtin_fmaf(wv[i], norm ? xv[i] * sc : xv[i], acc);
    return qg_tree32(acc);
}

// Router: grid (ceil(nt/RW) plane blocks + R x token groups of up to 5), RW
// waves per block (4; 1 at one token), R = 512 / (2 RW) row blocks.  The
// plane blocks come first, so they are dispatched, and their copies queued,
// before the router blocks' 4 MB.  Router block b (counted after the plane
// blocks) covers expert rows 2RW(b % R) .. +2RW-1 and the token group b / R
// (TPB tokens), so the blocks sharing a row block sit on one XCD and share its
// router rows through that L2.  Wave w owns rows 2RW(b % R) + 2w + h (32-lane
// half h), read into registers; the group's token rows are staged in shared
// memory by direct global->shared copies, each block starting at its own
// offset so the CUs do not read the same L2 lines at once.  Lane j
// accumulates columns k = j (mod 32) in ascending k with fma, then the
// 16/8/4/2/1 tree: the order of cpu.c:122-139, so logits equal the
// reference's qc_matmul bit for bit.  Plane blocks: one token per wave: the
// shared-expert gate logit (same order), and the (optionally normalised) row
// as fp16 hi/lo planes in the Q4_K fragment order plus hi/lo planes of the
// sums of each 32-group.
template <int TPB, int DW, int RW>
__global__ __launch_bounds__(256) void dec_router_kernel(RouterArgs A) {
    constexpr int KS = DW / 32, RBLK = QG_EXPERTS / (2 * RW);  // row blocks of 2 RW rows
    extern __shared__ float s_rt[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, j = lane & 31;
    const int nt = A.nt;
    constexpr int CPT = DW / 256;  // 1 KB copies per row
    // every argument in the entry batch of scalar loads (see entry_grid)
    asm volatile("" ::"s"(A.x), "s"(A.nt), "s"(A.D), "s"(A.rows), "s"(A.router), "s"(A.sh_row), "s"(A.logits), "s"(A.norm),
                 "s"(A.eps), "s"(A.xn), "s"(A.xp), "s"(A.xsp), "s"(A.plane_blocks), "s"(A.bias), "s"(A.emask));
    if (blockIdx.x < A.plane_blocks) {
        if (A.emask && blockIdx.x == 0)
            for (int i = threadIdx.x; i < QG_EXPERTS; i += 64 * RW) A.emask[i] = 0u;  // the routing kernel sets them
        const int t = blockIdx.x * RW + wave;
        if (t >= nt) return;  // whole wave; the plane blocks have no block barrier
        // the token row and the shared gate vector, copied into this wave's
        // part of shared memory by 2 CPT copies (all in flight at once, where
        // reading them with per-lane loads took three dependent rounds)
        float *xr = s_rt + (size_t)wave * 2 * DW, *gr = xr + DW;
        for (int c = 0; c < CPT; c++) dma16(A.x + (size_t)t * DW + c * 256 + lane * 4, xr + c * 256);
        if (A.sh_row)
            for (int c = 0; c < CPT; c++) dma16(A.sh_row + c * 256 + lane * 4, gr + c * 256);
        wait_vmem();
        const float sc = A.norm ? lds_rms_scale(xr, DW, A.eps, lane) : 1.0f;
        if (A.sh_row) {
            const float r = exact_row_dot<KS>(gr, xr, A.norm != 0, sc, j);
            if (lane == 0) A.logits[(size_t)t * A.rows + QG_EXPERTS] = r;
        }
        _Float16 *hi = A.xp + (size_t)t * 2 * DW, *shi = A.xsp + (size_t)t * 2 * (DW / 32);
        token_planes(xr, DW, A.norm != 0, sc, lane, hi, hi + DW, shi, shi + DW / 32, A.xn ? A.xn + (size_t)t * DW : nullptr);
        return;
    }
    const int b = blockIdx.x - A.plane_blocks, rb = b % RBLK, t0 = (b / RBLK) * TPB;
    const int ntg = min(TPB, nt - t0);  // tokens of this group (>= 1)
    const int row = rb * 2 * RW + 2 * wave + half;
    const float *wr = A.router + (size_t)row * DW;
    // the group's token rows, 1 KB per copy, rotated start
    const int ncp = ntg * CPT, rot = (int)((b * 37u) % (unsigned)ncp);
    for (int q = wave; q < ncp; q += RW) {
        int c = q + rot;
        if (c >= ncp) c -= ncp;
        dma16(A.x + (size_t)t0 * DW + c * 256 + lane * 4, s_rt + c * 256);
    }
    // the wave's router rows, in flight with the copies: a wave has at most
    // 63 vector-memory operations outstanding (issue stalls beyond, until
    // the oldest returns), so the first W0 go out now and the rest during
    // the first k-steps, long before the chains reach them
    constexpr int NCP = (TPB * CPT + RW - 1) / RW, W0 = KS < 63 - NCP ? KS : 63 - NCP;
    float wv[KS];
#pragma unroll
    for (int i = 0; i < W0; i++) wv[i] = wr[32 * i + j];
    wait_vmem();
    __syncthreads();
    // normalised input: wave w scales the rows of tokens w, w + RW, ... in
    // place (the product x * scale the reference's matmul reads, rounded as
    // there), so the chains run one fma per step
    if (A.norm) {
        for (int u = wave; u < ntg; u += RW) {
            float *xr = s_rt + u * DW;
            const float sc = lds_rms_scale(xr, DW, A.eps, lane);  // every lane's reads precede the sum it returns
            for (int k = lane; k < DW; k += 64) xr[k] *= sc;
        }
        __syncthreads();
    }
    // past the group the chains repeat its first token and are not stored
    float acc[TPB];
    const float *xb[TPB];
#pragma unroll
    for (int u = 0; u < TPB; u++) {
        xb[u] = s_rt + (u < ntg ? u : 0) * DW + j;
        acc[u] = 0.0f;
    }
    // the TPB chains advance together, 4 k-steps per group, with the next
    // group's token values read from shared memory before this group's fmas
    // run (the empty statements pin that order and, at the end of a group,
    // keep the compiler from running one chain ahead while the others' reads
    // pile up in registers)
    float xc[4][TPB], xn[4][TPB];
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
        for (int u = 0; u < TPB; u++) xc[s][u] = xb[u][32 * s];
#pragma unroll
    for (int g = 0; g < KS / 4; g++) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            if (4 * g + s + W0 < KS) wv[4 * g + s + W0] = wr[32 * (4 * g + s + W0) + j];  // the deferred rows' loads
#pragma unroll
            for (int u = 0; u < TPB; u++)
                if (g + 1 < KS / 4) xn[s][u] = xb[u][32 * (4 * g + 4 + s)];
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < TPB; u++) asm volatile("" : "+v"(acc[u]));
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int u = 0; u < TPB; u++) acc[u] = __builtin_fmaf(wv[4 * g + s], xc[s][u], acc[u]);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < TPB; u++) asm volatile("" : "+v"(acc[u]));
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int u = 0; u < TPB; u++) xc[s][u] = xn[s][u];
    }
#pragma unroll
    for (int u = 0; u < TPB; u++) {
        const float r = qg_tree32(acc[u]);
        if (j == 0 && u < ntg) A.logits[(size_t)(t0 + u) * A.rows + row] = A.bias ? r + A.bias[row] : r;
    }
}

// ---------------- KR: routing (B > 1), one block per token ----------------
struct RouteArgs {
    int nt; const float *logits; int ld;
    const uint8_t *resident; double thr;
    int *ids; float *w; uint8_t *flags_out; DecPlan *pl;
};

// Block t routes token t with one wave (top-10, coverage/prune, flags); the
// tokens run on separate CUs.  The expert plan is built from these results by
// every gate/up workgroup (dec_gateup_kernel).
__global__ __launch_bounds__(64) void dec_route_kernel(RouteArgs A) {
    __shared__ __align__(16) float s_rv[QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_ri[QG_ROUTE_SCRATCH];
    const int t = blockIdx.x, lane = threadIdx.x;
    int id, missing;
    float wv;
    double mass;
    qg_route_fast(A.logits + (size_t)t * A.ld, lane, id, wv, s_rv, s_ri);
    const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
    if (lane < QG_TOP) {
        A.ids[t * QG_TOP + lane] = id;
        A.w[t * QG_TOP + lane] = wv;
        // the gate/up kernel's plan: the tokens of each expert's eligible
        // selections (pruned selections carry -id-2; flag-2/3 tokens have none)
        if (flag < 2 && id >= 0 && id < QG_EXPERTS) atomicOr(&A.pl->emask[id], 1u << t);
    }
    if (lane == 0) {
        A.pl->flag[t] = flag;
        A.pl->missing[t] = missing;
        A.pl->mass[t] = mass;
        if (A.flags_out) A.flags_out[t] = (uint8_t)flag;
    }
}

// ---------------- K2: gate/up + SwiGLU ----------------
struct GuArgs {
    int nt, D, F;
    // routing inside the kernel: 1 the one token (template INL kernels),
    // 2 the batch (dec_gateup3_kernel), 0 none (the routing kernel ran)
    int inline_route; const float *logits; int ld; const uint8_t *resident; double thr;
    int *ids; float *w; uint8_t *flags_out; DecPlan *pl;
    const uint8_t *gate, *up, *sh_gate, *sh_up; size_t rb;
    const _Float16 *xp, *xsp;
    _Float16 *midp; float *msum8;    // mid planes [ME][2][F] in the down format's order; sums of 8 rows [ME][F/8]
    int fmt, sh_fmt;                 // down formats of the routed and shared experts
    // one token, when the next kernel is dec_down1_kernel: the down matrices
    // (288-byte rows), whose rows that kernel's workgroup g reads are read here
    // once this workgroup's own copies have landed (HBM is idle while its
    // products run), so that kernel finds them in the Infinity Cache; or null
    const uint8_t *dn_pre, *sh_dn_pre;
};

constexpr int GU_ROWS = 8;           // F rows of gate and of up per wave
constexpr int GU_WROWS = 4 * GU_ROWS; // F rows per workgroup (4 waves)

// ---- pieces shared by the gate/up kernels ----

// The grid size, read at kernel entry: the compiler otherwise loads this
// hidden kernel argument where it is first used, and its round trip then sits
// after the routing or the expert list (scalar loads return out of order, so
// the next shared-memory wait there waits for it too).
QG_DEV uint32_t entry_grid() {
    const uint32_t G = gridDim.x;
    asm volatile("" ::"s"(G));
    return G;
}
// Every gate/up argument in the entry batch of scalar loads, for the same
// reason: a field first read after the routing (the logits pointer, the plan
// fields) would cost a round trip there.
QG_DEV void entry_args(const GuArgs &A) {
    asm volatile("" ::"s"(A.nt), "s"(A.D), "s"(A.F), "s"(A.inline_route), "s"(A.logits), "s"(A.ld), "s"(A.resident),
                 "s"(A.ids), "s"(A.w), "s"(A.flags_out), "s"(A.pl));
    asm volatile("" ::"s"(A.gate), "s"(A.up), "s"(A.sh_gate), "s"(A.sh_up), "s"(A.rb), "s"(A.xp), "s"(A.xsp), "s"(A.midp),
                 "s"(A.msum8), "s"(A.fmt), "s"(A.sh_fmt));
}

// Warm this XCD's L2 with the batch's activation and sum planes while the
// plan is built (workgroups b, b + 8, ... share an XCD; each takes 4 KB); the
// returned word is consumed once the loads are needed to have landed.  Used
// by the D = 2560 kernel; at D = 2048 the warm loads measured slower (they
// compete with the plan's own reads).
QG_DEV uint32_t gu_warm(const GuArgs &A, int tid) {
    uint32_t warm = 0;
    const size_t pb = (size_t)A.nt * 2 * A.D * 2, tb = pb + (size_t)A.nt * 2 * (A.D / 32) * 2;
    const size_t step = (size_t)((gridDim.x + 7) / 8) * 4096;
    for (size_t off = (size_t)(blockIdx.x / 8) * 4096 + (size_t)tid * 16; off < tb; off += step) {
        const uint4 v = off < pb ? *(const uint4 *)((const uint8_t *)A.xp + off)
                                 : *(const uint4 *)((const uint8_t *)A.xsp + (off - pb));
        warm ^= v.x;
    }
    return warm;
}

// One token (wave 0 of every workgroup): its routing; entry k = k-th eligible
// rank (s_rank, s_rid, *s_nent).  Workgroup 0 publishes ids, weights, flags
// and the plan.
QG_DEV void gu_route_inline(const GuArgs &A, int lane, float *s_rv, int *s_ri, int *s_rank, int *s_rid, int *s_nent) {
    int id, missing;
    float wv;
    double mass;
    qg_route_fast(A.logits, lane, id, wv, s_rv, s_ri, blockIdx.x == 0 || A.resident != nullptr);
    const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
    const bool el = lane < QG_TOP && flag < 2 && id >= 0 && id < QG_EXPERTS;
    const unsigned long long b = __ballot(el);
    const int k = __popcll(b & ((1ULL << lane) - 1ULL));
    if (el) { s_rank[k] = lane; s_rid[k] = id; }
    if (lane == 0) *s_nent = __popcll(b);
    if (blockIdx.x == 0) {
        if (lane < QG_TOP) { A.ids[lane] = id; A.w[lane] = wv; }
        if (el) { A.pl->tile[k].e = id; A.pl->tile[k].n = 1; A.pl->tile[k].q[0] = lane; }
        if (lane == 0) {
            A.pl->flag[0] = flag;
            A.pl->missing[0] = missing;
            A.pl->mass[0] = mass;
            A.pl->n_tiles = __popcll(b);
            if (A.flags_out) A.flags_out[0] = (uint8_t)flag;
        }
    }
}

// B > 1: the plan from the routing kernel's ids and flags, built the same way
// in every workgroup (256 threads; scratch in shared memory): an expert's
// eligible selections form tiles of up to 8 in token order, experts in order
// of their first eligible selection.  A selection is eligible when its id is
// an expert and its token is computed here (flag 0 or 1; pruned selections
// carry -id-2).  p_mask[512]: tokens choosing each expert; p_ids[MS]:
// eligible id or -1; p_tile[MAX_TILES]: expert | tile-in-expert << 16.
struct GuPlan { uint32_t *mask; int *ids, *tile, *ntiles; };
QG_DEV GuPlan gu_plan_at(void *base) {
    GuPlan P;
    P.mask = (uint32_t *)base;
    P.ids = (int *)(P.mask + QG_EXPERTS);
    P.tile = P.ids + MS;
    P.ntiles = P.tile + MAX_TILES;
    return P;
}
constexpr int GU_PLAN_BYTES = (QG_EXPERTS + MS + MAX_TILES + 1) * 4;
QG_DEV void gu_build_plan(const GuArgs &A, int tid, const GuPlan &P) {
    const int wave = tid >> 6, lane = tid & 63, ns = A.nt * QG_TOP;
    for (int i = tid; i < QG_EXPERTS; i += 256) P.mask[i] = 0u;
    int eq = -1;
    if (tid < ns) {
        const int id = A.ids[tid], fl = A.pl->flag[tid / QG_TOP];
        eq = id >= 0 && id < QG_EXPERTS && fl < 2 ? id : -1;
        P.ids[tid] = eq;
    }
    __syncthreads();
    if (eq >= 0) atomicOr(&P.mask[eq], 1u << (tid / QG_TOP));
    __syncthreads();
    if (wave == 0) {
        const unsigned long long below = (1ULL << lane) - 1ULL;
        int tiles = 0;
        for (int c0 = 0; c0 < ns; c0 += 64) {
            const int q = c0 + lane, e = q < ns ? P.ids[q] : -1;
            const uint32_t m = e >= 0 ? P.mask[e] : 0u;
            // the expert's first eligible selection: its lowest token
            const bool own = e >= 0 && (m & ((1u << (q / QG_TOP)) - 1u)) == 0u;
            const int nt8 = own ? (__popc(m) + TILE_TOK - 1) / TILE_TOK : 0;  // 0..3
            const unsigned long long b0 = __ballot(nt8 & 1), b1 = __ballot(nt8 & 2);
            const int base = tiles + __popcll(b0 & below) + 2 * __popcll(b1 & below);
            for (int x = 0; x < nt8; x++) P.tile[base + x] = e | (x << 16);
            tiles += __popcll(b0) + 2 * __popcll(b1);
        }
        if (lane == 0) *P.ntiles = tiles;
    }
    __syncthreads();
}

// Tile T of the layer (the shared expert's tiles first): expert e (-1:
// shared), token count n (-1: past the plan) and, for list slot < n, its
// selection q (shared expert: MS + token).  With `publish`, the routed tile is
// written to the plan for the down kernel.
template <bool INL>
QG_DEV void gu_tile(const GuArgs &A, int T, int sh_tiles, int slot, const int *s_rank, const int *s_rid, int nent,
                    const GuPlan &P, bool publish, int &e, int &n, int &q) {
    e = -1;
    n = -1;
    q = -1;
    if (T < sh_tiles) {
        n = min(TILE_TOK, A.nt - TILE_TOK * T);
        if (slot < n) q = MS + TILE_TOK * T + slot;
    } else if (INL) {
        const int k = T - sh_tiles;
        if (k < nent) {
            e = s_rid[k];
            n = 1;
            if (slot == 0) q = s_rank[k];
        }
    } else if (T - sh_tiles < *P.ntiles) {
        const int k = T - sh_tiles, te = P.tile[k], jt = te >> 16;
        e = te & 0xffff;
        const uint32_t m = P.mask[e];
        n = min(TILE_TOK, __popc(m) - TILE_TOK * jt);
        if (slot < n) {
            // the (8 jt + slot)-th token choosing e, and the rank it gave e
            uint32_t mm = m;
            for (int x = TILE_TOK * jt + slot; x > 0; x--) mm &= mm - 1u;
            const int t = __builtin_ctz(mm);
            int r = 0;
#pragma unroll
            for (int rr = 0; rr < QG_TOP; rr++) r = P.ids[t * QG_TOP + rr] == e ? rr : r;
            q = t * QG_TOP + r;
        }
        if (publish) {
            if (slot < n) A.pl->tile[k].q[slot] = q;
            if (slot == 0) { A.pl->tile[k].e = e; A.pl->tile[k].n = n; }
        }
    }
}

// ---- K2 at D = 2048: pipelined K split ----
constexpr int GU2_ROWS = 16;                  // F rows per item (16 gate + 16 up weight rows)
constexpr int GU2_SL = 32 * 18;              // 16-byte slots per item and wave: 32 rows x 2 superblocks of 144 bytes
constexpr int GU2_NT = 4;                     // tiles a workgroup's item range may touch
constexpr size_t GU2_LDS = (size_t)4 * 2 * GU2_SL * 16;  // 4 waves x 2 buffers
constexpr int GU2_CPH = (GU2_SL / 2 + 63) / 64;  // copies per wave and superblock half of an item
constexpr int DN1_PRE_ROWS = 8;                   // output rows per dec_down1_kernel workgroup (DN1_ROWS)

// One token (INL) at D = 2048.
// Persistent: the layer's items (tile, 16 F rows) in tile order, split into
// contiguous ranges, one per workgroup, so a workgroup keeps a tile's
// activation fragments in registers across its row blocks.  Wave w takes
// superblocks 2w, 2w + 1 (the K split) of the item's 32 weight rows (column
// block 0: gate rows, 1: up rows): their bytes come by direct global->shared
// copies into the wave's own double buffer (each row's 288 bytes one
// contiguous run, rotated by row group to spread the fragment reads), the next
// item's copies in flight while this item's products run; partial sums meet
// in shared memory and wave 0 applies SwiGLU.
template <bool INL>
__global__ __launch_bounds__(256, 2) void dec_gateup2_kernel(GuArgs A) {
    extern __shared__ uint4 s_dyn[];
    __shared__ int s_te[GU2_NT][2];          // per tile of the range: expert, token count
    __shared__ int s_tl[GU2_NT][TILE_TOK];   // and its selections
    __shared__ __align__(16) float s_rv[QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_ri[QG_ROUTE_SCRATCH];
    __shared__ int s_rank[QG_TOP], s_rid[QG_TOP];
    __shared__ int s_nent;
    const uint32_t G = entry_grid();
    entry_args(A);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int D = A.D, D32 = D / 32, RBK = A.F / GU2_ROWS;
    const GuPlan P = gu_plan_at(s_dyn);
    if (INL) {
        if (wave == 0) gu_route_inline(A, lane, s_rv, s_ri, s_rank, s_rid, &s_nent);
        __syncthreads();
    } else {
        gu_build_plan(A, tid, P);
    }
    const int sh_tiles = A.sh_gate ? (A.nt + TILE_TOK - 1) / TILE_TOK : 0;
    const int ntl = sh_tiles + (INL ? s_nent : *P.ntiles), N = ntl * RBK;
    // N <= (3 + 170) * F / 16 items and at most 1024 workgroups: 32-bit products suffice
    const int i0 = (int)((uint32_t)N * blockIdx.x / G), i1 = (int)((uint32_t)N * (blockIdx.x + 1) / G);
    const int T0 = i0 / RBK;
    if (wave == 0) {
        // the range's tiles (lane l: tile T0 + l / 8, list slot l % 8); the
        // workgroup holding a tile's first row block publishes it
        const int ti = lane >> 3, slot = lane & 7, T = T0 + ti;
        if (ti < GU2_NT && i1 > i0 && T * RBK < i1) {
            int e, n, q;
            const bool pub = T * RBK >= i0;
            gu_tile<INL>(A, T, sh_tiles, slot, s_rank, s_rid, INL ? s_nent : 0, P, pub, e, n, q);
            if (slot < n) s_tl[ti][slot] = q;
            if (slot == 0) { s_te[ti][0] = e; s_te[ti][1] = n; }
        }
        if (!INL && blockIdx.x == 0 && lane == 0) A.pl->n_tiles = *P.ntiles;
    }
    __syncthreads();
    if (i1 <= i0) return;  // block-uniform
    uint4 *wl = s_dyn + (size_t)wave * 2 * GU2_SL;  // this wave's two buffers
    // superblock sb of an item's 32 weight rows -> the wave's copies into
    // buffer b: 9 pieces per row (header, 8 nibble chunks), superblock 1's
    // rows after superblock 0's, each row rotated by row / 8 pieces so the 16
    // rows of a fragment read spread over the banks; GU2_CPH copies per half
    auto copy_half = [&](int item, int b, int sb) {
        const int ti = item / RBK - T0, rb = item % RBK, e = s_te[ti][0];
        const uint8_t *gm = e < 0 ? A.sh_gate : A.gate + (size_t)e * A.F * A.rb;
        const uint8_t *um = e < 0 ? A.sh_up : A.up + (size_t)e * A.F * A.rb;
#pragma unroll
        for (int i = 0; i < GU2_CPH; i++) {
            const int s = i * 64 + lane, row = s / 9, pc = s - 9 * row, rot = row >> 3;
            const int c = pc - rot + (pc < rot ? 9 : 0);
            if (s < GU2_SL / 2)
                dma16_ordered((row < 16 ? gm : um) + (size_t)(rb * GU2_ROWS + (row & 15)) * A.rb + (size_t)wave * 288 +
                                  (size_t)sb * 144 + 16 * c,
                              wl + (size_t)b * GU2_SL + (size_t)sb * (GU2_SL / 2) + i * 64);
        }
    };
    // the tile's activation fragments for superblock sb of this wave: plane
    // row r = (token r/2, plane r%2).  Buffer loads: rows past the tile's
    // tokens take an offset past the planes and read zeros without a memory
    // access, and every load is issued by every lane (a load under a branch
    // would keep the compiler from counting it in its waits below)
    const __amdgpu_buffer_rsrc_t xpr = __builtin_amdgcn_make_buffer_rsrc((void *)A.xp, (short)0, A.nt * 2 * D * 2, QG_BUF_DW3);
    const __amdgpu_buffer_rsrc_t xsr = __builtin_amdgcn_make_buffer_rsrc((void *)A.xsp, (short)0, A.nt * 2 * D32 * 2, QG_BUF_DW3);
    qg_half8 af[2][8], sf[2];
    auto load_af = [&](int ti, int sb) {
        const int n = s_te[ti][1], e = s_te[ti][0];
        const bool real = (j >> 1) < n;
        const int r = 2 * min(j >> 1, n - 1) + (j & 1), sl0 = s_tl[ti][r >> 1];
        const int tok = e < 0 ? sl0 - MS : sl0 / QG_TOP;
        const int xo = ((tok * 2 + (r & 1)) * D + wave * 512 + sb * 256 + kq * 8) * 2;
        const int so = ((tok * 2 + (r & 1)) * D32 + wave * 16 + sb * 8) * 2;
#pragma unroll
        for (int m = 0; m < 8; m++) af[sb][m] = buf_frag(xpr, real ? xo + m * 64 : QG_BUF_OOB);
        sf[sb] = buf_frag(xsr, (kq || !real) ? QG_BUF_OOB : so);
    };
    // the first item: superblock 0's fragments and copies go out before
    // superblock 1's, so its products can start while superblock 1 streams
    // (the compiler's own waits for the fragments then cover no copies)
    load_af(0, 0);
    copy_half(i0, 0, 0);
    load_af(0, 1);
    copy_half(i0, 0, 1);
    // down1's rows prefetched by workgroups g < D / DN1_PRE_ROWS with a single item
    const bool pre = INL && A.dn_pre != nullptr && i1 - i0 == 1 && (int)blockIdx.x < D / DN1_PRE_ROWS;
    // item k of the range; the first one is a separate instance, so the
    // compiler's waits there see only the loads above (a shared loop would
    // merge in the later items' fragment reloads)
    int cur = 0;
    auto item_body = [&](int k, auto first) {
        constexpr bool FIRST = decltype(first)::value;
        const int item = i0 + k, ti = item / RBK - T0, rb = item % RBK, b = k & 1;
        const int e = s_te[ti][0], n = s_te[ti][1];
        if (!FIRST && ti != cur) {
            load_af(ti, 0);
            load_af(ti, 1);
            cur = ti;
        }
        const uint4 *wb = wl + (size_t)b * GU2_SL;
        qg_f4 y[2] = {qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, qg_f4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            if (sb == 0) {
                if (FIRST) wait_vmem_but<GU2_CPH>();  // all but superblock 1's copies
                else wait_vmem();  // this item's copies (issued during the previous item) and fragments
            } else {
                wait_vmem();  // this item's copies and fragments
                if (i0 + k + 1 < i1) {  // the next item streams during this superblock's products and the epilogue
                    copy_half(item + 1, b ^ 1, 0);
                    copy_half(item + 1, b ^ 1, 1);
                } else if (FIRST && INL && pre) {
                    // down1's rows for workgroup g = blockIdx.x of every entry
                    // (the plan's eligible ranks, then the shared expert), into
                    // the unused second buffer, whose contents nothing reads
                    const int E = s_nent + (A.sh_dn_pre ? 1 : 0);
                    for (int x = wave; x < E; x += 4) {
                        const uint8_t *W = (x < s_nent ? A.dn_pre + (size_t)s_rid[x] * D * 288 : A.sh_dn_pre) +
                                           (size_t)blockIdx.x * DN1_PRE_ROWS * 288;
#pragma unroll
                        for (int c = 0; c < (DN1_PRE_ROWS * 288 / 16 + 63) / 64; c++) {
                            const int ch = c * 64 + lane;
                            if (ch < DN1_PRE_ROWS * 288 / 16) dma16_ordered(W + 16 * ch, wl + (size_t)(b ^ 1) * GU2_SL + c * 64);
                        }
                    }
                }
            }
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                const int row = cb * 16 + j, rot = row >> 3;
                // piece c of the row's superblock (0: header, 1..8: nibbles)
                auto piece = [&](int c) { const int x = c + rot; return wb[(size_t)sb * (GU2_SL / 2) + 9 * row + (x >= 9 ? x - 9 : x)]; };
                const Q4kHeader h = q4k_header(piece(0));
                const uint4 ch0 = piece(1 + kq), ch1 = piece(5 + kq);
                qg_half2 scA, ofA, scB, ofB;  // scales of groups gA, gA + 1 and gB, gB + 1
                gq_scales(h.S[0], kq, scA, ofA);
                gq_scales(h.S[1], kq, scB, ofB);
                qg_f4 p0 = qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, p1 = p0, mm = p0;
#pragma unroll
                for (int f = 0; f < 4; f++) {
                    p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[sb][f], gq_frag(ch0, f, scA[f >> 1], ofA[f >> 1]), p0, 0, 0, 0);
                    p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[sb][4 + f], gq_frag(ch1, f, scB[f >> 1], ofB[f >> 1]), p1, 0, 0, 0);
                }
                mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(sf[sb], q4k_min_frag(h), mm, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) y[cb][i] = __builtin_fmaf(h.d, p0[i] + p1[i], __builtin_fmaf(-h.dmin, mm[i], y[cb][i]));
            }
        }
        // partial sums into this wave's buffer b (its reads are done)
        float4 *pw = (float4 *)(wl + (size_t)b * GU2_SL);
        pw[lane] = make_float4(y[0][0], y[0][1], y[0][2], y[0][3]);
        pw[64 + lane] = make_float4(y[1][0], y[1][1], y[1][2], y[1][3]);
        __syncthreads();
        if (wave == 0) {
            // the 4 partials in wave order; F row rb 16 + j
            float g[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float4 *pr = (const float4 *)(s_dyn + (size_t)w * 2 * GU2_SL + (size_t)b * GU2_SL);
                const float4 ga = pr[lane], ua = pr[64 + lane];
                g[0] += ga.x; g[1] += ga.y; g[2] += ga.z; g[3] += ga.w;
                u[0] += ua.x; u[1] += ua.y; u[2] += ua.z; u[3] += ua.w;
            }
            const int fmt = e < 0 ? A.sh_fmt : A.fmt, frow = rb * GU2_ROWS + j, pos = plane_pos(fmt, frow);
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const float m = qg_swiglu_fast(g[2 * t2] + g[2 * t2 + 1], u[2 * t2] + u[2 * t2 + 1]);
                // the sum over the 8 rows of this lane's group: only a Q4_K down reads it
                const bool q4k = fmt == QT_Q4_K;  // workgroup-uniform
                float s8 = m;
                if (q4k) {
                    s8 += __shfl_xor(s8, 1);
                    s8 += __shfl_xor(s8, 2);
                    s8 += __shfl_xor(s8, 4);
                }
                const int idx = 2 * kq + t2;
                if (idx < n) {
                    const int sl = s_tl[ti][idx];
                    _Float16 *mp = A.midp + (size_t)sl * 2 * A.F;
                    const _Float16 hv = (_Float16)m;
                    mp[pos] = hv;
                    mp[A.F + pos] = (_Float16)(m - (float)hv);
                    if (q4k && (j & 7) == 0) A.msum8[(size_t)sl * (A.F / GU_ROWS) + frow / GU_ROWS] = s8;
                }
            }
        }
        __syncthreads();  // buffer b is free for the item after next
    };
    item_body(0, std::true_type{});
    for (int k = 1; i0 + k < i1; k++) item_body(k, std::false_type{});
    if (pre) wait_vmem();  // no copy may land in shared memory after the workgroup ends
}

// ---- K2 at D = 2048, one expert per workgroup ----
// Every workgroup (one per CU) owns a contiguous run of one expert's 16-row F
// blocks and computes each block for all of the expert's token tiles (up to
// three tiles of 8 tokens) against a single copy of its weights, so an
// expert's weight rows are read from HBM once.  The experts' blocks are dealt
// to the workgroups in proportion to their cost (blocks x (GU3_COST + tiles):
// a block's copies, then its products and epilogue once per tile): workgroup
// g takes the expert whose cost range holds the midpoint of g's equal share.
// Wave w (of 8, two per SIMD) multiplies superblock w (the K split) of the
// block's 16 gate and 16 up rows; their bytes come by direct global->shared
// copies into the wave's own ring of GU3_RING buffers, issued GU3_RING - 1
// blocks ahead.  Each dequantised weight fragment feeds the MFMAs of every
// tile.  The tiles' activation fragments are loaded once, before the first
// copies.  Partial sums (hi and lo planes already added) meet in shared
// memory; 2M waves apply SwiGLU, one per tile and token of each lane pair.
constexpr int GU3_W = 8;                                          // waves per workgroup
constexpr int GU3_RING = 3;
constexpr int GU3_SLOT = 32 * 9;                                  // 16-byte pieces of one block and wave
constexpr int GU3_CPB = (GU3_SLOT + 63) / 64;                     // copies per block and wave
constexpr int GU3_MAXT = 3;                                       // tiles of 8 tokens per expert (17 tokens)
constexpr size_t GU3_RING_BYTES = (size_t)GU3_W * GU3_RING * GU3_SLOT * 16;
constexpr size_t GU3_RED_BYTES = (size_t)GU3_W * 2 * GU3_MAXT * 64 * 8;  // wave x gate/up x tile x lane: float2
constexpr size_t GU3_LDS = GU3_RING_BYTES + 2 * GU3_RED_BYTES;          // rings, two partial-sum buffers
constexpr int GU3_MAXX = MAX_TILES + 1;                           // experts in the plan, the shared one included
static_assert((size_t)(5 * GU3_MAXX + 1 + MS) * 4 <= GU3_RED_BYTES, "the expert list and ids fit a partial-sum buffer");
constexpr int GU3_COST = 1;                                       // a block's copy cost in units of one tile's compute (measured best of 0..8)

// The block's products for the M tiles: y[cb][m] = the wave's partial sums
// over its superblock for the 16 gate (cb 0) or up (cb 1) rows, column j,
// as (token 2kq, token 2kq + 1) with the hi and lo plane rows added.
template <int M>
QG_DEV void gu3_products(const uint4 *wb, const qg_half8 (&af)[GU3_MAXT][8], const qg_half8 (&sf)[GU3_MAXT], int j,
                         int kq, float2 (&y)[2][GU3_MAXT]) {
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
        const int row = cb * 16 + j, rot = row >> 3;
        // piece c of the row (0: header, 1..8: nibbles), rotated by row / 8
        auto piece = [&](int c) { const int x = c + rot; return wb[9 * row + (x >= 9 ? x - 9 : x)]; };
        const Q4kHeader h = q4k_header(piece(0));
        const uint4 ch0 = piece(1 + kq), ch1 = piece(5 + kq);
        qg_half2 scA, ofA, scB, ofB;  // scales of groups gA, gA + 1 and gB, gB + 1
        gq_scales(h.S[0], kq, scA, ofA);
        gq_scales(h.S[1], kq, scB, ofB);
        qg_f4 p0[M], p1[M], mm[M];
#pragma unroll
        for (int m = 0; m < M; m++) p0[m] = p1[m] = mm[m] = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int f = 0; f < 4; f++) {
            const qg_half8 b0 = gq_frag(ch0, f, scA[f >> 1], ofA[f >> 1]), b1 = gq_frag(ch1, f, scB[f >> 1], ofB[f >> 1]);
#pragma unroll
            for (int m = 0; m < M; m++) {
                p0[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[m][f], b0, p0[m], 0, 0, 0);
                p1[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[m][4 + f], b1, p1[m], 0, 0, 0);
            }
        }
        const qg_half8 bm = q4k_min_frag(h);
#pragma unroll
        for (int m = 0; m < M; m++) {
            mm[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sf[m], bm, mm[m], 0, 0, 0);
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = __builtin_fmaf(h.d, p0[m][i] + p1[m][i], -h.dmin * mm[m][i]);
            y[cb][m] = make_float2(v[0] + v[1], v[2] + v[3]);
        }
    }
}

// This wave's copies of F block rb of an expert (gate rows gm, up rows um)
// into its ring slot: each row's 144 bytes of the wave's superblock as one
// run, rotated by row / 8 pieces so that the 16 rows of a fragment read
// spread over the banks.
QG_DEV void gu3_copy(const GuArgs &A, const uint8_t *gm, const uint8_t *um, int rb, uint4 *slot, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < GU3_CPB; i++) {
        const int sl = i * 64 + lane, row = sl / 9, pc = sl - 9 * row, rot = row >> 3;
        const int c = pc - rot + (pc < rot ? 9 : 0);
        if (sl < GU3_SLOT)
            dma16_ordered((row < 16 ? gm : um) + (size_t)(rb * GU2_ROWS + (row & 15)) * A.rb + (size_t)wave * 144 + 16 * c,
                          slot + i * 64);
    }
}

// The selection of each of the expert's tile slots (t*10 + the rank token t
// gave expert e, from the routing ids; shared expert: MS + t), by one wave
// (lane l: tile l / 8, slot l % 8); with k0 >= 0 the tiles are also published
// as routed tiles k0 .. k0 + M - 1 of the plan for the down kernel.
QG_DEV void gu3_selections(const GuArgs &A, const int *ids, int e, int M, const int *tn, const int (*tt)[TILE_TOK],
                           int (*tq)[TILE_TOK], int k0, int lane) {
    const int m = lane >> 3, slot = lane & 7;
    if (m >= M) return;
    const int n = tn[m];
    int q = -1;
    if (slot < n) {
        const int t = tt[m][slot];
        if (e < 0) {
            q = MS + t;
        } else {
            const int2 *row = (const int2 *)(ids + t * QG_TOP);  // shared memory, 8-byte aligned
            int r = 0;
#pragma unroll
            for (int i = 0; i < QG_TOP / 2; i++) {
                const int2 v = row[i];
                r = v.x == e ? 2 * i : v.y == e ? 2 * i + 1 : r;
            }
            q = t * QG_TOP + r;
        }
        tq[m][slot] = q;
    }
    if (k0 >= 0) {
        if (slot < n) A.pl->tile[k0 + m].q[slot] = q;
        if (slot == 0) { A.pl->tile[k0 + m].e = e; A.pl->tile[k0 + m].n = n; }
    }
}

// The workgroup's blocks rb0 .. rb1 - 1 of one expert with M tiles, whose
// first GU3_RING - 1 blocks' copies are in flight; tn / tt: the tiles' token
// counts and tokens, tq: their selections (written by wave 0 here, read after
// the first block's barrier), all in shared memory.
template <int M>
QG_DEV void gu3_run(const GuArgs &A, const int *ids, int e, int rb0, int rb1, const int *tn, const int (*tt)[TILE_TOK],
                    int (*tq)[TILE_TOK], int k0, uint4 *s_dyn, int tid) {
    const int wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int D = A.D, D32 = D / 32, nb = rb1 - rb0;
    const uint8_t *gm = e < 0 ? A.sh_gate : A.gate + (size_t)e * A.F * A.rb;
    const uint8_t *um = e < 0 ? A.sh_up : A.up + (size_t)e * A.F * A.rb;
    uint4 *ring = s_dyn + (size_t)wave * GU3_RING * GU3_SLOT;
    float2 *red0 = (float2 *)(s_dyn + GU3_RING_BYTES / 16);
    // the tiles' activation fragments for this wave's superblock: plane row
    // r = (token r/2, plane r%2); rows past a tile's tokens are zeros, not
    // loaded (their products are never kept), so a one-token tile reads 2 of
    // the 16 rows
    qg_half8 af[GU3_MAXT][8], sf[GU3_MAXT];
#pragma unroll
    for (int m = 0; m < M; m++) {
        const bool real = (j >> 1) < tn[m];
        const int r = 2 * min(j >> 1, tn[m] - 1) + (j & 1), tok = tt[m][r >> 1];
        const _Float16 *xr = A.xp + ((size_t)tok * 2 + (r & 1)) * D + (size_t)wave * 256 + kq * 8;
        const _Float16 *xs = A.xsp + ((size_t)tok * 2 + (r & 1)) * D32 + (size_t)wave * 8;
#pragma unroll
        for (int f = 0; f < 8; f++) af[m][f] = real ? ld_frag(xr + f * 32) : qg_half8{};
        sf[m] = (kq || !real) ? qg_half8{} : ld_frag(xs);
    }
    if (wave == 0) gu3_selections(A, ids, e, M, tn, tt, tq, k0, lane);
    auto copy_block = [&](int rb, int s) { gu3_copy(A, gm, um, rb, ring + (size_t)s * GU3_SLOT, wave, lane); };
    const int fmt = e < 0 ? A.sh_fmt : A.fmt;
    for (int it = 0; it < nb; it++) {
        // the block GU3_RING - 1 ahead into the slot the previous block used
        if (it + GU3_RING - 1 < nb) copy_block(rb0 + it + GU3_RING - 1, (it + GU3_RING - 1) % GU3_RING);
        const int ahead = min(GU3_RING - 1, nb - 1 - it);  // later blocks in flight
        if (ahead >= 2) wait_vmem_but<2 * GU3_CPB>();
        else if (ahead == 1) wait_vmem_but<GU3_CPB>();
        else wait_vmem();
        float2 y[2][GU3_MAXT];
        gu3_products<M>(ring + (size_t)(it % GU3_RING) * GU3_SLOT, af, sf, j, kq, y);
        // partial sums alternate between two buffers: block it + 2 rewrites
        // this one only after every wave has passed block it + 1's barrier,
        // so this block's epilogue needs no barrier of its own
        float2 *red = red0 + (size_t)(it & 1) * (GU3_RED_BYTES / 8);
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int m = 0; m < M; m++) red[((wave * 2 + cb) * GU3_MAXT + m) * 64 + lane] = y[cb][m];
        __syncthreads();
        if (wave < 2 * M) {
            // tile m = wave / 2, token 2 kq + t2 of lane's pair, F row j of the block
            const int m = wave >> 1, t2 = wave & 1, n = tn[m];
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int w = 0; w < GU3_W; w++) {
                const float2 ga = red[((w * 2 + 0) * GU3_MAXT + m) * 64 + lane], ua = red[((w * 2 + 1) * GU3_MAXT + m) * 64 + lane];
                g += t2 ? ga.y : ga.x;
                u += t2 ? ua.y : ua.x;
            }
            const int rb = rb0 + it, frow = rb * GU2_ROWS + j, pos = plane_pos(fmt, frow);
            const float mv = qg_swiglu_fast(g, u);
            // the sum over the 8 rows of this lane's group, which only a Q4_K
            // down reads (its min term); an IQ4_NL down needs none
            const bool q4k = fmt == QT_Q4_K;  // workgroup-uniform
            float s8 = mv;
            if (q4k) {
                s8 += __shfl_xor(s8, 1);
                s8 += __shfl_xor(s8, 2);
                s8 += __shfl_xor(s8, 4);
            }
            const int idx = 2 * kq + t2;
            if (idx < n) {
                const int sl = tq[m][idx];
                _Float16 *mp = A.midp + (size_t)sl * 2 * A.F;
                const _Float16 hv = (_Float16)mv;
                mp[pos] = hv;
                mp[A.F + pos] = (_Float16)(mv - (float)hv);
                if (q4k && (j & 7) == 0) A.msum8[(size_t)sl * (A.F / GU_ROWS) + frow / GU_ROWS] = s8;
            }
        }
    }
}

// B = 2..17 at D = 2048.  The expert list: the shared expert, then the routed
// experts in ascending id, each with the tokens whose eligible selections
// chose it (the routing kernel's per-expert masks), cut into tiles of up to 8
// tokens in token order; the routed tiles are numbered in list order and
// published by each expert's first workgroup for the down kernel.
__global__ __launch_bounds__(512, 1) void dec_gateup3_kernel(GuArgs A) {
    extern __shared__ uint4 s_dyn[];
    // the expert list, in the second partial-sum buffer (first written after
    // the barrier that ends the list's use)
    int *s_xe = (int *)(s_dyn + (GU3_RING_BYTES + GU3_RED_BYTES) / 16), *s_xk = s_xe + GU3_MAXX, *s_xm = s_xk + GU3_MAXX;
    int *s_cum = s_xm + GU3_MAXX;
    uint32_t *s_xt = (uint32_t *)(s_cum + GU3_MAXX + 1);
    int *s_ids = (int *)(s_xt + GU3_MAXX);  // the routing ids, so the selections need no global reads behind the copies
    __shared__ int s_nx;
    __shared__ int s_tq[GU3_MAXT][TILE_TOK], s_tt[GU3_MAXT][TILE_TOK], s_tn[GU3_MAXT];
    const uint32_t G = entry_grid();
    entry_args(A);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int RBK = A.F / GU2_ROWS;
    const int sh = A.sh_gate ? 1 : 0, sh_tiles = sh ? (A.nt + TILE_TOK - 1) / TILE_TOK : 0;
    uint32_t em[QG_EXPERTS / 64];
    if (A.inline_route == 2) {
        // the workgroup routes the batch itself (wave w: token w; the host
        // takes this path for up to 8 tokens), every workgroup alike;
        // workgroup 0 publishes ids, weights and flags.  The per-expert token
        // masks and the routing scratch sit in the rings, which nothing
        // writes before the list's barrier below.
        static_assert(64 * GU3_W == QG_EXPERTS, "one mask per thread");
        static_assert((QG_EXPERTS + 2 * QG_ROUTE_SCRATCH * GU3_W) * 4 <= GU3_RING_BYTES, "masks and scratch fit the rings");
        uint32_t *s_em = (uint32_t *)s_dyn;
        float *s_rv = (float *)s_dyn + QG_EXPERTS + 2 * QG_ROUTE_SCRATCH * wave;
        int *s_ri = (int *)(s_rv + QG_ROUTE_SCRATCH);
        s_em[tid] = 0u;
        __syncthreads();
        const bool pub = blockIdx.x == 0;
        for (int t = wave; t < A.nt; t += GU3_W) {
            int id, missing;
            float wv = 0.0f;
            double mass;
            // only the ids unless this workgroup publishes or the flags need the mass
            qg_route_fast(A.logits + (size_t)t * A.ld, lane, id, wv, s_rv, s_ri, pub || A.resident != nullptr);
            const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
            if (lane < QG_TOP) {
                s_ids[t * QG_TOP + lane] = id;
                if (flag < 2 && id >= 0 && id < QG_EXPERTS) atomicOr(&s_em[id], 1u << t);
                if (pub) {
                    A.ids[t * QG_TOP + lane] = id;
                    A.w[t * QG_TOP + lane] = wv;
                }
            }
            if (pub && lane == 0) {
                A.pl->flag[t] = flag;
                A.pl->missing[t] = missing;
                A.pl->mass[t] = mass;
                if (A.flags_out) A.flags_out[t] = (uint8_t)flag;
            }
        }
        __syncthreads();
        if (wave == 0)
#pragma unroll
            for (int i = 0; i < QG_EXPERTS / 64; i++) em[i] = s_em[64 * i + lane];
    } else {
        // the masks, then the routing ids (read before any copy is in
        // flight), in one memory round trip
        if (wave == 0)
#pragma unroll
            for (int i = 0; i < QG_EXPERTS / 64; i++) em[i] = A.pl->emask[64 * i + lane];
        if (tid < A.nt * QG_TOP) s_ids[tid] = A.ids[tid];
    }
    if (wave == 0) {
        if (lane == 0 && sh) { s_xe[0] = -1; s_xk[0] = -1; s_xm[0] = sh_tiles; s_xt[0] = 0u; }
        const unsigned long long below = (1ULL << lane) - 1ULL;
        int nx = sh, ntl = 0;
#pragma unroll
        for (int i = 0; i < QG_EXPERTS / 64; i++) {
            // tiles per expert (1..3 for up to 17 tokens) as bit-sliced ballots
            const int mx = em[i] ? (__popc(em[i]) + TILE_TOK - 1) / TILE_TOK : 0;
            const unsigned long long b = __ballot(em[i] != 0u), b0 = __ballot(mx & 1), b1 = __ballot(mx & 2);
            const int x = nx + __popcll(b & below);
            if (em[i] && x < GU3_MAXX) {
                s_xe[x] = 64 * i + lane;
                s_xm[x] = mx;
                s_xk[x] = ntl + __popcll(b0 & below) + 2 * __popcll(b1 & below);
                s_xt[x] = em[i];
            }
            nx += __popcll(b);
            ntl += __popcll(b0) + 2 * __popcll(b1);
        }
        // at most one tile per eligible selection when the masks are this
        // layer's; anything larger (masks not cleared) computes nothing
        // rather than overrun the plan
        if (nx > GU3_MAXX || ntl > MAX_TILES) nx = ntl = 0;
        if (blockIdx.x == 0 && lane == 0) A.pl->n_tiles = ntl;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // cost prefix, RBK (GU3_COST + M) per expert: a block's copies (the
        // same for every tile count) plus its products and epilogue per tile;
        // tile counts (1..3) summed by bit-sliced ballots
        int carry = 0;
        for (int c0 = 0; c0 < nx; c0 += 64) {
            const int x = c0 + lane, mx = x < nx ? s_xm[x] : 0;
            const unsigned long long b0 = __ballot(mx & 1), b1 = __ballot(mx & 2), bv = __ballot(x < nx);
            const unsigned long long upto = below | (1ULL << lane);
            if (x < nx)
                s_cum[x + 1] = RBK * (carry + GU3_COST * __popcll(bv & upto) + __popcll(b0 & upto) + 2 * __popcll(b1 & upto));
            carry += GU3_COST * __popcll(bv) + __popcll(b0) + 2 * __popcll(b1);
        }
        if (lane == 0) { s_cum[0] = 0; s_nx = nx; }
    }
    __syncthreads();
    const int nx = s_nx;
    if (nx == 0) return;  // block-uniform: nothing computed on the device
    // this workgroup's expert: the one whose cost range holds the midpoint of
    // its share; its blocks are split evenly over the expert's workgroups
    // (C <= RBK (GU3_COST + 3) 173 and G <= 1024: 32-bit products suffice)
    const uint32_t C = (uint32_t)s_cum[nx], g = blockIdx.x;
    const uint32_t pos = ((2 * g + 1) * C) / (2 * G);
    int x = 0;
    for (int c0 = 0; c0 < nx; c0 += 64) {
        const int xx = c0 + lane;
        x += __popcll(__ballot(xx < nx && (uint32_t)s_cum[xx + 1] <= pos));
    }
    // first workgroup of expert x: the smallest g' with (2g'+1) C >= 2 G cum[x]
    auto first_wg = [&](int xx) -> uint32_t {
        if (xx >= nx) return G;
        const uint32_t t = 2 * G * (uint32_t)s_cum[xx];
        return t <= C ? 0u : (t - C + 2 * C - 1) / (2 * C);
    };
    const uint32_t gA = first_wg(x), gB = first_wg(x + 1), W = gB - gA, kx = g - gA;
    const int rb0 = (int)(RBK * kx / W), rb1 = (int)(RBK * (kx + 1) / W);
    const int e = s_xe[x], M = s_xm[x], k0 = kx == 0 && e >= 0 ? s_xk[x] : -1;
    // the first blocks' weights go out first
    {
        const uint8_t *gm = e < 0 ? A.sh_gate : A.gate + (size_t)e * A.F * A.rb;
        const uint8_t *um = e < 0 ? A.sh_up : A.up + (size_t)e * A.F * A.rb;
        uint4 *ring = s_dyn + (size_t)wave * GU3_RING * GU3_SLOT;
        for (int i = 0; i < GU3_RING - 1 && rb0 + i < rb1; i++) gu3_copy(A, gm, um, rb0 + i, ring + (size_t)i * GU3_SLOT, wave, lane);
    }
    if (wave == 0) {
        // the expert's tiles: n tokens each, in token order
        const int m = lane >> 3, slot = lane & 7;
        if (m < M) {
            int n, t = 0;
            if (e < 0) {
                n = min(TILE_TOK, A.nt - TILE_TOK * m);
                t = TILE_TOK * m + slot;
            } else {
                const uint32_t msk = s_xt[x];
                n = min(TILE_TOK, __popc(msk) - TILE_TOK * m);
                // the (8 m + slot)-th set bit of the mask, found by halving
                int k = TILE_TOK * m + slot;
#pragma unroll
                for (int w = 16; w >= 1; w >>= 1) {
                    const int c = __popc((msk >> t) & ((1u << w) - 1u));
                    if (k >= c) { k -= c; t += w; }
                }
            }
            if (slot < n) s_tt[m][slot] = t;
            if (slot == 0) s_tn[m] = n;
        }
    }
    __syncthreads();
    if (rb1 <= rb0) {  // block-uniform: no blocks here; the first workgroup still publishes
        if (wave == 0 && k0 >= 0) gu3_selections(A, s_ids, e, M, s_tn, s_tt, s_tq, k0, lane);
        return;
    }
    if (M == 1) gu3_run<1>(A, s_ids, e, rb0, rb1, s_tn, s_tt, s_tq, k0, s_dyn, tid);
    else if (M == 2) gu3_run<2>(A, s_ids, e, rb0, rb1, s_tn, s_tt, s_tq, k0, s_dyn, tid);
    else gu3_run<3>(A, s_ids, e, rb0, rb1, s_tn, s_tt, s_tq, k0, s_dyn, tid);
}

// Shared-memory layout of the gate/up kernel (fp16 units): 16 staged plane
// rows (8 tokens x {hi, lo}) of D values each padded by 8, then 16 rows of
// D/32 group sums each padded by 8.  The padding puts the 16 rows of every
// fragment read in distinct banks while each read keeps a constant offset.
// Copies into it are direct global->shared with the lanes of padding slots
// masked off.  Before the first stage the area holds the plan scratch.
struct GuLds { int arow, srow, sums, total; };  // strides and offsets in fp16 units
static __host__ __device__ inline GuLds gu_lds(int D) {
    GuLds L;
    L.arow = D + 8;
    L.srow = D / 32 + 8;
    L.sums = 16 * L.arow;
    L.total = L.sums + 16 * L.srow;
    return L;
}

// Persistent; item = (tile, 32 F rows): the shared expert's tiles first (no
// routing needed), then the plan's routed tiles.  The item's weight rows go to
// registers (8 gate and the same 8 up rows per wave, headers included), while
// the tile's activation planes and sum planes are staged by direct
// global->shared copies; then the products on the matrix cores.  In
// a wave, MFMA columns 0..7 are the gate rows and 8..15 the up rows, so lanes
// l and l^8 hold gate and up of one (row, token) pair.  Tiles of one expert
// and row block are items rblocks apart, on workgroups of one XCD, so their
// repeated weight reads meet in that XCD's L2.
template <int NSB, bool INL>
__global__ __launch_bounds__(256, 2) void dec_gateup_kernel(GuArgs A) {
    extern __shared__ uint4 s_dyn[];
    __shared__ int s_item[GU_NI][2];     // per item: expert (-1: shared), token count (-1: past the plan)
    __shared__ int s_list[GU_NI][TILE_TOK];  // per item: its selections (shared expert: MS + t)
    __shared__ int s_nitems;
    __shared__ __align__(16) float s_rv[QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_ri[QG_ROUTE_SCRATCH];
    __shared__ int s_rank[QG_TOP], s_rid[QG_TOP];
    __shared__ int s_nent;
    __shared__ uint4 s_zero[NSB];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int D = A.D, D32 = D / 32, cps = D / 256, bpr = D / 512;
    if (tid < NSB) s_zero[tid] = make_uint4(0u, 0u, 0u, 0u);  // read after the first barrier
    const int rblocks = A.F / GU_WROWS;
    const GuLds LY = gu_lds(D);
    _Float16 *act = (_Float16 *)s_dyn;
    _Float16 *acts = act + LY.sums;
    const uint32_t warm = gu_warm(A, tid);
    const GuPlan P = gu_plan_at(s_dyn);  // scratch in the stage area, free until the first stage
    if (INL) {
        if (wave == 0) gu_route_inline(A, lane, s_rv, s_ri, s_rank, s_rid, &s_nent);
        __syncthreads();
    } else {
        gu_build_plan(A, tid, P);
    }
    const int sh_tiles = A.sh_gate ? (A.nt + TILE_TOK - 1) / TILE_TOK : 0;
    // the workgroup's items (blockIdx.x + i * gridDim.x, i < GU_NI) -> expert
    // (-1: shared), token count (-1: past the plan) and selection list, by
    // wave 0: lane l takes item l / 8, list slot l % 8.  The workgroup with an
    // item in a tile's first row block publishes the tile for the down kernel.
    if (wave == 0) {
        const int i = lane >> 3, slot = lane & 7, item = blockIdx.x + i * gridDim.x, T = item / rblocks;
        int e, n, q;
        gu_tile<INL>(A, T, sh_tiles, slot, s_rank, s_rid, INL ? s_nent : 0, P, item % rblocks == 0, e, n, q);
        if (slot < n) s_list[i][slot] = q;
        if (!INL && blockIdx.x == 0 && lane == 0) A.pl->n_tiles = *P.ntiles;
        if (slot == 0) { s_item[i][0] = e; s_item[i][1] = n; }
        // items ascend in tile order, so the valid ones are a prefix
        const unsigned long long v = __ballot(slot == 0 && n >= 0);
        if (lane == 0) s_nitems = __popcll(v);
    }
    auto mats = [&](int e, const uint8_t *&gm, const uint8_t *&um) {
        gm = e < 0 ? A.sh_gate : A.gate + (size_t)e * A.F * A.rb;
        um = e < 0 ? A.sh_up : A.up + (size_t)e * A.F * A.rb;
    };
    // this wave's 8 gate and 8 up rows of an item into registers, superblock
    // by superblock: the header (every lane of a row loads the same 16 bytes,
    // one memory request) and the lane's two 16-byte chunks of nibbles
    auto load_weights = [&](int e, int rb0, uint4 *hd, uint4 *w0, uint4 *w1) {
        const uint8_t *gm, *um;
        mats(e, gm, um);
        const uint8_t *wrow = (j < 8 ? gm : um) + (size_t)(rb0 * GU_WROWS + wave * GU_ROWS + (j & 7)) * A.rb;
#pragma unroll
        for (int sb = 0; sb < NSB; sb++) {
            hd[sb] = qg_ld16(wrow + sb * 144);
            w0[sb] = qg_ld16(wrow + sb * 144 + 16 + 16 * kq);
            w1[sb] = qg_ld16(wrow + sb * 144 + 16 + 16 * (kq + 4));
            asm volatile("" ::: "memory");  // issue in superblock order
        }
    };
    // the tile's rows r < 2n (token r/2, plane r%2) with their sum rows,
    // straight into shared memory
    auto stage = [&](int e, int n, const int *list) {
        for (int q = wave; q < 2 * n * bpr; q += 4) {
            const int r = q / bpr, b = q - r * bpr;
            const int sl = list[r >> 1], tok = e < 0 ? sl - MS : sl / QG_TOP;
            dma16_ordered(A.xp + ((size_t)tok * 2 + (r & 1)) * D + (size_t)(b * 64 + lane) * 8, act + (size_t)r * LY.arow + b * 512);
        }
        for (int q = wave; q * 64 < 2 * n * (cps + 1); q += 4) {
            const int slot = q * 64 + lane, r = slot / (cps + 1), c = slot - r * (cps + 1);
            if (r < 2 * n && c < cps) {
                const int sl = list[r >> 1], tok = e < 0 ? sl - MS : sl / QG_TOP;
                dma16_ordered(A.xsp + ((size_t)tok * 2 + (r & 1)) * D32 + (size_t)c * 8, acts + (size_t)q * 512);
            }
        }
    };
    // Per item: the stage (untracked copies), then the weight rows; a wait for
    // the stage alone (the 3 NSB weight loads behind it may still be in
    // flight) and a barrier; then the products, each superblock waiting only
    // for its own rows (loads complete in issue order), so they run while the
    // later superblocks stream in.
    __syncthreads();
    asm volatile("" ::"v"(warm));  // the warming loads have landed
    const int nit = s_nitems;
    if (nit == 0) return;  // block-uniform
    uint4 hd[NSB], c0[NSB], c1[NSB];
    stage(s_item[0][0], s_item[0][1], s_list[0]);
    asm volatile("" ::: "memory");
    load_weights(s_item[0][0], blockIdx.x % rblocks, hd, c0, c1);
    for (int it = 0;; it++) {
        const int item = blockIdx.x + it * gridDim.x;
        wait_vmem_but<3 * NSB>();
        __syncthreads();
        const int e = s_item[it][0], n = s_item[it][1], rb0 = item % rblocks;
        const bool shared = e < 0;
        const int fmt = shared ? A.sh_fmt : A.fmt;
        const int pos = plane_pos(fmt, rb0 * GU_WROWS + wave * GU_ROWS + (j & 7));
        const int r = 2 * min(j >> 1, n - 1) + (j & 1);
        // the min-term product takes its 8 group sums from lanes kq = 0; the
        // other lanes read zeros
        const _Float16 *ap = act + (size_t)r * LY.arow + kq * 8, *sp = kq ? (const _Float16 *)s_zero : acts + (size_t)r * LY.srow;
        qg_f4 y = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sb = 0; sb < NSB; sb++) {
            const Q4kHeader h = q4k_header(hd[sb]);
            qg_half2 scA, ofA, scB, ofB;  // scales of groups gA, gA + 1 and gB, gB + 1
            gq_scales(h.S[0], kq, scA, ofA);
            gq_scales(h.S[1], kq, scB, ofB);
            qg_f4 p0 = qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, p1 = p0, mm = p0;
#pragma unroll
            for (int f = 0; f < 4; f++) {
                p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(ap + sb * 256 + f * 32),
                                                            gq_frag(c0[sb], f, scA[f >> 1], ofA[f >> 1]), p0, 0, 0, 0);
                p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(ap + sb * 256 + (4 + f) * 32),
                                                            gq_frag(c1[sb], f, scB[f >> 1], ofB[f >> 1]), p1, 0, 0, 0);
            }
            mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(sp + sb * 8), q4k_min_frag(h), mm, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(h.d, p0[i] + p1[i], __builtin_fmaf(-h.dmin, mm[i], y[i]));
            // one superblock at a time: its sums are taken and no later read is
            // hoisted above it
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < 4; i++) asm volatile("" : "+v"(y[i]));
        }
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const float v = y[2 * t2] + y[2 * t2 + 1];  // gate (j < 8) or up (j >= 8)
            const float u = __shfl_xor(v, 8);
            const float m = qg_swiglu_fast(v, u);
            // sum of the wave's 8 rows for this token (lanes j = 0..7)
            float s8 = m;
            s8 += __shfl_xor(s8, 1);
            s8 += __shfl_xor(s8, 2);
            s8 += __shfl_xor(s8, 4);
            const int idx = 2 * kq + t2;
            if (j < 8 && idx < n) {
                const int sl = s_list[it][idx];
                _Float16 *mp = A.midp + (size_t)sl * 2 * A.F;
                const _Float16 hv = (_Float16)m;
                mp[pos] = hv;
                mp[A.F + pos] = (_Float16)(m - (float)hv);
                if (j == 0) A.msum8[(size_t)sl * (A.F / GU_ROWS) + rb0 * 4 + wave] = s8;
            }
        }
        __syncthreads();  // the stage is free
        if (it + 1 == nit) break;  // block-uniform
        stage(s_item[it + 1][0], s_item[it + 1][1], s_list[it + 1]);
        asm volatile("" ::: "memory");
        load_weights(s_item[it + 1][0], (item + gridDim.x) % rblocks, hd, c0, c1);
    }
}

// ---------------- K3: down ----------------
struct DnArgs {
    int nt, D, F;
    const float *w; const DecPlan *pl;
    const uint8_t *down, *sh_down; size_t rb, sh_rb;
    const _Float16 *midp; const float *msum8;
    float *slots;                        // [ME][D]: selection t*10+k (weighted), shared rows MS+t
};

constexpr int DN_ROWS = 64;              // output rows per item (16 per wave)

// A fragment of staged plane row r (0..15 = token r/2, plane r%2), 16-byte
// chunk c; rows are F fp16 long, chunk c of row r stored at c ^ (r & 15).
QG_DEV qg_half8 dn_frag(const uint8_t *ast, int F, int r, int c) {
    return ld_frag((const _Float16 *)(ast + (size_t)r * F * 2 + 16 * (c ^ (r & 15))));
}

// y (rows 4kq..4kq+3 = tokens 2kq, 2kq+1 x {hi, lo}) of weight row wr
// (shared memory) against the staged tile; F/32 IQ4_NL blocks or F/256 Q4_K
// superblocks.  Q4_K min terms from the 8-row sums of the tile's tokens,
// staged as rows of F/8 floats padded by 4 (token mrow[t2]).
template <int FMT>
QG_DEV qg_f4 dn_tile(const uint8_t *wr, const uint8_t *ast, int F, int j, int kq, const float *ms, const int *mrow) {
    qg_f4 y = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
    if (FMT == QT_Q4_K) {
        for (int sb = 0; sb < F / 256; sb++) {
            qg_half8 af[8];
#pragma unroll
            for (int m = 0; m < 8; m++) af[m] = dn_frag(ast, F, j, sb * 32 + m * 4 + kq);
            const uint8_t *p = wr + sb * 144;
            const Q4kHeader h = q4k_header(*(const uint4 *)p);
            const uint4 ca = *(const uint4 *)(p + 16 + 16 * kq), cb = *(const uint4 *)(p + 16 + 16 * (kq + 4));
            qg_half2 scA, ofA, scB, ofB;  // scales of groups 2 (kq / 2) + {0, 1} and 4 + the same
            gq_scales(h.S[0], kq, scA, ofA);
            gq_scales(h.S[1], kq, scB, ofB);
            qg_f4 acc = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int f = 0; f < 4; f++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[f], gq_frag(ca, f, scA[f >> 1], ofA[f >> 1]), acc, 0, 0, 0);
#pragma unroll
            for (int f = 0; f < 4; f++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[4 + f], gq_frag(cb, f, scB[f >> 1], ofB[f >> 1]), acc, 0, 0, 0);
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                // group sums of mid: 4 partial sums of 8 rows per 32-group
                const float4 *X = (const float4 *)(ms + mrow[t2] * (F / 8 + 4) + sb * 32);
                float M = 0.0f;
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    const float4 q = X[g];
                    M = __builtin_fmaf((float)q4k_m(h, g), ((q.x + q.y) + (q.z + q.w)), M);
                }
                y[2 * t2] = __builtin_fmaf(h.d, acc[2 * t2], __builtin_fmaf(-h.dmin, M, y[2 * t2]));
                y[2 * t2 + 1] = __builtin_fmaf(h.d, acc[2 * t2 + 1], y[2 * t2 + 1]);
            }
        }
    } else {
        // per 8 blocks: every fragment and every product first, then the block scales
        for (int b0 = 0; b0 < F / 32; b0 += 8) {
            const int nb = min(8, F / 32 - b0);
            qg_half8 af[8];
            qg_f4 acc[8];
            float d[8];
#pragma unroll
            for (int b = 0; b < 8; b++)
                if (b < nb) af[b] = dn_frag(ast, F, j, (b0 + b) * 4 + kq);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                if (b < nb) {
                    const uint16_t *p16 = (const uint16_t *)(wr + 18 * (b0 + b));  // 2-byte aligned
                    d[b] = qg_half_u16(p16[0]);
                    const uint32_t q = (uint32_t)p16[1 + 2 * kq] | ((uint32_t)p16[2 + 2 * kq] << 16);
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[b], iq4_frag4(q), qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                }
            }
#pragma unroll
            for (int b = 0; b < 8; b++)
                if (b < nb)
#pragma unroll
                    for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(d[b], acc[b][i], y[i]);
        }
    }
    return y;
}

// Persistent; item = (tile, 64 output rows): the shared expert's tiles first,
// then the plan's routed tiles.  An item's 64-row weight slab (contiguous) and
// the tile's mid planes (up to 8 tokens) are staged in shared memory by direct
// global->shared copies; each of
// the 4 waves takes 16 rows (MFMA columns).  Results go to the selection's
// slot, weighted by its routing weight (shared rows unweighted); the combine
// kernel sums the slots in router-rank order.
template <int FMT, int SFMT, int FF>
__global__ __launch_bounds__(256, 2) void dec_down_kernel(DnArgs A) {
    extern __shared__ uint4 s_dyn[];
    __shared__ int s_list[TILE_TOK];   // the tile's selections
    __shared__ float s_wt[TILE_TOK];  // and routing weights (1 for the shared expert)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    constexpr int F = FF;  // the layer's F (512 or 640): a constant, so the staging splits need no division
    const uint32_t G = entry_grid();
    // every argument in the entry batch of scalar loads (see entry_grid)
    asm volatile("" ::"s"(A.nt), "s"(A.D), "s"(A.F), "s"(A.w), "s"(A.pl), "s"(A.down), "s"(A.sh_down), "s"(A.rb), "s"(A.sh_rb),
                 "s"(A.midp), "s"(A.msum8), "s"(A.slots));
    const int sh = A.sh_down != nullptr ? 1 : 0;
    const int dblocks = A.D / DN_ROWS;
    const int rbmax = (int)(A.rb > A.sh_rb ? A.rb : A.sh_rb);
    const int slab = (DN_ROWS * rbmax + 1023) & ~1023;
    uint8_t *wbuf = (uint8_t *)s_dyn, *abuf = wbuf + slab;
    float *mbuf = (float *)(abuf + 16 * F * 2);
    const int cpr = F / 8;  // 16-byte chunks per staged plane row
    const int sh_tiles = sh ? (A.nt + TILE_TOK - 1) / TILE_TOK : 0;
    // every wave holds the plan entry of the workgroup's next item in
    // registers (lane l: tile slot l % 8), loaded while the current item
    // streams (routed tiles only), so no barrier precedes an item's copies.
    // The tile's expert and token count sit in lanes 0 and 1 of p_en: a value
    // that differs across lanes stays in a vector register, so nothing waits
    // for the load until the next item reads it (a wave-uniform one would be
    // moved to a scalar register, with a wait, right after the load).
    int p_ntl = 0, p_en = -1, p_q = 0;
    auto fetch = [&](int item) {
        const int k = item / dblocks - sh_tiles;
        if (k >= 0 && k < MAX_TILES) {
            p_ntl = A.pl->n_tiles;
            p_en = (&A.pl->tile[k].e)[lane & 1];
            p_q = A.pl->tile[k].q[lane & (TILE_TOK - 1)];
        }
    };
    fetch(blockIdx.x);
    for (int item = blockIdx.x;; item += G) {
        const int T = item / dblocks, d0 = (item - T * dblocks) * DN_ROWS;
        // this item's expert e (-1: shared), token count n (-1: past the
        // plan) and the selection qs of tile slot lane % 8, alike in every wave
        int e = -1, n = -1, qs = MS;
        if (T < sh_tiles) {
            n = min(TILE_TOK, A.nt - TILE_TOK * T);
            qs = MS + TILE_TOK * T + (lane & (TILE_TOK - 1));
        } else if (T - sh_tiles < MAX_TILES && T - sh_tiles < p_ntl) {
            e = __builtin_amdgcn_readlane(p_en, 0);
            n = __builtin_amdgcn_readlane(p_en, 1);
            qs = p_q;
        }
        fetch(item + G);
        if (n < 0) break;  // block-uniform; every later item is past the plan too
        float wq = 1.0f;  // wave 0: the routing weight of tile slot `lane`, loaded behind the copies
        if (wave == 0 && lane < n) {
            s_list[lane] = qs;
            if (e >= 0) wq = A.w[qs];
        }
        auto sel = [&](int slot) { return __shfl(qs, slot); };  // the selection of tile slot `slot` (all lanes active)
        const bool shared = e < 0;
        const int rb = (int)(shared ? A.sh_rb : A.rb);
        // the item's weight slab: 64 consecutive rows, one flat copy
        {
            const uint8_t *W = shared ? A.sh_down + (size_t)d0 * rb : A.down + ((size_t)e * A.D + d0) * rb;
            const int nch = DN_ROWS * rb / 16;
            for (int q = wave; q * 64 < nch; q += 4) {
                const int c = q * 64 + lane;
                if (c < nch) dma16(W + 16 * (size_t)c, wbuf + (size_t)q * 1024);
            }
        }
        // the tile's 2n plane rows (token r/2, plane r%2) of mid, swizzled; rows
        // past them are not read into any kept result
        for (int q = wave; q * 64 < 2 * n * cpr; q += 4) {
            const int C = q * 64 + lane, r = C / cpr, pos = C - r * cpr;
            const int sq = sel(min(r, 2 * n - 1) >> 1);
            if (r < 2 * n) dma16(A.midp + ((size_t)sq * 2 + (r & 1)) * F + (size_t)(pos ^ (r & 15)) * 8, abuf + (size_t)q * 1024);
        }
        if ((shared ? SFMT : FMT) == QT_Q4_K) {
            // the tile tokens' 8-row sums of mid (Q4_K min terms), padded rows
            const int cpm = F / 32;  // 16-byte chunks per row
            for (int q = wave; q * 64 < n * (cpm + 1); q += 4) {
                const int slot = q * 64 + lane, r = slot / (cpm + 1), c = slot - r * (cpm + 1);
                const int sq = sel(min(r, n - 1));
                if (r < n && c < cpm) dma16(A.msum8 + (size_t)sq * (F / 8) + c * 4, mbuf + q * 256);
            }
        }
        wait_vmem();
        if (wave == 0 && lane < TILE_TOK) s_wt[lane] = wq;
        __syncthreads();
        const uint8_t *wr = wbuf + (size_t)(16 * wave + j) * rb;
        int mrow[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) mrow[t2] = min(2 * kq + t2, n - 1);
        const qg_f4 y = shared ? dn_tile<SFMT>(wr, abuf, F, j, kq, mbuf, mrow) : dn_tile<FMT>(wr, abuf, F, j, kq, mbuf, mrow);
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const int idx = 2 * kq + t2;
            if (idx < n) {
                const int sl = s_list[idx];
                const float v = y[2 * t2] + y[2 * t2 + 1];
                A.slots[(size_t)sl * A.D + d0 + 16 * wave + j] = shared ? v : v * s_wt[idx];
            }
        }
        __syncthreads();  // s_list, s_wt, the slab and the stage are rewritten by the next item
    }
}

// ---------------- K4: router-rank combine + shared + residual ----------------
struct CombArgs {
    int nt, D;
    const int *ids; const DecPlan *pl;
    const float *slots;
    const float *sh_logit; int ld; int has_shared;
    float *out, *resid;
    qg_prune_stats *stats;               // accumulated by block (0, 0) when pruning is active
};

// out[t] = sum over ranks k of the weighted slots (cpu.c:257-259 order), then
// + y_sh * sigmoid(logit) (gpu.cu:552-553), then the optional residual add.
// Flag 2 rows (host handoff, qwen.c:658-678) get the shared part only, flag 3
// rows 0.
__global__ __launch_bounds__(256) void dec_combine_kernel(CombArgs A) {
    const int t = blockIdx.y, d = (blockIdx.x * 256 + threadIdx.x) * 4;
    // every argument in the entry batch of scalar loads (see entry_grid)
    asm volatile("" ::"s"(A.nt), "s"(A.D), "s"(A.ids), "s"(A.pl), "s"(A.slots), "s"(A.sh_logit), "s"(A.ld), "s"(A.has_shared));
    asm volatile("" ::"s"(A.out), "s"(A.resid), "s"(A.stats));
    if (d < A.D) {
        // every load is independent of the others (slot addresses do not depend
        // on the ids): one memory round trip; invalid selections are selected away
        const int flag = A.pl->flag[t];
        int e[QG_TOP];
        float4 v[QG_TOP];
#pragma unroll
        for (int k = 0; k < QG_TOP; k++) {
            e[k] = A.ids[t * QG_TOP + k];
            v[k] = *(const float4 *)(A.slots + (size_t)(t * QG_TOP + k) * A.D + d);
        }
        float4 vs = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float lg = 0.0f;
        if (A.has_shared) {
            vs = *(const float4 *)(A.slots + (size_t)(MS + t) * A.D + d);
            lg = A.sh_logit[(size_t)t * A.ld];
        }
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (flag < 2) {
#pragma unroll
            for (int k = 0; k < QG_TOP; k++) {
                const bool ok = e[k] >= 0 && e[k] < QG_EXPERTS;
                acc.x += ok ? v[k].x : 0.0f;
                acc.y += ok ? v[k].y : 0.0f;
                acc.z += ok ? v[k].z : 0.0f;
                acc.w += ok ? v[k].w : 0.0f;
            }
        }
        if (A.has_shared && flag != 3) {
            const float sg = qg_sig(lg);
            acc.x = __builtin_fmaf(vs.x, sg, acc.x);
            acc.y = __builtin_fmaf(vs.y, sg, acc.y);
            acc.z = __builtin_fmaf(vs.z, sg, acc.z);
            acc.w = __builtin_fmaf(vs.w, sg, acc.w);
        }
        const size_t o = (size_t)t * A.D + d;
        if (A.out) *(float4 *)(A.out + o) = acc;
        if (A.resid) {
            float4 h = *(float4 *)(A.resid + o);
            h.x += acc.x; h.y += acc.y; h.z += acc.z; h.w += acc.w;
            *(float4 *)(A.resid + o) = h;
        }
    }
    if (A.stats && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64) {
        // counters (deterministic, unlike the reference's atomics): lane u
        // loads token u's record, all in flight at once; counts by ballots,
        // the skipped mass summed in token order, each added once
        const int u = threadIdx.x;
        int f = 3, mi = 0;
        double mu = 0.0;
        if (u < A.nt) {
            f = A.pl->flag[u];
            mi = A.pl->missing[u];
            mu = A.pl->mass[u];
        }
        const bool counted = f != 3, skipped = f == 1;
        int ms = counted ? mi : 0, ss = skipped ? mi : 0;
        ms = (int)qg_sum_lanes<64>((float)ms);  // small integers: exact in fp32
        ss = (int)qg_sum_lanes<64>((float)ss);
        const uint64_t tl = (uint64_t)__popcll(__ballot(counted)), av = (uint64_t)__popcll(__ballot(skipped));
        // the skipped mass in token order, by every lane (the readlanes run
        // with the whole wave active), stored by lane 0
        const uint64_t bits = (uint64_t)__double_as_longlong(skipped ? mu : 0.0);
        const int mhi = (int)(bits >> 32), mlo = (int)(uint32_t)bits, sk = skipped ? 1 : 0;
        double mass = A.stats->skipped_mass;
        for (int v = 0; v < A.nt; v++) {
            const double m = __longlong_as_double((long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(mhi, v) << 32) |
                                                              (uint32_t)__builtin_amdgcn_readlane(mlo, v)));
            if (__builtin_amdgcn_readlane(sk, v)) mass += m;
        }
        if (u == 0) {
            A.stats->token_layers += tl;
            A.stats->missing_selections += (uint64_t)ms;
            A.stats->skipped_selections += (uint64_t)ss;
            A.stats->avoided_token_handoffs += av;
            A.stats->skipped_mass = mass;
        }
    }
}

// ---------------- K3+K4 at one token: down and combine in one kernel ----------------
struct Dn1Args {
    int D, F;
    const float *w; const DecPlan *pl;
    const uint8_t *down, *sh_down; size_t rb, sh_rb;
    const _Float16 *midp; const float *msum8;
    const float *sh_logit;               // the shared-gate logit (with a shared expert)
    float *out, *resid;
    qg_prune_stats *stats;
};
constexpr int DN1_ROWS = 8;              // output rows per workgroup (MFMA columns 8..15 repeat 0..7)
static_assert(DN1_ROWS == DN1_PRE_ROWS, "gate/up prefetches the rows of this kernel's workgroups");
constexpr int DN1_SL = DN1_ROWS * 288 / 16;  // 16-byte slots of the rows (288 bytes each)
constexpr int DN1_W = 16;                // waves per workgroup
constexpr int DN1_EPW = 1;               // entries per wave (10 routed + 1 shared, each on its own wave)
// weight rows per wave and entry, then every entry's mid planes (F = 512) and 8-row sums
constexpr size_t DN1_LDS = (size_t)DN1_W * DN1_EPW * DN1_SL * 16 + (size_t)(QG_TOP + 1) * 2 * 512 * 2 + (size_t)(QG_TOP + 1) * 64 * 4;

// One token (the plan's entries k = eligible ranks in order, then the shared
// expert): workgroup b owns output rows 8b .. 8b + 7 (256 workgroups at
// D = 2048, one per CU); wave w (of 16)
// computes entry k = w (its 16 weight rows, the entries' mid planes
// and 8-row sums all copied into shared memory by direct global->shared
// copies at once), each weighted by its routing weight; wave 0 then sums them in
// rank order, adds sigmoid(logit) times the shared expert's row and the
// optional residual, as the combine kernel does.  F = 512 (288-byte rows).
template <int FMT, int SFMT>
__global__ __launch_bounds__(64 * DN1_W) void dec_down1_kernel(Dn1Args A) {
    extern __shared__ uint4 s_dyn[];
    __shared__ float s_v[QG_TOP + 1][DN1_ROWS];
    // every argument in the entry batch of scalar loads (see entry_grid)
    asm volatile("" ::"s"(A.D), "s"(A.F), "s"(A.w), "s"(A.pl), "s"(A.down), "s"(A.sh_down), "s"(A.rb), "s"(A.sh_rb),
                 "s"(A.midp), "s"(A.msum8), "s"(A.sh_logit), "s"(A.out), "s"(A.resid), "s"(A.stats));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int F = A.F, d0 = blockIdx.x * DN1_ROWS, sh = A.sh_down ? 1 : 0;
    uint4 *wl = s_dyn + (size_t)wave * DN1_EPW * DN1_SL;
    _Float16 *mids = (_Float16 *)(s_dyn + (size_t)DN1_W * DN1_EPW * DN1_SL);  // [E][2][F] mid planes
    float *msl = (float *)(mids + (size_t)(QG_TOP + 1) * 2 * F);          // [E][F/8] 8-row sums
    // the wave's plan entries, read with the entry count in one round trip
    // (entries k < DN1_W * DN1_EPW <= MAX_TILES always lie in the plan; those
    // past the count are then dropped)
    int ee[DN1_EPW], qq[DN1_EPW];
#pragma unroll
    for (int x = 0; x < DN1_EPW; x++) {
        const int k = wave + DN1_W * x;
        ee[x] = A.pl->tile[k].e;
        qq[x] = A.pl->tile[k].q[0];
    }
    const int nent = A.pl->n_tiles, flag = A.pl->flag[0], E = nent + sh;
#pragma unroll
    for (int x = 0; x < DN1_EPW; x++) {
        const int k = wave + DN1_W * x;
        ee[x] = k < nent ? ee[x] : -1;
        qq[x] = k < nent ? qq[x] : MS;
    }
    // every copy at once: this wave's entries' weight rows, and (spread over the
    // waves) each entry's two mid plane rows and its 8-row sums
#pragma unroll
    for (int x = 0; x < DN1_EPW; x++) {
        const int k = wave + DN1_W * x;
        if (k < E) {
            const uint8_t *W = (ee[x] < 0 ? A.sh_down : A.down + (size_t)ee[x] * A.D * A.rb) + (size_t)d0 * 288;
#pragma unroll
            for (int i = 0; i < (DN1_SL + 63) / 64; i++) {
                const int sl = i * 64 + lane;
                if (sl < DN1_SL) dma16_ordered(W + 16 * (size_t)sl, wl + (size_t)x * DN1_SL + i * 64);
            }
            // the entry's mid planes (2 x 1 KB) and sums (256 bytes)
            const int q = qq[x];
            const _Float16 *mg = A.midp + (size_t)q * 2 * F;
#pragma unroll
            for (int pl = 0; pl < 2; pl++) dma16_ordered(mg + (size_t)pl * F + lane * 8, mids + ((size_t)k * 2 + pl) * F);
            if (lane < F / 32) dma16_ordered(A.msum8 + (size_t)q * (F / 8) + lane * 4, msl + (size_t)k * (F / 8));
        }
    }
    // the entries' routing weights, read while the copies stream (read
    // before them, the dependent load would delay their issue; read at the
    // end, it would add a round trip after the products)
    float wq[DN1_EPW];
#pragma unroll
    for (int x = 0; x < DN1_EPW; x++) wq[x] = wave + DN1_W * x < nent ? A.w[qq[x]] : 1.0f;
    wait_vmem();
    __syncthreads();
#pragma unroll
    for (int x = 0; x < DN1_EPW; x++) {
        const int k = wave + DN1_W * x;
        if (k < E) {
            const bool shared = ee[x] < 0, q4k = (shared ? SFMT : FMT) == QT_Q4_K;
            const int q = qq[x];
            // A rows: 0 = hi plane, 1 = lo plane of the token's mid (others repeat them)
            const _Float16 *mr = mids + ((size_t)k * 2 + (j & 1)) * F + kq * 8;
            qg_half8 af[16];
#pragma unroll
            for (int i = 0; i < 16; i++) af[i] = ld_frag(mr + i * 32);
            float xg[16];
            if (q4k) {
#pragma unroll
                for (int g = 0; g < 16; g++) {
                    const float4 m4 = *(const float4 *)(msl + (size_t)k * (F / 8) + 4 * g);
                    xg[g] = (m4.x + m4.y) + (m4.z + m4.w);
                }
            }
            const uint8_t *wb = (const uint8_t *)(wl + (size_t)x * DN1_SL) + (size_t)(j % DN1_ROWS) * 288;
            qg_f4 y = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
            if (q4k) {
#pragma unroll
                for (int sb = 0; sb < 2; sb++) {
                    const uint8_t *p = wb + sb * 144;
                    const Q4kHeader h = q4k_header(*(const uint4 *)p);
                    const uint4 ca = *(const uint4 *)(p + 16 + 16 * kq), cb = *(const uint4 *)(p + 16 + 16 * (kq + 4));
                    qg_half2 scA, ofA, scB, ofB;  // scales of groups 2 (kq / 2) + {0, 1} and 4 + the same
                    gq_scales(h.S[0], kq, scA, ofA);
                    gq_scales(h.S[1], kq, scB, ofB);
                    qg_f4 acc = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int f = 0; f < 4; f++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[sb * 8 + f], gq_frag(ca, f, scA[f >> 1], ofA[f >> 1]), acc, 0, 0, 0);
#pragma unroll
                    for (int f = 0; f < 4; f++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[sb * 8 + 4 + f], gq_frag(cb, f, scB[f >> 1], ofB[f >> 1]), acc, 0, 0, 0);
                    float M = 0.0f;
#pragma unroll
                    for (int g = 0; g < 8; g++) M = __builtin_fmaf((float)q4k_m(h, g), xg[sb * 8 + g], M);
                    y[0] = __builtin_fmaf(h.d, acc[0], __builtin_fmaf(-h.dmin, M, y[0]));
                    y[1] = __builtin_fmaf(h.d, acc[1], y[1]);
                }
            } else {
#pragma unroll
                for (int b0 = 0; b0 < 16; b0 += 8) {
                    qg_f4 acc[8];
                    float d[8];
#pragma unroll
                    for (int bb = 0; bb < 8; bb++) {
                        const uint16_t *p16 = (const uint16_t *)(wb + 18 * (b0 + bb));  // 2-byte aligned
                        d[bb] = qg_half_u16(p16[0]);
                        const uint32_t qv = (uint32_t)p16[1 + 2 * kq] | ((uint32_t)p16[2 + 2 * kq] << 16);
                        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[b0 + bb], iq4_frag4(qv), qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    }
#pragma unroll
                    for (int bb = 0; bb < 8; bb++) {
                        y[0] = __builtin_fmaf(d[bb], acc[bb][0], y[0]);
                        y[1] = __builtin_fmaf(d[bb], acc[bb][1], y[1]);
                    }
                }
            }
            // lanes kq = 0 hold rows 0 (hi) and 1 (lo) of weight row j
            const float v = y[0] + y[1];
            if (kq == 0 && j < DN1_ROWS) s_v[k][j] = shared ? v : v * wq[x];
        }
    }
    __syncthreads();
    if (tid < DN1_ROWS) {
        float acc = 0.0f;
        if (flag < 2)
            for (int k = 0; k < nent; k++) acc += s_v[k][tid];
        // a handed-off token (flag 2, no routed entries) keeps the shared part
        if (sh && flag != 3) acc = __builtin_fmaf(s_v[nent][tid], qg_sig(A.sh_logit[0]), acc);
        if (A.out) A.out[d0 + tid] = acc;
        if (A.resid) A.resid[d0 + tid] += acc;
    }
    if (A.stats && blockIdx.x == 0 && tid == 0 && flag != 3) {
        A.stats->token_layers += 1;
        A.stats->missing_selections += (uint64_t)A.pl->missing[0];
        if (flag == 1) {
            A.stats->skipped_selections += (uint64_t)A.pl->missing[0];
            A.stats->avoided_token_handoffs += 1;
            A.stats->skipped_mass += A.pl->mass[0];
        }
    }
}

bool fmt_down_ok(int t, int F) { return (t == QT_Q4_K && F % 256 == 0) || t == QT_IQ4_NL; }

bool dec_ok(const qg_moe_layer *L) {
    const int D = L->width, F = L->ff;
    if ((D != 2048 && D != 2560) || (F != 512 && F != 640)) return false;
    if (L->gate_type != QT_Q4_K || L->up_type != QT_Q4_K || !fmt_down_ok(L->down_type, F)) return false;
    if (L->sh_gate && (L->sh_gate_type != QT_Q4_K || L->sh_up_type != QT_Q4_K || !fmt_down_ok(L->sh_down_type, F))) return false;
    return true;
}

template <int FF>
void launch_down_f(const DnArgs &DA, int fr, int fs, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(256);
    if (fr == QT_IQ4_NL && fs == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_IQ4_NL, QT_IQ4_NL, FF>, grid, block, lds, s, DA);
    else if (fr == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_IQ4_NL, QT_Q4_K, FF>, grid, block, lds, s, DA);
    else if (fs == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_Q4_K, QT_IQ4_NL, FF>, grid, block, lds, s, DA);
    else dec_launch(3, dec_down_kernel<QT_Q4_K, QT_Q4_K, FF>, grid, block, lds, s, DA);
}
// F is 512 or 640 on this path (dec_ok)
void launch_down(const DnArgs &DA, int fr, int fs, dim3 grid, size_t lds, hipStream_t s) {
    if (DA.F == 512) launch_down_f<512>(DA, fr, fs, grid, lds, s);
    else launch_down_f<640>(DA, fr, fs, grid, lds, s);
}

template <int DW>
void router_launch(int TPB, dim3 grid, dim3 block, size_t lds, hipStream_t s, const RouterArgs &R) {
    switch (TPB) {
    case 1: dec_launch(0, dec_router_kernel<1, DW, 1>, grid, block, lds, s, R); break;
    case 2: dec_launch(0, dec_router_kernel<2, DW, 4>, grid, block, lds, s, R); break;
    case 3: dec_launch(0, dec_router_kernel<3, DW, 4>, grid, block, lds, s, R); break;
    case 4: dec_launch(0, dec_router_kernel<4, DW, 4>, grid, block, lds, s, R); break;
    default: dec_launch(0, dec_router_kernel<5, DW, 4>, grid, block, lds, s, R); break;
    }
}

int dec_forward(float *out, float *resid, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                const float *x, float *xn_out, int norm, int nt, const qg_moe_layer *L, uint8_t *ws) {
    const int D = L->width, F = L->ff;
    const bool sh = L->sh_gate != nullptr;
    const DecLayout lay = dec_layout(D, F);
    hipStream_t s = qg_stream();
    DecPlan *pl = (DecPlan *)(ws + lay.tok);
    float *logits = (float *)(ws + lay.logits);
    _Float16 *xp = (_Float16 *)(ws + lay.xp);
    _Float16 *xsp = (_Float16 *)(ws + lay.xsum);
    const int rows = QG_EXPERTS + (sh ? 1 : 0);
    // token groups of up to 5: 64 row blocks of 4 waves each (128 blocks of 2
    // waves: 6.3 -> 6.7 us at 17 tokens); one token: 256 one-wave row blocks
    // (fewer rows per CU, so more of the router's 4 MB in flight at once)
    const int ngr = (nt + 4) / 5, TPB = (nt + ngr - 1) / ngr, RW = TPB == 1 ? 1 : 4;
    const int row_blocks = QG_EXPERTS / (2 * RW) * ngr, plane_blocks = (nt + RW - 1) / RW;
    // one token: every gate/up workgroup routes it; 2..8 tokens at D = 2048:
    // every dec_gateup3_kernel workgroup routes the batch, a token per wave
    // (a second token per wave costs the kernel more than the routing kernel
    // takes); otherwise the routing kernel sets the plan's token masks,
    // cleared by the router
    const bool inl = nt <= INLINE_MAX, gu3r = !inl && D == 2048 && nt <= GU3_W, rk = !inl && !gu3r;
    RouterArgs R{x, nt, D, rows, L->router, sh ? L->sh_gate_inp : nullptr, logits, norm, 1e-6f, xn_out, xp, xsp, plane_blocks,
                 L->router_bias, rk ? pl->emask : nullptr};
    const dim3 rgrid(plane_blocks + row_blocks), rblock(64 * RW);
    const size_t rlds = (size_t)(TPB > 2 * RW ? TPB : 2 * RW) * D * 4;  // router blocks: the group's rows; plane blocks: two rows per wave
    if (D == 2048) router_launch<2048>(TPB, rgrid, rblock, rlds, s, R);
    else router_launch<2560>(TPB, rgrid, rblock, rlds, s, R);
    int rc = hipGetLastError();
    if (rc) return rc;
    if (rk) {
        RouteArgs RA{nt, logits, rows, L->resident, L->threshold, ids, weights, flags, pl};
        dec_launch(1, dec_route_kernel, dim3(nt), dim3(64), 0, s, RA);
        if ((rc = hipGetLastError())) return rc;
    }
    _Float16 *midp = (_Float16 *)(ws + lay.midp);
    float *msum8 = (float *)(ws + lay.msum);
    GuArgs G2{nt, D, F, inl ? 1 : gu3r ? 2 : 0, logits, rows, L->resident, L->threshold, ids, weights, flags, pl,
              (const uint8_t *)L->gate, (const uint8_t *)L->up, sh ? (const uint8_t *)L->sh_gate : nullptr,
              sh ? (const uint8_t *)L->sh_up : nullptr, qg_row_bytes_host(QT_Q4_K, D), xp, xsp, midp, msum8,
              L->down_type, sh ? L->sh_down_type : L->down_type, nullptr, nullptr};
    const size_t rb = qg_row_bytes_host(L->down_type, F), srb = sh ? qg_row_bytes_host(L->sh_down_type, F) : 0;
    const bool down1 = inl && F == 512 && rb == 288 && (!sh || srb == 288) && D % DN1_ROWS == 0;
    if (down1) {
        G2.dn_pre = (const uint8_t *)L->down;
        G2.sh_dn_pre = sh ? (const uint8_t *)L->sh_down : nullptr;
    }
    // upper bound of the tiles: the shared expert's, and every selection its own tile
    const int tiles = (sh ? (nt + TILE_TOK - 1) / TILE_TOK : 0) + nt * QG_TOP;
    const int items = tiles * (F / GU_WROWS);
    int nwg = items < GU_WGS ? items : GU_WGS;
    if (nwg * GU_NI < items) nwg = (items + GU_NI - 1) / GU_NI;  // each workgroup resolves GU_NI items at most
    // the pipelined kernel: contiguous ranges of 16-row items, at most GU2_NT tiles each
    const int items2 = tiles * (F / GU2_ROWS), per2 = (GU2_NT - 1) * (F / GU2_ROWS);
    int nwg2 = items2 < GU_WGS ? items2 : GU_WGS;
    if ((long long)nwg2 * per2 < items2) nwg2 = (items2 + per2 - 1) / per2;
    if (D == 2048) {
        // F is a multiple of 32 (validate_layer), so of GU2_ROWS; one
        // workgroup per CU, each on one expert's run of F blocks
        // (one token: the per-tile kernel with its finer split, 512 workgroups)
        if (inl) dec_launch(2, dec_gateup2_kernel<true>, dim3(nwg2), dim3(256), GU2_LDS, s, G2);
        else dec_launch(2, dec_gateup3_kernel, dim3(qg_cu_count()), dim3(64 * GU3_W), GU3_LDS, s, G2);
    } else {
        // D = 2560 (dec_ok): the register-weight kernel, 10 superblocks per row
        const size_t gu_bytes = (size_t)gu_lds(D).total * 2;
        if (inl) dec_launch(2, dec_gateup_kernel<10, true>, dim3(nwg), dim3(256), gu_bytes, s, G2);
        else dec_launch(2, dec_gateup_kernel<10, false>, dim3(nwg), dim3(256), gu_bytes, s, G2);
    }
    if ((rc = hipGetLastError())) return rc;
    float *slots = (float *)(ws + lay.slots);
    DnArgs DA{nt, D, F, weights, pl, (const uint8_t *)L->down, sh ? (const uint8_t *)L->sh_down : nullptr, rb, srb,
              midp, msum8, slots};
    const size_t rbmax = rb > srb ? rb : srb;
    // slab, 16 staged plane rows, 8 padded rows of 8-row sums (rounded up to whole 1 KB copies)
    const size_t dn_lds = ((DN_ROWS * rbmax + 1023) & ~(size_t)1023) + (size_t)16 * F * 2 +
                          (((size_t)8 * (F / 8 + 4) * 4 + 1023) & ~(size_t)1023);
    const int fr = L->down_type, fs = sh ? L->sh_down_type : fr;
    if (down1) {
        // one token: down and the combine in one kernel
        Dn1Args D1{D, F, weights, pl, (const uint8_t *)L->down, sh ? (const uint8_t *)L->sh_down : nullptr, rb, srb,
                   midp, msum8, logits + QG_EXPERTS, out, resid, (L->resident && stats) ? stats : nullptr};
        const dim3 g1(D / DN1_ROWS), b1(64 * DN1_W);
        if (fr == QT_IQ4_NL && fs == QT_IQ4_NL) dec_launch(3, dec_down1_kernel<QT_IQ4_NL, QT_IQ4_NL>, g1, b1, DN1_LDS, s, D1);
        else if (fr == QT_IQ4_NL) dec_launch(3, dec_down1_kernel<QT_IQ4_NL, QT_Q4_K>, g1, b1, DN1_LDS, s, D1);
        else if (fs == QT_IQ4_NL) dec_launch(3, dec_down1_kernel<QT_Q4_K, QT_IQ4_NL>, g1, b1, DN1_LDS, s, D1);
        else dec_launch(3, dec_down1_kernel<QT_Q4_K, QT_Q4_K>, g1, b1, DN1_LDS, s, D1);
        return hipGetLastError();
    }
    const int dn_items = tiles * (D / DN_ROWS);
    launch_down(DA, fr, fs, dim3(dn_items < DN_WGS ? dn_items : DN_WGS), dn_lds, s);
    if ((rc = hipGetLastError())) return rc;
    CombArgs CA{nt, D, ids, pl, slots, logits + QG_EXPERTS, rows, sh ? 1 : 0, out, resid,
                (L->resident && stats) ? stats : nullptr};
    dec_launch(4, dec_combine_kernel, dim3((D / 4 + 255) / 256, nt), dim3(256), 0, s, CA);
    return hipGetLastError();
}

// The layer kernels copy weight, activation and output rows with 16-byte
// direct global->shared copies and vector accesses.
bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

int validate_layer(const qg_moe_layer *L, int nt) {
    if (!L || nt < 1 || nt > QG_MAX_TOKENS) return hipErrorInvalidValue;
    if (!al16(L->router) || !al16(L->gate) || !al16(L->up) || !al16(L->down) || !al16(L->sh_gate) || !al16(L->sh_up) ||
        !al16(L->sh_down) || !al16(L->sh_gate_inp) || !al16(L->router_bias))
        return hipErrorInvalidValue;
    const int D = L->width, F = L->ff;
    if (D < 256 || D % 256 || D > 8192 || F < 32 || F % 32 || F > 4096) return hipErrorInvalidValue;
    if (!L->router || !L->gate || !L->up || !L->down) return hipErrorInvalidValue;
    if (!qg_row_bytes_host(L->gate_type, D) || !qg_row_bytes_host(L->up_type, D) || !qg_row_bytes_host(L->down_type, F))
        return hipErrorInvalidValue;
    if (L->sh_gate && (!L->sh_up || !L->sh_down || !L->sh_gate_inp || !qg_row_bytes_host(L->sh_gate_type, D) ||
                       !qg_row_bytes_host(L->sh_up_type, D) || !qg_row_bytes_host(L->sh_down_type, F)))
        return hipErrorInvalidValue;
    if (L->resident && (L->threshold < 0 || L->threshold > 0.1 || !__builtin_isfinite(L->threshold))) return hipErrorInvalidValue;
    if (nt > MB && !qg_prefill_ok(L)) return hipErrorInvalidValue;
    return hipSuccess;
}

__global__ void add_rows_kernel(float *h, const float *o, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = h[i] + o[i];
}

}  // namespace

// Library-held workspace for qg_moe_forward_noalloc: one copy per GPU in
// the code object's device memory (it lives until the process ends).  Host
// code never passes `scratch` itself to a kernel: its host-side name is a
// stand-in, not a device address.  The device address of each GPU's copy is
// looked up once per device (hipGetSymbolAddress with that device current)
// and kept in noalloc_ptr.
constexpr size_t NOALLOC_BYTES = (size_t)16 << 20;
constexpr int NOALLOC_DEVICES = 64;
__device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];
void *noalloc_ptr[NOALLOC_DEVICES] = {nullptr};
std::mutex noalloc_mu;

int noalloc_workspace(void **ws) {
    int dev = 0, rc = hipGetDevice(&dev);
    if (rc) return rc;
    if (dev < 0 || dev >= NOALLOC_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(noalloc_mu);
    if (!noalloc_ptr[dev]) {
        void *p = nullptr;
        if ((rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))) return rc;
        if (!p) return hipErrorInvalidSymbol;
        noalloc_ptr[dev] = p;
    }
    *ws = noalloc_ptr[dev];
    return hipSuccess;
}

bool qg_kernel_event_pair(int slot, void **begin, void **end) {
    if (slot < 0 || 2 * slot + 1 >= tl_kev_n || !tl_kev[2 * slot] || !tl_kev[2 * slot + 1]) return false;
    *begin = tl_kev[2 * slot];
    *end = tl_kev[2 * slot + 1];
    return true;
}

extern "C" {

size_t qg_moe_workspace_bytes(int width, int ff, int tokens) {
    if (tokens > MB) return qg_prefill_workspace_bytes(width, ff, tokens);
    const size_t g = qg_generic_workspace_bytes(width, ff, tokens);
    if (!g) return 0;
    // the residual form keeps the normalised input and the layer output of the
    // generic path after its own workspace
    const size_t extra = 2 * (((size_t)MB * width * 4 + 255) & ~(size_t)255);
    const size_t d = dec_layout(width, ff).total;
    return (g + extra > d ? g + extra : d);
}

int qg_moe_kernel_events(void **events, int n) {
    if (n < 0 || n > 32 || (n && !events)) return hipErrorInvalidValue;
    for (int i = 0; i < 32; i++) tl_kev[i] = i < n ? events[i] : nullptr;
    tl_kev_n = n;
    return hipSuccess;
}

int qg_moe_forward(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, const float *x, int nt,
                   const qg_moe_layer *L, void *workspace, size_t ws_bytes) {
    int rc = validate_layer(L, nt);
    if (rc) return rc;
    if (!out || !ids || !weights || !x || !workspace || ws_bytes < qg_moe_workspace_bytes(L->width, L->ff, nt) ||
        !al16(out) || !al16(x) || !al16(workspace))
        return hipErrorInvalidValue;
    if (nt > MB) return qg_prefill_forward(out, nullptr, ids, weights, flags, stats, x, nullptr, 0, nt, L, workspace);
    if (!dec_ok(L)) return qg_generic_forward(out, ids, weights, flags, stats, x, nt, L, workspace, ws_bytes);
    return dec_forward(out, nullptr, ids, weights, flags, stats, x, nullptr, 0, nt, L, (uint8_t *)workspace);
}

// qg_moe_forward with the library's static per-device workspace: no
// allocation of any kind, for callers that cannot allocate.  Rejects (invalid
// value, nothing launched) a layer whose workspace at `nt` tokens exceeds
// NOALLOC_BYTES.  The workspace needs no initialisation (every kernel writes
// what it later reads), so nothing is cleared between calls; calls that
// overlap on one GPU share it and race.
int qg_moe_forward_noalloc(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, const float *x,
                           int nt, const qg_moe_layer *L) {
    int rc = validate_layer(L, nt);
    if (rc) return rc;
    const size_t need = qg_moe_workspace_bytes(L->width, L->ff, nt);
    if (!need || need > NOALLOC_BYTES) return hipErrorInvalidValue;
    void *ws = nullptr;
    if ((rc = noalloc_workspace(&ws))) return rc;
    return qg_moe_forward(out, ids, weights, flags, stats, x, nt, L, ws, NOALLOC_BYTES);
}

int qg_moe_forward_residual(float *h, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, float *xn_out,
                            float *out, int nt, const qg_moe_layer *L, void *workspace, size_t ws_bytes) {
    int rc = validate_layer(L, nt);
    if (rc) return rc;
    if (!h || !ids || !weights || !workspace || ws_bytes < qg_moe_workspace_bytes(L->width, L->ff, nt) || !al16(h) ||
        !al16(xn_out) || !al16(out) || !al16(workspace))
        return hipErrorInvalidValue;
    if (nt > MB) return qg_prefill_forward(out, h, ids, weights, flags, stats, h, xn_out, 1, nt, L, workspace);
    if (dec_ok(L)) return dec_forward(out, h, ids, weights, flags, stats, h, xn_out, 1, nt, L, (uint8_t *)workspace);
    // generic form: normalise into the workspace tail, run the layer, add
    const int D = L->width;
    const size_t g = qg_generic_workspace_bytes(D, L->ff, nt), act = ((size_t)MB * D * 4 + 255) & ~(size_t)255;
    float *xn = (float *)((uint8_t *)workspace + g), *o = (float *)((uint8_t *)workspace + g + act);
    if ((rc = qg_norm(xn, h, nullptr, D, 1, nt, 0, 0, 1e-6f))) return rc;
    if (xn_out && (rc = qg_copy(xn_out, xn, (size_t)nt * D * 4))) return rc;
    if ((rc = qg_generic_forward(o, ids, weights, flags, stats, xn, nt, L, workspace, g))) return rc;
    if (out && (rc = qg_copy(out, o, (size_t)nt * D * 4))) return rc;
    const size_t n = (size_t)nt * D;
    add_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, qg_stream()>>>(h, o, n);
    return hipGetLastError();
}

}  // extern "C"
