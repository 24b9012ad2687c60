// Device-driven routed-MoE layer for decode batches (1..17 tokens): the fast
// path of qg_moe_forward (and qg_moe_forward_residual) for Q4_K gate/up and
// Q4_K or IQ4_NL down.  It replaces moe()/grouped_moe()/shared_direct() of
// qwen.c:633-735 for one layer without any host round trip.
//
// Kernels per layer (3 for B <= 4, 4 above).  No kernel waits on another block
// of its own grid: on MI355X a grid-wide ticket costs ~12 ns per block of
// serialised atomics and a device-scope fence ~17 us per 1000 waves, more than
// a kernel boundary (~1.7-2.4 us).
//   K1 router  : the 512 router rows (plus the shared-expert gate vector as
//                row 512) for every token in the reference's fixed summation
//                order, so logits, ids and weights are bit-exact.  Extra
//                blocks write the fp16 hi/lo activation planes and per-32
//                sums; optionally the input is RMS-normalised first.
//   KR route   : B > 4 only; one wave per token: top-10, coverage/prune, flags.
//   K2 gate/up : one workgroup per (selection, 32 rows of F).  A selection
//                computes its expert only if it is the expert's first
//                eligible selection (no dispatch list needed), for every token
//                that chose the expert.  B <= 4 routes inline.  Products on the
//                matrix cores (v_mfma_f32_16x16x32_f16) with exact integer
//                weights; SwiGLU; mid rows written as fp16 hi/lo planes.
//   K3 down    : one workgroup per 16 output rows, owning every selected
//                expert for those rows: down products on the matrix cores,
//                then the router-rank sum of the 10 slots, the sigmoid-gated
//                shared expert and the optional residual add, in-block.
//
// Operand conventions and the K order of the weight formats are those of
// qg_frag.h; here A row j = (token j/2, plane j%2), so a lane's D rows
// 4kq..4kq+3 are tokens 2kq, 2kq+1 (hi, lo) of weight row j.
#include "qg_internal.h"
#include "qg_frag.h"
#include <hip/hip_ext.h>

namespace {

constexpr int MB = QG_MAX_DECODE;         // 17 tokens
constexpr int MS = MB * QG_TOP;           // 170 selections
constexpr int ME = MS + MB;               // selection rows + shared-expert rows
constexpr int RCH = 64;                   // router k-steps held in registers
constexpr int INLINE_MAX = 1;             // tokens routed inside the gate/up kernel
constexpr int GU_WGS = 512;               // gate/up grid cap (workgroups)

struct TokRoute { int flag[MB]; int missing[MB]; double mass[MB]; };

struct DecLayout { size_t tok, logits, xp, xsum, midp, msum, total; };
DecLayout dec_layout(int D, int F) {
    DecLayout L;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += (n + 255) & ~(size_t)255; return o; };
    L.tok = take(sizeof(TokRoute));
    L.logits = take((size_t)MB * (QG_EXPERTS + 1) * 4);
    L.xp = take((size_t)MB * 2 * D * 2);
    L.xsum = take((size_t)MB * 2 * (D / 32) * 2);
    L.midp = take((size_t)ME * 2 * F * 2);
    L.msum = take((size_t)ME * (F / 8) * 4);
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
    int row_pairs;                  // blockIdx.x < row_pairs: router rows; == row_pairs: planes
    const float *bias;              // F32 [512] added to the expert logits, or null
};

// Grid (row_pairs + 1, ceil(nt/4)), 4 waves per block, wave w = token
// 4*blockIdx.y + w.  Router block x: each 32-lane half owns row 2x+half; lane j
// accumulates columns k = j (mod 32) in ascending k with fma, then the
// 16/8/4/2/1 tree: the order of cpu.c:122-139, so logits equal the
// reference's qc_matmul bit for bit.  All 64 weight and 64 input loads of a
// lane (D = 2048) are issued before the first fma.  Block x = row_pairs: the
// token's (optionally normalised) row as fp16 hi/lo planes in the Q4_K
// fragment order, plus hi/lo planes of the sums of each 32-group.
__global__ __launch_bounds__(256) void dec_router_kernel(RouterArgs A) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, j = lane & 31;
    const int t = blockIdx.y * 4 + wave;
    if (t >= A.nt) return;  // whole wave; no block barrier in this kernel
    const float *xr = A.x + (size_t)t * A.D;
    const float sc = A.norm ? row_rms_scale(xr, A.D, A.eps, lane) : 1.0f;
    if (blockIdx.x == A.row_pairs) {
        _Float16 *hi = A.xp + (size_t)t * 2 * A.D, *shi = A.xsp + (size_t)t * 2 * (A.D / 32);
        token_planes(xr, A.D, A.norm != 0, sc, lane, hi, hi + A.D, shi, shi + A.D / 32, A.xn ? A.xn + (size_t)t * A.D : nullptr);
        return;
    }
    const int row = blockIdx.x * 2 + half;
    const bool rok = row < A.rows;
    const float *wr = !rok ? A.router : row == QG_EXPERTS ? A.sh_row : A.router + (size_t)row * A.D;
    float acc = 0.0f;
    int k0 = 0;
    for (; k0 + 32 * RCH <= A.D; k0 += 32 * RCH) {
        float wv[RCH], xv[RCH];
#pragma unroll
        for (int i = 0; i < RCH; i++) {
            wv[i] = wr[k0 + 32 * i + j];
            xv[i] = xr[k0 + 32 * i + j];
        }
        if (A.norm)
#pragma unroll
            for (int i = 0; i < RCH; i++) xv[i] = xv[i] * sc;
#pragma unroll
        for (int i = 0; i < RCH; i++) acc = __builtin_fmaf(wv[i], xv[i], acc);
    }
    for (; k0 < A.D; k0 += 32) {
        const float xv = A.norm ? xr[k0 + j] * sc : xr[k0 + j];
        acc = __builtin_fmaf(wr[k0 + j], xv, acc);
    }
    const float r = qg_tree32(acc);
    if (j == 0 && rok) A.logits[(size_t)t * A.rows + row] = A.bias && row < QG_EXPERTS ? r + A.bias[row] : r;
}

// ---------------- KR: routing, one wave per token (B > 4) ----------------
struct RouteArgs {
    int nt; const float *logits; int ld;
    const uint8_t *resident; double thr;
    int *ids; float *w; uint8_t *flags_out; TokRoute *tr;
};

__global__ __launch_bounds__(256) void dec_route_kernel(RouteArgs A) {
    __shared__ float s_rv[4][64];
    __shared__ int s_ri[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = blockIdx.x * 4 + wave;
    if (t >= A.nt) return;  // the whole wave; this kernel has no block barrier
    int id, missing;
    float wv;
    double mass;
    qg_route_fast(A.logits + (size_t)t * A.ld, lane, id, wv, s_rv[wave], s_ri[wave]);
    const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
    if (lane < QG_TOP) { A.ids[t * QG_TOP + lane] = id; A.w[t * QG_TOP + lane] = wv; }
    if (lane == 0) {
        A.tr->flag[t] = flag;
        A.tr->missing[t] = missing;
        A.tr->mass[t] = mass;
        if (A.flags_out) A.flags_out[t] = (uint8_t)flag;
    }
}

// ---------------- K2: gate/up + SwiGLU ----------------
struct GuArgs {
    int nt, D, F;
    int inline_route; const float *logits; int ld; const uint8_t *resident; double thr;
    int *ids; float *w; uint8_t *flags_out; TokRoute *tr;
    const uint8_t *gate, *up, *sh_gate, *sh_up; size_t rb;
    const _Float16 *xp, *xsp;
    _Float16 *midp; float *msum8;    // mid planes [ME][2][F] in the down format's order; sums of 8 rows [ME][F/8]
    int fmt, sh_fmt;                 // down formats of the routed and shared experts
    int tt;                          // tokens per tile (8)
};

constexpr int GU_ROWS = 8;           // F rows of gate and of up per wave
constexpr int GU_WROWS = 4 * GU_ROWS; // F rows per workgroup (4 waves)

// Workgroup = 4 waves, persistent over work items.  Item = (expert, tile of
// tt <= 8 of its tokens, 32 F rows): the shared expert's items first (no routing
// needed), then the routed experts in order of their owning selection (the
// expert's first eligible selection).  The tile's activation planes (real
// tokens only) are staged in shared memory while every wave loads its weight
// rows into registers; MFMA A fragments are then shared-memory reads.  In a
// wave, MFMA columns 0..7 are 8 gate rows and 8..15 the same 8 up rows, so
// lane l and lane l^8 hold gate and up of one (row, token) pair.
template <int NSB>
__global__ __launch_bounds__(256, 2) void dec_gateup_kernel(GuArgs A) {
    // dynamic shared memory: [tt tokens][2 planes][D] fp16 activations, the
    // tokens' [2][D/32] sum planes (rounded up to 1 KB), then per wave the
    // 16 rows x NSB Q4_K superblock headers (16 B each)
    extern __shared__ uint4 s_act[];
    // planning scratch shares the staging buffer (planning precedes any staging
    // of the same item, and every item ends with a barrier)
    int *s_first = (int *)s_act, *s_cnt = s_first + QG_EXPERTS;
    float *s_rv = (float *)(s_cnt + QG_EXPERTS);
    int *s_ri = (int *)(s_rv + 64);
    __shared__ int s_nown;
    __shared__ int s_ids[MS];
    __shared__ int s_flag[MB];
    __shared__ int s_owner[MS];      // owning selection of routed expert k
    __shared__ int s_tbase[MS + 1];  // first tile of routed expert k (prefix over owners)
    __shared__ int s_slot[MB];
    __shared__ int s_item[3];        // expert (-1 shared), list length n, tile
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int ns = A.nt * QG_TOP, rblocks = A.F / GU_WROWS, D = A.D, D32 = A.D / 32;
    const int TT = A.tt, sh_tiles = A.sh_gate ? (A.nt + TT - 1) / TT : 0;
    _Float16 *act = (_Float16 *)s_act;
    _Float16 *acts = act + TT * 2 * D;
    uint8_t *hbuf = (uint8_t *)acts + (((size_t)TT * 2 * D32 * 2 + 1023) & ~(size_t)1023) + (size_t)wave * 16 * NSB * 16;
    bool planned = false;
    for (int item = blockIdx.x;; item += gridDim.x) {
        const int tile_g = item / rblocks, rb0 = item % rblocks;
        if (tile_g >= sh_tiles && !planned) {
            // routing of this batch (inline for one token, else from the routing kernel)
            if (A.inline_route) {
                if (wave == 0) {
                    int id, missing;
                    float wv;
                    double mass;
                    qg_route_fast(A.logits, lane, id, wv, s_rv, s_ri);
                    const int flag = qg_route_cover(id, wv, A.resident, A.thr, missing, mass);
                    if (lane < QG_TOP) s_ids[lane] = id;
                    if (lane == 0) s_flag[0] = flag;
                    if (blockIdx.x == 0) {
                        if (lane < QG_TOP) { A.ids[lane] = id; A.w[lane] = wv; }
                        if (lane == 0) {
                            A.tr->flag[0] = flag;
                            A.tr->missing[0] = missing;
                            A.tr->mass[0] = mass;
                            if (A.flags_out) A.flags_out[0] = (uint8_t)flag;
                        }
                    }
                }
            } else {
                for (int i = tid; i < ns; i += 256) s_ids[i] = A.ids[i];
                if (tid < A.nt) s_flag[tid] = A.tr->flag[tid];
            }
            for (int i = tid; i < QG_EXPERTS; i += 256) { s_first[i] = 0x7fffffff; s_cnt[i] = 0; }
            __syncthreads();
            for (int i = tid; i < ns; i += 256) {
                const int e = s_ids[i];
                if (e >= 0 && e < QG_EXPERTS && s_flag[i / QG_TOP] < 2) { atomicMin(&s_first[e], i); atomicAdd(&s_cnt[e], 1); }
            }
            __syncthreads();
            if (wave == 0) {
                int n = 0, tiles = 0;
                for (int c0 = 0; c0 < ns; c0 += 64) {
                    const int q = c0 + lane;
                    const int e = q < ns ? s_ids[q] : -1;
                    const bool own = e >= 0 && e < QG_EXPERTS && s_flag[q / QG_TOP] < 2 && s_first[e] == q;
                    const int nt8 = own ? (min(s_cnt[e], MB) + TT - 1) / TT : 0;
                    int incl = nt8;
#pragma unroll
                    for (int d = 1; d < 64; d <<= 1) {
                        const int o = __shfl_up(incl, d);
                        if (lane >= d) incl += o;
                    }
                    const unsigned long long b = __ballot(own);
                    if (own) {
                        const int k = n + __popcll(b & ((1ULL << lane) - 1ULL));
                        s_owner[k] = q;
                        s_tbase[k] = tiles + incl - nt8;
                    }
                    n += __popcll(b);
                    tiles += __shfl(incl, 63);
                }
                if (lane == 0) { s_tbase[n] = tiles; s_nown = n; }
            }
            __syncthreads();
            planned = true;
        }
        // item -> expert, token list, tile (wave 0), shared with the other waves
        if (wave == 0) {
            int e = -1, n, tile = tile_g;
            bool done = false;
            if (tile_g >= sh_tiles) {
                const int n_owner = s_nown, rt = tile_g - sh_tiles;
                if (rt >= s_tbase[n_owner]) done = true;
                else {
                    int k = 0;
                    while (s_tbase[k + 1] <= rt) k++;
                    e = s_ids[s_owner[k]];
                    tile = rt - s_tbase[k];
                }
            }
            if (done) n = -1;
            else if (e < 0) {
                n = A.nt;
                if (lane < A.nt) s_slot[lane] = MS + lane;
            } else {
                n = 0;
                for (int c0 = 0; c0 < ns; c0 += 64) {
                    const int q = c0 + lane;
                    const bool m = q < ns && s_ids[q] == e && s_flag[q / QG_TOP] < 2;
                    const unsigned long long b = __ballot(m);
                    const int pos = n + __popcll(b & ((1ULL << lane) - 1ULL));
                    if (m && pos < MB) s_slot[pos] = q;  // a token lists an expert at most once
                    n += __popcll(b);
                }
                n = min(n, MB);
            }
            if (lane == 0) { s_item[0] = e; s_item[1] = n; s_item[2] = tile; }
        }
        __syncthreads();
        const int e = s_item[0], n = s_item[1], tile = s_item[2];
        if (n < 0) break;  // block-uniform
        const bool shared = e < 0;
        const int t0 = tile * TT, nl = min(TT, n - t0);
        // weight rows of this wave into registers
        const int row = rb0 * GU_WROWS + wave * GU_ROWS + (j & 7);
        const uint8_t *mat = j < 8 ? (shared ? A.sh_gate : A.gate) : (shared ? A.sh_up : A.up);
        const uint8_t *wrow = mat + (shared ? 0 : (size_t)e * A.F * A.rb) + (size_t)row * A.rb;
        uint4 c0[NSB], c1[NSB];
#pragma unroll
        for (int sb = 0; sb < NSB; sb++) {
            const uint8_t *p = wrow + sb * 144;
            c0[sb] = qg_ld16(p + 16 + 16 * kq);
            c1[sb] = qg_ld16(p + 16 + 16 * (kq + 4));
        }
        // the wave's 16 x NSB superblock headers, straight into shared memory
        for (int q = 0; q * 64 < 16 * NSB; q++) {
            int h = q * 64 + lane;
            if (h >= 16 * NSB) h = 0;  // lanes past the end copy header 0 into unused space
            const int rr = h / NSB, sb = h - rr * NSB;
            const uint8_t *hm = rr < 8 ? (shared ? A.sh_gate : A.gate) : (shared ? A.sh_up : A.up);
            dma16(hm + (shared ? 0 : (size_t)e * A.F * A.rb) + (size_t)(rb0 * GU_WROWS + wave * GU_ROWS + (rr & 7)) * A.rb + sb * 144,
                  hbuf + (size_t)q * 64 * 16);
        }
        // stage the nl tokens' planes and sum planes by direct global->shared
        // copies (1 KB per wave instruction), in flight with the weight loads
        {
            const int per = 2 * D / 8, pers = 2 * D32 / 8;  // 16-byte chunks per token
            for (int q = wave; q * 64 < nl * per; q += 4) {
                const int c = q * 64 + lane, ti = c / per, off = c - ti * per;
                const int sl = s_slot[t0 + ti], tok = shared ? sl - MS : sl / QG_TOP;
                dma16(A.xp + (size_t)tok * 2 * D + (size_t)off * 8, act + (size_t)q * 64 * 8);
            }
            for (int q = wave; q * 64 < nl * pers; q += 4) {
                int c = q * 64 + lane;
                if (c >= nl * pers) c = 0;  // lanes past the tile copy a valid chunk into unused space
                const int ti = c / pers, off = c - ti * pers;
                const int sl = s_slot[t0 + ti], tok = shared ? sl - MS : sl / QG_TOP;
                dma16(A.xsp + (size_t)tok * 2 * D32 + (size_t)off * 8, acts + (size_t)q * 64 * 8);
            }
        }
        wait_vmem();
        __syncthreads();
        const int ti = min(j >> 1, nl - 1);
        const _Float16 *ap = act + ((size_t)ti * 2 + (j & 1)) * D + kq * 8;
        const _Float16 *sp = acts + ((size_t)ti * 2 + (j & 1)) * D32;
        qg_f4 y = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sb = 0; sb < NSB; sb++) {
            const Q4kHeader h = q4k_header(*(const uint4 *)(hbuf + ((size_t)j * NSB + sb) * 16));
            const int gA = 2 * (kq >> 1), gB = gA + 4;
            qg_f4 p = qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, mm = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int f = 0; f < 4; f++)
                p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(ap + sb * 256 + f * 32),
                                                           q4k_chunk_frag(c0[sb], f, (_Float16)q4k_s(h, gA + (f >> 1))), p, 0, 0, 0);
#pragma unroll
            for (int f = 0; f < 4; f++)
                p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(ap + sb * 256 + (4 + f) * 32),
                                                           q4k_chunk_frag(c1[sb], f, (_Float16)q4k_s(h, gB + (f >> 1))), p, 0, 0, 0);
            qg_half8 mf;
#pragma unroll
            for (int g = 0; g < 8; g++) mf[g] = kq == 0 ? (_Float16)q4k_m(h, g) : (_Float16)0.0f;
            mm = __builtin_amdgcn_mfma_f32_16x16x32_f16(ld_frag(sp + sb * 8), mf, mm, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(h.d, p[i], __builtin_fmaf(-h.dmin, mm[i], y[i]));
        }
        const int fmt = shared ? A.sh_fmt : A.fmt;
        const int pos = plane_pos(fmt, row);
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const float v = y[2 * t2] + y[2 * t2 + 1];  // gate (j < 8) or up (j >= 8)
            const float u = __shfl_xor(v, 8);
            const float m = qg_swiglu(v, u);
            // sum of the wave's 8 rows for this token (lanes j = 0..7)
            float s8 = m;
            s8 += __shfl_xor(s8, 1);
            s8 += __shfl_xor(s8, 2);
            s8 += __shfl_xor(s8, 4);
            const int idx = 2 * kq + t2;
            if (j < 8 && idx < nl) {
                const int sl = s_slot[t0 + idx];
                _Float16 *hp = A.midp + (size_t)sl * 2 * A.F;
                const _Float16 hv = (_Float16)m;
                hp[pos] = hv;
                hp[A.F + pos] = (_Float16)(m - (float)hv);
                if (j == 0) A.msum8[(size_t)sl * (A.F / GU_ROWS) + rb0 * 4 + wave] = s8;
            }
        }
        __syncthreads();  // shared buffers are rewritten by the next item
    }
}

// ---------------- K3: down + router-rank combine + shared + residual ----------------
struct DnArgs {
    int nt, D, F;
    const int *ids; const float *w; const TokRoute *tr;
    qg_prune_stats *stats;               // accumulated by block 0 when pruning is active
    const uint8_t *down, *sh_down; size_t rb, sh_rb;
    const _Float16 *midp; const float *msum8;
    const float *sh_logit; int ld;       // shared-expert gate logit of token t at sh_logit[t*ld]
    float *out;                          // [nt][D] or null
    float *resid;                        // [nt][D] residual updated in place, or null
};

constexpr int DN_ROWS = 8;               // output rows per workgroup
constexpr int DN_WAVES = 8;              // waves per down workgroup
constexpr int DN_LDS = 144 * 1024;       // shared memory for staged weight slabs

// y (hi and lo planes) of one item for one 8-token tile (NB = F/32 blocks).  W: the item's 8
// rows in LDS (row stride rb); MFMA columns j and j+8 both read row j&7.
template <int FMT, int NB>
QG_DEV qg_f4 down_tile(const DnArgs &A, const uint8_t *W, int rb, int j, int kq, int arow_slot, const int *oslot) {
    qg_f4 y = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t *wr = W + (j & 7) * rb;
    const _Float16 *ap = A.midp + ((size_t)arow_slot * 2 + (j & 1)) * A.F;
    if (FMT == QT_Q4_K) {
        for (int sb = 0; sb < A.F / 256; sb++) {
            qg_half8 af[8];
#pragma unroll
            for (int m = 0; m < 8; m++) af[m] = ld_frag(ap + sb * 256 + (m * 4 + kq) * 8);
            const uint8_t *p = wr + sb * 144;
            const Q4kHeader h = q4k_header(*(const uint4 *)p);
            const uint4 ca = *(const uint4 *)(p + 16 + 16 * kq), cb = *(const uint4 *)(p + 16 + 16 * (kq + 4));
            const int gA = 2 * (kq >> 1), gB = gA + 4;
            qg_f4 acc = qg_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int f = 0; f < 4; f++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[f], q4k_chunk_frag(ca, f, (_Float16)q4k_s(h, gA + (f >> 1))), acc, 0, 0, 0);
#pragma unroll
            for (int f = 0; f < 4; f++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[4 + f], q4k_chunk_frag(cb, f, (_Float16)q4k_s(h, gB + (f >> 1))), acc, 0, 0, 0);
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                // group sums of mid: 4 partial sums of 8 rows per 32-group
                const float4 *X = (const float4 *)(A.msum8 + (size_t)oslot[t2] * (A.F / GU_ROWS) + sb * 32);
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
        // all NB activation fragments and all NB block products first, then the
        // block scales: the products do not wait on one another
        qg_half8 af[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) af[b] = ld_frag(ap + b * 32 + kq * 8);
        qg_f4 acc[NB];
        float d[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint16_t *p16 = (const uint16_t *)(wr + 18 * b);  // 2-byte aligned
            d[b] = qg_half_u16(p16[0]);
            const uint32_t q = (uint32_t)p16[1 + 2 * kq] | ((uint32_t)p16[2 + 2 * kq] << 16);
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[b], iq4_frag4(q), qg_f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(d[b], acc[b][i], y[i]);
    }
    return y;
}

// Workgroup = 8 waves owning output rows r0..r0+7 of every selected expert.
// Items (the shared expert first, then each expert at its owning selection)
// are staged in batches: one flat direct global->shared copy of every item's
// 8-row weight slab (contiguous in memory), then the waves take the items
// round robin; a wave loads an item's activation fragments in one batch.
template <int FMT, int SFMT, int NB>
__global__ __launch_bounds__(DN_WAVES * 64) void dec_down_kernel(DnArgs A) {
    extern __shared__ uint4 s_wbuf[];   // slabs of 8 rows x rb bytes, slab stride rbmax*8
    __shared__ int s_first[QG_EXPERTS];
    __shared__ int s_ids[MS];
    __shared__ int s_flag[MB];
    __shared__ int s_items[MS + 1];
    __shared__ int s_nitems;
    __shared__ int s_list[DN_WAVES][MB];
    __shared__ float s_val[ME][DN_ROWS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kq = lane >> 4;
    const int ns = A.nt * QG_TOP, r0 = blockIdx.x * DN_ROWS;
    const bool has_shared = A.sh_down != nullptr;
    for (int i = tid; i < QG_EXPERTS; i += DN_WAVES * 64) s_first[i] = 0x7fffffff;
    for (int i = tid; i < ns; i += DN_WAVES * 64) s_ids[i] = A.ids[i];
    if (tid < A.nt) s_flag[tid] = A.tr->flag[tid];
    __syncthreads();
    for (int i = tid; i < ns; i += DN_WAVES * 64) {
        const int e = s_ids[i];
        if (e >= 0 && e < QG_EXPERTS && s_flag[i / QG_TOP] < 2) atomicMin(&s_first[e], i);
    }
    __syncthreads();
    if (wave == 0) {
        int n = 0;
        if (has_shared) {
            if (lane == 0) s_items[0] = MS;
            n = 1;
        }
        for (int c0 = 0; c0 < ns; c0 += 64) {
            const int q = c0 + lane;
            const int e = q < ns ? s_ids[q] : -1;
            const bool own = e >= 0 && e < QG_EXPERTS && s_flag[q / QG_TOP] < 2 && s_first[e] == q;
            const unsigned long long b = __ballot(own);
            if (own) s_items[n + __popcll(b & ((1ULL << lane) - 1ULL))] = q;
            n += __popcll(b);
        }
        if (lane == 0) s_nitems = n;
    }
    __syncthreads();
    const int nitems = s_nitems;
    const int rbmax = (int)(A.rb > A.sh_rb ? A.rb : A.sh_rb);
    const int slab = DN_ROWS * rbmax;                 // bytes per staged item (multiple of 16)
    const int cps = slab / 16;                        // 16-byte chunks per slab
    const int cap = (DN_LDS - 1024) / slab;           // items per batch (a partial last copy spills < 1 KB)
    uint8_t *wbuf = (uint8_t *)s_wbuf;
    for (int b0 = 0; b0 < nitems; b0 += cap) {
        const int nb = min(cap, nitems - b0);
        // one flat copy of nb slabs; chunks past a shorter slab copy its first chunk
        for (int q = wave; q * 64 < nb * cps; q += DN_WAVES) {
            int c = q * 64 + lane;
            if (c >= nb * cps) c = 0;
            const int bi = c / cps, off = c - bi * cps;
            const int sidx = s_items[b0 + bi];
            const bool shared = sidx == MS;
            const int rb = (int)(shared ? A.sh_rb : A.rb);
            const uint8_t *W = shared ? A.sh_down + (size_t)r0 * rb : A.down + ((size_t)s_ids[sidx] * A.D + r0) * rb;
            dma16(W + 16 * (size_t)(off < DN_ROWS * rb / 16 ? off : 0), wbuf + (size_t)q * 64 * 16);
        }
        wait_vmem();
        __syncthreads();
        for (int bi = wave; bi < nb; bi += DN_WAVES) {
            const int s = s_items[b0 + bi];
            const bool shared = s == MS;
            int n;
            if (shared) {
                n = A.nt;
                if (lane < A.nt) s_list[wave][lane] = MS + lane;
            } else {
                const int e = s_ids[s];
                n = 0;
                for (int c0 = 0; c0 < ns; c0 += 64) {
                    const int q = c0 + lane;
                    const bool m = q < ns && s_ids[q] == e && s_flag[q / QG_TOP] < 2;
                    const unsigned long long b = __ballot(m);
                    const int pos = n + __popcll(b & ((1ULL << lane) - 1ULL));
                    if (m && pos < MB) s_list[wave][pos] = q;  // a token lists an expert at most once
                    n += __popcll(b);
                }
                n = min(n, MB);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int rb = (int)(shared ? A.sh_rb : A.rb);
            const uint8_t *W = wbuf + (size_t)bi * slab;
            for (int c = 0; 8 * c < n; c++) {
                const int arow = s_list[wave][min(8 * c + (j >> 1), n - 1)];
                int oslot[2];
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++) oslot[t2] = s_list[wave][min(8 * c + 2 * kq + t2, n - 1)];
                const qg_f4 y = shared ? down_tile<SFMT, NB>(A, W, rb, j, kq, arow, oslot) : down_tile<FMT, NB>(A, W, rb, j, kq, arow, oslot);
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++) {
                    const int idx = 8 * c + 2 * kq + t2;
                    if (idx < n && j < DN_ROWS) {
                        const int sl = oslot[t2];
                        const float v = y[2 * t2] + y[2 * t2 + 1];
                        s_val[sl][j] = shared ? v : v * A.w[sl];
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        __syncthreads();  // the slabs are overwritten by the next batch
    }
    for (int i = tid; i < A.nt * DN_ROWS; i += DN_WAVES * 64) {
        const int t = i / DN_ROWS, r = i % DN_ROWS;
        float acc = 0.0f;
        if (s_flag[t] < 2) {
#pragma unroll
            for (int k = 0; k < QG_TOP; k++) {
                const int sl = t * QG_TOP + k, e = s_ids[sl];
                acc += (e >= 0 && e < QG_EXPERTS) ? s_val[sl][r] : 0.0f;
            }
            if (has_shared) acc = __builtin_fmaf(s_val[MS + t][r], qg_sig(A.sh_logit[(size_t)t * A.ld]), acc);
        }
        const size_t o = (size_t)t * A.D + r0 + r;
        if (A.out) A.out[o] = acc;
        if (A.resid) A.resid[o] = A.resid[o] + acc;
    }
    if (A.stats && blockIdx.x == 0 && tid == 0) {
        // counters in token order (deterministic, unlike the reference's atomics)
        for (int t = 0; t < A.nt; t++) {
            const int f = A.tr->flag[t];
            if (f == 3) continue;
            A.stats->token_layers += 1;
            A.stats->missing_selections += (uint64_t)A.tr->missing[t];
            if (f == 1) {
                A.stats->skipped_selections += (uint64_t)A.tr->missing[t];
                A.stats->avoided_token_handoffs += 1;
                A.stats->skipped_mass += A.tr->mass[t];
            }
        }
    }
}

// Tokens per gate/up tile (MFMA rows = tokens x {hi, lo}); the staged planes
// of 8 tokens take 8 x 2 x (D + D/32) x 2 bytes of shared memory (68 KB at
// D = 2048; a workgroup may use 160 KB on gfx950).
int gu_tile_tokens(int) { return 8; }

bool fmt_down_ok(int t, int F) { return (t == QT_Q4_K && F % 256 == 0) || t == QT_IQ4_NL; }

bool dec_ok(const qg_moe_layer *L) {
    const int D = L->width, F = L->ff;
    if ((D != 2048 && D != 2560) || (F != 512 && F != 640)) return false;
    if (L->gate_type != QT_Q4_K || L->up_type != QT_Q4_K || !fmt_down_ok(L->down_type, F)) return false;
    if (L->sh_gate && (L->sh_gate_type != QT_Q4_K || L->sh_up_type != QT_Q4_K || !fmt_down_ok(L->sh_down_type, F))) return false;
    return true;
}

template <int NB>
void launch_down(const DnArgs &DA, int fr, int fs, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(DN_WAVES * 64);
    if (fr == QT_IQ4_NL && fs == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_IQ4_NL, QT_IQ4_NL, NB>, grid, block, lds, s, DA);
    else if (fr == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_IQ4_NL, QT_Q4_K, NB>, grid, block, lds, s, DA);
    else if (fs == QT_IQ4_NL) dec_launch(3, dec_down_kernel<QT_Q4_K, QT_IQ4_NL, NB>, grid, block, lds, s, DA);
    else dec_launch(3, dec_down_kernel<QT_Q4_K, QT_Q4_K, NB>, grid, block, lds, s, DA);
}

int dec_forward(float *out, float *resid, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats,
                const float *x, float *xn_out, int norm, int nt, const qg_moe_layer *L, uint8_t *ws) {
    const int D = L->width, F = L->ff;
    const bool sh = L->sh_gate != nullptr;
    const DecLayout lay = dec_layout(D, F);
    hipStream_t s = qg_stream();
    TokRoute *tr = (TokRoute *)(ws + lay.tok);
    float *logits = (float *)(ws + lay.logits);
    _Float16 *xp = (_Float16 *)(ws + lay.xp);
    _Float16 *xsp = (_Float16 *)(ws + lay.xsum);
    const int rows = QG_EXPERTS + (sh ? 1 : 0);
    const int row_pairs = (rows + 1) / 2;
    RouterArgs R{x, nt, D, rows, L->router, sh ? L->sh_gate_inp : nullptr, logits, norm, 1e-6f, xn_out, xp, xsp, row_pairs,
                 L->router_bias};
    dec_launch(0, dec_router_kernel, dim3(row_pairs + 1, (nt + 3) / 4), dim3(256), 0, s, R);
    int rc = hipGetLastError();
    if (rc) return rc;
    const bool inl = nt <= INLINE_MAX;
    if (!inl) {
        RouteArgs RA{nt, logits, rows, L->resident, L->threshold, ids, weights, flags, tr};
        dec_launch(1, dec_route_kernel, dim3((nt + 3) / 4), dim3(256), 0, s, RA);
        if ((rc = hipGetLastError())) return rc;
    }
    _Float16 *midp = (_Float16 *)(ws + lay.midp);
    float *msum8 = (float *)(ws + lay.msum);
    GuArgs G2{nt, D, F, inl ? 1 : 0, logits, rows, L->resident, L->threshold, ids, weights, flags, tr,
              (const uint8_t *)L->gate, (const uint8_t *)L->up, sh ? (const uint8_t *)L->sh_gate : nullptr,
              sh ? (const uint8_t *)L->sh_up : nullptr, qg_row_bytes_host(QT_Q4_K, D), xp, xsp, midp, msum8,
              L->down_type, sh ? L->sh_down_type : L->down_type, gu_tile_tokens(D)};
    // upper bound of the work items: every selection its own expert with one tile
    const int rblocks = F / GU_WROWS;
    const int TT = gu_tile_tokens(D);
    const int items = ((sh ? (nt + TT - 1) / TT : 0) + (nt * QG_TOP < QG_EXPERTS ? nt * QG_TOP : QG_EXPERTS)) * rblocks;
    const int nwg = items < GU_WGS ? items : GU_WGS;
    // planes, the sum planes rounded up to whole 1 KB copies, 4 waves' headers
    // (16 rows x NSB x 16 B, the last copy rounded up to 1 KB)
    const size_t act_lds = (size_t)TT * 2 * D * 2 + (((size_t)TT * 2 * (D / 32) * 2 + 1023) & ~(size_t)1023) +
                           4 * (((size_t)16 * (D / 256) * 16 + 1023) & ~(size_t)1023);
    if (D == 2048) dec_launch(2, dec_gateup_kernel<8>, dim3(nwg), dim3(256), act_lds, s, G2);
    else dec_launch(2, dec_gateup_kernel<10>, dim3(nwg), dim3(256), act_lds, s, G2);
    if ((rc = hipGetLastError())) return rc;
    const size_t rb = qg_row_bytes_host(L->down_type, F), srb = sh ? qg_row_bytes_host(L->sh_down_type, F) : 0;
    DnArgs DA{nt, D, F, ids, weights, tr, (L->resident && stats) ? stats : nullptr,
              (const uint8_t *)L->down, sh ? (const uint8_t *)L->sh_down : nullptr, rb, srb, midp, msum8,
              logits + QG_EXPERTS, rows, out, resid};
    const size_t lds = DN_LDS;
    const int fr = L->down_type, fs = sh ? L->sh_down_type : fr;
    const dim3 grid(D / DN_ROWS);
    if (F == 512) launch_down<16>(DA, fr, fs, grid, lds, s);
    else launch_down<20>(DA, fr, fs, grid, lds, s);
    return hipGetLastError();
}

int validate_layer(const qg_moe_layer *L, int nt) {
    if (!L || nt < 1 || nt > QG_MAX_TOKENS) return hipErrorInvalidValue;
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
    if (!out || !ids || !weights || !x || !workspace || ws_bytes < qg_moe_workspace_bytes(L->width, L->ff, nt))
        return hipErrorInvalidValue;
    if (nt > MB) return qg_prefill_forward(out, nullptr, ids, weights, flags, stats, x, nullptr, 0, nt, L, workspace);
    if (!dec_ok(L)) return qg_generic_forward(out, ids, weights, flags, stats, x, nt, L, workspace, ws_bytes);
    return dec_forward(out, nullptr, ids, weights, flags, stats, x, nullptr, 0, nt, L, (uint8_t *)workspace);
}

int qg_moe_forward_residual(float *h, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, float *xn_out,
                            float *out, int nt, const qg_moe_layer *L, void *workspace, size_t ws_bytes) {
    int rc = validate_layer(L, nt);
    if (rc) return rc;
    if (!h || !ids || !weights || !workspace || ws_bytes < qg_moe_workspace_bytes(L->width, L->ff, nt))
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
