// Device-driven routed-MoE layer for decode batches (1..17 tokens) and the
// reference's fused MTP entry point (gpu.cu:528-551), plus the CSR dispatch.
//
// Layer = 4 kernels, no host round trip (the reference reads routing ids back
// every layer, qwen.c:649):
//   1. router GEMV (F32, reference order; the shared-expert gate row rides
//      along as row 512)                               -> logits [B][513]
//   2. route + coverage/prune + dispatch, one block     -> ids, weights,
//      flags, CSR of (expert -> ascending token) entries
//   3. gate/up + SwiGLU per (active expert, row block)  -> mid [entry][F]
//   4. down per (active expert, row block) -> weighted slot rows; the last
//      block to finish a row block sums its 10 slots per token in router-rank
//      order and adds the sigmoid-gated shared expert   -> out [B][D]
// Each expert's weights are read once per layer however many tokens chose it.
//
// Expert products are fp32 over exactly dequantised weights, factorised per
// Q4_K group: sum_l (d*s*q_l - dmin*m) x_l = d*s*sum_l q_l x_l - dmin*m*sum_l x_l,
// so nibbles convert straight to float and each group costs one scale step.
#include "qg_internal.h"
#include <string.h>

namespace {

constexpr int MAXB = QG_MAX_DECODE;       // 17 tokens (anchor + 16 drafts, qwen.h:10)
constexpr int MAXS = MAXB * QG_TOP;       // 170 routed selections
constexpr int ROWS_DOWN = 32;             // output rows per down block
constexpr int RD_THREADS = 1024;          // route/dispatch block

struct Disp {
    int n_active, n_entries, status, has_shared;
    int4 act[QG_EXPERTS];                 // active expert a: (expert id, first entry, entries, 0)
    int ent_token[MAXS];
    int ent_slot[MAXS];
    int slot_ent[MAXS];
    int tok_flag[MAXB];
};

struct WsLayout { size_t logits, disp, mid, slots, xh, xs, midh, mids, total; };
WsLayout ws_layout(int D, int F) {
    WsLayout L;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += (n + 255) & ~(size_t)255; return o; };
    L.logits = take((size_t)MAXB * (QG_EXPERTS + 1) * 4);
    L.disp = take(sizeof(Disp));
    L.mid = take((size_t)(MAXS + MAXB) * F * 4);
    L.slots = take((size_t)(MAXS + MAXB) * D * 4);
    L.xh = take((size_t)MAXB * 2 * D * 2);
    L.xs = take((size_t)MAXB * (D / 32) * 4);
    L.midh = take((size_t)(MAXS + MAXB) * 2 * F * 2);
    L.mids = take((size_t)(MAXS + MAXB) * (F / 32) * 4);
    L.total = off;
    return L;
}

// Optional per-phase timing (benchmark support): events recorded on the
// launch stream after each kernel of qg_moe_forward.
thread_local void *tl_phase_ev[8] = {nullptr};
thread_local int tl_phase_n = 0;
void phase_mark(int i, hipStream_t s) {
    if (i < tl_phase_n && tl_phase_ev[i]) (void)hipEventRecord((hipEvent_t)tl_phase_ev[i], s);
}

QG_DEV void route_token(int *s_ids, float *s_w, const float *s, int t, int lane, float *lds_v, int *lds_i) {
    qg_route_wave(s_ids + t * QG_TOP, s_w + t * QG_TOP, s, lane, lds_v, lds_i);
}

QG_DEV void act_planes_group(const float *x, int K, int r, int g, _Float16 *xh, float *xs);

// logits[t][e] += bias[e] for the 512 expert logits of token blockIdx.x.
__global__ __launch_bounds__(QG_EXPERTS) void logit_bias_kernel(float *logits, int ld, const float *bias) {
    logits[(size_t)blockIdx.x * ld + threadIdx.x] += bias[threadIdx.x];
}

// Inclusive scan of one int per thread over a RD_THREADS-thread block.
QG_DEV int block_scan(int v, int *s_tmp) {
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

// CSR dispatch of the ids in LDS, every step parallel (RD_THREADS threads):
// selection i is eligible if 0<=id<512 and its token's flag is 0 or 1; its
// rank within its expert is the number of earlier eligible selections of the
// same expert, so entries of an expert come in ascending (token, rank) order.
QG_DEV void build_dispatch(const int *s_ids, const int *s_flag, int nt, Disp *ds, int *s_cnt, int *s_rank, int *s_tmp) {
    const int tid = threadIdx.x, n = nt * QG_TOP, lane = tid & 63;
    if (tid < QG_EXPERTS) s_cnt[tid] = 0;
    __syncthreads();
    // One wave ranks 64 selections at a time: the lanes holding the same
    // expert are found with nine ballots (one per id bit); a selection's rank
    // is the count from earlier chunks plus its same-expert lanes below it.
    if (tid < 64) {
        for (int c0 = 0; c0 < n; c0 += 64) {
            const int i = c0 + lane;
            int e = 0;
            bool el = false;
            if (i < n) { e = s_ids[i]; el = e >= 0 && e < QG_EXPERTS && s_flag[i / QG_TOP] < 2; }
            unsigned long long peers = __ballot(el);
#pragma unroll
            for (int b = 0; b < 9; b++) {
                const bool bit = (e >> b) & 1;
                const unsigned long long bal = __ballot(el && bit);
                peers &= bit ? bal : ~bal;
            }
            const int base = el ? s_cnt[e] : 0;
            if (i < n) s_rank[i] = el ? base + __popcll(peers & ((1ULL << lane) - 1ULL)) : -1;
            if (el && lane == 63 - __builtin_clzll(peers)) s_cnt[e] = base + __popcll(peers);
        }
    }
    __syncthreads();
    const int c = tid < QG_EXPERTS ? s_cnt[tid] : 0;
    const int local = ((c > 0) << 16) | c;
    const int incl = block_scan(local, s_tmp);
    const int excl = incl - local;
    if (c) {
        ds->act[excl >> 16] = make_int4(tid, excl & 0xffff, c, 0);
        s_cnt[tid] = excl & 0xffff;  // becomes the expert's first entry
    }
    if (tid == RD_THREADS - 1) { ds->n_active = incl >> 16; ds->n_entries = incl & 0xffff; }
    __syncthreads();
    if (tid < MAXS) {
        int ent = -1;
        if (tid < n && s_rank[tid] >= 0) {
            ent = s_cnt[s_ids[tid]] + s_rank[tid];
            ds->ent_token[ent] = tid / QG_TOP;
            ds->ent_slot[ent] = tid;
        }
        ds->slot_ent[tid] = ent;
    }
}

// ---------------- kernel 2: route + coverage + dispatch (one block) ----------------
__global__ __launch_bounds__(RD_THREADS) void route_dispatch_kernel(int *ids_out, float *w_out, uint8_t *flags_out,
                                                                    qg_prune_stats *stats, const float *logits, int ld, int nt,
                                                                    const uint8_t *resident, double thr, Disp *ds, int has_shared,
                                                                    const float *x, int D, _Float16 *xh, float *xs) {
    __shared__ int s_ids[MAXS], s_rank[MAXS], s_cnt[QG_EXPERTS];
    __shared__ float s_w[MAXS];
    __shared__ int s_flag[MAXB], s_missing[MAXB];
    __shared__ double s_mass[MAXB];
    __shared__ int s_tmp[RD_THREADS / 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (xh)  // fp16 hi/lo planes of the inputs for the matrix-core expert kernels
        for (int i = tid; i < nt * (D / 32); i += RD_THREADS) act_planes_group(x, D, i / (D / 32), i % (D / 32), xh, xs);
    __shared__ __align__(16) float s_rv[RD_THREADS / 64][QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_ri[RD_THREADS / 64][QG_ROUTE_SCRATCH];
    for (int t = wave; t < nt; t += RD_THREADS / 64) route_token(s_ids, s_w, logits + (size_t)t * ld, t, lane, s_rv[wave], s_ri[wave]);
    __syncthreads();
    // Coverage (gpu.cu:470-478): mass of non-resident selections in rank order.
    if (tid < nt) {
        const int t = tid;
        int missing = 0, bad = 0;
        double mass = 0;
        for (int k = 0; k < QG_TOP; k++) {
            const int e = s_ids[t * QG_TOP + k];
            if (e < 0 || e >= QG_EXPERTS) { bad = 1; break; }
            if (resident && !resident[e]) { missing++; mass += (double)s_w[t * QG_TOP + k]; }
        }
        const int flag = bad ? 3 : !missing ? 0 : (thr > 0 && mass < thr) ? 1 : 2;
        if (flag == 1)
            for (int k = 0; k < QG_TOP; k++) {
                const int e = s_ids[t * QG_TOP + k];
                if (!resident[e]) { s_ids[t * QG_TOP + k] = -e - 2; s_w[t * QG_TOP + k] = 0.0f; }
            }
        s_flag[t] = flag;
        s_missing[t] = missing;
        s_mass[t] = mass;
        ds->tok_flag[t] = flag;
        if (flags_out) flags_out[t] = (uint8_t)flag;
    }
    __syncthreads();
    // Counters in token order (deterministic, unlike the reference's atomics).
    if (tid == 0) {
        int bad = 0;
        for (int t = 0; t < nt; t++) {
            if (s_flag[t] == 3) { bad = 1; continue; }
            if (resident && stats) {
                stats->token_layers += 1;
                stats->missing_selections += (uint64_t)s_missing[t];
                if (s_flag[t] == 1) {
                    stats->skipped_selections += (uint64_t)s_missing[t];
                    stats->avoided_token_handoffs += 1;
                    stats->skipped_mass += s_mass[t];
                }
            }
        }
        ds->status = bad;
        ds->has_shared = has_shared;
    }
    for (int i = tid; i < nt * QG_TOP; i += RD_THREADS) { ids_out[i] = s_ids[i]; w_out[i] = s_w[i]; }
    build_dispatch(s_ids, s_flag, nt, ds, s_cnt, s_rank, s_tmp);
}

// ---------------- dispatch from given ids (qg_mtp_moe front end) ----------------
// Every selection with 0<=id<512 dispatches (duplicates included, as the
// reference computes each (token, rank) independently); invalid slots get
// NaN in mid and slots (gpu.cu:531,539).
__global__ __launch_bounds__(RD_THREADS) void dispatch_ids_kernel(const int *ids, int nt, Disp *ds, float *mid_slot,
                                                                  float *slots_out, int D, int F, const float *x, _Float16 *xh,
                                                                  float *xs) {
    __shared__ int s_ids[MAXS], s_rank[MAXS], s_cnt[QG_EXPERTS];
    __shared__ int s_flag[MAXB];
    __shared__ int s_tmp[RD_THREADS / 64];
    const int tid = threadIdx.x;
    if (xh)
        for (int i = tid; i < nt * (D / 32); i += RD_THREADS) act_planes_group(x, D, i / (D / 32), i % (D / 32), xh, xs);
    if (tid < nt * QG_TOP) s_ids[tid] = ids[tid];
    if (tid < MAXB) s_flag[tid] = 0;
    if (tid == 0) { ds->status = 0; ds->has_shared = 0; }
    if (tid < nt) ds->tok_flag[tid] = 0;
    __syncthreads();
    build_dispatch(s_ids, s_flag, nt, ds, s_cnt, s_rank, s_tmp);
    const float nan = __builtin_nanf("");
    for (int s = 0; s < nt * QG_TOP; s++) {
        const int e = s_ids[s];
        if (e >= 0 && e < QG_EXPERTS) continue;
        for (int r = tid; r < F; r += RD_THREADS) mid_slot[(size_t)s * F + r] = nan;
        for (int d = tid; d < D; d += RD_THREADS) slots_out[(size_t)s * D + d] = nan;
    }
}

// ---------------- Q4_K chunk arithmetic ----------------
// Chunk q (0..7) of a superblock: qs bytes 16q..16q+15 hold elements
// l = 16(q&1)+0..15 of group ga = 2(q>>1) (low nibbles) and gb = ga+1 (high
// nibbles) (layout of cpu.c:56-64).  Scales decoded four bytes at a time.
struct Q4kScale { float dsa, dma, dsb, dmb; };
QG_DEV Q4kScale q4k_scale(uint4 hd, int q) {
    const float d = qg_half_u16(hd.x & 0xffffu), dmin = qg_half_u16(hd.x >> 16);
    const int p = q >> 1;
    uint32_t S, M;
    if (p < 2) { S = hd.y & 0x3F3F3F3Fu; M = hd.z & 0x3F3F3F3Fu; }
    else {
        S = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        M = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    }
    const int sh = (p & 1) * 16;
    Q4kScale r;
    r.dsa = d * (float)((S >> sh) & 0xffu);
    r.dsb = d * (float)((S >> (sh + 8)) & 0xffu);
    r.dma = dmin * (float)((M >> sh) & 0xffu);
    r.dmb = dmin * (float)((M >> (sh + 8)) & 0xffu);
    return r;
}

// x slice of one lane for one Q4_K chunk: 16 values of group ga and 16 of gb,
// plus their sums (for the per-group minimum term).
struct Q4kSlice { float a[16], b[16], sa, sb; };

QG_DEV void q4k_load_slice(Q4kSlice &s, const float *xrow, int koff, bool valid) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 16; i++) { s.a[i] = 0.0f; s.b[i] = 0.0f; }
        s.sa = s.sb = 0.0f;
        return;
    }
    const float4 *pa = (const float4 *)(xrow + koff), *pb = (const float4 *)(xrow + koff + 32);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 va = pa[i], vb = pb[i];
        s.a[4 * i] = va.x; s.a[4 * i + 1] = va.y; s.a[4 * i + 2] = va.z; s.a[4 * i + 3] = va.w;
        s.b[4 * i] = vb.x; s.b[4 * i + 1] = vb.y; s.b[4 * i + 2] = vb.z; s.b[4 * i + 3] = vb.w;
    }
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) { sa += s.a[i]; sb += s.b[i]; }
    s.sa = sa;
    s.sb = sb;
}

// Nibbles of a chunk as floats: qa = group ga (low nibbles), qb = group gb.
struct Q4kVals { float qa[16], qb[16]; };
QG_DEV void q4k_unpack(Q4kVals &v, uint4 qv) {
    const uint32_t w4[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = w4[i] & 0x0F0F0F0Fu, hi = (w4[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            v.qa[4 * i + b] = (float)((lo >> (8 * b)) & 0xffu);
            v.qb[4 * i + b] = (float)((hi >> (8 * b)) & 0xffu);
        }
    }
}
// d*s_a*sum(q x) - dmin*m_a*sum(x) + (same for gb), added to p.
QG_DEV float q4k_dot(float p, const Q4kVals &v, const Q4kScale &sc, const Q4kSlice &x) {
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) { sa = __builtin_fmaf(v.qa[i], x.a[i], sa); sb = __builtin_fmaf(v.qb[i], x.b[i], sb); }
    p = __builtin_fmaf(sc.dsa, sa, p);
    p = __builtin_fmaf(-sc.dma, x.sa, p);
    p = __builtin_fmaf(sc.dsb, sb, p);
    p = __builtin_fmaf(-sc.dmb, x.sb, p);
    return p;
}

// koff of chunk `ch` (16-byte qs chunk index along a row of Q4_K superblocks)
QG_DEV int q4k_koff(int ch) { const int sb = ch >> 3, q = ch & 7; return sb * 256 + (q >> 1) * 64 + (q & 1) * 16; }
QG_DEV size_t q4k_qoff(int ch) { const int sb = ch >> 3, q = ch & 7; return (size_t)sb * 144 + 16 + 16 * q; }
QG_DEV size_t q4k_hoff(int ch) { return (size_t)(ch >> 3) * 144; }

template <int W>
QG_DEV float group_sum(float v) {
#pragma unroll
    for (int d = W / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, W);
    return v;
}

// Eight per-lane partial sums -> the full wave sum of value r(lane) in every
// lane, r = 4*bit5 + 2*bit4 + bit3 of the lane id.  A transposed butterfly:
// 10 shuffles instead of 48.
QG_DEV float reduce8(float (&v)[8], int lane) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bool up = lane & 32;
        const float send = up ? v[i] : v[i + 4], keep = up ? v[i + 4] : v[i];
        v[i] = keep + __shfl_xor(send, 32);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bool up = lane & 16;
        const float send = up ? v[i] : v[i + 2], keep = up ? v[i + 2] : v[i];
        v[i] = keep + __shfl_xor(send, 16);
    }
    {
        const bool up = lane & 8;
        const float send = up ? v[0] : v[1], keep = up ? v[1] : v[0];
        v[0] = keep + __shfl_xor(send, 8);
    }
    float r = v[0];
    r += __shfl_xor(r, 4);
    r += __shfl_xor(r, 2);
    r += __shfl_xor(r, 1);
    return r;
}

// ---------------- kernel 3: gate/up + SwiGLU (Q4_K, D = 2048*CPL) ----------------
struct GateUpArgs {
    const float *x;
    int nt, D, F, maxa;
    const uint8_t *gate, *up, *sh_gate, *sh_up;
    size_t rb;  // row bytes of a D-column Q4_K row
    const Disp *ds;
    float *mid;       // [MAXS+MAXB][F], entry-indexed; shared rows at MAXS+t
    float *mid_slot;  // slot layout [(t*10+k)][F] or null
};

// Block = 4 waves x 4 (gate row, up row) pairs = 16 rows of the expert.
// All 16 row loads are issued before any arithmetic and stay in registers
// while the expert's tokens are processed TC at a time.
template <int TC, int CPL>
__global__ __launch_bounds__(256) void gateup_q4k_kernel(GateUpArgs A) {
    constexpr int RPW = 4;
    const int a = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool shared = A.sh_gate && a == A.maxa;
    int n, ent0 = 0;
    const uint8_t *G, *U;
    if (shared) { n = A.nt; G = A.sh_gate; U = A.sh_up; }
    else {
        if (a >= A.ds->n_active) return;
        const int4 info = A.ds->act[a];
        ent0 = info.y;
        n = info.z;
        G = A.gate + (size_t)info.x * A.F * A.rb;
        U = A.up + (size_t)info.x * A.F * A.rb;
    }
    const int row0 = (blockIdx.y * 4 + wave) * RPW;
    uint4 qg[RPW][CPL], hg[RPW][CPL], qu[RPW][CPL], hu[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const size_t rowoff = (size_t)(row0 + r) * A.rb;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = lane + 64 * c;
            qg[r][c] = qg_ld16(G + rowoff + q4k_qoff(ch)); hg[r][c] = qg_ld16(G + rowoff + q4k_hoff(ch));
            qu[r][c] = qg_ld16(U + rowoff + q4k_qoff(ch)); hu[r][c] = qg_ld16(U + rowoff + q4k_hoff(ch));
        }
    }
    for (int t0 = 0; t0 < n; t0 += TC) {
        Q4kSlice xs[TC][CPL];
#pragma unroll
        for (int i = 0; i < TC; i++) {
            const bool valid = t0 + i < n;
            const int tok = !valid ? 0 : shared ? t0 + i : A.nt == 1 ? 0 : A.ds->ent_token[ent0 + t0 + i];
#pragma unroll
            for (int c = 0; c < CPL; c++) q4k_load_slice(xs[i][c], A.x + (size_t)tok * A.D, q4k_koff(lane + 64 * c), valid);
        }
        float v[TC][2 * RPW];
#pragma unroll
        for (int i = 0; i < TC; i++)
#pragma unroll
            for (int r = 0; r < 2 * RPW; r++) v[i][r] = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const int q = (lane + 64 * c) & 7;
                Q4kVals vals;
                q4k_unpack(vals, qg[r][c]);
                const Q4kScale sg = q4k_scale(hg[r][c], q);
#pragma unroll
                for (int i = 0; i < TC; i++) v[i][r] = q4k_dot(v[i][r], vals, sg, xs[i][c]);
                q4k_unpack(vals, qu[r][c]);
                const Q4kScale su = q4k_scale(hu[r][c], q);
#pragma unroll
                for (int i = 0; i < TC; i++) v[i][RPW + r] = q4k_dot(v[i][RPW + r], vals, su, xs[i][c]);
            }
        }
#pragma unroll
        for (int i = 0; i < TC; i++) {
            const float s = reduce8(v[i], lane);          // gate (bit5=0) or up (bit5=1) row (lane>>3)&3
            const float u = __shfl_xor(s, 32);
            if ((lane & 39) == 0 && t0 + i < n) {
                const int row = row0 + ((lane >> 3) & 3);
                const float m = qg_swiglu(s, u);
                if (shared) A.mid[(size_t)(MAXS + t0 + i) * A.F + row] = m;
                else {
                    const int ent = ent0 + t0 + i;
                    A.mid[(size_t)ent * A.F + row] = m;
                    if (A.mid_slot) A.mid_slot[(size_t)A.ds->ent_slot[ent] * A.F + row] = m;
                }
            }
        }
    }
}

// ---------------- kernel 4: down -> weighted slot rows ----------------
struct DownArgs {
    int nt, D, F, maxa;
    const uint8_t *down, *sh_down;
    size_t rb, sh_rb;          // row bytes of an F-column row (routed, shared)
    const Disp *ds;
    const float *mid;
    const float *route_w;      // [nt][10] after pruning
    float *slots;              // workspace [MAXS+MAXB][D] (entry-indexed)
    float *slots_out;          // slot mode: caller's [(t*10+k)][D], or null
};

// IQ4_NL: 8 lanes per 512-column row, a lane owns a pair of 18-byte blocks
// (64 columns).  The table is shifted by +128 to unsigned bytes so v_perm can
// look it up and cvt_f32_ubyte convert; the shift is removed with the block's
// x sum.

struct Iq4Slice { float v[64]; float s0, s1; };

QG_DEV void iq4_load_slice(Iq4Slice &s, const float *xrow, int koff) {
    const float4 *p = (const float4 *)(xrow + koff);
#pragma unroll
    for (int i = 0; i < 16; i++) { const float4 f = p[i]; s.v[4*i] = f.x; s.v[4*i+1] = f.y; s.v[4*i+2] = f.z; s.v[4*i+3] = f.w; }
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) { a += s.v[i]; b += s.v[32 + i]; }
    s.s0 = a;
    s.s1 = b;
}

// 36 bytes at p (4-byte aligned): block0 = d0 | qs0[16], block1 = d1 | qs1[16].
struct Iq4Raw { uint32_t w[9]; };
QG_DEV Iq4Raw iq4_load(const uint8_t *p) {
    Iq4Raw r;
    const uint32_t *q = (const uint32_t *)p;
#pragma unroll
    for (int i = 0; i < 9; i++) r.w[i] = q[i];
    return r;
}
struct Iq4Vals { float val[64]; float d0, d1; };
QG_DEV void iq4_unpack(Iq4Vals &v, const Iq4Raw &r) {
    v.d0 = qg_half_u16(r.w[0] & 0xffffu);
    v.d1 = qg_half_u16(r.w[4] >> 16);
    uint32_t qs[8];
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
#pragma unroll
    for (int i = 0; i < 4; i++) qs[4 + i] = r.w[5 + i];
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = qs[blk * 4 + i];
            const uint32_t lo = iq4_lookup(w & 0x0F0F0F0Fu), hi = iq4_lookup((w >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                v.val[blk * 32 + 4 * i + b] = (float)((lo >> (8 * b)) & 0xffu);
                v.val[blk * 32 + 16 + 4 * i + b] = (float)((hi >> (8 * b)) & 0xffu);
            }
        }
    }
}
QG_DEV float iq4_dot(const Iq4Vals &v, const Iq4Slice &x) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) { s0 = __builtin_fmaf(v.val[i], x.v[i], s0); s1 = __builtin_fmaf(v.val[32 + i], x.v[32 + i], s1); }
    s0 = __builtin_fmaf(-128.0f, x.s0, s0);
    s1 = __builtin_fmaf(-128.0f, x.s1, s1);
    return __builtin_fmaf(v.d0, s0, v.d1 * s1);
}

#include "qg_mfma.hip"

QG_DEV void down_store(const DownArgs &A, bool shared, int mrow, int row, float y) {
    if (shared) { A.slots[(size_t)mrow * A.D + row] = y; return; }
    const int slot = A.ds->ent_slot[mrow];
    const float v = y * A.route_w[slot];
    if (A.slots_out) A.slots_out[(size_t)slot * A.D + row] = v;
    else A.slots[(size_t)mrow * A.D + row] = v;
}

// Rows [rowbase, rowbase+32) of one expert (or the shared expert) for all of
// its tokens.  Weights are loaded and unpacked once, then reused per token.
template <int FMT>
QG_DEV void down_rows(const DownArgs &A, const uint8_t *W, size_t rb, int n, int ent0, bool shared, int rowbase) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (FMT == QT_IQ4_NL) {
        const int c = lane & 7, row = rowbase + wave * 8 + (lane >> 3);
        Iq4Vals vals;
        iq4_unpack(vals, iq4_load(W + (size_t)row * rb + 36 * c));
        for (int t = 0; t < n; t++) {
            const int mrow = shared ? MAXS + t : ent0 + t;
            Iq4Slice xs;
            iq4_load_slice(xs, A.mid + (size_t)mrow * A.F, 64 * c);
            const float y = group_sum<8>(iq4_dot(vals, xs));
            if (c == 0) down_store(A, shared, mrow, row, y);
        }
    } else {
        const int c = lane & 15;
        const int rowA = rowbase + wave * 8 + (lane >> 4), rowB = rowA + 4;
        const uint8_t *pa = W + (size_t)rowA * rb, *pb = W + (size_t)rowB * rb;
        const uint4 qa = qg_ld16(pa + q4k_qoff(c)), ha = qg_ld16(pa + q4k_hoff(c));
        const uint4 qb = qg_ld16(pb + q4k_qoff(c)), hb = qg_ld16(pb + q4k_hoff(c));
        Q4kVals va, vb;
        q4k_unpack(va, qa);
        q4k_unpack(vb, qb);
        const Q4kScale sa = q4k_scale(ha, c & 7), sb = q4k_scale(hb, c & 7);
        for (int t = 0; t < n; t++) {
            const int mrow = shared ? MAXS + t : ent0 + t;
            Q4kSlice xs;
            q4k_load_slice(xs, A.mid + (size_t)mrow * A.F, q4k_koff(c), true);
            const float ya = group_sum<16>(q4k_dot(0.0f, va, sa, xs));
            const float yb = group_sum<16>(q4k_dot(0.0f, vb, sb, xs));
            if (c == 0) { down_store(A, shared, mrow, rowA, ya); down_store(A, shared, mrow, rowB, yb); }
        }
    }
}

template <int FR, int FS>
__global__ __launch_bounds__(256) void down_kernel(DownArgs A) {
    const int a = blockIdx.x, rowbase = blockIdx.y * ROWS_DOWN;
    if (A.sh_down && a == A.maxa) { down_rows<FS>(A, A.sh_down, A.sh_rb, A.nt, 0, true, rowbase); return; }
    if (a >= A.ds->n_active) return;
    const int4 info = A.ds->act[a];
    down_rows<FR>(A, A.down + (size_t)info.x * A.D * A.rb, A.rb, info.z, info.y, false, rowbase);
}

// ---------------- kernel 5: router-rank combine + shared expert ----------------
// out[t,d] = sum over k=0..9 of the weighted slots from 0.0f in router-rank
// order (gpu.cu:521-527, cpu.c:227-230; pruned ranks add +0), then the
// sigmoid-gated shared expert added with one fma (gpu.cu:552).  Handoff
// tokens (flag 2) get the shared part only, invalid ones (flag 3) a zero row.
__global__ __launch_bounds__(256) void combine_kernel(float *out, const float *slots, const Disp *ds, const float *sh_logit,
                                                      int ld, int nt, int D) {
    const int i = blockIdx.x * 256 + threadIdx.x, q = D / 4;
    if (i >= nt * q) return;
    const int t = i / q, d4 = (i % q) * 4;
    int se[QG_TOP];
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) se[k] = ds->slot_ent[t * QG_TOP + k];  // issued together
    const int flag = ds->tok_flag[t], has_shared = ds->has_shared;
    const float g = has_shared ? qg_sig(sh_logit[(size_t)t * ld]) : 0.0f;
    float4 v[QG_TOP];
#pragma unroll
    for (int k = 0; k < QG_TOP; k++)
        v[k] = *(const float4 *)(slots + (size_t)(se[k] >= 0 ? se[k] : 0) * D + d4);
    const float4 s = *(const float4 *)(slots + (size_t)(MAXS + t) * D + d4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (flag < 2) {
#pragma unroll
        for (int k = 0; k < QG_TOP; k++) {
            const bool ok = se[k] >= 0;
            acc.x += ok ? v[k].x : 0.0f; acc.y += ok ? v[k].y : 0.0f; acc.z += ok ? v[k].z : 0.0f; acc.w += ok ? v[k].w : 0.0f;
        }
    }
    if (has_shared && flag != 3) {
        acc.x = __builtin_fmaf(s.x, g, acc.x); acc.y = __builtin_fmaf(s.y, g, acc.y);
        acc.z = __builtin_fmaf(s.z, g, acc.z); acc.w = __builtin_fmaf(s.w, g, acc.w);
    }
    *(float4 *)(out + (size_t)t * D + d4) = acc;
}

// ---------------- generic fallback (any format, any width) ----------------
// Exact reference order per (row, token), one 32-lane half per row: the same
// arithmetic as cpu.c's dot_group for every format.
QG_DEV float exact_dot(const uint8_t *row, int type, int cols, const float *x, int j) {
    float acc = 0.0f;
    for (int k = 0; k < cols; k += 32) acc = __builtin_fmaf(qg_weight_at(row, type, k + j), x[k + j], acc);
    return qg_tree32(acc);
}

struct GenericArgs {
    const float *x;
    int nt, D, F, maxa;
    const uint8_t *gate, *up, *sh_gate, *sh_up; int gt, ut, sgt, sut; size_t grb, urb, sgrb, surb;
    const Disp *ds;
    float *mid, *mid_slot;
};

__global__ __launch_bounds__(64) void gateup_generic_kernel(GenericArgs A) {
    const int a = blockIdx.x, half = threadIdx.x >> 5, j = threadIdx.x & 31, row = blockIdx.y * 2 + half;
    if (row >= A.F) return;
    const bool shared = A.sh_gate && a == A.maxa;
    int n, ent0 = 0;
    const uint8_t *G, *U;
    int gt, ut;
    size_t grb, urb;
    if (shared) { n = A.nt; G = A.sh_gate; U = A.sh_up; gt = A.sgt; ut = A.sut; grb = A.sgrb; urb = A.surb; }
    else {
        if (a >= A.ds->n_active) return;
        const int4 info = A.ds->act[a];
        ent0 = info.y;
        n = info.z;
        gt = A.gt; ut = A.ut; grb = A.grb; urb = A.urb;
        G = A.gate + (size_t)info.x * A.F * grb;
        U = A.up + (size_t)info.x * A.F * urb;
    }
    for (int i = 0; i < n; i++) {
        const int tok = shared ? i : A.ds->ent_token[ent0 + i];
        const float *xr = A.x + (size_t)tok * A.D;
        const float g = exact_dot(G + (size_t)row * grb, gt, A.D, xr, j), u = exact_dot(U + (size_t)row * urb, ut, A.D, xr, j);
        if (j == 0) {
            const float m = qg_swiglu(g, u);
            if (shared) A.mid[(size_t)(MAXS + i) * A.F + row] = m;
            else {
                A.mid[(size_t)(ent0 + i) * A.F + row] = m;
                if (A.mid_slot) A.mid_slot[(size_t)A.ds->ent_slot[ent0 + i] * A.F + row] = m;
            }
        }
    }
}

struct GenericDownArgs { DownArgs d; int dt, sdt; };

__global__ __launch_bounds__(64) void down_generic_kernel(GenericDownArgs G) {
    const DownArgs &A = G.d;
    const int a = blockIdx.x, half = threadIdx.x >> 5, j = threadIdx.x & 31, row = blockIdx.y * 2 + half;
    if (row >= A.D) return;
    if (A.sh_down && a == A.maxa) {
        for (int t = 0; t < A.nt; t++) {
            const float y = exact_dot(A.sh_down + (size_t)row * A.sh_rb, G.sdt, A.F, A.mid + (size_t)(MAXS + t) * A.F, j);
            if (j == 0) A.slots[(size_t)(MAXS + t) * A.D + row] = y;
        }
        return;
    }
    if (a >= A.ds->n_active) return;
    const int4 info = A.ds->act[a];
    const uint8_t *W = A.down + (size_t)info.x * A.D * A.rb;
    for (int i = 0; i < info.z; i++) {
        const int ent = info.y + i;
        const float y = exact_dot(W + (size_t)row * A.rb, G.dt, A.F, A.mid + (size_t)ent * A.F, j);
        if (j == 0) down_store(A, false, ent, row, y);
    }
}

// ---------------- expert-phase launcher shared by forward and mtp_moe ----------------
struct ExpertPhase {
    const float *x; int nt, D, F;
    _Float16 *xh; float *xs; _Float16 *midh; float *mids;
    const uint8_t *gate, *up, *down; int gt, ut, dt;
    const uint8_t *sh_gate, *sh_up, *sh_down; int sgt, sut, sdt;
    Disp *ds; float *mid, *mid_slot, *slots, *slots_out; const float *route_w;
    const float *sh_logit; int ld; float *out;
};

bool mfma_ok(const ExpertPhase &P) {
    auto dn_ok = [&](int t) { return (t == QT_IQ4_NL && P.F % 64 == 0) || (t == QT_Q4_K && P.F % 256 == 0); };
    return P.xh && P.gt == QT_Q4_K && P.ut == QT_Q4_K && P.D % 256 == 0 && P.D % 64 == 0 && P.F % 64 == 0 && dn_ok(P.dt) &&
           (!P.sh_gate || (P.sgt == QT_Q4_K && P.sut == QT_Q4_K && dn_ok(P.sdt)));
}

int launch_experts(const ExpertPhase &P, hipStream_t s) {
    const int maxa = P.nt * QG_TOP < QG_EXPERTS ? P.nt * QG_TOP : QG_EXPERTS;
    const int gx = maxa + (P.sh_gate ? 1 : 0);
    if (mfma_ok(P)) {
        MfmaGU G{P.xh, P.xs, P.nt, P.D, P.F, maxa, P.gate, P.up, P.sh_gate, P.sh_up, qg_row_bytes_host(QT_Q4_K, P.D), P.ds,
                 nullptr, P.mid_slot, P.midh, P.mids, P.ds->ent_token, MAXS};
        gateup_mfma_kernel<3><<<dim3(gx, P.F / 64), 256, 0, s>>>(G);
        int rc = hipGetLastError();
        if (rc) return rc;
        phase_mark(3, s);
        MfmaDown Dn{P.nt, P.D, P.F, maxa, P.down, P.sh_down, qg_row_bytes_host(P.dt, P.F),
                    P.sh_down ? qg_row_bytes_host(P.sdt, P.F) : 0, P.ds, P.midh, P.mids, P.route_w, P.slots, P.slots_out, MAXS};
        const int fs = P.sh_down ? P.sdt : P.dt;
        const dim3 grid(gx, P.D / 64);
        if (P.dt == QT_IQ4_NL && fs == QT_IQ4_NL) down_mfma_kernel<QT_IQ4_NL, QT_IQ4_NL, 3><<<grid, 256, 0, s>>>(Dn);
        else if (P.dt == QT_IQ4_NL) down_mfma_kernel<QT_IQ4_NL, QT_Q4_K, 3><<<grid, 256, 0, s>>>(Dn);
        else if (fs == QT_IQ4_NL) down_mfma_kernel<QT_Q4_K, QT_IQ4_NL, 3><<<grid, 256, 0, s>>>(Dn);
        else down_mfma_kernel<QT_Q4_K, QT_Q4_K, 3><<<grid, 256, 0, s>>>(Dn);
        if ((rc = hipGetLastError())) return rc;
        phase_mark(4, s);
        if (P.out) {
            const int quads = P.nt * P.D / 4;
            combine_kernel<<<(quads + 255) / 256, 256, 0, s>>>(P.out, P.slots, P.ds, P.sh_logit, P.ld, P.nt, P.D);
            rc = hipGetLastError();
        }
        phase_mark(5, s);
        return rc;
    }
    const bool fast_gu = P.gt == QT_Q4_K && P.ut == QT_Q4_K && (!P.sh_gate || (P.sgt == QT_Q4_K && P.sut == QT_Q4_K)) &&
                         P.D == 2048 && P.F % 16 == 0;
    const bool fast_dn = (P.dt == QT_IQ4_NL || P.dt == QT_Q4_K) && (!P.sh_down || P.sdt == QT_IQ4_NL || P.sdt == QT_Q4_K) &&
                         P.F == 512 && P.D % ROWS_DOWN == 0;
    if (fast_gu) {
        GateUpArgs A{P.x, P.nt, P.D, P.F, maxa, P.gate, P.up, P.sh_gate, P.sh_up, qg_row_bytes_host(QT_Q4_K, P.D), P.ds, P.mid, P.mid_slot};
        dim3 grid(gx, P.F / 16);
        gateup_q4k_kernel<1, 1><<<grid, 256, 0, s>>>(A);
    } else {
        GenericArgs A{P.x, P.nt, P.D, P.F, maxa, P.gate, P.up, P.sh_gate, P.sh_up, P.gt, P.ut, P.sgt, P.sut,
                      qg_row_bytes_host(P.gt, P.D), qg_row_bytes_host(P.ut, P.D),
                      P.sh_gate ? qg_row_bytes_host(P.sgt, P.D) : 0, P.sh_up ? qg_row_bytes_host(P.sut, P.D) : 0,
                      P.ds, P.mid, P.mid_slot};
        gateup_generic_kernel<<<dim3(gx, (P.F + 1) / 2), 64, 0, s>>>(A);
    }
    int rc = hipGetLastError();
    if (rc) return rc;
    phase_mark(3, s);
    DownArgs D{P.nt, P.D, P.F, maxa, P.down, P.sh_down, qg_row_bytes_host(P.dt, P.F),
               P.sh_down ? qg_row_bytes_host(P.sdt, P.F) : 0, P.ds, P.mid, P.route_w, P.slots, P.slots_out};
    if (fast_dn) {
        dim3 grid(gx, P.D / ROWS_DOWN);
        const int fs = P.sh_down ? P.sdt : P.dt;
        if (P.dt == QT_IQ4_NL && fs == QT_IQ4_NL) down_kernel<QT_IQ4_NL, QT_IQ4_NL><<<grid, 256, 0, s>>>(D);
        else if (P.dt == QT_IQ4_NL) down_kernel<QT_IQ4_NL, QT_Q4_K><<<grid, 256, 0, s>>>(D);
        else if (fs == QT_IQ4_NL) down_kernel<QT_Q4_K, QT_IQ4_NL><<<grid, 256, 0, s>>>(D);
        else down_kernel<QT_Q4_K, QT_Q4_K><<<grid, 256, 0, s>>>(D);
    } else {
        GenericDownArgs G{D, P.dt, P.sh_down ? P.sdt : 0};
        down_generic_kernel<<<dim3(gx, (P.D + 1) / 2), 64, 0, s>>>(G);
    }
    if ((rc = hipGetLastError())) return rc;
    phase_mark(4, s);
    if (P.out) {
        const int quads = P.nt * P.D / 4;
        combine_kernel<<<(quads + 255) / 256, 256, 0, s>>>(P.out, P.slots, P.ds, P.sh_logit, P.ld, P.nt, P.D);
        rc = hipGetLastError();
    }
    phase_mark(5, s);
    return rc;
}

}  // namespace

extern "C" {

int qg_moe_phase_events(void **events, int n) {
    if (n < 0 || n > 6 || (n && !events)) return hipErrorInvalidValue;
    for (int i = 0; i < 8; i++) tl_phase_ev[i] = i < n ? events[i] : nullptr;
    tl_phase_n = n;
    return hipSuccess;
}

size_t qg_generic_workspace_bytes(int width, int ff, int tokens) {
    if (width < 256 || width % 256 || width > 8192 || ff < 32 || ff % 32 || ff > 4096 || tokens < 1 || tokens > MAXB) return 0;
    return ws_layout(width, ff).total;
}

// The layer for any supported format and width (the fallback of
// qg_moe_forward); arguments already validated by the caller.
int qg_generic_forward(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, const float *x, int nt,
                       const qg_moe_layer *L, void *workspace, size_t ws_bytes) {
    if (!out || !ids || !weights || !x || !L || !workspace || nt < 1 || nt > MAXB) return hipErrorInvalidValue;
    const int D = L->width, F = L->ff;
    const size_t need = qg_generic_workspace_bytes(D, F, nt);
    if (!need || ws_bytes < need || !L->router || !L->gate || !L->up || !L->down) return hipErrorInvalidValue;
    if (!qg_row_bytes_host(L->gate_type, D) || !qg_row_bytes_host(L->up_type, D) || !qg_row_bytes_host(L->down_type, F))
        return hipErrorInvalidValue;
    const bool sh = L->sh_gate != nullptr;
    if (sh && (!L->sh_up || !L->sh_down || !L->sh_gate_inp || !qg_row_bytes_host(L->sh_gate_type, D) ||
               !qg_row_bytes_host(L->sh_up_type, D) || !qg_row_bytes_host(L->sh_down_type, F)))
        return hipErrorInvalidValue;
    if (L->resident && (L->threshold < 0 || L->threshold > 0.1 || !__builtin_isfinite(L->threshold))) return hipErrorInvalidValue;
    hipStream_t s = qg_stream();
    const WsLayout lay = ws_layout(D, F);
    uint8_t *ws = (uint8_t *)workspace;
    float *logits = (float *)(ws + lay.logits);
    Disp *ds = (Disp *)(ws + lay.disp);
    const int rows = QG_EXPERTS + (sh ? 1 : 0);
    phase_mark(0, s);
    int rc = qg_launch_matmul_exact(logits, (const uint8_t *)L->router, QT_F32, rows, D, x, nt,
                                    sh ? (const uint8_t *)L->sh_gate_inp : nullptr, s);
    if (rc) return rc;
    if (L->router_bias) {
        logit_bias_kernel<<<nt, QG_EXPERTS, 0, s>>>(logits, rows, L->router_bias);
        if ((rc = hipGetLastError())) return rc;
    }
    phase_mark(1, s);
    _Float16 *xh = (_Float16 *)(ws + lay.xh);
    float *xs = (float *)(ws + lay.xs);
    route_dispatch_kernel<<<1, RD_THREADS, 0, s>>>(ids, weights, flags, stats, logits, rows, nt, L->resident, L->threshold, ds,
                                                   sh ? 1 : 0, x, D, xh, xs);
    if ((rc = hipGetLastError())) return rc;
    phase_mark(2, s);
    ExpertPhase P{x, nt, D, F, xh, xs, (_Float16 *)(ws + lay.midh), (float *)(ws + lay.mids),
                  (const uint8_t *)L->gate, (const uint8_t *)L->up, (const uint8_t *)L->down, L->gate_type, L->up_type, L->down_type,
                  sh ? (const uint8_t *)L->sh_gate : nullptr, sh ? (const uint8_t *)L->sh_up : nullptr,
                  sh ? (const uint8_t *)L->sh_down : nullptr, L->sh_gate_type, L->sh_up_type, L->sh_down_type,
                  ds, (float *)(ws + lay.mid), nullptr, (float *)(ws + lay.slots), nullptr, weights,
                  logits + QG_EXPERTS, rows, out};
    return launch_experts(P, s);
}

// Fused MTP MoE (gpu.cu:528-551): slots[t,k,:] = down_e(silu(gate_e x_t) *
// up_e x_t) * w[t,k], mid[t,k,:] the SwiGLU rows, e = ids[t,k]; invalid ids
// give NaN rows; tokens 1..17; widths from qg_moe_configure.  Experts shared
// by several tokens are read once.
int qg_mtp_moe(float *slots, float *mid, const float *x, const int *ids, const float *weights, const void *g, int gt,
               const void *u, int ut, const void *d, int dt, int nt) {
    const int D = qg_cfg_width(), F = qg_cfg_ff();
    if (!qg_row_bytes_host(gt, D) || !qg_row_bytes_host(ut, D) || !qg_row_bytes_host(dt, F) || nt < 1 || nt > MAXB)
        return hipErrorInvalidValue;
    if (!slots || !mid || !x || !ids || !weights || !g || !u || !d) return hipErrorInvalidValue;
    // Scratch for the dispatch and the entry-indexed rows, grown on demand
    // (never inside a capture: the first call per shape must be eager; an
    // outgrown buffer stays allocated for graphs captured with it).
    static thread_local void *scratch = nullptr;
    static thread_local size_t scratch_bytes = 0;
    const WsLayout lay = ws_layout(D, F);
    int grc = qg_scratch_grow(&scratch, &scratch_bytes, lay.total);
    if (grc) return grc;
    hipStream_t s = qg_stream();
    uint8_t *ws = (uint8_t *)scratch;
    Disp *ds = (Disp *)(ws + lay.disp);
    _Float16 *xh = (_Float16 *)(ws + lay.xh);
    float *xs = (float *)(ws + lay.xs);
    const bool planes = nt > 4;  // matrix-core expert kernels for groups above four tokens
    dispatch_ids_kernel<<<1, RD_THREADS, 0, s>>>(ids, nt, ds, mid, slots, D, F, x, planes ? xh : nullptr, xs);
    int rc = hipGetLastError();
    if (rc) return rc;
    const int saved_n = tl_phase_n;
    tl_phase_n = 0;  // phase timing covers qg_moe_forward only
    ExpertPhase P{x, nt, D, F, planes ? xh : nullptr, xs, (_Float16 *)(ws + lay.midh), (float *)(ws + lay.mids),
                  (const uint8_t *)g, (const uint8_t *)u, (const uint8_t *)d, gt, ut, dt,
                  nullptr, nullptr, nullptr, 0, 0, 0,
                  ds, (float *)(ws + lay.mid), mid, (float *)(ws + lay.slots), slots, weights,
                  nullptr, 0, nullptr};
    rc = launch_experts(P, s);
    tl_phase_n = saved_n;
    return rc;
}

// CSR dispatch for any batch (per-chunk histogram, prefix sums, stable fill).
int qg_moe_dispatch(int *offsets, int *row_token, int *row_slot, int *status, const int *ids, int nt) {
    if (!offsets || !row_token || !row_slot || !status || !ids || nt < 1 || nt > QG_MAX_TOKENS) return hipErrorInvalidValue;
    // chunk histograms, grown on demand (never inside a capture: the first
    // call per size must be eager; an outgrown buffer stays allocated for
    // graphs captured with it)
    static thread_local void *scratch = nullptr;
    static thread_local size_t scratch_bytes = 0;
    int grc = qg_scratch_grow(&scratch, &scratch_bytes, qg_prefill_dispatch_scratch(nt));
    if (grc) return grc;
    return qg_prefill_dispatch(offsets, row_token, row_slot, status, ids, nt, scratch);
}

}  // extern "C"
