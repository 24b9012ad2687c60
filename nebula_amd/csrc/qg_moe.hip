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

struct Disp {
    int n_active, n_entries, status, has_shared;
    int act_expert[QG_EXPERTS];
    int act_off[QG_EXPERTS + 1];
    int ent_token[MAXS];
    int ent_slot[MAXS];
    int slot_ent[MAXS];
    int tok_flag[MAXB];
};

struct WsLayout { size_t logits, disp, mid, slots, arrive, total; };
WsLayout ws_layout(int D, int F) {
    WsLayout L;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += (n + 255) & ~(size_t)255; return o; };
    L.logits = take((size_t)MAXB * (QG_EXPERTS + 1) * 4);
    L.disp = take(sizeof(Disp));
    L.mid = take((size_t)(MAXS + MAXB) * F * 4);
    L.slots = take((size_t)(MAXS + MAXB) * D * 4);
    L.arrive = take((size_t)(D / 2 + 1) * 4);
    L.total = off;
    return L;
}

// ---------------- routing of one token by one wave (gpu.cu:456-465) ----------------
QG_DEV void route_token(int *s_ids, float *s_w, const float *s, int t, int lane) {
    float v[8];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) { v[i] = s[lane + 64 * i]; bad |= !__builtin_isfinite(v[i]); }
    if (__any(bad)) {
        if (lane < QG_TOP) { s_ids[t * QG_TOP + lane] = -1; s_w[t * QG_TOP + lane] = 0.0f; }
        return;
    }
    float largest = v[0];
#pragma unroll
    for (int i = 1; i < 8; i++) largest = fmaxf(largest, v[i]);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) largest = fmaxf(largest, __shfl_xor(largest, d));
    float num[QG_TOP], total = 0.0f;
    int best_id[QG_TOP];
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) {
        float bv = v[0];
        int bi = 0;
#pragma unroll
        for (int i = 1; i < 8; i++) if (v[i] > bv) { bv = v[i]; bi = i; }
        int bidx = lane + 64 * bi;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const float ov = __shfl_xor(bv, d);
            const int oi = __shfl_xor(bidx, d);
            if (ov > bv || (ov == bv && oi < bidx)) { bv = ov; bidx = oi; }
        }
        best_id[k] = bidx;
        num[k] = qg_expf(bv - largest);
        total += num[k];
        if ((bidx & 63) == lane) {
#pragma unroll
            for (int i = 0; i < 8; i++) if (i == (bidx >> 6)) v[i] = -__builtin_inff();
        }
    }
#pragma unroll
    for (int k = 0; k < QG_TOP; k++)
        if (lane == k) { s_ids[t * QG_TOP + k] = best_id[k]; s_w[t * QG_TOP + k] = num[k] / total; }
}

// Inclusive scan of one int per thread over a 256-thread block.
QG_DEV int block_scan256(int v, int *s_tmp) {
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

// Build the CSR dispatch from ids in LDS.  eligible(t) excludes tokens whose
// flag is 2 (handoff) or 3 (invalid); ids outside [0,512) never dispatch.
// Entries of each expert are in ascending (token, rank) order.
QG_DEV void build_dispatch(const int *s_ids, const int *s_flag, int nt, Disp *ds, int *s_tmp) {
    const int tid = threadIdx.x, n = nt * QG_TOP;
    for (int i = tid; i < MAXS; i += 256) ds->slot_ent[i] = -1;
    const int e0 = 2 * tid, e1 = 2 * tid + 1;
    int c0 = 0, c1 = 0;
    for (int i = 0; i < n; i++) {
        const int id = s_ids[i];
        if ((id >> 1) == tid && id >= 0 && s_flag[i / QG_TOP] < 2) { c0 += id == e0; c1 += id == e1; }
    }
    const int local = (((c0 > 0) + (c1 > 0)) << 16) | (c0 + c1);
    const int incl = block_scan256(local, s_tmp);
    const int excl = incl - local;
    int act = excl >> 16, off = excl & 0xffff;
    __syncthreads();  // slot_ent initialisation above is complete
    for (int h = 0; h < 2; h++) {
        const int e = h ? e1 : e0, c = h ? c1 : c0;
        if (!c) continue;
        ds->act_expert[act] = e;
        ds->act_off[act] = off;
        int i = off;
        for (int t = 0; t < nt; t++) {
            if (s_flag[t] >= 2) continue;
            for (int k = 0; k < QG_TOP; k++)
                if (s_ids[t * QG_TOP + k] == e) { ds->ent_token[i] = t; ds->ent_slot[i] = t * QG_TOP + k; ds->slot_ent[t * QG_TOP + k] = i; i++; }
        }
        act++;
        off += c;
    }
    if (tid == 255) {
        ds->n_active = incl >> 16;
        ds->n_entries = incl & 0xffff;
        ds->act_off[incl >> 16] = incl & 0xffff;
    }
}

// ---------------- kernel 2: route + coverage + dispatch (one block) ----------------
__global__ __launch_bounds__(256) void route_dispatch_kernel(int *ids_out, float *w_out, uint8_t *flags_out,
                                                             qg_prune_stats *stats, const float *logits, int ld, int nt,
                                                             const uint8_t *resident, double thr, Disp *ds,
                                                             int *arrive, int n_arrive, int has_shared) {
    __shared__ int s_ids[MAXS];
    __shared__ float s_w[MAXS];
    __shared__ int s_flag[MAXB], s_missing[MAXB];
    __shared__ double s_mass[MAXB];
    __shared__ int s_tmp[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < n_arrive; i += 256) arrive[i] = 0;
    for (int t = wave; t < nt; t += 4) route_token(s_ids, s_w, logits + (size_t)t * ld, t, lane);
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
    }
    __syncthreads();
    // Counters in token order (deterministic, unlike the reference's atomics).
    if (tid == 0 && resident && stats) {
        for (int t = 0; t < nt; t++) {
            if (s_flag[t] == 3) continue;
            stats->token_layers += 1;
            stats->missing_selections += (uint64_t)s_missing[t];
            if (s_flag[t] == 1) {
                stats->skipped_selections += (uint64_t)s_missing[t];
                stats->avoided_token_handoffs += 1;
                stats->skipped_mass += s_mass[t];
            }
        }
    }
    for (int i = tid; i < nt * QG_TOP; i += 256) { ids_out[i] = s_ids[i]; w_out[i] = s_w[i]; }
    if (flags_out && tid < nt) flags_out[tid] = (uint8_t)s_flag[tid];
    if (tid == 0) { ds->status = 0; ds->has_shared = has_shared; }
    for (int t = 0; t < nt; t++) if (s_flag[t] == 3 && tid == 0) ds->status = 1;
    build_dispatch(s_ids, s_flag, nt, ds, s_tmp);
}

// ---------------- dispatch from given ids (qg_mtp_moe front end) ----------------
// Every selection with 0<=id<512 dispatches (duplicates included, as the
// reference computes each (token, rank) independently); invalid slots get
// NaN in mid and slots (gpu.cu:531,539).
__global__ __launch_bounds__(256) void dispatch_ids_kernel(const int *ids, int nt, Disp *ds, float *mid_slot, float *slots_out,
                                                           int D, int F) {
    __shared__ int s_ids[MAXS];
    __shared__ int s_flag[MAXB];
    __shared__ int s_tmp[4];
    const int tid = threadIdx.x;
    for (int i = tid; i < nt * QG_TOP; i += 256) s_ids[i] = ids[i];
    if (tid < MAXB) s_flag[tid] = 0;
    if (tid == 0) { ds->status = 0; ds->has_shared = 0; }
    __syncthreads();
    // duplicates: the CSR keeps ascending (token, rank); a duplicate id within
    // a token yields two entries of that expert, both computed.
    build_dispatch(s_ids, s_flag, nt, ds, s_tmp);
    const float nan = __builtin_nanf("");
    for (int s = 0; s < nt * QG_TOP; s++) {
        const int e = s_ids[s];
        if (e >= 0 && e < QG_EXPERTS) continue;
        for (int r = tid; r < F; r += 256) mid_slot[(size_t)s * F + r] = nan;
        for (int d = tid; d < D; d += 256) slots_out[(size_t)s * D + d] = nan;
    }
}

// ---------------- Q4_K chunk arithmetic ----------------
// Chunk q (0..7) of a superblock: qs bytes 16q..16q+15 hold elements
// l = 16(q&1)+0..15 of group ga = 2(q>>1) (low nibbles) and gb = ga+1 (high
// nibbles) (cpu.c:56-64 layout).  Scales decoded four bytes at a time.
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

template <int TC>
QG_DEV void q4k_chunk_dot(float (&part)[TC], uint4 qv, const Q4kScale &sc, const Q4kSlice (&xs)[TC]) {
    float qa[16], qb[16];
    const uint32_t w4[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = w4[i] & 0x0F0F0F0Fu, hi = (w4[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            qa[4 * i + b] = (float)((lo >> (8 * b)) & 0xffu);
            qb[4 * i + b] = (float)((hi >> (8 * b)) & 0xffu);
        }
    }
#pragma unroll
    for (int t = 0; t < TC; t++) {
        float sa = 0.0f, sb = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) { sa = __builtin_fmaf(qa[i], xs[t].a[i], sa); sb = __builtin_fmaf(qb[i], xs[t].b[i], sb); }
        float p = part[t];
        p = __builtin_fmaf(sc.dsa, sa, p);
        p = __builtin_fmaf(-sc.dma, xs[t].sa, p);
        p = __builtin_fmaf(sc.dsb, sb, p);
        p = __builtin_fmaf(-sc.dmb, xs[t].sb, p);
        part[t] = p;
    }
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

template <int TC, int CPL>
__global__ __launch_bounds__(256) void gateup_q4k_kernel(GateUpArgs A) {
    constexpr int RPW = 2;  // row pairs (gate row + up row) per wave
    const int a = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool shared = A.sh_gate && a == A.maxa;
    int n, ent0 = 0;
    const uint8_t *G, *U;
    if (shared) { n = A.nt; G = A.sh_gate; U = A.sh_up; }
    else {
        if (a >= A.ds->n_active) return;
        const int e = A.ds->act_expert[a];
        ent0 = A.ds->act_off[a];
        n = A.ds->act_off[a + 1] - ent0;
        G = A.gate + (size_t)e * A.F * A.rb;
        U = A.up + (size_t)e * A.F * A.rb;
    }
    const int row0 = (blockIdx.y * 4 + wave) * RPW;
    if (row0 >= A.F) return;
    int koff[CPL];
    size_t qoff[CPL], hoff[CPL];
    int qsel[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int ch = lane + 64 * c;
        koff[c] = q4k_koff(ch); qoff[c] = q4k_qoff(ch); hoff[c] = q4k_hoff(ch); qsel[c] = ch & 7;
    }
    for (int t0 = 0; t0 < n; t0 += TC) {
        Q4kSlice xs[CPL][TC];
        int tok[TC];
#pragma unroll
        for (int i = 0; i < TC; i++) {
            const bool valid = t0 + i < n;
            tok[i] = valid ? (shared ? t0 + i : A.ds->ent_token[ent0 + t0 + i]) : 0;
#pragma unroll
            for (int c = 0; c < CPL; c++) q4k_load_slice(xs[c][i], A.x + (size_t)tok[i] * A.D, koff[c], valid);
        }
        uint4 qg[RPW][CPL], hg[RPW][CPL], qu[RPW][CPL], hu[RPW][CPL];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const size_t rowoff = (size_t)(row0 + r) * A.rb;
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                qg[r][c] = qg_ld16(G + rowoff + qoff[c]); hg[r][c] = qg_ld16(G + rowoff + hoff[c]);
                qu[r][c] = qg_ld16(U + rowoff + qoff[c]); hu[r][c] = qg_ld16(U + rowoff + hoff[c]);
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float pg[TC], pu[TC];
#pragma unroll
            for (int i = 0; i < TC; i++) { pg[i] = 0.0f; pu[i] = 0.0f; }
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                q4k_chunk_dot<TC>(pg, qg[r][c], q4k_scale(hg[r][c], qsel[c]), xs[c]);
                q4k_chunk_dot<TC>(pu, qu[r][c], q4k_scale(hu[r][c], qsel[c]), xs[c]);
            }
            float gsel = 0.0f, usel = 0.0f;
#pragma unroll
            for (int i = 0; i < TC; i++) {
                const float g = group_sum<64>(pg[i]), u = group_sum<64>(pu[i]);
                if (lane == i) { gsel = g; usel = u; }
            }
            if (lane < TC && t0 + lane < n) {
                const int row = row0 + r;
                const float m = qg_swiglu(gsel, usel);
                if (shared) A.mid[(size_t)(MAXS + t0 + lane) * A.F + row] = m;
                else {
                    const int ent = ent0 + t0 + lane;
                    A.mid[(size_t)ent * A.F + row] = m;
                    if (A.mid_slot) A.mid_slot[(size_t)A.ds->ent_slot[ent] * A.F + row] = m;
                }
            }
        }
    }
}

// ---------------- kernel 4: down + weighted slots + rank-order combine ----------------
struct DownArgs {
    int nt, D, F, maxa;
    const uint8_t *down, *sh_down;
    size_t rb, sh_rb;          // row bytes of an F-column row (routed, shared)
    const Disp *ds;
    const float *mid;
    const float *route_w;      // [nt][10] after pruning
    float *slots;              // workspace [MAXS+MAXB][D] (entry-indexed)
    float *slots_out;          // slot mode: caller's [(t*10+k)][D], or null
    int *arrive;               // per row block arrival counters (fused mode)
    const float *sh_logit;     // logits + 512, stride ld
    int ld;
    float *out;                // [nt][D] (fused mode)
};

// IQ4_NL: 8 lanes per 512-column row, a lane owns a pair of 18-byte blocks
// (64 columns).  The table is shifted by +128 to unsigned bytes so v_perm can
// look it up and cvt_f32_ubyte can convert; the shift is removed with the
// block's x sum.
QG_DEV uint32_t iq4_lookup(uint32_t idx) {
    // lut + 128 = {1,24,45,63, 79,93,106,118, 129,141,153,166, 181,197,217,241}
    const uint32_t T0 = 0x3F2D1801u, T1 = 0x766A5D4Fu, T2 = 0xA6998D81u, T3 = 0xF1D9C5B5u;
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

struct Iq4Slice { float v[64]; float s0, s1; };

QG_DEV void iq4_load_slice(Iq4Slice &s, const float *xrow, int koff, bool valid) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 64; i++) s.v[i] = 0.0f;
        s.s0 = s.s1 = 0.0f;
        return;
    }
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

template <int TC>
QG_DEV void iq4_pair_dot(float (&part)[TC], const Iq4Raw &r, const Iq4Slice (&xs)[TC]) {
    const float d0 = qg_half_u16(r.w[0] & 0xffffu), d1 = qg_half_u16(r.w[4] >> 16);
    uint32_t qs[8];
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
#pragma unroll
    for (int i = 0; i < 4; i++) qs[4 + i] = r.w[5 + i];
    float val[64];
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = qs[blk * 4 + i];
            const uint32_t lo = iq4_lookup(w & 0x0F0F0F0Fu), hi = iq4_lookup((w >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                val[blk * 32 + 4 * i + b] = (float)((lo >> (8 * b)) & 0xffu);
                val[blk * 32 + 16 + 4 * i + b] = (float)((hi >> (8 * b)) & 0xffu);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TC; t++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) { s0 = __builtin_fmaf(val[i], xs[t].v[i], s0); s1 = __builtin_fmaf(val[32 + i], xs[t].v[32 + i], s1); }
        s0 = __builtin_fmaf(-128.0f, xs[t].s0, s0);
        s1 = __builtin_fmaf(-128.0f, xs[t].s1, s1);
        part[t] = __builtin_fmaf(d0, s0, __builtin_fmaf(d1, s1, part[t]));
    }
}

// Rows [rowbase, rowbase+32) of one expert (or the shared expert).  FMT is the
// row format: 20 (IQ4_NL, 8 lanes/row) or 12 (Q4_K, 16 lanes/row).
template <int FMT, int TC>
QG_DEV void down_rows(const DownArgs &A, const uint8_t *W, size_t rb, int n, int ent0, bool shared, int rowbase) {
    constexpr int LPR = FMT == QT_IQ4_NL ? 8 : 16, RPW = 64 / LPR, PASSES = ROWS_DOWN / (4 * RPW);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane % LPR, rsub = lane / LPR;
    for (int t0 = 0; t0 < n; t0 += TC) {
        int mrow[TC];
        bool valid[TC];
#pragma unroll
        for (int i = 0; i < TC; i++) {
            valid[i] = t0 + i < n;
            mrow[i] = valid[i] ? (shared ? MAXS + t0 + i : ent0 + t0 + i) : 0;
        }
        if (FMT == QT_IQ4_NL) {
            Iq4Slice xs[TC];
#pragma unroll
            for (int i = 0; i < TC; i++) iq4_load_slice(xs[i], A.mid + (size_t)mrow[i] * A.F, 64 * c, valid[i]);
#pragma unroll
            for (int ps = 0; ps < PASSES; ps++) {
                const int row = rowbase + (ps * 4 + wave) * RPW + rsub;
                const Iq4Raw raw = iq4_load(W + (size_t)row * rb + 36 * c);
                float part[TC];
#pragma unroll
                for (int i = 0; i < TC; i++) part[i] = 0.0f;
                iq4_pair_dot<TC>(part, raw, xs);
#pragma unroll
                for (int i = 0; i < TC; i++) {
                    const float y = group_sum<LPR>(part[i]);
                    if (c == i && valid[i]) {
                        if (shared) A.slots[(size_t)mrow[i] * A.D + row] = y;
                        else {
                            const int slot = A.ds->ent_slot[mrow[i]];
                            const float v = y * A.route_w[slot];
                            if (A.slots_out) A.slots_out[(size_t)slot * A.D + row] = v;
                            else A.slots[(size_t)mrow[i] * A.D + row] = v;
                        }
                    }
                }
            }
        } else {
            Q4kSlice xs[1][TC];
            const int koff = q4k_koff(c);
#pragma unroll
            for (int i = 0; i < TC; i++) q4k_load_slice(xs[0][i], A.mid + (size_t)mrow[i] * A.F, koff, valid[i]);
#pragma unroll
            for (int ps = 0; ps < PASSES; ps++) {
                const int row = rowbase + (ps * 4 + wave) * RPW + rsub;
                const uint8_t *rp = W + (size_t)row * rb;
                const uint4 qv = qg_ld16(rp + q4k_qoff(c)), hd = qg_ld16(rp + q4k_hoff(c));
                float part[TC];
#pragma unroll
                for (int i = 0; i < TC; i++) part[i] = 0.0f;
                q4k_chunk_dot<TC>(part, qv, q4k_scale(hd, c & 7), xs[0]);
#pragma unroll
                for (int i = 0; i < TC; i++) {
                    const float y = group_sum<LPR>(part[i]);
                    if (c == i && valid[i]) {
                        if (shared) A.slots[(size_t)mrow[i] * A.D + row] = y;
                        else {
                            const int slot = A.ds->ent_slot[mrow[i]];
                            const float v = y * A.route_w[slot];
                            if (A.slots_out) A.slots_out[(size_t)slot * A.D + row] = v;
                            else A.slots[(size_t)mrow[i] * A.D + row] = v;
                        }
                    }
                }
            }
        }
    }
}

// Sum the 10 weighted slots of each token in router-rank order from 0.0f
// (gpu.cu:521-527, cpu.c:227-230; pruned ranks add +0), then add the
// sigmoid-gated shared expert with one fma (gpu.cu:552).  Tokens flagged
// handoff/invalid get a zero row.
QG_DEV void combine_rows(const DownArgs &A, int rowbase) {
    const int has_shared = A.ds->has_shared;
    for (int idx = threadIdx.x; idx < A.nt * ROWS_DOWN; idx += 256) {
        const int t = idx / ROWS_DOWN, d = rowbase + idx % ROWS_DOWN;
        float acc = 0.0f;
        const int flag = A.ds->tok_flag[t];
        if (flag < 2) {
#pragma unroll
            for (int k = 0; k < QG_TOP; k++) {
                const int se = A.ds->slot_ent[t * QG_TOP + k];
                acc += se >= 0 ? A.slots[(size_t)se * A.D + d] : 0.0f;
            }
            if (has_shared)
                acc = __builtin_fmaf(A.slots[(size_t)(MAXS + t) * A.D + d],
                                     qg_sig(A.sh_logit[(size_t)t * A.ld]), acc);
        }
        A.out[(size_t)t * A.D + d] = acc;
    }
}

template <int FR, int FS, int TC>
__global__ __launch_bounds__(256) void down_kernel(DownArgs A) {
    const int a = blockIdx.x, rowbase = blockIdx.y * ROWS_DOWN;
    const bool shared = A.sh_down && a == A.maxa;
    if (shared) down_rows<FS, TC>(A, A.sh_down, A.sh_rb, A.nt, 0, true, rowbase);
    else {
        if (a >= A.ds->n_active) return;
        const int e = A.ds->act_expert[a], ent0 = A.ds->act_off[a], n = A.ds->act_off[a + 1] - ent0;
        down_rows<FR, TC>(A, A.down + (size_t)e * A.D * A.rb, A.rb, n, ent0, false, rowbase);
    }
    if (!A.out) return;
    // Last block of this row block combines (release/acquire at agent scope).
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int expected = A.ds->n_active + (A.sh_down ? 1 : 0);
        s_last = atomicAdd(&A.arrive[blockIdx.y], 1) == expected - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    combine_rows(A, rowbase);
    if (threadIdx.x == 0) A.arrive[blockIdx.y] = 0;
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
        const int e = A.ds->act_expert[a];
        ent0 = A.ds->act_off[a];
        n = A.ds->act_off[a + 1] - ent0;
        gt = A.gt; ut = A.ut; grb = A.grb; urb = A.urb;
        G = A.gate + (size_t)e * A.F * grb;
        U = A.up + (size_t)e * A.F * urb;
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
    const int a = blockIdx.x, half = threadIdx.x >> 5, j = threadIdx.x & 31;
    const int rowbase = blockIdx.y * 2, row = rowbase + half;
    const bool shared = A.sh_down && a == A.maxa;
    bool active = true;
    if (shared) {
        if (row < A.D)
            for (int t = 0; t < A.nt; t++) {
                const float y = exact_dot(A.sh_down + (size_t)row * A.sh_rb, G.sdt, A.F, A.mid + (size_t)(MAXS + t) * A.F, j);
                if (j == 0) A.slots[(size_t)(MAXS + t) * A.D + row] = y;
            }
    } else if (a < A.ds->n_active) {
        const int e = A.ds->act_expert[a], ent0 = A.ds->act_off[a], n = A.ds->act_off[a + 1] - ent0;
        const uint8_t *W = A.down + (size_t)e * A.D * A.rb;
        if (row < A.D)
            for (int i = 0; i < n; i++) {
                const int ent = ent0 + i;
                const float y = exact_dot(W + (size_t)row * A.rb, G.dt, A.F, A.mid + (size_t)ent * A.F, j);
                if (j == 0) {
                    const int slot = A.ds->ent_slot[ent];
                    const float v = y * A.route_w[slot];
                    if (A.slots_out) A.slots_out[(size_t)slot * A.D + row] = v;
                    else A.slots[(size_t)ent * A.D + row] = v;
                }
            }
    } else active = false;
    if (!A.out || !active) return;
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int expected = A.ds->n_active + (A.sh_down ? 1 : 0);
        s_last = atomicAdd(&A.arrive[blockIdx.y], 1) == expected - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int has_shared = A.ds->has_shared;
    for (int idx = threadIdx.x; idx < A.nt * 2; idx += 64) {
        const int t = idx / 2, d = rowbase + idx % 2;
        if (d >= A.D) continue;
        float acc = 0.0f;
        if (A.ds->tok_flag[t] < 2) {
            for (int k = 0; k < QG_TOP; k++) {
                const int se = A.ds->slot_ent[t * QG_TOP + k];
                acc += se >= 0 ? A.slots[(size_t)se * A.D + d] : 0.0f;
            }
            if (has_shared)
                acc = __builtin_fmaf(A.slots[(size_t)(MAXS + t) * A.D + d],
                                     qg_sig(A.sh_logit[(size_t)t * A.ld]), acc);
        }
        A.out[(size_t)t * A.D + d] = acc;
    }
    if (threadIdx.x == 0) A.arrive[blockIdx.y] = 0;
}

// ---------------- expert-phase launcher shared by forward and mtp_moe ----------------
struct ExpertPhase {
    const float *x; int nt, D, F;
    const uint8_t *gate, *up, *down; int gt, ut, dt;
    const uint8_t *sh_gate, *sh_up, *sh_down; int sgt, sut, sdt;
    Disp *ds; float *mid, *mid_slot, *slots, *slots_out; const float *route_w;
    int *arrive; const float *sh_logit; int ld; float *out;
};

int launch_experts(const ExpertPhase &P, hipStream_t s) {
    const int maxa = P.nt * QG_TOP < QG_EXPERTS ? P.nt * QG_TOP : QG_EXPERTS;
    const int gx = maxa + (P.sh_gate ? 1 : 0);
    const bool fast_gu = P.gt == QT_Q4_K && P.ut == QT_Q4_K && (!P.sh_gate || (P.sgt == QT_Q4_K && P.sut == QT_Q4_K)) &&
                         (P.D == 2048 || P.D == 4096) && P.F % 8 == 0;
    const bool fast_dn = (P.dt == QT_IQ4_NL || P.dt == QT_Q4_K) && (!P.sh_down || P.sdt == QT_IQ4_NL || P.sdt == QT_Q4_K) &&
                         P.F == 512 && P.D % ROWS_DOWN == 0;
    if (fast_gu) {
        GateUpArgs A{P.x, P.nt, P.D, P.F, maxa, P.gate, P.up, P.sh_gate, P.sh_up, qg_row_bytes_host(QT_Q4_K, P.D), P.ds, P.mid, P.mid_slot};
        dim3 grid(gx, P.F / 8);
        if (P.D == 2048) {
            if (P.nt == 1) gateup_q4k_kernel<1, 1><<<grid, 256, 0, s>>>(A);
            else gateup_q4k_kernel<4, 1><<<grid, 256, 0, s>>>(A);
        } else {
            if (P.nt == 1) gateup_q4k_kernel<1, 2><<<grid, 256, 0, s>>>(A);
            else gateup_q4k_kernel<2, 2><<<grid, 256, 0, s>>>(A);
        }
    } else {
        GenericArgs A{P.x, P.nt, P.D, P.F, maxa, P.gate, P.up, P.sh_gate, P.sh_up, P.gt, P.ut, P.sgt, P.sut,
                      qg_row_bytes_host(P.gt, P.D), qg_row_bytes_host(P.ut, P.D),
                      P.sh_gate ? qg_row_bytes_host(P.sgt, P.D) : 0, P.sh_up ? qg_row_bytes_host(P.sut, P.D) : 0,
                      P.ds, P.mid, P.mid_slot};
        gateup_generic_kernel<<<dim3(gx, (P.F + 1) / 2), 64, 0, s>>>(A);
    }
    int rc = hipGetLastError();
    if (rc) return rc;
    DownArgs D{P.nt, P.D, P.F, maxa, P.down, P.sh_down, qg_row_bytes_host(P.dt, P.F),
               P.sh_down ? qg_row_bytes_host(P.sdt, P.F) : 0, P.ds, P.mid, P.route_w, P.slots, P.slots_out,
               P.arrive, P.sh_logit, P.ld, P.out};
    if (fast_dn) {
        dim3 grid(gx, P.D / ROWS_DOWN);
        const int fs = P.sh_down ? P.sdt : P.dt;
#define NB_DOWN(FR, FS)                                                                     \
        if (P.nt == 1) down_kernel<FR, FS, 1><<<grid, 256, 0, s>>>(D);                      \
        else down_kernel<FR, FS, 2><<<grid, 256, 0, s>>>(D);
        if (P.dt == QT_IQ4_NL && fs == QT_IQ4_NL) { NB_DOWN(QT_IQ4_NL, QT_IQ4_NL) }
        else if (P.dt == QT_IQ4_NL) { NB_DOWN(QT_IQ4_NL, QT_Q4_K) }
        else if (fs == QT_IQ4_NL) { NB_DOWN(QT_Q4_K, QT_IQ4_NL) }
        else { NB_DOWN(QT_Q4_K, QT_Q4_K) }
#undef NB_DOWN
    } else {
        GenericDownArgs G{D, P.dt, P.sh_down ? P.sdt : 0};
        down_generic_kernel<<<dim3(gx, (P.D + 1) / 2), 64, 0, s>>>(G);
    }
    return hipGetLastError();
}

// ---------------- general CSR dispatch (any token count) ----------------
// counts[e] = tokens selecting e, with bit 30 set if some token lists e twice
// and bit 29 (expert 0's word) set if any id is neither valid nor a pruned
// encoding (the validation of cpu.c:242-244).
__global__ __launch_bounds__(64) void csr_count_kernel(int *counts, const int *ids, int nt) {
    const int e = blockIdx.x, lane = threadIdx.x;
    int c = 0, dup = 0, bad = 0;
    for (int t = lane; t < nt; t += 64) {
        int m = 0;
        for (int k = 0; k < QG_TOP; k++) {
            const int id = ids[t * QG_TOP + k];
            m += id == e;
            if (e == 0 && (id >= QG_EXPERTS || (id < 0 && !(id <= -2 && id >= -QG_EXPERTS - 1)))) bad = 1;
        }
        c += m > 0;
        dup |= m > 1;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) { c += __shfl_xor(c, d); dup |= __shfl_xor(dup, d); bad |= __shfl_xor(bad, d); }
    if (lane == 0) counts[e] = c | (dup << 30) | (bad << 29);
}
__global__ __launch_bounds__(256) void csr_scan_kernel(int *offsets, int *status, const int *counts) {
    __shared__ int s_tmp[4];
    __shared__ int s_bad;
    const int tid = threadIdx.x;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    const int w0 = counts[2 * tid], w1 = counts[2 * tid + 1];
    if ((w0 | w1) & (3 << 29)) atomicOr(&s_bad, 1);
    const int c0 = w0 & 0x1fffffff, c1 = w1 & 0x1fffffff;
    const int incl = block_scan256(c0 + c1, s_tmp);
    offsets[2 * tid] = incl - c0 - c1;
    offsets[2 * tid + 1] = incl - c1;
    if (tid == 255) offsets[QG_EXPERTS] = incl;
    __syncthreads();
    if (tid == 0) *status = s_bad;
}
__global__ __launch_bounds__(64) void csr_fill_kernel(int *row_token, int *row_slot, const int *offsets, const int *ids, int nt) {
    const int e = blockIdx.x, lane = threadIdx.x;
    int carry = offsets[e];
    for (int base = 0; base < nt; base += 64) {
        const int t = base + lane;
        int k_sel = -1;
        if (t < nt)
            for (int k = QG_TOP - 1; k >= 0; k--) if (ids[t * QG_TOP + k] == e) k_sel = k;
        // a token lists one entry per matching rank (duplicates are rejected upstream)
        const unsigned long long mask = __ballot(k_sel >= 0);
        if (k_sel >= 0) {
            const int pos = carry + __popcll(mask & ((1ULL << lane) - 1ULL));
            row_token[pos] = t;
            row_slot[pos] = t * QG_TOP + k_sel;
        }
        carry += __popcll(mask);
    }
}

}  // namespace

extern "C" {

size_t qg_moe_workspace_bytes(int width, int ff, int tokens) {
    if (width < 256 || width % 256 || width > 8192 || ff < 32 || ff % 32 || ff > 4096 || tokens < 1 || tokens > MAXB) return 0;
    return ws_layout(width, ff).total;
}

int qg_moe_forward(float *out, int *ids, float *weights, unsigned char *flags, qg_prune_stats *stats, const float *x, int nt,
                   const qg_moe_layer *L, void *workspace, size_t ws_bytes) {
    if (!out || !ids || !weights || !x || !L || !workspace || nt < 1 || nt > MAXB) return hipErrorInvalidValue;
    const int D = L->width, F = L->ff;
    const size_t need = qg_moe_workspace_bytes(D, F, nt);
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
    int rc = qg_launch_matmul_exact(logits, (const uint8_t *)L->router, QT_F32, rows, D, x, nt,
                                    sh ? (const uint8_t *)L->sh_gate_inp : nullptr, s);
    if (rc) return rc;
    int *arrive = (int *)(ws + lay.arrive);
    route_dispatch_kernel<<<1, 256, 0, s>>>(ids, weights, flags, stats, logits, rows, nt, L->resident, L->threshold, ds,
                                            arrive, D / 2 + 1, sh ? 1 : 0);
    if ((rc = hipGetLastError())) return rc;
    ExpertPhase P{x, nt, D, F,
                  (const uint8_t *)L->gate, (const uint8_t *)L->up, (const uint8_t *)L->down, L->gate_type, L->up_type, L->down_type,
                  sh ? (const uint8_t *)L->sh_gate : nullptr, sh ? (const uint8_t *)L->sh_up : nullptr,
                  sh ? (const uint8_t *)L->sh_down : nullptr, L->sh_gate_type, L->sh_up_type, L->sh_down_type,
                  ds, (float *)(ws + lay.mid), nullptr, (float *)(ws + lay.slots), nullptr, weights,
                  arrive, logits + QG_EXPERTS, rows, out};
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
    // (never inside a capture: the first call per shape must be eager).
    static thread_local void *scratch = nullptr;
    static thread_local size_t scratch_bytes = 0;
    const WsLayout lay = ws_layout(D, F);
    if (scratch_bytes < lay.total) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (qg_stream() && hipStreamIsCapturing(qg_stream(), &st) == hipSuccess && st != hipStreamCaptureStatusNone)
            return hipErrorInvalidValue;
        if (scratch) (void)hipFree(scratch);
        scratch = nullptr;
        scratch_bytes = 0;
        if (hipMalloc(&scratch, lay.total) != hipSuccess) return hipErrorOutOfMemory;
        scratch_bytes = lay.total;
    }
    hipStream_t s = qg_stream();
    uint8_t *ws = (uint8_t *)scratch;
    Disp *ds = (Disp *)(ws + lay.disp);
    dispatch_ids_kernel<<<1, 256, 0, s>>>(ids, nt, ds, mid, slots, D, F);
    int rc = hipGetLastError();
    if (rc) return rc;
    ExpertPhase P{x, nt, D, F, (const uint8_t *)g, (const uint8_t *)u, (const uint8_t *)d, gt, ut, dt,
                  nullptr, nullptr, nullptr, 0, 0, 0,
                  ds, (float *)(ws + lay.mid), mid, (float *)(ws + lay.slots), slots, weights,
                  nullptr, nullptr, 0, nullptr};
    return launch_experts(P, s);
}

// CSR dispatch for any batch (histogram per expert, prefix sum, ordered fill).
int qg_moe_dispatch(int *offsets, int *row_token, int *row_slot, int *status, const int *ids, int nt) {
    if (!offsets || !row_token || !row_slot || !status || !ids || nt < 1 || nt > QG_MAX_TOKENS) return hipErrorInvalidValue;
    hipStream_t s = qg_stream();
    // counts live in offsets[0..511] until the scan overwrites them in place
    static thread_local int *counts = nullptr;
    if (!counts && hipMalloc((void **)&counts, QG_EXPERTS * sizeof(int)) != hipSuccess) { counts = nullptr; return hipErrorOutOfMemory; }
    csr_count_kernel<<<QG_EXPERTS, 64, 0, s>>>(counts, ids, nt);
    csr_scan_kernel<<<1, 256, 0, s>>>(offsets, status, counts);
    csr_fill_kernel<<<QG_EXPERTS, 64, 0, s>>>(row_token, row_slot, offsets, ids, nt);
    return hipGetLastError();
}

}  // extern "C"
