// Expert products on the CDNA4 matrix cores (v_mfma_f32_16x16x32_f16) for
// token groups larger than a few tokens: the decode batches of 5..17 tokens
// and the grouped prefill.  Included by qg_moe.hip (shares its dispatch
// structures).
//
// Operand roles (lane layouts checked on gfx950): A = activations, 16 rows =
// 8 tokens x {hi, lo} fp16 planes; B = weights, 16 columns = 16 weight rows;
// D[token-plane][weight row].  Lane l holds column j = l%16 (its own weight
// row, so that row's Q4_K/IQ4_NL scales are lane-local) and D rows
// 4*(l/16)+0..3 = both planes of tokens 2*(l/16) and 2*(l/16)+1.
//
// Exactness: Q4_K weights enter as w' = s_g*q (an integer <= 945, exact in
// fp16) and the superblock scale d and the min term dmin*m_g*sum(x) are
// applied in fp32 per superblock; IQ4_NL weights enter as their table value
// (an integer in [-127,113]) with the block scale applied per 32 columns.
// Activations x = hi + lo with hi = fp16(x), lo = fp16(x - hi), carrying
// ~22 significant bits; products are exact and accumulate in fp32.
//
// Element order: a weight fragment's 8 consecutive elements come out of the
// nibble->fp16 conversion as pairs (0,2),(1,3),(4,6),(5,7); activation planes
// are stored with the same order inside every 8-element chunk.


QG_DEV void act_planes_group(const float *x, int K, int r, int g, _Float16 *xh, float *xs) {
    const float *src = x + (size_t)r * K + g * 32;
    _Float16 *hi = xh + ((size_t)r * 2) * K + g * 32, *lo = hi + K;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) {
        const float v = src[e];
        s += v;
        const _Float16 h = (_Float16)v;
        const int pos = (e & ~7) | qg_perm8(e & 7);
        hi[pos] = h;
        lo[pos] = (_Float16)(v - (float)h);
    }
    xs[(size_t)r * (K / 32) + g] = s;
}

// fp32 rows -> fp16 hi/lo planes (permuted chunks) and per-32 sums.
// out planes: [row][2][K]; sums: [row][K/32].  One thread per 32-group.
__global__ __launch_bounds__(256) void act_planes_kernel(const float *x, int rows, int K, _Float16 *xh, float *xs) {
    const int i = blockIdx.x * 256 + threadIdx.x, groups = K / 32;
    if (i >= rows * groups) return;
    const int r = i / groups, g = i % groups;
    const float *src = x + (size_t)r * K + g * 32;
    _Float16 *hi = xh + ((size_t)r * 2) * K + g * 32, *lo = hi + K;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) {
        const float v = src[e];
        s += v;
        const _Float16 h = (_Float16)v;
        const int pos = (e & ~7) | qg_perm8(e & 7);
        hi[pos] = h;
        lo[pos] = (_Float16)(v - (float)h);
    }
    xs[(size_t)r * groups + g] = s;
}

// Activation fragment: row (token, plane), k-chunk starting at k.
QG_DEV qg_half8 act_frag(const _Float16 *planes, int K, int row, int plane, int k) {
    return __builtin_bit_cast(qg_half8, *(const uint4 *)(planes + ((size_t)row * 2 + plane) * K + k));
}


// ---------------- gate/up + SwiGLU on MFMA ----------------
struct MfmaGU {
    const _Float16 *xh; const float *xs;   // token planes [nt][2][D], sums [nt][D/32]
    int nt, D, F, maxa;
    const uint8_t *gate, *up, *sh_gate, *sh_up;
    size_t rb;
    const Disp *ds;
    float *mid;                 // entry-indexed [MAXS+MAXB][F] (shared at MAXS+t)
    float *mid_slot;            // slot layout or null
    _Float16 *midh;             // planes of mid rows [MAXS+MAXB][2][F]
    float *mids;                // sums of mid rows [MAXS+MAXB][F/32]
    const int *tok_of;          // entry -> token, or null when entries are tokens
    int ent_base_shared;        // first mid row of the shared expert
};

// Block: 4 waves x 16 weight rows (gate and up) = 64 rows of F; all tokens
// of the expert, TG tiles of 8 tokens per pass.
template <int TG>
__global__ __launch_bounds__(256) void gateup_mfma_kernel(MfmaGU A) {
    __shared__ float s_mid[8 * TG][64];
    const int a = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = lane & 15, kq = lane >> 4;
    const bool shared = A.sh_gate && a == A.maxa;
    int n, ent0 = 0;
    const uint8_t *G, *U;
    if (shared) { n = A.nt; G = A.sh_gate; U = A.sh_up; ent0 = A.ent_base_shared; }
    else {
        if (a >= A.ds->n_active) return;
        const int4 info = A.ds->act[a];
        ent0 = info.y;
        n = info.z;
        G = A.gate + (size_t)info.x * A.F * A.rb;
        U = A.up + (size_t)info.x * A.F * A.rb;
    }
    const int rbase = blockIdx.y * 64, row = rbase + wave * 16 + j;
    const uint8_t *gr = G + (size_t)row * A.rb, *ur = U + (size_t)row * A.rb;
    for (int c0 = 0; c0 < n; c0 += 8 * TG) {
        // the token (activation row) each lane feeds as A row l%16 of tile c
        int arow[TG];
#pragma unroll
        for (int c = 0; c < TG; c++) {
            const int idx = c0 + c * 8 + (j >> 1);
            const int e = idx < n ? idx : n - 1;
            arow[c] = shared ? e : (A.tok_of ? A.tok_of[ent0 + e] : ent0 + e);
        }
        const float *Xrow[TG][2];  // sums of the two tokens whose hi-plane rows this lane holds
#pragma unroll
        for (int c = 0; c < TG; c++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const int idx = c0 + c * 8 + kq * 2 + t2;
                const int e = idx < n ? idx : n - 1;
                const int tok = shared ? e : (A.tok_of ? A.tok_of[ent0 + e] : ent0 + e);
                Xrow[c][t2] = A.xs + (size_t)tok * (A.D / 32);
            }
        qg_f4 yg[TG], yu[TG];
#pragma unroll
        for (int c = 0; c < TG; c++) { yg[c] = qg_f4{0, 0, 0, 0}; yu[c] = qg_f4{0, 0, 0, 0}; }
        for (int sb = 0; sb < A.D / 256; sb++) {
            const Q4kHeader hg = q4k_header(qg_ld16(gr + (size_t)sb * 144)), hu = q4k_header(qg_ld16(ur + (size_t)sb * 144));
            qg_f4 pg[TG], pu[TG];
#pragma unroll
            for (int c = 0; c < TG; c++) { pg[c] = qg_f4{0, 0, 0, 0}; pu[c] = qg_f4{0, 0, 0, 0}; }
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const size_t qoff = (size_t)sb * 144 + 16 + (g >> 1) * 32 + kq * 8;
                const uint2 bg = *(const uint2 *)(gr + qoff), bu = *(const uint2 *)(ur + qoff);
                const qg_half8 wg = q4_frag(bg, g & 1, (_Float16)q4k_s(hg, g));
                const qg_half8 wu = q4_frag(bu, g & 1, (_Float16)q4k_s(hu, g));
                const int k = sb * 256 + g * 32 + kq * 8;
#pragma unroll
                for (int c = 0; c < TG; c++) {
                    const qg_half8 x = act_frag(A.xh, A.D, arow[c], j & 1, k);
                    pg[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, wg, pg[c], 0, 0, 0);
                    pu[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, wu, pu[c], 0, 0, 0);
                }
            }
            // superblock epilogue: d * P - dmin * sum_g m_g * X_g (hi-plane rows only)
#pragma unroll
            for (int c = 0; c < TG; c++) {
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++) {
                    const float *X = Xrow[c][t2] + sb * 8;
                    float mg = 0.0f, mu = 0.0f;
#pragma unroll
                    for (int g = 0; g < 8; g++) {
                        mg = __builtin_fmaf((float)q4k_m(hg, g), X[g], mg);
                        mu = __builtin_fmaf((float)q4k_m(hu, g), X[g], mu);
                    }
                    yg[c][2 * t2] = __builtin_fmaf(hg.d, pg[c][2 * t2], __builtin_fmaf(-hg.dmin, mg, yg[c][2 * t2]));
                    yg[c][2 * t2 + 1] = __builtin_fmaf(hg.d, pg[c][2 * t2 + 1], yg[c][2 * t2 + 1]);
                    yu[c][2 * t2] = __builtin_fmaf(hu.d, pu[c][2 * t2], __builtin_fmaf(-hu.dmin, mu, yu[c][2 * t2]));
                    yu[c][2 * t2 + 1] = __builtin_fmaf(hu.d, pu[c][2 * t2 + 1], yu[c][2 * t2 + 1]);
                }
            }
        }
        // planes combine, SwiGLU, stage the 64 rows x tokens in LDS
#pragma unroll
        for (int c = 0; c < TG; c++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const float gv = yg[c][2 * t2] + yg[c][2 * t2 + 1], uv = yu[c][2 * t2] + yu[c][2 * t2 + 1];
                s_mid[c * 8 + kq * 2 + t2][wave * 16 + j] = qg_swiglu(gv, uv);
            }
        __syncthreads();
        // write mid rows (fp32, planes, sums of the two 32-row groups of this block)
        const int ntile = min(8 * TG, n - c0);
        for (int i = threadIdx.x; i < ntile * 64; i += 256) {
            const int tt = i >> 6, r = i & 63;
            const int mrow = ent0 + c0 + tt;
            const float v = s_mid[tt][r];
            const int f = rbase + r;
            if (A.mid) A.mid[(size_t)mrow * A.F + f] = v;
            if (A.mid_slot && !shared) A.mid_slot[(size_t)A.ds->ent_slot[mrow] * A.F + f] = v;
            const _Float16 h = (_Float16)v;
            const int pos = (f & ~7) | qg_perm8(f & 7);
            A.midh[((size_t)mrow * 2) * A.F + pos] = h;
            A.midh[((size_t)mrow * 2 + 1) * A.F + pos] = (_Float16)(v - (float)h);
        }
        if (threadIdx.x < ntile * 2) {
            const int tt = threadIdx.x >> 1, gsel = threadIdx.x & 1;
            float s = 0.0f;
            for (int r = 0; r < 32; r++) s += s_mid[tt][gsel * 32 + r];
            A.mids[(size_t)(ent0 + c0 + tt) * (A.F / 32) + rbase / 32 + gsel] = s;
        }
        __syncthreads();
    }
}

// ---------------- down on MFMA ----------------
struct MfmaDown {
    int nt, D, F, maxa;
    const uint8_t *down, *sh_down;
    size_t rb, sh_rb;
    const Disp *ds;
    const _Float16 *midh; const float *mids;
    const float *route_w;
    float *slots;      // entry-indexed [MAXS+MAXB][D]
    float *slots_out;  // slot layout or null
    int ent_base_shared;
};

template <int FMT, int TG>
QG_DEV void down_mfma_rows(const MfmaDown &A, const uint8_t *W, size_t rb, int n, int ent0, bool shared, int rbase) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15, kq = lane >> 4;
    const int row = rbase + wave * 16 + j;
    const uint8_t *wr = W + (size_t)row * rb;
    for (int c0 = 0; c0 < n; c0 += 8 * TG) {
        int arow[TG];
#pragma unroll
        for (int c = 0; c < TG; c++) {
            const int idx = c0 + c * 8 + (j >> 1);
            arow[c] = ent0 + (idx < n ? idx : n - 1);
        }
        qg_f4 y[TG];
#pragma unroll
        for (int c = 0; c < TG; c++) y[c] = qg_f4{0, 0, 0, 0};
        if (FMT == QT_IQ4_NL) {
            for (int bp = 0; bp < A.F / 64; bp++) {
                const Iq4Raw raw = iq4_load(wr + 36 * bp);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    // block 2bp+h: d and 16 qs bytes; this lane's 8 elements are
                    // nibble half kq>>1 of qs bytes (kq&1)*8 .. +8
                    float d;
                    uint32_t q0, q1;
                    if (h == 0) {
                        d = qg_half_u16(raw.w[0] & 0xffffu);
                        const uint32_t a0 = __builtin_amdgcn_alignbyte(raw.w[1], raw.w[0], 2), a1 = __builtin_amdgcn_alignbyte(raw.w[2], raw.w[1], 2);
                        const uint32_t a2 = __builtin_amdgcn_alignbyte(raw.w[3], raw.w[2], 2), a3 = __builtin_amdgcn_alignbyte(raw.w[4], raw.w[3], 2);
                        q0 = (kq & 1) ? a2 : a0;
                        q1 = (kq & 1) ? a3 : a1;
                    } else {
                        d = qg_half_u16(raw.w[4] >> 16);
                        q0 = (kq & 1) ? raw.w[7] : raw.w[5];
                        q1 = (kq & 1) ? raw.w[8] : raw.w[6];
                    }
                    const qg_half8 w = iq4_frag(q0, q1, kq >> 1);
                    const int k = (2 * bp + h) * 32 + kq * 8;
#pragma unroll
                    for (int c = 0; c < TG; c++) {
                        const qg_half8 x = act_frag(A.midh, A.F, arow[c], j & 1, k);
                        const qg_f4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, w, qg_f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) y[c][r] = __builtin_fmaf(d, p[r], y[c][r]);
                    }
                }
            }
        } else {
            for (int sb = 0; sb < A.F / 256; sb++) {
                const Q4kHeader hd = q4k_header(qg_ld16(wr + (size_t)sb * 144));
                qg_f4 p[TG];
#pragma unroll
                for (int c = 0; c < TG; c++) p[c] = qg_f4{0, 0, 0, 0};
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    const uint2 b = *(const uint2 *)(wr + (size_t)sb * 144 + 16 + (g >> 1) * 32 + kq * 8);
                    const qg_half8 w = q4_frag(b, g & 1, (_Float16)q4k_s(hd, g));
                    const int k = sb * 256 + g * 32 + kq * 8;
#pragma unroll
                    for (int c = 0; c < TG; c++)
                        p[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(act_frag(A.midh, A.F, arow[c], j & 1, k), w, p[c], 0, 0, 0);
                }
#pragma unroll
                for (int c = 0; c < TG; c++)
#pragma unroll
                    for (int t2 = 0; t2 < 2; t2++) {
                        const int idx = c0 + c * 8 + kq * 2 + t2;
                        const float *X = A.mids + (size_t)(ent0 + (idx < n ? idx : n - 1)) * (A.F / 32) + sb * 8;
                        float m = 0.0f;
#pragma unroll
                        for (int g = 0; g < 8; g++) m = __builtin_fmaf((float)q4k_m(hd, g), X[g], m);
                        y[c][2 * t2] = __builtin_fmaf(hd.d, p[c][2 * t2], __builtin_fmaf(-hd.dmin, m, y[c][2 * t2]));
                        y[c][2 * t2 + 1] = __builtin_fmaf(hd.d, p[c][2 * t2 + 1], y[c][2 * t2 + 1]);
                    }
            }
        }
#pragma unroll
        for (int c = 0; c < TG; c++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const int idx = c0 + c * 8 + kq * 2 + t2;
                if (idx >= n) continue;
                const float v = y[c][2 * t2] + y[c][2 * t2 + 1];
                const int mrow = ent0 + idx;
                if (shared) { A.slots[(size_t)mrow * A.D + row] = v; continue; }
                const int slot = A.ds->ent_slot[mrow];
                const float sv = v * A.route_w[slot];
                if (A.slots_out) A.slots_out[(size_t)slot * A.D + row] = sv;
                else A.slots[(size_t)mrow * A.D + row] = sv;
            }
    }
}

template <int FR, int FS, int TG>
__global__ __launch_bounds__(256) void down_mfma_kernel(MfmaDown A) {
    const int a = blockIdx.x, rbase = blockIdx.y * 64;
    if (A.sh_down && a == A.maxa) { down_mfma_rows<FS, TG>(A, A.sh_down, A.sh_rb, A.nt, A.ent_base_shared, true, rbase); return; }
    if (a >= A.ds->n_active) return;
    const int4 info = A.ds->act[a];
    down_mfma_rows<FR, TG>(A, A.down + (size_t)info.x * A.D * A.rb, A.rb, info.z, info.y, false, rbase);
}
