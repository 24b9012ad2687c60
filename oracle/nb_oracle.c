/* CPU restatement of nebula's routed-MoE layer: TEST INFRASTRUCTURE ONLY.
 *
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * as the parity checker; the product never links or calls it.  Paths in the
 * citations are under /root/reference/qwen/.
 *
 * How each part is pinned (tests/test_oracle_cpu.py):
 *  - nbo_weight_at, nbo_matmul: bit-exact against the reference's own
 *    qc_matmul/qc_weight_at built from cpu.c into oracle/_ref, all 11 formats;
 *    closed-form dequant of hand-built blocks; all 65,536 fp16 encodings.
 *  - nbo_moe: bit-exact against the reference's qc_moe (2560/640 unpatched
 *    build and the 2048/512 build), both sides of nt=17, pruned ids skipped,
 *    duplicate/out-of-range ids rejected.
 *  - nbo_route: the KAT of test_gpu.py:338-346 (ids = stable argsort of
 *    -logits, weights = softmax of the winners, NaN row -> all -1), plus
 *    invariants (sum of weights, first numerator exactly 1).
 *  - nbo_prune / nbo_coverage: the KAT of test_gpu.py:84-95 (counters
 *    (5,10,4,2), strict threshold cases) and brute-force mass sums.
 *  - nbo_moe_map / nbo_dispatch: brute force (np.flatnonzero per expert, as
 *    in test_gpu.py:352-359).
 *  - nbo_exp_d / nbo_expf: against glibc exp/expf over dense samples.
 *  - nbo_shared: no CPU implementation exists in the reference (qwen.c:708-713
 *    runs it on the GPU only); pinned by the float64 closed form of the same
 *    products (tolerance) and by nbo_matmul for each product.
 */
#include "nb_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------- formats (cpu.c:17-67) ---------------- */

size_t nbo_row_bytes(int type, int cols) { /* cpu.c:17-30 */
    if (cols < 1) return 0;
    if (type == 0) return (size_t)cols * 4;
    if (type == 1 || type == 30) return (size_t)cols * 2;
    if (cols % 32) return 0;
    if (type == 2 || type == 20) return (size_t)cols / 32 * 18;
    if (type == 6) return (size_t)cols / 32 * 22;
    if (type == 12) return cols % 256 ? 0 : (size_t)cols / 256 * 144;
    if (type == 13) return cols % 256 ? 0 : (size_t)cols / 256 * 176;
    if (type == 14) return cols % 256 ? 0 : (size_t)cols / 256 * 210;
    if (type == 7) return (size_t)cols / 32 * 24;
    if (type == 8) return (size_t)cols / 32 * 34;
    return 0;
}

float nbo_half(const uint8_t *p) { /* scalar branch of cpu.c:31-42 */
    uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 31, m = h & 1023, bits;
    if (!e) {
        if (!m) bits = sign;
        else {
            int ex = -14;
            while (!(m & 1024)) { m <<= 1; ex--; }
            bits = sign | ((uint32_t)(ex + 127) << 23) | ((m & 1023) << 13);
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0);
    else bits = sign | ((e + 112) << 23) | (m << 13);
    float v; memcpy(&v, &bits, 4); return v;
}

static const int8_t IQ4NL_LUT[16] = {-127,-104,-83,-65,-49,-35,-22,-10,1,13,25,38,53,69,89,113}; /* cpu.c:53 */

float nbo_weight_at(const void *ptr, int type, int i) { /* cpu.c:43-67 */
    const uint8_t *row = ptr;
    if (type == 0) { float f; memcpy(&f, row + (size_t)i * 4, 4); return f; }
    if (type == 1) return nbo_half(row + (size_t)i * 2);
    if (type == 30) { uint32_t u = (uint32_t)(row[2*i] | (row[2*i+1] << 8)) << 16; float f; memcpy(&f, &u, 4); return f; }
    if (type == 8) { const uint8_t *p = row + (size_t)(i / 32) * 34; return nbo_half(p) * (float)(int8_t)p[2 + i % 32]; }
    if (type == 2 || type == 20 || type == 6 || type == 7) {
        int bytes = type == 7 ? 24 : type == 6 ? 22 : 18, j = i % 32, off = type == 7 ? 8 : type == 6 ? 6 : 2;
        const uint8_t *p = row + (size_t)(i / 32) * bytes;
        int q = (p[off + j % 16] >> ((j / 16) * 4)) & 15;
        if (type == 6 || type == 7) {
            const uint8_t *hp = p + (type == 7 ? 4 : 2);
            uint32_t high = (uint32_t)hp[0] | ((uint32_t)hp[1] << 8) | ((uint32_t)hp[2] << 16) | ((uint32_t)hp[3] << 24);
            q |= ((high >> j) & 1) << 4;
        }
        if (type == 20) return nbo_half(p) * (float)IQ4NL_LUT[q];
        return type == 7 ? fmaf(nbo_half(p), (float)q, nbo_half(p + 2))
                         : nbo_half(p) * (float)(q - (type == 2 ? 8 : type == 6 ? 16 : 0));
    }
    int k = i % 256, g = k / 32, l = k % 32;
    const uint8_t *p = row + (size_t)(i / 256) * (type == 12 ? 144 : type == 13 ? 176 : 210);
    if (type == 14) {
        int h = k / 128, s = (k % 128) / 32;
        int lo = (p[h*64 + (s%2)*32 + l] >> ((s/2)*4)) & 15, hi = (p[128 + h*32 + l] >> (s*2)) & 3;
        return nbo_half(p + 208) * (float)(int8_t)p[192 + h*8 + s*2 + l/16] * (float)((lo | (hi << 4)) - 32);
    }
    const uint8_t *sc = p + 4;
    int s = g < 4 ? (sc[g] & 63) : ((sc[g+4] & 15) | ((sc[g-4] >> 6) << 4));
    int m = g < 4 ? (sc[g+4] & 63) : ((sc[g+4] >> 4) | ((sc[g] >> 6) << 4));
    int q = (p[(type == 12 ? 16 : 48) + (g/2)*32 + l] >> ((g%2)*4)) & 15;
    if (type == 13) q |= ((p[16 + l] >> g) & 1) << 4;
    return fmaf(nbo_half(p) * (float)s, (float)q, -nbo_half(p + 2) * (float)m);
}

/* The reference's one summation order (cpu.c:122-139, cpu_portable.h:326-335,
 * gpu.cu:89-92,159-163): lane j in 0..31 accumulates k = j (mod 32) in
 * ascending k with fused multiply-add, then the 32 lanes are added pairwise
 * with strides 16, 8, 4, 2, 1. */
static float dot32(const uint8_t *row, int type, int cols, const float *x) {
    float acc[32] = {0};
    for (int k = 0; k < cols; k += 32)
        for (int j = 0; j < 32; j++) acc[j] = fmaf(nbo_weight_at(row, type, k + j), x[k + j], acc[j]);
    for (int stride = 16; stride; stride /= 2)
        for (int j = 0; j < stride; j++) acc[j] += acc[j + stride];
    return acc[0];
}

int nbo_matmul(float *out, const void *w, int type, int rows, int cols, const float *x, int nt) {
    size_t stride = nbo_row_bytes(type, cols); /* validation as cpu.c:121 without the 2048-token cap */
    if (!out || !w || !x || !stride || cols % 32 || rows < 1 || nt < 1) return -1;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < rows; r++)
        for (int t = 0; t < nt; t++)
            out[(size_t)t * rows + r] = dot32((const uint8_t *)w + (size_t)r * stride, type, cols, x + (size_t)t * cols);
    return 0;
}

/* ---------------- exp ----------------
 * The reference's routing and shared-expert gate use CUDA's expf, which has
 * no CPU counterpart here.  The build defines exp as the double-precision
 * exponential rounded once to float; this is the oracle's statement of it:
 * Cody-Waite reduction by ln 2 (split into the fdlibm hi/lo constants) and a
 * degree-17 Taylor polynomial on |r| <= ln2/2 (truncation < 1e-24 relative),
 * evaluated by Horner with fused multiply-adds, then an exact 2^k scaling. */
double nbo_exp_d(double x) {
    if (x != x) return x;
    if (x > 709.782712893384) return INFINITY;
    if (x < -745.1332191019412) return 0.0;
    const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
    double kd = rint(x * 1.44269504088896338700e+00);
    double r = fma(-kd, ln2_hi, x);
    r = fma(-kd, ln2_lo, r);
    static const double inv_fact[18] = {
        1.0, 1.0, 1.0/2.0, 1.0/6.0, 1.0/24.0, 1.0/120.0, 1.0/720.0, 1.0/5040.0, 1.0/40320.0,
        1.0/362880.0, 1.0/3628800.0, 1.0/39916800.0, 1.0/479001600.0, 1.0/6227020800.0,
        1.0/87178291200.0, 1.0/1307674368000.0, 1.0/20922789888000.0, 1.0/355687428096000.0};
    double p = inv_fact[17];
    for (int n = 16; n >= 0; n--) p = fma(p, r, inv_fact[n]);
    int k = (int)kd;
    /* p in [0.70, 1.42]; scale by 2^k in at most two exact steps. */
    if (k > 1023) { k -= 1023; p *= 8.98846567431157953865e+307; } /* 2^1023 */
    if (k < -1022) { k += 1022; p *= 2.22507385850720138309e-308; } /* 2^-1022 */
    uint64_t bits = (uint64_t)(k + 1023) << 52;
    double scale; memcpy(&scale, &bits, 8);
    return p * scale;
}

float nbo_expf(float x) { return (float)nbo_exp_d((double)x); }

/* ---------------- routing (gpu.cu:456-465) ----------------
 * Per token: any non-finite logit -> ids -1, weights 0.  Otherwise the 10
 * winners by repeated strict-greater argmax (lowest index among maxima),
 * numerators exp(s - max) summed in rank order, then divided by that sum. */
void nbo_route(int *ids, float *weights, const float *logits, int nt) {
    for (int t = 0; t < nt; t++) {
        float s[NBO_EXPERTS]; memcpy(s, logits + (size_t)t * NBO_EXPERTS, sizeof s);
        float largest = -INFINITY; int bad = 0;
        for (int j = 0; j < NBO_EXPERTS; j++) { if (!isfinite(s[j])) { bad = 1; break; } largest = fmaxf(largest, s[j]); }
        int *id = ids + (size_t)t * NBO_TOP; float *w = weights + (size_t)t * NBO_TOP;
        if (bad) { for (int k = 0; k < NBO_TOP; k++) { id[k] = -1; w[k] = 0; } continue; }
        float total = 0;
        for (int k = 0; k < NBO_TOP; k++) {
            int best = 0;
            for (int j = 1; j < NBO_EXPERTS; j++) if (s[j] > s[best]) best = j;
            id[k] = best; w[k] = nbo_expf(s[best] - largest); total += w[k]; s[best] = -INFINITY;
        }
        for (int k = 0; k < NBO_TOP; k++) w[k] /= total;
    }
}

/* ---------------- pruning (gpu.cu:467-488) ----------------
 * Tokens with any id outside [0,512) are skipped before counting.  mass is
 * the double sum, in rank order, of weights whose expert is not resident.
 * If missing>0, threshold>0 and mass<threshold, non-resident ids become
 * -id-2 and their weights 0 (no renormalisation).  The device adds
 * skipped_mass with atomics (order-dependent); here it is summed in token
 * order. */
void nbo_prune(int *ids, float *weights, const uint8_t *resident, int nt, double threshold, nbo_prune_stats *st) {
    for (int t = 0; t < nt; t++) {
        int *id = ids + (size_t)t * NBO_TOP; float *w = weights + (size_t)t * NBO_TOP;
        int missing = 0, bad = 0; double mass = 0;
        for (int k = 0; k < NBO_TOP; k++) {
            int e = id[k]; if (e < 0 || e >= NBO_EXPERTS) { bad = 1; break; }
            if (!resident[e]) { missing++; mass += (double)w[k]; }
        }
        if (bad) continue;
        if (st) { st->token_layers++; st->missing_selections += (uint64_t)missing; }
        if (missing && threshold > 0 && mass < threshold) {
            for (int k = 0; k < NBO_TOP; k++) if (!resident[id[k]]) { id[k] = -id[k] - 2; w[k] = 0; }
            if (st) { st->skipped_selections += (uint64_t)missing; st->avoided_token_handoffs++; st->skipped_mass += mass; }
        }
    }
}

/* Coverage classification with the 0.10 rule of gpu.cu:470-478 and
 * config.py:9 (called with 0.10 at qwen.c:647-648):
 * 0 = every selection resident, 1 = pruned (missing mass < 0.10),
 * 2 = handoff (missing and !(mass < 0.10): coverage below 90 %),
 * 3 = invalid ids (the kernel returns before counting). */
void nbo_coverage(uint8_t *flags, double *mass_out, const int *ids, const float *weights, const uint8_t *resident, int nt) {
    for (int t = 0; t < nt; t++) {
        const int *id = ids + (size_t)t * NBO_TOP; const float *w = weights + (size_t)t * NBO_TOP;
        int missing = 0, bad = 0; double mass = 0;
        for (int k = 0; k < NBO_TOP; k++) {
            int e = id[k]; if (e < 0 || e >= NBO_EXPERTS) { bad = 1; break; }
            if (!resident[e]) { missing++; mass += (double)w[k]; }
        }
        if (mass_out) mass_out[t] = bad ? NAN : mass;
        flags[t] = bad ? 3 : !missing ? 0 : (mass < 0.10 ? 1 : 2);
    }
}

/* ---------------- dispatch ----------------
 * gpu.cu:489-500: row e of map lists, in ascending order, the tokens t with
 * some ids[t,k]==e; negative (pruned/invalid) ids never match. */
void nbo_moe_map(int *map, int *counts, const int *ids, int nt) {
    for (int e = 0; e < NBO_EXPERTS; e++) {
        int c = 0;
        for (int t = 0; t < nt; t++) {
            int sel = 0;
            for (int k = 0; k < NBO_TOP; k++) sel |= ids[(size_t)t * NBO_TOP + k] == e;
            if (sel) map[(size_t)e * nt + c++] = t;
        }
        if (counts) counts[e] = c;
    }
}

/* CSR of the same permutation with the validation of cpu.c:241-246:
 * offsets[513]; entries of expert e are offsets[e]..offsets[e+1]-1 in
 * ascending token order; row_slot = t*10+k.  Pruned encodings (-2..-513 with
 * weight 0) are skipped by the caller's weights check; here any id in
 * [-513,-2] is skipped.  Returns the entry count, or -1 on an id outside
 * [0,512) that is not a pruned encoding, or on a duplicate within a token. */
int nbo_dispatch(int *offsets, int *row_token, int *row_slot, const int *ids, int nt) {
    int counts[NBO_EXPERTS] = {0};
    for (int t = 0; t < nt; t++) for (int k = 0; k < NBO_TOP; k++) {
        int e = ids[(size_t)t * NBO_TOP + k];
        if (e <= -2 && e >= -NBO_EXPERTS - 1) continue;
        if (e < 0 || e >= NBO_EXPERTS) return -1;
        for (int j = 0; j < k; j++) if (ids[(size_t)t * NBO_TOP + j] == e) return -1;
        counts[e]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < NBO_EXPERTS; e++) offsets[e + 1] = offsets[e] + counts[e];
    int fill[NBO_EXPERTS]; memcpy(fill, offsets, sizeof fill);
    for (int t = 0; t < nt; t++) for (int k = 0; k < NBO_TOP; k++) {
        int e = ids[(size_t)t * NBO_TOP + k];
        if (e < 0) continue;
        int i = fill[e]++; row_token[i] = t; row_slot[i] = t * NBO_TOP + k;
    }
    return offsets[NBO_EXPERTS];
}

/* ---------------- routed experts (cpu.c:235-261) ----------------
 * Validation and slot map of cpu.c:238-246; per (expert, token):
 * gate/up rows with the fixed order, mid = (g*(1/(1+expf(-g))))*u with
 * libm expf (cpu.c:216,253), down rows with the fixed order, slot value
 * result*weight (cpu.c:224,255); then out = sum over k=0..9 from 0.0f in
 * router-rank order (cpu.c:227-230,257-259).  The nt<=17 and nt>17 branches
 * of the reference perform identical arithmetic. */
int nbo_moe(float *out, const float *x, const int *ids, const float *weights, int nt, int D, int F,
            const void *gate, int gt, const void *up, int ut, const void *down, int dt) {
    size_t gs = nbo_row_bytes(gt, D), us = nbo_row_bytes(ut, D), ds = nbo_row_bytes(dt, F);
    if (!out || !x || !ids || !weights || !gate || !up || !down || nt < 1 || !gs || !us || !ds) return -1;
    for (int t = 0; t < nt; t++) for (int k = 0; k < NBO_TOP; k++) {
        int e = ids[t * NBO_TOP + k]; float w = weights[t * NBO_TOP + k];
        if (e <= -2 && e >= -NBO_EXPERTS - 1 && w == 0) continue;
        if (e < 0 || e >= NBO_EXPERTS || !isfinite(w) || w < 0) return -1;
        for (int j = 0; j < k; j++) if (ids[t * NBO_TOP + j] == e) return -1;
    }
    float *slots = calloc((size_t)nt * NBO_TOP * D, sizeof(float));
    if (!slots) return -1;
    int failed = 0;
    #pragma omp parallel
    {
        float *mid = malloc((size_t)F * sizeof(float));
        if (!mid) {
            #pragma omp atomic write
            failed = 1;
        }
        #pragma omp for schedule(dynamic)
        for (int s = 0; s < nt * NBO_TOP; s++) {
            int e = ids[s]; if (e < 0 || !mid) continue;
            const float *xt = x + (size_t)(s / NBO_TOP) * D;
            const uint8_t *ge = (const uint8_t *)gate + (size_t)e * F * gs, *ue = (const uint8_t *)up + (size_t)e * F * us;
            const uint8_t *de = (const uint8_t *)down + (size_t)e * D * ds;
            for (int r = 0; r < F; r++) {
                float g = dot32(ge + (size_t)r * gs, gt, D, xt), u = dot32(ue + (size_t)r * us, ut, D, xt);
                mid[r] = (g * (1.0f / (1.0f + expf(-g)))) * u;
            }
            for (int d = 0; d < D; d++) slots[(size_t)s * D + d] = dot32(de + (size_t)d * ds, dt, F, mid) * weights[s];
        }
        free(mid);
    }
    if (!failed)
        for (int t = 0; t < nt; t++) for (int d = 0; d < D; d++) {
            float sum = 0;
            for (int k = 0; k < NBO_TOP; k++) sum += slots[((size_t)t * NBO_TOP + k) * D + d];
            out[(size_t)t * D + d] = sum;
        }
    free(slots);
    return failed ? -1 : 0;
}

/* ---------------- shared expert (qwen.c:708-713) ----------------
 * g = gate.x, u = up.x (qg_matmul order), mid = (g*sig(g))*u
 * (qg_unary op0 then qg_binary op1, gpu.cu:215-226), s = down.mid,
 * gate logit = sh_inp.x (F32 [1,D]), out += s*sig(logit) (gpu.cu:552-553).
 * sig(a) = 1/(1+exp(-a)) with the build's exp.  nvcc contracts the
 * `o[i]+=x[i]*sig(..)` of gpu.cu:552 into one fused multiply-add; so does
 * this statement. */
static float sigf(float a) { return 1.0f / (1.0f + nbo_expf(-a)); }

int nbo_shared(float *out, const float *x, int nt, int D, int F, const void *gate, int gt,
               const void *up, int ut, const void *down, int dt, const float *gate_inp) {
    float *g = malloc((size_t)nt * F * 4), *u = malloc((size_t)nt * F * 4), *s = malloc((size_t)nt * D * 4), *lg = malloc((size_t)nt * 4);
    int rc = -1;
    if (!g || !u || !s || !lg) goto done;
    if (nbo_matmul(g, gate, gt, F, D, x, nt) || nbo_matmul(u, up, ut, F, D, x, nt)) goto done;
    for (size_t i = 0; i < (size_t)nt * F; i++) { float a = g[i] * 1.0f; g[i] = (a * sigf(a)) * u[i]; }
    if (nbo_matmul(s, down, dt, D, F, g, nt) || nbo_matmul(lg, gate_inp, 0, 1, D, x, nt)) goto done;
    for (int t = 0; t < nt; t++) {
        float sg = sigf(lg[t]);
        for (int d = 0; d < D; d++) out[(size_t)t * D + d] = fmaf(s[(size_t)t * D + d], sg, out[(size_t)t * D + d]);
    }
    rc = 0;
done:
    free(g); free(u); free(s); free(lg);
    return rc;
}

/* ---------------- one layer (qwen.c:714-735) ----------------
 * router matmul (F32, qwen.c:716) -> route -> [prune with the resident mask,
 * qwen.c:647-648] -> routed experts -> rank-order reduce -> shared expert. */
int nbo_layer(float *out, int *ids_out, float *w_out, float *logits_out, uint8_t *flags,
              const nbo_layer_desc *L, const float *x, int nt, const uint8_t *resident,
              double threshold, nbo_prune_stats *stats) {
    int rc = -1;
    float *logits = malloc((size_t)nt * NBO_EXPERTS * 4), *w = malloc((size_t)nt * NBO_TOP * 4);
    int *ids = malloc((size_t)nt * NBO_TOP * 4);
    if (!logits || !w || !ids) goto done;
    if (nbo_matmul(logits, L->router, 0, NBO_EXPERTS, L->D, x, nt)) goto done;
    if (L->router_bias)
        for (int t = 0; t < nt; t++)
            for (int e = 0; e < NBO_EXPERTS; e++) logits[(size_t)t * NBO_EXPERTS + e] += L->router_bias[e];
    nbo_route(ids, w, logits, nt);
    if (resident) {
        if (flags) nbo_coverage(flags, NULL, ids, w, resident, nt);
        nbo_prune(ids, w, resident, nt, threshold, stats);
    }
    if (nbo_moe(out, x, ids, w, nt, L->D, L->F, L->gate, L->gt, L->up, L->ut, L->down, L->dt)) goto done;
    if (L->sh_gate && nbo_shared(out, x, nt, L->D, L->F, L->sh_gate, L->sgt, L->sh_up, L->sut, L->sh_down, L->sdt, L->sh_inp)) goto done;
    if (ids_out) memcpy(ids_out, ids, (size_t)nt * NBO_TOP * 4);
    if (w_out) memcpy(w_out, w, (size_t)nt * NBO_TOP * 4);
    if (logits_out) memcpy(logits_out, logits, (size_t)nt * NBO_EXPERTS * 4);
    rc = 0;
done:
    free(logits); free(w); free(ids);
    return rc;
}

/* Input normalisation (the RMSNorm of gpu.cu:204-214 with weight 1), evaluated
 * in double and rounded once; used only to build "RMS-normalised" inputs. */
void nbo_rmsnorm(float *out, const float *x, int nt, int D, float eps) {
    for (int t = 0; t < nt; t++) {
        double ss = 0;
        for (int d = 0; d < D; d++) ss += (double)x[(size_t)t * D + d] * x[(size_t)t * D + d];
        double scale = 1.0 / sqrt(ss / D + (double)eps);
        for (int d = 0; d < D; d++) out[(size_t)t * D + d] = (float)(x[(size_t)t * D + d] * scale);
    }
}
