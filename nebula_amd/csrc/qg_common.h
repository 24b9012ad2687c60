// Device-side helpers shared by the HIP translation units of libqwen_gpu.so.
// CDNA4 (gfx950) only: 64-lane wavefronts, DPP/ds_swizzle cross-lane ops.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#define QG_DEV static __device__ __forceinline__

enum { QG_EXPERTS = 512, QG_TOP = 10, QG_MAX_DECODE = 17, QG_MAX_TOKENS = 8192 };

// GGML type ids on the path (cpu.c:17-30): 0 F32, 12 Q4_K, 20 IQ4_NL; the
// generic path also handles 1 F16, 30 BF16, 2 Q4_0, 6 Q5_0, 7 Q4_1, 8 Q8_0,
// 13 Q5_K, 14 Q6_K.
enum { QT_F32 = 0, QT_F16 = 1, QT_Q4_0 = 2, QT_Q5_0 = 6, QT_Q4_1 = 7, QT_Q8_0 = 8,
       QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14, QT_IQ4_NL = 20, QT_BF16 = 30 };

static inline size_t qg_row_bytes_host(int type, int cols) {  // cpu.c:17-30 / gpu.cu:105-113
    if (cols < 1) return 0;
    switch (type) {
    case QT_F32: return (size_t)cols * 4;
    case QT_F16: case QT_BF16: return (size_t)cols * 2;
    case QT_Q4_0: case QT_IQ4_NL: return cols % 32 ? 0 : (size_t)cols / 32 * 18;
    case QT_Q5_0: return cols % 32 ? 0 : (size_t)cols / 32 * 22;
    case QT_Q4_1: return cols % 32 ? 0 : (size_t)cols / 32 * 24;
    case QT_Q8_0: return cols % 32 ? 0 : (size_t)cols / 32 * 34;
    case QT_Q4_K: return cols % 256 ? 0 : (size_t)cols / 256 * 144;
    case QT_Q5_K: return cols % 256 ? 0 : (size_t)cols / 256 * 176;
    case QT_Q6_K: return cols % 256 ? 0 : (size_t)cols / 256 * 210;
    default: return 0;
    }
}

// fp16 bits -> float, exact for every encoding (cpu.c:31-42 semantics).
QG_DEV float qg_half(const uint8_t *p) {
    uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    return (float)__builtin_bit_cast(_Float16, h);
}
QG_DEV float qg_half_u16(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__constant__ static const int8_t qg_iq4nl_lut[16] = {-127,-104,-83,-65,-49,-35,-22,-10,1,13,25,38,53,69,89,113};

// One dequantised weight, element i of a row (cpu.c:43-67, gpu.cu:121-153).
// Q4_K/Q5_K use fma(d*s, q, -(dmin*m)) as cpu.c:66 does.
QG_DEV float qg_weight_at(const uint8_t *row, int type, int i) {
    if (type == QT_F32) return ((const float *)row)[i];
    if (type == QT_F16) return qg_half(row + 2 * i);
    if (type == QT_BF16) return __uint_as_float((uint32_t)((const uint16_t *)row)[i] << 16);
    if (type == QT_Q8_0) { const uint8_t *p = row + (size_t)(i / 32) * 34; return qg_half(p) * (float)(int8_t)p[2 + i % 32]; }
    if (type == QT_Q4_0 || type == QT_IQ4_NL || type == QT_Q5_0 || type == QT_Q4_1) {
        int bytes = type == QT_Q4_1 ? 24 : type == QT_Q5_0 ? 22 : 18, j = i % 32, off = type == QT_Q4_1 ? 8 : type == QT_Q5_0 ? 6 : 2;
        const uint8_t *p = row + (size_t)(i / 32) * bytes;
        int q = (p[off + j % 16] >> ((j / 16) * 4)) & 15;
        if (type == QT_Q5_0 || type == QT_Q4_1) {
            const uint8_t *hp = p + (type == QT_Q4_1 ? 4 : 2);
            uint32_t high = (uint32_t)hp[0] | ((uint32_t)hp[1] << 8) | ((uint32_t)hp[2] << 16) | ((uint32_t)hp[3] << 24);
            q |= ((high >> j) & 1) << 4;
        }
        if (type == QT_IQ4_NL) return qg_half(p) * (float)qg_iq4nl_lut[q];
        return type == QT_Q4_1 ? __builtin_fmaf(qg_half(p), (float)q, qg_half(p + 2))
                               : qg_half(p) * (float)(q - (type == QT_Q4_0 ? 8 : type == QT_Q5_0 ? 16 : 0));
    }
    int k = i % 256, g = k / 32, l = k % 32;
    const uint8_t *p = row + (size_t)(i / 256) * (type == QT_Q4_K ? 144 : type == QT_Q5_K ? 176 : 210);
    if (type == QT_Q6_K) {
        int h = k / 128, s = (k % 128) / 32;
        int lo = (p[h * 64 + (s % 2) * 32 + l] >> ((s / 2) * 4)) & 15, hi = (p[128 + h * 32 + l] >> (s * 2)) & 3;
        return qg_half(p + 208) * (float)(int8_t)p[192 + h * 8 + s * 2 + l / 16] * (float)((lo | (hi << 4)) - 32);
    }
    const uint8_t *sc = p + 4;
    int s = g < 4 ? (sc[g] & 63) : ((sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4));
    int m = g < 4 ? (sc[g + 4] & 63) : ((sc[g + 4] >> 4) | ((sc[g] >> 6) << 4));
    int q = (p[(type == QT_Q4_K ? 16 : 48) + (g / 2) * 32 + l] >> ((g % 2) * 4)) & 15;
    if (type == QT_Q5_K) q |= ((p[16 + l] >> g) & 1) << 4;
    return __builtin_fmaf(qg_half(p) * (float)s, (float)q, -(qg_half(p + 2) * (float)m));
}

// exp(x) evaluated in double and rounded once to float.  Cody-Waite
// reduction by ln 2 (fdlibm's hi/lo split) and a degree-17 Taylor polynomial
// on |r| <= ln2/2, Horner with fused multiply-adds, exact 2^k scaling.  The
// same statement runs on the host in the test oracle, so routing weights are
// bit-identical on both sides.
QG_DEV double qg_exp_d(double x) {
    if (x != x) return x;
    if (x > 709.782712893384) return __builtin_inf();
    if (x < -745.1332191019412) return 0.0;
    const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
    double kd = __builtin_rint(x * 1.44269504088896338700e+00);
    double r = __builtin_fma(-kd, ln2_hi, x);
    r = __builtin_fma(-kd, ln2_lo, r);
    const double c[18] = {
        1.0, 1.0, 1.0/2.0, 1.0/6.0, 1.0/24.0, 1.0/120.0, 1.0/720.0, 1.0/5040.0, 1.0/40320.0,
        1.0/362880.0, 1.0/3628800.0, 1.0/39916800.0, 1.0/479001600.0, 1.0/6227020800.0,
        1.0/87178291200.0, 1.0/1307674368000.0, 1.0/20922789888000.0, 1.0/355687428096000.0};
    double p = c[17];
#pragma unroll
    for (int n = 16; n >= 0; n--) p = __builtin_fma(p, r, c[n]);
    int k = (int)kd;
    if (k > 1023) { k -= 1023; p *= 8.98846567431157953865e+307; }
    if (k < -1022) { k += 1022; p *= 2.22507385850720138309e-308; }
    return p * __longlong_as_double((long long)((uint64_t)(k + 1023) << 52));
}
QG_DEV float qg_expf(float x) { return (float)qg_exp_d((double)x); }
QG_DEV float qg_sig(float a) { return 1.0f / (1.0f + qg_expf(-a)); }
// SwiGLU as cpu.c:216 writes it: (g*(1/(1+exp(-g))))*u.
QG_DEV float qg_swiglu(float g, float u) { return (g * (1.0f / (1.0f + qg_expf(-g)))) * u; }
// The same with the hardware base-2 exponential and reciprocal (about 1 ulp
// each) for the matrix-core kernels, whose outputs are held to a tolerance
// (the routing weights, which must match exactly, keep qg_expf); a few
// registers instead of the double-precision polynomial's constants.
QG_DEV float qg_swiglu_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// ---- cross-lane helpers (wave64) ----
// Sum over `width` consecutive lanes (power of two <= 64); result in every lane.
template <int WIDTH>
QG_DEV float qg_sum_lanes(float v) {
#pragma unroll
    for (int d = WIDTH / 2; d >= 1; d /= 2) v += __shfl_xor(v, d, WIDTH);
    return v;
}

// DPP-based wave reductions (VALU cross-lane moves instead of LDS-crossbar
// shuffles).  quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror leave every lane of a 16-lane row with the row's result; the
// four rows are then combined from lanes 0/16/32/48 via readlane.
#define QG_DPP_F(v, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false))
QG_DEV float qg_row_max(float v) {
    v = fmaxf(v, QG_DPP_F(v, 0xB1));
    v = fmaxf(v, QG_DPP_F(v, 0x4E));
    v = fmaxf(v, QG_DPP_F(v, 0x141));
    v = fmaxf(v, QG_DPP_F(v, 0x140));
    return v;
}
// Pairwise tree over 32-lane halves with strides 16,8,4,2,1: lane 0 (and 32)
// ends with ((a0+a16)+(a8+a24))+... exactly as cpu.c's reduction
// (cpu_portable.h:333, gpu.cu:89-92); only lanes 0 and 32 are meaningful.
// Stride 16 is a swizzle (lane ^ 16), strides 8..1 rotate within 16-lane
// rows, which gives lanes 0 and 32 the same partners as the strided tree.
QG_DEV float qg_tree32(float v) {
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
    v += QG_DPP_F(v, 0x128);
    v += QG_DPP_F(v, 0x124);
    v += QG_DPP_F(v, 0x122);
    v += QG_DPP_F(v, 0x121);
    return v;
}
QG_DEV float qg_wave_max(float v) {
    v = qg_row_max(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// Sum over each 16-lane row (every lane gets its row's sum).
QG_DEV float qg_row_sum(float v) {
    v += QG_DPP_F(v, 0xB1);
    v += QG_DPP_F(v, 0x4E);
    v += QG_DPP_F(v, 0x141);
    v += QG_DPP_F(v, 0x140);
    return v;
}
// Sum over groups of 8 lanes (every lane gets its group's sum).
QG_DEV float qg_oct_sum(float v) {
    v += QG_DPP_F(v, 0xB1);
    v += QG_DPP_F(v, 0x4E);
    v += QG_DPP_F(v, 0x141);
    return v;
}

// Routing of one token by one wave (gpu.cu:456-465).  On return lane k < 10
// holds the rank-k winner: id (lowest index among equal maxima) and weight
// exp(s - max) / (sum of the 10 numerators in rank order); a token with any
// non-finite logit gets id -1, weight 0 in every rank.  Lanes >= 10 get -1/0.
// Lane l holds logits l, l+64, ..., l+448.  Each of the 10 rounds takes the
// wave maximum (DPP), then the lowest index holding it from per-slot ballots
// (scalar work: the first slot i with a match, its lowest lane), which is the
// winner of the reference's strict-greater scan from index 0.
QG_DEV void qg_route_lane(const float *s, int lane, int &id_out, float &w_out) {
    float v[8];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) { v[i] = s[lane + 64 * i]; bad |= !__builtin_isfinite(v[i]); }
    id_out = -1;
    w_out = 0.0f;
    if (__any(bad)) return;
    float num[QG_TOP], total = 0.0f, largest = 0.0f;
    int best_id[QG_TOP];
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) {
        float lm = v[0];
#pragma unroll
        for (int i = 1; i < 8; i++) lm = fmaxf(lm, v[i]);
        const float m = qg_wave_max(lm);
        if (k == 0) largest = m;
        int bidx = -1;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const unsigned long long b = __ballot(v[i] == m);
            if (bidx < 0 && b) bidx = 64 * i + __builtin_ctzll(b);
        }
        best_id[k] = bidx;
        num[k] = qg_expf(m - largest);
        total += num[k];
#pragma unroll
        for (int i = 0; i < 8; i++) if (bidx == lane + 64 * i) v[i] = -__builtin_inff();
    }
#pragma unroll
    for (int k = 0; k < QG_TOP; k++)
        if (lane == k) { id_out = best_id[k]; w_out = num[k] / total; }
}

// The same routing as qg_route_lane, faster: a threshold T that every top-10
// logit reaches, then an exact rank by (value desc, index asc) among the
// candidates >= T, which is the order of the reference's repeated
// strict-greater argmax.  T: each 16-lane row's three largest distinct lane
// maxima are 12 values held by 12 different lanes; the third smallest of
// them has at least 10 of the 12 lanes at or above it, so at least 10 logits
// reach it and the 10th largest logit does.  (Typically 10-14 candidates; a
// row with fewer than three distinct lane maxima gives -inf, every logit a
// candidate, and the fallback.)  The numerators exp(s - max) are computed in
// parallel (lane k: rank k) and summed in rank order; with weights false they
// are skipped (w_out 0).  lds_v/lds_i: QG_ROUTE_SCRATCH (128) floats / ints
// of wave-private shared memory (entries 64 + lane take the lane's
// non-candidates, so the compaction has no branches).  More than 64
// candidates (heavy ties) falls back to qg_route_lane.  qg_route_vals takes
// the lane's 8 logits s[lane + 64 i] already loaded (s itself is read again
// only by that fallback).
constexpr int QG_ROUTE_SCRATCH = 128;  // entries of each routing scratch array
QG_DEV void qg_route_vals(const float (&v)[8], const float *s, int lane, int &id_out, float &w_out, float *lds_v, int *lds_i,
                          bool weights = true) {
    auto rl = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
    id_out = -1;
    w_out = 0.0f;
    bool bad = false;
    float lm = v[0];
#pragma unroll
    for (int i = 0; i < 8; i++) { bad |= !__builtin_isfinite(v[i]); lm = fmaxf(lm, v[i]); }
    if (__any(bad)) return;
    // the rows' three largest distinct lane maxima (-inf where a row has fewer)
    float cur = lm;
    const float r1 = qg_row_max(cur);
    cur = cur == r1 ? -__builtin_inff() : cur;
    const float r2 = qg_row_max(cur);
    cur = cur == r2 ? -__builtin_inff() : cur;
    const float r3 = qg_row_max(cur);
    float a[12];
#pragma unroll
    for (int rw = 0; rw < 4; rw++) { a[3 * rw] = rl(r1, 16 * rw); a[3 * rw + 1] = rl(r2, 16 * rw); a[3 * rw + 2] = rl(r3, 16 * rw); }
    const float largest = fmaxf(fmaxf(a[0], a[3]), fmaxf(a[6], a[9]));
    // T = the third smallest of the 12 (the three smallest kept in order)
    float m0 = a[0], m1 = __builtin_inff(), m2 = __builtin_inff();
#pragma unroll
    for (int i = 1; i < 12; i++) {
        m2 = fminf(m2, fmaxf(m1, a[i]));
        m1 = fminf(m1, fmaxf(m0, a[i]));
        m0 = fminf(m0, a[i]);
    }
    const float T = m2;
    // candidates v >= T, compacted in lane order: exclusive prefix sum of the
    // lane's count (0..8) from bit-sliced ballots
    int c = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) c += v[i] >= T;
    int pos = 0, total_c = 0;
#pragma unroll
    for (int bit = 0; bit < 4; bit++) {
        const unsigned long long b = __ballot((c >> bit) & 1);
        pos += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u)) << bit;
        total_c += __popcll(b) << bit;
    }
    if (total_c > 64) { qg_route_lane(s, lane, id_out, w_out); return; }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const bool cand = v[i] >= T;
        const int at = cand ? pos : 64 + lane;
        lds_v[at] = v[i];
        lds_i[at] = lane + 64 * i;
        pos += cand;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rank of candidate `lane` among the total_c candidates, every lane
    // reading candidates 0..15 from shared memory at once (the same
    // addresses in every lane; entries past total_c are not counted), then
    // any further ones one by one
    const float cv = lane < total_c ? lds_v[lane] : 0.0f;
    const int ci = lane < total_c ? lds_i[lane] : 0;
    int rank = 0;
    {
        float4 ov[4];
        int4 oi[4];
#pragma unroll
        for (int c4 = 0; c4 < 4; c4++) {
            ov[c4] = ((const float4 *)lds_v)[c4];
            oi[c4] = ((const int4 *)lds_i)[c4];
        }
#pragma unroll
        for (int c4 = 0; c4 < 4; c4++) {
            const float o_v[4] = {ov[c4].x, ov[c4].y, ov[c4].z, ov[c4].w};
            const int o_i[4] = {oi[c4].x, oi[c4].y, oi[c4].z, oi[c4].w};
#pragma unroll
            for (int u = 0; u < 4; u++)
                rank += (4 * c4 + u < total_c) & ((o_v[u] > cv) | ((o_v[u] == cv) & (o_i[u] < ci)));
        }
    }
    for (int q = 16; q < total_c; q++) {
        const float ov = lds_v[q];
        const int oi = lds_i[q];
        rank += (ov > cv) | ((ov == cv) & (oi < ci));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < total_c && rank < QG_TOP) { lds_v[rank] = cv; lds_i[rank] = ci; }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < QG_TOP) id_out = lds_i[lane];
    if (!weights) return;  // wave-uniform
    // the numerators (lane k: rank k) through shared memory, summed in rank
    // order by every lane
    const float num = lane < QG_TOP ? qg_expf(lds_v[lane] - largest) : 0.0f;
    if (lane < QG_TOP) lds_v[lane] = num;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float nk[12];
    *(float4 *)&nk[0] = ((const float4 *)lds_v)[0];
    *(float4 *)&nk[4] = ((const float4 *)lds_v)[1];
    *(float4 *)&nk[8] = ((const float4 *)lds_v)[2];
    static_assert(QG_TOP <= 12, "the numerators fit three 16-byte reads");
    float total = 0.0f;
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) total += nk[k];
    if (lane < QG_TOP) w_out = num / total;
}
QG_DEV void qg_route_fast(const float *s, int lane, int &id_out, float &w_out, float *lds_v, int *lds_i, bool weights = true) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = s[lane + 64 * i];
    qg_route_vals(v, s, lane, id_out, w_out, lds_v, lds_i, weights);
}

// Two tokens per wave, one per 32-lane half h: the routing of qg_route_fast
// with 16 logits per lane (lane l of half h holds row_h[l], row_h[l+32], ...).
// The threshold is the 10th largest of the half's 32 lane maxima (counting
// equal values separately), so at least 10 logits reach it; the candidates
// >= T are ranked exactly as there.  On return lane 32h + k (k < 10) holds the
// rank-k id and weight of token h, other lanes -1/0.  A half with a
// non-finite logit gets -1/0; a half with more than 32 candidates (heavy
// ties) is not routed here: fb_h is set (wave-uniform) and the caller routes
// that token with qg_route_lane.  lds_v/lds_i: 64 floats / 64 ints of
// wave-private shared memory (32 per half).
QG_DEV void qg_route_pair(const float *row, int lane, int &id_out, float &w_out, float *lds_v, int *lds_i, bool &fb0,
                          bool &fb1) {
    const int h = lane >> 5, l = lane & 31;
    const unsigned long long hm = h ? 0xFFFFFFFF00000000ull : 0x00000000FFFFFFFFull;
    const unsigned long long below = (1ull << lane) - 1ull;
    float v[16];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 16; i++) { v[i] = row[l + 32 * i]; bad |= !__builtin_isfinite(v[i]); }
    const unsigned long long bb = __ballot(bad);
    const bool bad0 = (bb & 0xFFFFFFFFull) != 0, bad1 = (bb >> 32) != 0, mybad = h ? bad1 : bad0;
    if (mybad) {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.0f;  // a harmless routing whose result is discarded
    }
    float lm = v[0];
#pragma unroll
    for (int i = 1; i < 16; i++) lm = fmaxf(lm, v[i]);
    // threshold per half: walk down the distinct lane maxima until 10 lanes are covered
    float largest = 0.0f, T = 0.0f, cur = lm;
    int remaining = QG_TOP;
    bool done = false;
    for (int r = 0; r < QG_TOP; r++) {
        const float rm = qg_row_max(cur);
        const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 0));
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 16));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 32));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 48));
        const float m = h ? fmaxf(r2, r3) : fmaxf(r0, r1);
        if (r == 0) largest = m;
        const int cnt = __popcll(__ballot(cur == m) & hm);
        if (!done) {
            T = m;
            if (cnt >= remaining) done = true;
            else remaining -= cnt;
        }
        if (__ballot(!done) == 0) break;
        cur = (!done && cur == m) ? -__builtin_inff() : cur;
    }
    // candidates v >= T, compacted in lane order within the half
    int c = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) c += v[i] >= T;
    int pos = 0, tc0 = 0, tc1 = 0;
#pragma unroll
    for (int bit = 0; bit < 5; bit++) {
        const unsigned long long b = __ballot((c >> bit) & 1);
        pos += __popcll(b & hm & below) << bit;
        tc0 += __popcll(b & 0xFFFFFFFFull) << bit;
        tc1 += __popcll(b >> 32) << bit;
    }
    fb0 = !bad0 && tc0 > 32;
    fb1 = !bad1 && tc1 > 32;
    const int total_c = h ? tc1 : tc0;
    const bool ok = total_c <= 32;
    float *hv = lds_v + 32 * h;
    int *hi = lds_i + 32 * h;
    if (ok) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (v[i] >= T) { hv[pos] = v[i]; hi[pos] = l + 32 * i; pos++; }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rank of candidate l among the half's candidates
    const bool mine = ok && l < total_c;
    const float cv = mine ? hv[l] : 0.0f;
    const int ci = mine ? hi[l] : 0;
    const int qm = max(tc0 <= 32 ? tc0 : 0, tc1 <= 32 ? tc1 : 0);
    int rank = 0;
    for (int q = 0; q < qm; q++) {  // candidate q of each half from its lane's registers (wave-uniform q)
        const float o0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), q));
        const float o1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), 32 + q));
        const int i0 = __builtin_amdgcn_readlane(ci, q), i1 = __builtin_amdgcn_readlane(ci, 32 + q);
        const float ov = h ? o1 : o0;
        const int oi = h ? i1 : i0;
        if (q < total_c) rank += (ov > cv) | ((ov == cv) & (oi < ci));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (mine && rank < QG_TOP) { hv[rank] = cv; hi[rank] = ci; }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool win = ok && !mybad && l < QG_TOP;
    const float num = win ? qg_expf(hv[l] - largest) : 0.0f;
    float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) {
        t0 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), k));
        t1 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), 32 + k));
    }
    id_out = win ? hi[l] : -1;
    w_out = win ? num / (h ? t1 : t0) : 0.0f;
}

// Routing of one token written to ids[0..9] / w[0..9] by lanes 0..9
// (lds_v/lds_i as for qg_route_fast).
QG_DEV void qg_route_wave(int *ids, float *w, const float *s, int lane, float *lds_v, int *lds_i) {
    int id;
    float wv;
    qg_route_fast(s, lane, id, wv, lds_v, lds_i);
    if (lane < QG_TOP) { ids[lane] = id; w[lane] = wv; }
}

// Routing of tokens ta (lanes 0-31) and tb (lanes 32-63; tb == ta routes one
// token) of a [nt][ld] logit matrix, written to rows ta/tb of ids and w; a
// half with heavy ties is routed again by the whole wave.
QG_DEV void qg_route_wave2(int *ids, float *w, const float *logits, int ld, int ta, int tb, int lane, float *lds_v,
                           int *lds_i) {
    int id;
    float wv;
    bool fb0, fb1;
    const int h = lane >> 5, k = lane & 31, t = h ? tb : ta;
    qg_route_pair(logits + (size_t)t * ld, lane, id, wv, lds_v, lds_i, fb0, fb1);
    if (k < QG_TOP && !(h ? fb1 : fb0) && (h == 0 || tb != ta)) {
        ids[(size_t)t * QG_TOP + k] = id;
        w[(size_t)t * QG_TOP + k] = wv;
    }
    if (fb0) qg_route_wave(ids + (size_t)ta * QG_TOP, w + (size_t)ta * QG_TOP, logits + (size_t)ta * ld, lane, lds_v, lds_i);
    if (fb1 && tb != ta)
        qg_route_wave(ids + (size_t)tb * QG_TOP, w + (size_t)tb * QG_TOP, logits + (size_t)tb * ld, lane, lds_v, lds_i);
}

// Coverage of one routed token (gpu.cu:467-483 with the 0.10 rule of
// config.py:9): lane k < 10 holds rank k's (id, weight).  mass is the double
// sum, in rank order, of the weights of non-resident experts.  Returns the
// flag 0 (all resident), 1 (pruned: missing > 0 and mass < threshold; the
// lane's non-resident id becomes -id-2 and its weight 0, no renormalisation),
// 2 (handoff: missing > 0 and !(mass < threshold)) or 3 (an id outside
// [0,512): uncounted).  resident == NULL means every expert is resident.
QG_DEV int qg_route_cover(int &id, float &wv, const uint8_t *resident, double thr, int &missing, double &mass) {
    const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const bool mine = lane < QG_TOP, valid = id >= 0 && id < QG_EXPERTS;
    // one residency lookup per lane, all in flight together
    const bool nonres = mine && valid && resident && !resident[id];
    const unsigned long long nb = __ballot(nonres);
    const bool bad = __ballot(mine && !valid) != 0;
    missing = __popcll(nb);
    mass = 0.0;
    if (nb) {  // wave-uniform
#pragma unroll
        for (int k = 0; k < QG_TOP; k++)
            if ((nb >> k) & 1) mass += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), k));
    }
    const int flag = bad ? 3 : !missing ? 0 : (thr > 0 && mass < thr) ? 1 : 2;
    if (flag == 1 && nonres) { id = -id - 2; wv = 0.0f; }
    return flag;
}

// qg_route_cover for the two tokens of qg_route_pair: lane 32h + k (k < 10)
// holds rank k of token h; each half gets its own flag, missing and mass
// (same rank-order double sum).
QG_DEV int qg_route_cover_half(int &id, float &wv, const uint8_t *resident, double thr, int &missing, double &mass) {
    const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int h = lane >> 5;
    const bool mine = (lane & 31) < QG_TOP, valid = id >= 0 && id < QG_EXPERTS;
    const bool nonres = mine && valid && resident && !resident[id];
    const unsigned long long nb = __ballot(nonres), vb = __ballot(mine && !valid);
    const uint32_t nb0 = (uint32_t)nb, nb1 = (uint32_t)(nb >> 32);
    const bool bad = (h ? (uint32_t)(vb >> 32) : (uint32_t)vb) != 0u;
    missing = __popc(h ? nb1 : nb0);
    double m0 = 0.0, m1 = 0.0;
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) {
        const double a = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), k));
        const double b = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), 32 + k));
        if ((nb0 >> k) & 1) m0 += a;
        if ((nb1 >> k) & 1) m1 += b;
    }
    mass = h ? m1 : m0;
    const int flag = bad ? 3 : !missing ? 0 : (thr > 0 && mass < thr) ? 1 : 2;
    if (flag == 1 && nonres) { id = -id - 2; wv = 0.0f; }
    return flag;
}

// 16 bytes from global memory with one 128-bit load (address 4-byte aligned).
QG_DEV uint4 qg_ld16(const uint8_t *p) { return *(const uint4 *)p; }

// ---- operand helpers shared by the matrix-core kernels ----
typedef _Float16 qg_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 qg_half2 __attribute__((ext_vector_type(2)));
typedef float qg_f4 __attribute__((ext_vector_type(4)));
typedef int qg_i4 __attribute__((ext_vector_type(4)));

QG_DEV int qg_perm8(int e) { return (e & 4) | ((e & 1) << 1) | ((e & 2) >> 1); }  // 0,2,1,3,4,6,5,7 self-inverse

// IQ4_NL table lookup of four 4-bit indices (one per byte) with v_perm: the
// table is stored +128 as unsigned bytes; callers remove the bias.
QG_DEV uint32_t iq4_lookup(uint32_t idx) {
    // lut + 128 = {1,24,45,63, 79,93,106,118, 129,141,153,166, 181,197,217,241}
    const uint32_t T0 = 0x3F2D1801u, T1 = 0x766A5D4Fu, T2 = 0xA6998D81u, T3 = 0xF1D9C5B5u;
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    // byte i from hi (permute selector 4 + i) where bit 3 of index i is set,
    // else from lo (selector i); the identity selector as an opaque register
    // value makes the mask-and-insert one v_and_or_b32
    uint32_t I;
    asm("v_mov_b32 %0, 0x03020100" : "=v"(I));
    return __builtin_amdgcn_perm(hi, lo, ((idx >> 1) & 0x04040404u) | I);
}

// 8 nibbles of one byte octet (low or high half) times s -> fp16 fragment,
// element order (0,2),(1,3),(4,6),(5,7).  Each nibble is masked in place under
// the exponent byte 0x64: a low nibble q reads as fp16 1024 + q, a high one as
// 1024 + 16q, and (1024+q)*s - 1024*s, (1024+16q)*(s/16) - 64*s are both q*s,
// exact (q*s <= 945; one rounding in the fused multiply-add).
QG_DEV qg_half8 q4_frag(uint2 b, int hi_nib, _Float16 s) {
    // E as an opaque register value lets each mask-and-insert be one v_and_or_b32
    // (a VOP3 instruction takes at most one literal or scalar operand here)
    uint32_t E;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(E));
    const uint32_t m = hi_nib ? 0x00F000F0u : 0x000F000Fu;
    const uint32_t u[4] = {(b.x & m) | E, ((b.x >> 8) & m) | E, (b.y & m) | E, ((b.y >> 8) & m) | E};
    const _Float16 sc = hi_nib ? s * (_Float16)0.0625f : s, of = hi_nib ? (_Float16)(-64.0f) * s : (_Float16)(-1024.0f) * s;
    const qg_half2 sv = {sc, sc}, off = {of, of};
    qg_half8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const qg_half2 h = __builtin_bit_cast(qg_half2, u[i]);
        const qg_half2 v = __builtin_elementwise_fma(h, sv, off);
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// 8 IQ4_NL nibbles (4 bytes, one half) -> table values as fp16, same order.
QG_DEV qg_half8 iq4_frag(uint32_t b0, uint32_t b1, int hi_nib) {
    const uint32_t i0 = (hi_nib ? b0 >> 4 : b0) & 0x0F0F0F0Fu, i1 = (hi_nib ? b1 >> 4 : b1) & 0x0F0F0F0Fu;
    const uint32_t l0 = iq4_lookup(i0), l1 = iq4_lookup(i1);  // lut + 128 as bytes
    const uint32_t u[4] = {(l0 & 0x00FF00FFu) | 0x64006400u, ((l0 >> 8) & 0x00FF00FFu) | 0x64006400u,
                           (l1 & 0x00FF00FFu) | 0x64006400u, ((l1 >> 8) & 0x00FF00FFu) | 0x64006400u};
    const qg_half2 off = {(_Float16)(-1152.0f), (_Float16)(-1152.0f)};
    qg_half8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const qg_half2 v = __builtin_bit_cast(qg_half2, u[i]) + off;
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}


// The 8 scales and mins of a Q4_K superblock header as integers.
struct Q4kHeader { float d, dmin; uint32_t S[2], M[2]; };
QG_DEV Q4kHeader q4k_header(uint4 hd) {
    Q4kHeader h;
    h.d = qg_half_u16(hd.x & 0xffffu);
    h.dmin = qg_half_u16(hd.x >> 16);
    h.S[0] = hd.y & 0x3F3F3F3Fu;
    h.M[0] = hd.z & 0x3F3F3F3Fu;
    h.S[1] = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    h.M[1] = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    return h;
}
QG_DEV int q4k_s(const Q4kHeader &h, int g) { return (h.S[g >> 2] >> (8 * (g & 3))) & 0xff; }
QG_DEV int q4k_m(const Q4kHeader &h, int g) { return (h.M[g >> 2] >> (8 * (g & 3))) & 0xff; }
// The 8 mins m_0..m_7 of a superblock as an fp16 fragment in group order: a
// byte permute puts each 6-bit value under the exponent byte 0x64 (1024 + m),
// one packed add removes the 1024.
QG_DEV qg_half8 q4k_min_frag(const Q4kHeader &h) {
    const uint32_t X = 0x64646464u;
    const uint32_t u[4] = {__builtin_amdgcn_perm(X, h.M[0], 0x04010400u), __builtin_amdgcn_perm(X, h.M[0], 0x04030402u),
                           __builtin_amdgcn_perm(X, h.M[1], 0x04010400u), __builtin_amdgcn_perm(X, h.M[1], 0x04030402u)};
    const qg_half2 off = {(_Float16)(-1024.0f), (_Float16)(-1024.0f)};
    qg_half8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const qg_half2 v = __builtin_bit_cast(qg_half2, u[i]) + off;
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}
// the same 6-bit values as fp16 (one integer-to-half conversion)
QG_DEV _Float16 q4k_sh(const Q4kHeader &h, int g) { return (_Float16)(unsigned short)q4k_s(h, g); }
QG_DEV _Float16 q4k_mh(const Q4kHeader &h, int g) { return (_Float16)(unsigned short)q4k_m(h, g); }
