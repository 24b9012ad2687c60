// Device generator of synthetic layer inputs (benchmark and test support; not
// a reference interface).  Gaussian values come from Box-Muller over a
// splitmix64 hash of (seed, stream, index) with this file's own double
// ln/cos/sqrt; encoders write legal GGML Q4_K / IQ4_NL blocks.  Only integer
// ops and correctly rounded IEEE ops (+,-,*,/,fma,rint,floor) are used, with
// contraction off, so the bytes equal the host statement in the test oracle.
#include "qg_internal.h"

#pragma clang fp contract(off)

namespace {

QG_DEV uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
QG_DEV uint64_t hash3(uint64_t seed, uint64_t stream, uint64_t index) { return mix64(mix64(mix64(seed) ^ stream) ^ index); }
QG_DEV double from_bits(uint64_t b) { return __longlong_as_double((long long)b); }
QG_DEV uint64_t to_bits(double d) { return (uint64_t)__double_as_longlong(d); }

QG_DEV double syn_log(double u) {
    const uint64_t b = to_bits(u);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = from_bits((b & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL);
    if (m > 1.4142135623730951) { m *= 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double p = 1.0 / 25.0;
    for (int k = 11; k >= 0; k--) p = __builtin_fma(p, s2, 1.0 / (double)(2 * k + 1));
    const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
    return __builtin_fma((double)e, ln2_hi, __builtin_fma((double)e, ln2_lo, 2.0 * s * p));
}
QG_DEV double syn_sqrt(double v) {
    double y = from_bits((to_bits(v) >> 1) + 0x1FF8000000000000ULL);
    for (int i = 0; i < 6; i++) y = 0.5 * (y + v / y);
    return y;
}
QG_DEV double syn_sin(double a) {
    const double c[9] = {1.0, -1.0/6.0, 1.0/120.0, -1.0/5040.0, 1.0/362880.0, -1.0/39916800.0,
                         1.0/6227020800.0, -1.0/1307674368000.0, 1.0/355687428096000.0};
    double a2 = a * a, p = -1.0 / 121645100408832000.0;
    for (int k = 8; k >= 0; k--) p = __builtin_fma(p, a2, c[k]);
    return a * p;
}
QG_DEV double syn_cos(double a) {
    const double c[9] = {1.0, -1.0/2.0, 1.0/24.0, -1.0/720.0, 1.0/40320.0, -1.0/3628800.0,
                         1.0/479001600.0, -1.0/87178291200.0, 1.0/20922789888000.0};
    double a2 = a * a, p = 1.0 / 6402373705728000.0;
    for (int k = 8; k >= 0; k--) p = __builtin_fma(p, a2, c[k]);
    return p;
}
QG_DEV double syn_cos2pi(double t) {
    const double t4 = 4.0 * t, q = __builtin_floor(t4), f = t4 - q;
    const double half_pi = 1.57079632679489661923;
    const double c = f <= 0.5 ? syn_cos(half_pi * f) : syn_sin(half_pi * (1.0 - f));
    const double s = f <= 0.5 ? syn_sin(half_pi * f) : syn_cos(half_pi * (1.0 - f));
    const int qi = (int)q;
    return qi == 0 ? c : qi == 1 ? -s : qi == 2 ? -c : s;
}
QG_DEV double gauss(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t h = hash3(seed, stream, index);
    const double u1 = ((double)(h >> 32) + 0.5) * 2.3283064365386962890625e-10;
    const double u2 = (double)(h & 0xffffffffULL) * 2.3283064365386962890625e-10;
    return syn_sqrt(-2.0 * syn_log(u1)) * syn_cos2pi(u2);
}

QG_DEV uint32_t f32_to_f16(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000, ex = (x >> 23) & 0xff;
    uint32_t m = x & 0x7fffff;
    if (ex == 0xff) return sign | 0x7c00 | (m ? 0x200 : 0);
    const int e = (int)ex - 127 + 15;
    if (e >= 31) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        m |= 0x800000;
        const int shift = 14 - e;
        uint32_t hm = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return sign | hm;
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return h;
}
QG_DEV double f16_to_f64(uint32_t h) { return (double)qg_half_u16(h); }
QG_DEV double clampd(double v, double lo, double hi) { return v < lo ? lo : v > hi ? hi : v; }

// One Q4_K superblock from 256 values (same steps as the host encoder).
// Bytes are written straight to `blk`; every per-group array is indexed by
// unrolled loops only, so it lives in registers.
QG_DEV void encode_q4k(uint8_t *blk, const float *x) {
    double scale[8], offs[8], maxs = 0, maxm = 0;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        double lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) { const double v = x[g * 32 + l]; if (v < lo) lo = v; if (v > hi) hi = v; }
        scale[g] = (hi - lo) / 15.0;
        offs[g] = -lo;
        if (scale[g] > maxs) maxs = scale[g];
        if (offs[g] > maxm) maxm = offs[g];
    }
    const uint32_t d16 = f32_to_f16((float)(maxs / 63.0)), m16 = f32_to_f16((float)(maxm / 63.0));
    const double d = f16_to_f64(d16), dm = f16_to_f64(m16);
    int s[8], m[8];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        s[g] = d > 0 ? (int)clampd(__builtin_rint(scale[g] / d), 0, 63) : 0;
        m[g] = dm > 0 ? (int)clampd(__builtin_rint(offs[g] / dm), 0, 63) : 0;
    }
    blk[0] = (uint8_t)d16; blk[1] = (uint8_t)(d16 >> 8); blk[2] = (uint8_t)m16; blk[3] = (uint8_t)(m16 >> 8);
#pragma unroll
    for (int g = 0; g < 4; g++) {
        blk[4 + g] = (uint8_t)((s[g] & 63) | ((s[g + 4] >> 4) << 6));
        blk[8 + g] = (uint8_t)((m[g] & 63) | ((m[g + 4] >> 4) << 6));
        blk[12 + g] = (uint8_t)((s[g + 4] & 15) | ((m[g + 4] & 15) << 4));
    }
#pragma unroll
    for (int gp = 0; gp < 4; gp++) {
        const double step0 = d * (double)s[2 * gp], off0 = dm * (double)m[2 * gp];
        const double step1 = d * (double)s[2 * gp + 1], off1 = dm * (double)m[2 * gp + 1];
        for (int l = 0; l < 32; l++) {
            const int q0 = step0 > 0 ? (int)clampd(__builtin_rint(((double)x[2 * gp * 32 + l] + off0) / step0), 0, 15) : 0;
            const int q1 = step1 > 0 ? (int)clampd(__builtin_rint(((double)x[(2 * gp + 1) * 32 + l] + off1) / step1), 0, 15) : 0;
            blk[16 + gp * 32 + l] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// Nearest IQ4_NL table entry of v (lowest index on ties, the host encoder's
// strict-less scan).
QG_DEV int iq4nl_nearest(double v) {
    constexpr int lut[16] = {-127,-104,-83,-65,-49,-35,-22,-10,1,13,25,38,53,69,89,113};
    double err = __builtin_fabs(v - lut[0]);
    int best = 0;
#pragma unroll
    for (int q = 1; q < 16; q++) { const double e = __builtin_fabs(v - lut[q]); if (e < err) { err = e; best = q; } }
    return best;
}

QG_DEV void encode_iq4nl(uint8_t *blk, const float *x) {
    double amax = 0;
    for (int j = 0; j < 32; j++) { const double a = __builtin_fabs((double)x[j]); if (a > amax) amax = a; }
    const uint32_t d16 = f32_to_f16((float)(amax / 127.0));
    const double d = f16_to_f64(d16);
    blk[0] = (uint8_t)d16; blk[1] = (uint8_t)(d16 >> 8);
    for (int j = 0; j < 16; j++) {
        const int q0 = d > 0 ? iq4nl_nearest((double)x[j] / d) : 8;
        const int q1 = d > 0 ? iq4nl_nearest((double)x[j + 16] / d) : 8;
        blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

// One thread per quantisation block (256 values for Q4_K, 32 for IQ4_NL, 1
// for F32) of `experts` consecutive matrices: matrix e (stream base | e) sits
// e * rows * rb bytes after `out`.  A block's values are staged in shared
// memory (no per-thread scratch memory).
constexpr int SYN_THREADS = 32;
__global__ __launch_bounds__(SYN_THREADS) void synth_kernel(uint8_t *out, int type, uint64_t seed, uint64_t stream, int experts,
                                                            int rows, int cols, float sigma, size_t rb) {
    __shared__ float stage[SYN_THREADS * 256];
    const int block = type == QT_Q4_K ? 256 : type == QT_IQ4_NL ? 32 : 1;
    const size_t per_row = (size_t)(cols / block), per_expert = (size_t)rows * per_row;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= per_expert * (size_t)experts) return;
    const int e = (int)(i / per_expert);
    const size_t j = i % per_expert;
    const int r = (int)(j / per_row), c0 = (int)(j % per_row) * block;
    const uint64_t st = stream | (uint64_t)(uint32_t)e;
    float *v = stage + threadIdx.x * 256;
    for (int k = 0; k < block; k++) v[k] = (float)((double)sigma * gauss(seed, st, (uint64_t)r * cols + c0 + k));
    uint8_t *dst = out + ((size_t)e * rows + r) * rb;
    if (type == QT_F32) *(float *)(dst + (size_t)c0 * 4) = v[0];
    else if (type == QT_Q4_K) encode_q4k(dst + (size_t)(c0 / 256) * 144, v);
    else encode_iq4nl(dst + (size_t)(c0 / 32) * 18, v);
}

int synth_launch(void *out, int type, uint64_t seed, uint64_t stream, int experts, int rows, int cols, float sigma) {
    const size_t rb = qg_row_bytes_host(type, cols);
    if (!out || !rb || rows < 1 || experts < 1 || (type != QT_F32 && type != QT_Q4_K && type != QT_IQ4_NL)) return hipErrorInvalidValue;
    const int block = type == QT_Q4_K ? 256 : type == QT_IQ4_NL ? 32 : 1;
    const size_t n = (size_t)experts * rows * (cols / block);
    if ((n + SYN_THREADS - 1) / SYN_THREADS > 0x7fffffffULL) return hipErrorInvalidValue;
    synth_kernel<<<(unsigned)((n + SYN_THREADS - 1) / SYN_THREADS), SYN_THREADS, 0, qg_stream()>>>(
        (uint8_t *)out, type, seed, stream, experts, rows, cols, sigma, rb);
    return hipGetLastError();
}

}  // namespace

extern "C" int qg_synth_matrix(void *out, int type, uint64_t seed, uint64_t stream, int rows, int cols, float sigma) {
    return synth_launch(out, type, seed, stream, 1, rows, cols, sigma);
}

extern "C" int qg_synth_experts(void *out, int type, uint64_t seed, int tensor, int experts, int rows, int cols, float sigma) {
    if (tensor < 0) return hipErrorInvalidValue;
    return synth_launch(out, type, seed, (uint64_t)(uint32_t)tensor << 32, experts, rows, cols, sigma);
}
