/* CPU mirror of the device synthetic-input generator: TEST INFRASTRUCTURE.
 *
 * The bench generates its expert weights on the GPU (nebula_amd/csrc/
 * nb_synth.hip); this file states the same generator on the CPU so that
 * tests can (a) check the device bytes bit-for-bit at small sizes and
 * (b) build identical inputs without a GPU.  Every step uses only IEEE
 * operations that are exact or correctly rounded on both sides (integer
 * ops, +, -, *, /, fma, rint), so both sides produce identical bytes.
 *
 * Gaussian: Box-Muller, z = sqrt(-2 ln u1) cos(2 pi u2), with u1, u2 the two
 * 32-bit halves of a splitmix64 hash of (seed, stream, index).  ln, cos and
 * sqrt are this file's own double-precision routines (atanh series, Taylor
 * polynomials, Newton iteration), not libm's, so nothing depends on a math
 * library's last-bit behaviour.
 *
 * Encoders write legal GGML blocks (layouts of cpu.c:43-67): Q4_K with
 * per-group min/max scales quantised to 6 bits, IQ4_NL with the nearest
 * table entry.  They are this project's own simple encoders; the reference
 * quantises with GGML's ggml_quantize_chunk (third party, not vendored), and
 * layer parity does not depend on the encoder because both sides consume the
 * same bytes. */
#include "nb_oracle.h"
#include <math.h>
#include <string.h>

static uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

uint64_t nbs_hash(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(mix64(mix64(seed) ^ stream) ^ index);
}

uint64_t nbs_stream(int tensor, int expert) { return ((uint64_t)(uint32_t)tensor << 32) | (uint32_t)expert; }

static double from_bits(uint64_t b) { double d; memcpy(&d, &b, 8); return d; }
static uint64_t to_bits(double d) { uint64_t b; memcpy(&b, &d, 8); return b; }

/* ln(u) for normal u > 0: u = m 2^e, m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s),
 * s = (m-1)/(m+1), |s| <= 0.1716, series to s^25. */
static double syn_log(double u) {
    uint64_t b = to_bits(u);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = from_bits((b & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL);
    if (m > 1.4142135623730951) { m *= 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double p = 1.0 / 25.0;
    for (int k = 11; k >= 0; k--) p = fma(p, s2, 1.0 / (double)(2 * k + 1));
    const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
    return fma((double)e, ln2_hi, fma((double)e, ln2_lo, 2.0 * s * p));
}

/* sqrt(v), v > 0 normal: exponent-halving first guess, six Newton steps. */
static double syn_sqrt(double v) {
    double y = from_bits((to_bits(v) >> 1) + 0x1FF8000000000000ULL);
    for (int i = 0; i < 6; i++) y = 0.5 * (y + v / y);
    return y;
}

/* sin and cos of a in [0, pi/4]: Taylor to degree 19 / 18. */
static double syn_sin(double a) {
    double a2 = a * a, p = -1.0 / 121645100408832000.0; /* -1/19! */
    static const double c[9] = {1.0, -1.0/6.0, 1.0/120.0, -1.0/5040.0, 1.0/362880.0, -1.0/39916800.0,
                                1.0/6227020800.0, -1.0/1307674368000.0, 1.0/355687428096000.0};
    for (int k = 8; k >= 0; k--) p = fma(p, a2, c[k]);
    return a * p;
}
static double syn_cos(double a) {
    double a2 = a * a, p = 1.0 / 6402373705728000.0; /* 1/18! */
    static const double c[9] = {1.0, -1.0/2.0, 1.0/24.0, -1.0/720.0, 1.0/40320.0, -1.0/3628800.0,
                                1.0/479001600.0, -1.0/87178291200.0, 1.0/20922789888000.0};
    for (int k = 8; k >= 0; k--) p = fma(p, a2, c[k]);
    return p;
}

/* cos(2 pi t), t in [0,1): quadrant q = floor(4t), f = 4t - q (both exact). */
static double syn_cos2pi(double t) {
    double t4 = 4.0 * t, q = floor(t4), f = t4 - q;
    const double half_pi = 1.57079632679489661923;
    double c = f <= 0.5 ? syn_cos(half_pi * f) : syn_sin(half_pi * (1.0 - f));
    double s = f <= 0.5 ? syn_sin(half_pi * f) : syn_cos(half_pi * (1.0 - f));
    int qi = (int)q;
    return qi == 0 ? c : qi == 1 ? -s : qi == 2 ? -c : s;
}

double nbs_gauss(uint64_t seed, uint64_t stream, uint64_t index) {
    uint64_t h = nbs_hash(seed, stream, index);
    double u1 = ((double)(h >> 32) + 0.5) * 2.3283064365386962890625e-10; /* 2^-32 */
    double u2 = (double)(h & 0xffffffffULL) * 2.3283064365386962890625e-10;
    return syn_sqrt(-2.0 * syn_log(u1)) * syn_cos2pi(u2);
}

/* float -> fp16 bits, round to nearest even, with subnormals and overflow. */
uint16_t nbs_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000, ex = (x >> 23) & 0xff, m = x & 0x7fffff;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00 | (m ? 0x200 : 0));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000;
        int shift = 14 - e;
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (m >> 13), rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return (uint16_t)h;
}

float nbs_f16_to_f32(uint16_t h) { uint8_t b[2] = {(uint8_t)h, (uint8_t)(h >> 8)}; return nbo_half(b); }

static double clampd(double v, double lo, double hi) { return v < lo ? lo : v > hi ? hi : v; }

/* Q4_K: 8 groups of 32; group scale (max-min)/15 and offset -min (min<=0),
 * both quantised to 6 bits against fp16 super-scales d = max scale/63,
 * dmin = max offset/63; nibbles rint((x + dmin*m)/(d*s)) clamped to 0..15.
 * Packing inverts the decode of cpu.c:61-64. */
void nbs_encode_q4k(uint8_t *blk, const float *x) {
    double scale[8], offs[8], maxs = 0, maxm = 0;
    for (int g = 0; g < 8; g++) {
        double lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) { double v = x[g*32 + l]; if (v < lo) lo = v; if (v > hi) hi = v; }
        scale[g] = (hi - lo) / 15.0; offs[g] = -lo;
        if (scale[g] > maxs) maxs = scale[g];
        if (offs[g] > maxm) maxm = offs[g];
    }
    uint16_t d16 = nbs_f32_to_f16((float)(maxs / 63.0)), m16 = nbs_f32_to_f16((float)(maxm / 63.0));
    double d = nbs_f16_to_f32(d16), dm = nbs_f16_to_f32(m16);
    int s[8], m[8];
    for (int g = 0; g < 8; g++) {
        s[g] = d > 0 ? (int)clampd(rint(scale[g] / d), 0, 63) : 0;
        m[g] = dm > 0 ? (int)clampd(rint(offs[g] / dm), 0, 63) : 0;
    }
    memset(blk, 0, 144);
    blk[0] = (uint8_t)d16; blk[1] = (uint8_t)(d16 >> 8); blk[2] = (uint8_t)m16; blk[3] = (uint8_t)(m16 >> 8);
    uint8_t *sc = blk + 4;
    for (int g = 0; g < 4; g++) {
        sc[g] = (uint8_t)((s[g] & 63) | ((s[g + 4] >> 4) << 6));
        sc[g + 4] = (uint8_t)((m[g] & 63) | ((m[g + 4] >> 4) << 6));
        sc[g + 8] = (uint8_t)((s[g + 4] & 15) | ((m[g + 4] & 15) << 4));
    }
    for (int g = 0; g < 8; g++) {
        double step = d * (double)s[g], off = dm * (double)m[g];
        for (int l = 0; l < 32; l++) {
            int q = step > 0 ? (int)clampd(rint(((double)x[g*32 + l] + off) / step), 0, 15) : 0;
            blk[16 + (g/2)*32 + l] |= (uint8_t)(q << ((g % 2) * 4));
        }
    }
}

/* IQ4_NL: fp16 scale amax/127, each value the nearest table entry (ties to
 * the lower index); nibble j%16 of byte 2+j%16, high half for j>=16
 * (cpu.c:49-53). */
void nbs_encode_iq4nl(uint8_t *blk, const float *x) {
    static const int lut[16] = {-127,-104,-83,-65,-49,-35,-22,-10,1,13,25,38,53,69,89,113};
    double amax = 0;
    for (int j = 0; j < 32; j++) { double a = fabs((double)x[j]); if (a > amax) amax = a; }
    uint16_t d16 = nbs_f32_to_f16((float)(amax / 127.0));
    double d = nbs_f16_to_f32(d16);
    memset(blk, 0, 18);
    blk[0] = (uint8_t)d16; blk[1] = (uint8_t)(d16 >> 8);
    for (int j = 0; j < 32; j++) {
        int best = 8;
        if (d > 0) {
            double v = (double)x[j] / d, err = fabs(v - lut[0]); best = 0;
            for (int q = 1; q < 16; q++) { double e = fabs(v - lut[q]); if (e < err) { err = e; best = q; } }
        }
        blk[2 + j % 16] |= (uint8_t)(best << ((j / 16) * 4));
    }
}

int nbs_fill_matrix(void *out, int type, uint64_t seed, uint64_t stream, int rows, int cols, float sigma) {
    size_t rb = nbo_row_bytes(type, cols);
    if (!rb || (type != 0 && type != 12 && type != 20)) return -1;
    int block = type == 12 ? 256 : type == 20 ? 32 : 1;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float v[256];
        for (int c0 = 0; c0 < cols; c0 += block) {
            for (int j = 0; j < block; j++)
                v[j] = (float)((double)sigma * nbs_gauss(seed, stream, (uint64_t)r * cols + c0 + j));
            uint8_t *dst = (uint8_t *)out + (size_t)r * rb;
            if (type == 0) memcpy(dst + (size_t)c0 * 4, v, 4);
            else if (type == 12) nbs_encode_q4k(dst + (size_t)(c0 / 256) * 144, v);
            else nbs_encode_iq4nl(dst + (size_t)(c0 / 32) * 18, v);
        }
    }
    return 0;
}
