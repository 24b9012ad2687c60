// Matrix-core operand helpers shared by the decode and prefill kernels.
//
// Operand conventions (v_mfma_f32_16x16x32_f16, lane l: j = l%16, kq = l/16):
// A = activations (row j = one token, or one token-plane), lane supplies 8
// k-values; B = weights, column j = weight row j, lane supplies the same 8
// k-values; D[row][weight row]: lane holds rows 4kq..4kq+3 of column j.
// K order inside a Q4_K superblock: MFMA m (0..7), lane kq takes 16-byte qs
// chunks kq and kq+4; chunk c's fragment f (0..3) = (low/high nibbles) x
// (bytes 0-7 / 8-15).  Every weight enters as s_g*q (an integer <= 945, exact
// in fp16), so elements of different groups may share an MFMA; the superblock
// scale d and the min term dmin*sum_g m_g*X_g are applied in fp32.  IQ4_NL:
// one MFMA per 32-element block, lane kq takes qs bytes 4kq..4kq+3 (slots 0..3
// their low nibbles, 4..7 their high nibbles), the block scale is applied in
// fp32.  Activation planes (fp16 hi and lo = x - hi) are
// stored in the matching permuted order (pos_q4k / pos_iq4), so every A
// fragment is one 16-byte load.
#pragma once
#include "qg_common.h"

// Plane position of element e (0..255) of a Q4_K superblock.
QG_DEV int pos_q4k(int e) {
    const int g = e >> 5, l = e & 31, nib = g & 1, gp = g >> 1, h = l >> 4, p = l & 15;
    const int c = 2 * gp + h, kq = c & 3, ci = c >> 2, f = 2 * nib + (p >> 3);
    return ((4 * ci + f) * 4 + kq) * 8 + qg_perm8(p & 7);
}
QG_DEV int qg_perm4(int i) { return ((i & 1) << 1) | ((i & 2) >> 1); }  // 0,2,1,3
// Plane position of element e (0..31) of an IQ4_NL block: lane kq's 8 slots
// hold the low nibbles of its qs bytes 4kq..4kq+3 (elements 4kq..4kq+3), then
// their high nibbles (elements 16 + 4kq..16 + 4kq+3).
QG_DEV int pos_iq4(int e) {
    const int hi = e >> 4, r = e & 15;
    return (r >> 2) * 8 + 4 * hi + (r & 3);
}
QG_DEV int plane_pos(int fmt, int k) {
    return fmt == QT_IQ4_NL ? (k & ~31) | pos_iq4(k & 31) : (k & ~255) | pos_q4k(k & 255);
}

// The 8 fp16 values s*q of one fragment of a Q4_K qs chunk (c = 16 bytes):
// f bit 1 = high nibbles, f bit 0 = bytes 8..15.
QG_DEV qg_half8 q4k_chunk_frag(uint4 c, int f, _Float16 s) {
    return q4_frag((f & 1) ? make_uint2(c.z, c.w) : make_uint2(c.x, c.y), f >> 1, s);
}

// 4 IQ4_NL qs bytes -> 8 table values in fp16, slots 0..3 / 4..7 = low /
// high nibbles of bytes 0..3 (pos_iq4's order).  The table bytes (value +
// 128) are permuted in pairs under the exponent byte 0x64 (1024 + value +
// 128) and 1152 is taken off, exactly.
QG_DEV qg_half8 iq4_frag4(uint32_t q) {
    const uint32_t lo = iq4_lookup(q & 0x0F0F0F0Fu), hi = iq4_lookup((q >> 4) & 0x0F0F0F0Fu);  // lut + 128 as bytes
    uint32_t X;
    asm("v_mov_b32 %0, 0x64646464" : "=v"(X));
    const uint32_t u[4] = {__builtin_amdgcn_perm(X, lo, 0x04010400u), __builtin_amdgcn_perm(X, lo, 0x04030402u),
                           __builtin_amdgcn_perm(X, hi, 0x04010400u), __builtin_amdgcn_perm(X, hi, 0x04030402u)};
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
// The lane's two group scales of a half superblock as fp16 pairs: sc = {s_a,
// s_b / 16}, of = {-1024 s_a, -64 s_b}, where s_a is byte 2 (kq >> 1) of the
// half's scale word (the group of the lane's low nibbles) and s_b the next
// byte (the group of its high nibbles); a byte permute puts both under the
// exponent byte 0x64 (1024 + s, exact) and one packed add removes the 1024.
QG_DEV void gq_scales(uint32_t S, int kq, qg_half2 &sc, qg_half2 &of) {
    const uint32_t b = 2u * (uint32_t)(kq >> 1);
    const uint32_t u = __builtin_amdgcn_perm(0x64646464u, S, b | (4u << 8) | ((b + 1u) << 16) | (4u << 24));
    const qg_half2 sv = __builtin_bit_cast(qg_half2, u) + qg_half2{(_Float16)(-1024.0f), (_Float16)(-1024.0f)};
    sc = sv * qg_half2{(_Float16)1.0f, (_Float16)0.0625f};
    of = sv * qg_half2{(_Float16)(-1024.0f), (_Float16)(-64.0f)};
}
// 8 Q4_K nibbles of fragment f of a 16-byte qs chunk as s * q in fp16: the
// nibbles go under the exponent byte 0x64 (1024 + q, or 1024 + 16 q for the
// high nibbles) and one packed fma per pair applies the scale and removes the
// offset, exactly (s * q <= 945).
QG_DEV qg_half8 gq_frag(uint4 c, int f, _Float16 sc, _Float16 of) {
    uint32_t E;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(E));
    const uint32_t m = (f & 2) ? 0x00F000F0u : 0x000F000Fu;
    const uint32_t x = (f & 1) ? c.z : c.x, y = (f & 1) ? c.w : c.y;
    const uint32_t u[4] = {(x & m) | E, ((x >> 8) & m) | E, (y & m) | E, ((y >> 8) & m) | E};
    const qg_half2 sv = {sc, sc}, ov = {of, of};
    qg_half8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const qg_half2 v = __builtin_elementwise_fma(__builtin_bit_cast(qg_half2, u[i]), sv, ov);
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}
QG_DEV qg_half8 ld_frag(const _Float16 *p) { return __builtin_bit_cast(qg_half8, *(const uint4 *)p); }
// Raw buffer loads (no stride; the byte range is the descriptor's record
// count): an offset past the range reads zeros with no memory access.
// QG_BUF_DW3: descriptor word 3 for gfx9 raw buffers (32-bit data format).
constexpr int QG_BUF_DW3 = 0x00020000;
constexpr int QG_BUF_OOB = 0x7fff0000;  // an offset past any range used here
QG_DEV qg_half8 buf_frag(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(qg_half8, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

typedef __attribute__((address_space(3))) void qg_lds_void;

// Direct global->shared copy of 16 bytes per lane (gfx950 global_load_lds
// b128): lane l's 16 bytes land at lds_base + 16*l, lds_base uniform across
// the wave.  Completion is tracked by the vector-memory counter.
QG_DEV void dma16(const void *g, void *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (qg_lds_void *)lds_base, 16, 0, 0);
}
// The same copy issued from inline assembly: it stays in program order with
// the surrounding memory operations and the compiler does not track it, so
// it adds no waits of its own before later shared-memory reads; the caller
// waits for it with wait_vmem or wait_vmem_but before the data is read (and
// makes it visible to the other waves with a barrier).  M0, which holds the
// shared-memory base of the copy, is restored afterwards.
QG_DEV void dma16_ordered(const void *g, void *lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(qg_lds_void *)lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(base)
                 : "memory");
}
// Three dma16_ordered copies to lds_base, +1024 and +2048 under one M0 value:
// the instruction offset moves both the shared-memory and the global address,
// so copy t reads g_t through g_t - 1024 t + offset.
QG_DEV void dma16x3_ordered(const uint8_t *g0, const uint8_t *g1, const uint8_t *g2, void *lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(qg_lds_void *)lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %4\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, off\n\t"
                 "global_load_lds_dwordx4 %2, off offset:1024\n\t"
                 "global_load_lds_dwordx4 %3, off offset:2048\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g0), "v"(g1 - 1024), "v"(g2 - 2048), "s"(base)
                 : "memory");
}
// dma16_ordered for 4 bytes per lane (global_load_lds_dword): lane l's word
// lands at lds_base + 4*l.
QG_DEV void dma4_ordered(const void *g, void *lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(qg_lds_void *)lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(base)
                 : "memory");
}
QG_DEV void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }
// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order), leaving the other counters alone.
template <int N>
QG_DEV void wait_vmem_but() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 1/sqrt(mean(x^2) + eps) of one row, summed lane-strided then across the
// wave; every caller runs this same code, so all blocks agree bit for bit.
QG_DEV float row_rms_scale(const float *xr, int D, float eps, int lane) {
    float ss = 0.0f;
#pragma unroll 4
    for (int i = lane; i < D; i += 64) ss = __builtin_fmaf(xr[i], xr[i], ss);
    ss = qg_sum_lanes<64>(ss);
    return 1.0f / __builtin_sqrtf(ss / (float)D + eps);
}
// The same scale from a row held in shared memory (same values, same order).
QG_DEV float lds_rms_scale(const float *xl, int D, float eps, int lane) {
    float ss = 0.0f;
#pragma unroll 4
    for (int i = lane; i < D; i += 64) ss = __builtin_fmaf(xl[i], xl[i], ss);
    ss = qg_sum_lanes<64>(ss);
    return 1.0f / __builtin_sqrtf(ss / (float)D + eps);
}

// The fp16 hi/lo planes of one token row (Q4_K fragment order) and the hi/lo
// planes of its 32-group sums, optionally RMS-scaled by sc (written to xn);
// lane g handles groups g, g+64, ... with 8 float4 loads each.  In the Q4_K
// order every 16-byte chunk holds 8 consecutive elements of one group (in
// qg_perm8 order), so each group is written as 4 chunks per plane.
QG_DEV void token_planes(const float *xr, int D, bool norm, float sc, int lane, _Float16 *hi, _Float16 *lo,
                         _Float16 *shi, _Float16 *slo, float *xn) {
    for (int g = lane; g < D / 32; g += 64) {
        float v[32];
        const float4 *src = (const float4 *)(xr + 32 * g);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = src[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
        float s = 0.0f;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            if (norm) v[l] = v[l] * sc;
            s += v[l];
        }
        const _Float16 sh = (_Float16)s;
        shi[g] = sh;
        slo[g] = (_Float16)(s - (float)sh);
        if (norm && xn) {
            float4 *dst = (float4 *)(xn + 32 * g);
#pragma unroll
            for (int i = 0; i < 8; i++) dst[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            // elements 8q..8q+7 of the group form one chunk; pos_q4k of its first element
            const int p0 = (g & ~7) * 32 + pos_q4k((g & 7) * 32 + 8 * q);
            qg_half8 h8, l8;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = v[8 * q + qg_perm8(i)];
                const _Float16 h = (_Float16)x;
                h8[i] = h;
                l8[i] = (_Float16)(x - (float)h);
            }
            *(qg_half8 *)(hi + p0) = h8;
            *(qg_half8 *)(lo + p0) = l8;
        }
    }
}
