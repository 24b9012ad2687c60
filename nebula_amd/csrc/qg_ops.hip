// Drop-in operators of the reference's GPU C ABI on the routed-MoE path
// (gpu.h:37-43,62-78).  Each entry point keeps the reference's argument
// list, validation and semantics (gpu.cu lines cited per function); the
// kernels are written for CDNA4 wave64.
#include "qg_internal.h"
#include "qg_frag.h"

// The widths of the width-less entry points: a process-wide setting
// (qg_moe_configure), which a thread may override for its own calls
// (qg_moe_configure_thread), so a caller that configures on one thread and
// launches from another sees its setting, and two threads driving models of
// different shapes each keep their own.
#include <atomic>
static std::atomic<int> g_width{2560}, g_ff{640};  // gpu.cu:508-553 hard-code these
static thread_local int t_width = 0, t_ff = 0;     // 0: no per-thread override
int qg_cfg_width(void) { return t_width ? t_width : g_width.load(std::memory_order_relaxed); }
int qg_cfg_ff(void) { return t_width ? t_ff : g_ff.load(std::memory_order_relaxed); }

namespace {

// ------------------------------------------------------------------------
// qg_matmul: out[t,r] = sum_c deq(W)[r,c] x[t,c] in the reference's order.
// Each 32-lane half of a wave owns one row; lane j owns partial sum j
// (k = j mod 32, ascending k, fused multiply-add), then the stride
// 16/8/4/2/1 tree.  This is the order of cpu.c:122-139 and gpu.cu:154-180,
// so every result equals cpu.c's qc_matmul bit for bit.  A block is one
// wave (two rows) so that even the 512-row router fills all CUs.  TT tokens
// share each weight value.
// ------------------------------------------------------------------------
template <int TT>
struct Acc { float v[TT]; };

// Branch-free so that the loads of a chunk can all be in flight: tokens past
// the tile's end re-read the last valid row and their sums are never stored.
template <int TT>
QG_DEV void acc_step(Acc<TT> &a, float w, const float *x, size_t cols, int k, int n) {
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const int tt = t < n ? t : n - 1;
        a.v[t] = __builtin_fmaf(w, x[(size_t)tt * cols + k], a.v[t]);
    }
}

template <int TYPE, int TT>
__global__ __launch_bounds__(64) void mm_exact_kernel(float *__restrict__ out, const uint8_t *__restrict__ w, int type,
                                                      int rows, int cols, const float *__restrict__ x, int nt,
                                                      size_t stride, const uint8_t *extra_row) {
    const int half = threadIdx.x >> 5, j = threadIdx.x & 31;
    const int row = blockIdx.x * 2 + half;
    const int t0 = blockIdx.y * TT, n = min(nt - t0, TT);
    if (row >= rows) return;  // whole 32-lane half leaves; shuffles stay within halves
    const uint8_t *wr = (extra_row && row == rows - 1) ? extra_row : w + (size_t)row * stride;
    const float *xb = x + (size_t)t0 * cols;
    Acc<TT> a;
#pragma unroll
    for (int t = 0; t < TT; t++) a.v[t] = 0.0f;
    if (TYPE == QT_F32) {
        // Issue a whole chunk of weight (and x) loads before the dependent
        // FMAs so the GEMV is not one memory round trip per 32 columns.
        constexpr int CH = TT == 1 ? 64 : TT == 4 ? 32 : 8;
        const float *wf = (const float *)wr;
        int k = 0;
        for (; k + 32 * CH <= cols; k += 32 * CH) {
            float wv[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) wv[i] = wf[k + 32 * i + j];
#pragma unroll
            for (int i = 0; i < CH; i++) acc_step<TT>(a, wv[i], xb, cols, k + 32 * i + j, n);
        }
        for (; k < cols; k += 32) acc_step<TT>(a, wf[k + j], xb, cols, k + j, n);
    } else if (TYPE == QT_Q4_K) {
        for (int sb = 0; sb < cols / 256; sb++) {
            const uint8_t *p = wr + (size_t)sb * 144;
            const float d = qg_half(p), dmin = qg_half(p + 2);
            const uint8_t *sc = p + 4;
#pragma unroll
            for (int gp = 0; gp < 4; gp++) {
                const int byte = p[16 + gp * 32 + j];
#pragma unroll
                for (int hi = 0; hi < 2; hi++) {
                    const int g = gp * 2 + hi;
                    const int s = g < 4 ? (sc[g] & 63) : ((sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4));
                    const int m = g < 4 ? (sc[g + 4] & 63) : ((sc[g + 4] >> 4) | ((sc[g] >> 6) << 4));
                    const float wv = __builtin_fmaf(d * (float)s, (float)((byte >> (hi * 4)) & 15), -(dmin * (float)m));
                    acc_step<TT>(a, wv, xb, cols, sb * 256 + g * 32 + j, n);
                }
            }
        }
    } else if (TYPE == QT_IQ4_NL) {
        for (int b = 0; b < cols / 32; b++) {
            const uint8_t *p = wr + (size_t)b * 18;
            const int q = (p[2 + (j & 15)] >> ((j >> 4) * 4)) & 15;
            acc_step<TT>(a, qg_half(p) * (float)qg_iq4nl_lut[q], xb, cols, b * 32 + j, n);
        }
    } else {
        // generic formats; F32/F16/BF16 rows may end in a partial 32-column step
        // (lanes past the end add nothing, as gpu.cu:159's k<cols loop)
        for (int k = 0; k < cols; k += 32)
            if (k + j < cols) acc_step<TT>(a, qg_weight_at(wr, type, k + j), xb, cols, k + j, n);
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
        if (t < n) {
            const float s = qg_tree32(a.v[t]);
            if (j == 0) out[(size_t)(t0 + t) * rows + row] = s;
        }
    }
}

// qg_matmul for Q4_K and IQ4_NL rows with cols a multiple of 256, up to TT
// tokens per block: the arithmetic of mm_exact_kernel (the same weight value
// per element, lane j's chain over k = j (mod 32) in ascending k, the same
// tree).  A block holds 8 RPL rows: 32-lane half h runs rows h, h + 8, ...
// (RPL of them, sharing every x read).  Per chunk of KC columns: the rows'
// weight bytes and the tile's x rows arrive by direct global->shared copies,
// all in flight at once; then each group's d*s and -(dmin*m) (Q4_K) or each
// block's d (IQ4_NL) is formed once into shared memory, and the rows' chains
// run from shared memory.
template <int TT> struct MmTile;
template <> struct MmTile<1> { static constexpr int KC = 4096; };
template <> struct MmTile<4> { static constexpr int KC = 2048; };
template <> struct MmTile<8> { static constexpr int KC = 1024; };
template <> struct MmTile<16> { static constexpr int KC = 512; };
template <> struct MmTile<20> { static constexpr int KC = 512; };

template <int TYPE, int TT, int RPL, int KCO = 0>
__global__ __launch_bounds__(256) void mm_tile_kernel(float *__restrict__ out, const uint8_t *__restrict__ w, int rows,
                                                     int cols, const float *__restrict__ x, int nt, size_t stride) {
    constexpr int KC = KCO ? KCO : MmTile<TT>::KC, RB = 8 * RPL;  // chunk columns; rows per block
    constexpr int WB = KC / 256 * 144;                                       // chunk bytes of a row
    constexpr int NS = TYPE == QT_Q4_K ? RB * (KC / 256) * 8 : RB * (KC / 32);  // scale entries per chunk
    __shared__ __attribute__((aligned(16))) float xs[TT * KC];    // [token][k], row stride kc
    __shared__ __attribute__((aligned(16))) uint8_t ws[RB * WB];  // [row][bytes]
    __shared__ __attribute__((aligned(16))) float2 s_sc[TYPE == QT_Q4_K ? NS : 1];
    __shared__ float s_d[TYPE == QT_Q4_K ? 1 : NS];
    __shared__ float s_lut[16];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hw = tid >> 5, j = tid & 31;
    const int r0 = blockIdx.x * RB;
    const int t0 = blockIdx.y * TT, n = min(nt - t0, TT);
    if (TYPE == QT_IQ4_NL && tid < 16) s_lut[tid] = (float)qg_iq4nl_lut[tid];
    Acc<TT> a[RPL];
#pragma unroll
    for (int q = 0; q < RPL; q++)
#pragma unroll
        for (int t = 0; t < TT; t++) a[q].v[t] = 0.0f;
    for (int c0 = 0; c0 < cols; c0 += KC) {
        const int kc = min(KC, cols - c0), rb = kc / 256 * 144;  // this chunk's columns, bytes per row
        // the block's rows' bytes, contiguous per row (rows past the end repeat the last)
        const int wp = rb / 16;
        for (int base = wave * 64; base < RB * wp; base += 256) {
            const int i = base + lane, r = i / wp, pc = i - r * wp;
            if (i < RB * wp) dma16(w + (size_t)min(r0 + r, rows - 1) * stride + (size_t)c0 / 256 * 144 + 16 * pc, ws + 16 * base);
        }
        // the tile's n token rows of the chunk: piece i lands at 16 i bytes, so
        // token t starts at t * kc floats
        const int xp = kc / 4;
        for (int base = wave * 64; base < n * xp; base += 256) {
            const int i = base + lane, t = i / xp, pc = i - t * xp;
            if (i < n * xp) dma16(x + (size_t)(t0 + t) * cols + c0 + 4 * pc, xs + 4 * base);
        }
        wait_vmem();
        __syncthreads();
        // per-group (Q4_K) or per-block (IQ4_NL) scales of the chunk, once
        if (TYPE == QT_Q4_K) {
            const int nsb = kc / 256;
            for (int e = tid; e < RB * nsb * 8; e += 256) {
                const int r = e / (nsb * 8), sb = (e >> 3) - r * nsb, g = e & 7;
                const uint8_t *p = ws + r * rb + sb * 144, *sc = p + 4;
                const float d = qg_half(p), dmin = qg_half(p + 2);
                const int sv = g < 4 ? (sc[g] & 63) : ((sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4));
                const int mv = g < 4 ? (sc[g + 4] & 63) : ((sc[g + 4] >> 4) | ((sc[g] >> 6) << 4));
                s_sc[e] = make_float2(d * (float)sv, -(dmin * (float)mv));
            }
        } else {
            const int nb = kc / 32;
            for (int e = tid; e < RB * nb; e += 256) {
                const int r = e / nb, b = e - r * nb;
                s_d[e] = qg_half(ws + r * rb + b * 18);
            }
        }
        __syncthreads();
        // tokens past the tile's n re-read its last row, rows past the end the
        // last row (their sums are not stored)
        auto chains = [&](const float *wv, int k) {
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const float xv = xs[min(t, n - 1) * kc + k];
#pragma unroll
                for (int q = 0; q < RPL; q++) a[q].v[t] = __builtin_fmaf(wv[q], xv, a[q].v[t]);
            }
        };
        if (TYPE == QT_Q4_K) {
            const int nsb = kc / 256;
            for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
                for (int gp = 0; gp < 4; gp++) {
                    int byte[RPL];
#pragma unroll
                    for (int q = 0; q < RPL; q++) byte[q] = ws[(hw + 8 * q) * rb + sb * 144 + 16 + gp * 32 + j];
#pragma unroll
                    for (int hi = 0; hi < 2; hi++) {
                        float wv[RPL];
#pragma unroll
                        for (int q = 0; q < RPL; q++) {
                            const float2 ds = s_sc[((hw + 8 * q) * nsb + sb) * 8 + 2 * gp + hi];
                            wv[q] = __builtin_fmaf(ds.x, (float)((byte[q] >> (hi * 4)) & 15), ds.y);
                        }
                        chains(wv, sb * 256 + (2 * gp + hi) * 32 + j);
                    }
                }
            }
        } else {
            const int nb = kc / 32;
            for (int b = 0; b < nb; b++) {
                float wv[RPL];
#pragma unroll
                for (int q = 0; q < RPL; q++) {
                    const int r = hw + 8 * q;
                    const int qq = (ws[r * rb + b * 18 + 2 + (j & 15)] >> ((j >> 4) * 4)) & 15;
                    wv[q] = s_d[r * nb + b] * s_lut[qq];
                }
                chains(wv, b * 32 + j);
            }
        }
        __syncthreads();  // the chunk's buffers are rewritten next
    }
#pragma unroll
    for (int q = 0; q < RPL; q++) {
        const int row = r0 + hw + 8 * q;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float s = qg_tree32(a[q].v[t]);
            if (j == 0 && t < n && row < rows) out[(size_t)(t0 + t) * rows + row] = s;
        }
    }
}

// Two rows per lane halve the shared-memory reads per product (they pay off
// for the long token tiles), when the matrix still fills 512 blocks.
template <int TYPE, int TT>
void launch_mm_tile(float *out, const uint8_t *w, int rows, int cols, const float *x, int nt, size_t stride, hipStream_t s) {
    const int ty = (nt + TT - 1) / TT;
    const dim3 g8((rows + 7) / 8, ty);
    if constexpr (TT >= 16) {
        if (((rows + 15) / 16) * ty >= 512) {
            mm_tile_kernel<TYPE, TT, 2><<<dim3((rows + 15) / 16, ty), 256, 0, s>>>(out, w, rows, cols, x, nt, stride);
            return;
        }
    } else if constexpr (TT == 1) {
        if (cols <= 2560) {
            // one chunk of at most 2560 columns: a third less shared memory than
            // the 4096-column chunk, so 5 blocks per CU stay resident instead of 3
            mm_tile_kernel<TYPE, 1, 1, 2560><<<g8, 256, 0, s>>>(out, w, rows, cols, x, nt, stride);
            return;
        }
        if (cols > 4096 && cols <= 6144) {
            // one chunk instead of two (one copy round trip per block)
            mm_tile_kernel<TYPE, 1, 1, 6144><<<g8, 256, 0, s>>>(out, w, rows, cols, x, nt, stride);
            return;
        }
    } else {
        if (cols <= 2560) {
            // two 1280-column chunks: 5 (4 tokens) or 3 (8 tokens) blocks per CU
            // instead of 3 or 4, at the same or fewer copy rounds
            mm_tile_kernel<TYPE, TT, 1, 1280><<<g8, 256, 0, s>>>(out, w, rows, cols, x, nt, stride);
            return;
        }
    }
    mm_tile_kernel<TYPE, TT, 1><<<g8, 256, 0, s>>>(out, w, rows, cols, x, nt, stride);
}

template <int TYPE>
void launch_mm_exact(float *out, const uint8_t *w, int type, int rows, int cols, const float *x, int nt, size_t stride,
                     const uint8_t *extra, hipStream_t s) {
    if constexpr (TYPE == QT_Q4_K || TYPE == QT_IQ4_NL) {
        // the tiled kernel's 16-byte copies need 16-byte aligned rows and x
        if (!extra && cols % 256 == 0 && (((uintptr_t)w | (uintptr_t)x | stride) & 15) == 0) {
        if (nt == 1) launch_mm_tile<TYPE, 1>(out, w, rows, cols, x, nt, stride, s);
        else if (nt <= 4) launch_mm_tile<TYPE, 4>(out, w, rows, cols, x, nt, stride, s);
        else if (nt <= 8) launch_mm_tile<TYPE, 8>(out, w, rows, cols, x, nt, stride, s);
        else if (nt <= 16) launch_mm_tile<TYPE, 16>(out, w, rows, cols, x, nt, stride, s);
        else launch_mm_tile<TYPE, 20>(out, w, rows, cols, x, nt, stride, s);
        return;
        }
    }
    dim3 grid((rows + 1) / 2, 1);
    if (nt == 1) { mm_exact_kernel<TYPE, 1><<<grid, 64, 0, s>>>(out, w, type, rows, cols, x, nt, stride, extra); return; }
    if (nt <= 64) {
        grid.y = (nt + 3) / 4;
        mm_exact_kernel<TYPE, 4><<<grid, 64, 0, s>>>(out, w, type, rows, cols, x, nt, stride, extra);
        return;
    }
    grid.y = (nt + 15) / 16;
    mm_exact_kernel<TYPE, 16><<<grid, 64, 0, s>>>(out, w, type, rows, cols, x, nt, stride, extra);
}

// ------------------------------------------------------------------------
// Elementwise and row operators.
// ------------------------------------------------------------------------
__global__ void gather_kernel(float *o, const uint8_t *w, int type, int n, size_t stride, int row) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = qg_weight_at(w + (size_t)row * stride, type, i);
}
__global__ void dequant_kernel(float *o, const uint8_t *w, int type, int rows, int cols, size_t stride) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)rows * cols) o[i] = qg_weight_at(w + (i / cols) * stride, type, (int)(i % cols));
}

// RMS/L2 norm of gpu.cu:204-214: one block per (group, token).
__global__ __launch_bounds__(256) void norm_kernel(float *o, const float *x, const float *w, int width, int groups, int wg, int l2, float eps) {
    __shared__ float partial[4];
    const int g = blockIdx.x, base = g * width;
    float ss = 0;
    for (int i = threadIdx.x; i < width; i += 256) ss = __builtin_fmaf(x[base + i], x[base + i], ss);
    ss = qg_sum_lanes<64>(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float scale = 1.0f / __builtin_sqrtf(ss / (l2 ? 1.0f : (float)width) + eps);
    for (int i = threadIdx.x; i < width; i += 256)
        o[base + i] = x[base + i] * scale * (w ? w[(wg ? g % groups : 0) * width + i] : 1.0f);
}

// gpu.cu:215-220: a = x*scale; op0 a*sig(a), op1 sig(a), else a.
__global__ void unary_kernel(float *o, const float *x, int n, int op, float s) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { float a = x[i] * s; o[i] = op == 0 ? a * qg_sig(a) : op == 1 ? qg_sig(a) : a; }
}
// gpu.cu:221-226: op0 add, otherwise multiply.
__global__ void binary_kernel(float *o, const float *a, const float *b, int n, int op) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = op == 0 ? a[i] + b[i] : a[i] * b[i];
}

// ------------------------------------------------------------------------
// Routing (gpu.cu:456-465).  One wave per pair of tokens (qg_route_pair, a
// 32-lane half per token): the 10 winners by value with the lowest index
// among equal values (the reference's strict-greater scan from index 0),
// numerators exp(s - max) summed in rank order, then divided by the sum.
// ------------------------------------------------------------------------
__global__ __launch_bounds__(64) void route_kernel(int *ids, float *weights, const float *logits, int nt, int ld) {
    __shared__ __align__(16) float s_v[QG_ROUTE_SCRATCH];
    __shared__ __align__(16) int s_i[QG_ROUTE_SCRATCH];
    const int ta = 2 * blockIdx.x, tb = min(ta + 1, nt - 1);
    qg_route_wave2(ids, weights, logits, ld, ta, tb, threadIdx.x, s_v, s_i);
}

// Pruning (gpu.cu:467-483), one thread per token, device atomics for the
// counters exactly as the reference (skipped_mass is an order-dependent
// double atomic there too).
__global__ void prune_kernel(int *ids, float *w, const uint8_t *resident, int nt, double thr, qg_prune_stats *st) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nt) return;
    int missing = 0;
    double mass = 0;
    for (int k = 0; k < QG_TOP; k++) {
        const int e = ids[t * QG_TOP + k];
        if (e < 0 || e >= QG_EXPERTS) return;
        if (!resident[e]) { missing++; mass += (double)w[t * QG_TOP + k]; }
    }
    atomicAdd((unsigned long long *)&st->token_layers, 1ULL);
    atomicAdd((unsigned long long *)&st->missing_selections, (unsigned long long)missing);
    if (missing && thr > 0 && mass < thr) {
        for (int k = 0; k < QG_TOP; k++) {
            const int e = ids[t * QG_TOP + k];
            if (!resident[e]) { ids[t * QG_TOP + k] = -e - 2; w[t * QG_TOP + k] = 0.0f; }
        }
        atomicAdd((unsigned long long *)&st->skipped_selections, (unsigned long long)missing);
        atomicAdd((unsigned long long *)&st->avoided_token_handoffs, 1ULL);
        atomicAdd(&st->skipped_mass, mass);
    }
}

// Token map (gpu.cu:489-500): row e lists ascending tokens that selected e.
// One wave per expert; ordered compaction by ballot + popcount.
__global__ __launch_bounds__(64) void moe_map_kernel(int *map, const int *ids, int nt) {
    const int e = blockIdx.x, lane = threadIdx.x;
    int carry = 0;
    for (int base = 0; base < nt; base += 64) {
        const int t = base + lane;
        bool sel = false;
        if (t < nt) {
#pragma unroll
            for (int k = 0; k < QG_TOP; k++) sel |= ids[t * QG_TOP + k] == e;
        }
        const unsigned long long mask = __ballot(sel);
        if (sel) map[(size_t)e * nt + carry + __popcll(mask & ((1ULL << lane) - 1ULL))] = t;
        carry += __popcll(mask);
    }
}

// gpu.cu:506-512, width from qg_moe_configure.
__global__ void moe_gather_kernel(float *out, const float *x, const int *map, int width) {
    const int r = blockIdx.x, t = map[r];
    for (int d = threadIdx.x; d < width; d += blockDim.x) out[(size_t)r * width + d] = x[(size_t)t * width + d];
}
// gpu.cu:513-517: rank r -> token map[r] (or r), slot = last k with
// ids[t,k]==expert, slots[t,slot,:] = y[r,:]*w[t,slot].
__global__ void moe_scatter_kernel(float *slots, const float *y, const float *w, const int *ids, const int *map, int expert, int width) {
    const int r = blockIdx.x, t = map ? map[r] : r;
    int slot = -1;
    for (int k = 0; k < QG_TOP; k++) if (ids[t * QG_TOP + k] == expert) slot = k;
    if (slot < 0) return;
    const float wk = w[t * QG_TOP + slot];
    for (int d = threadIdx.x; d < width; d += blockDim.x)
        slots[((size_t)t * QG_TOP + slot) * width + d] = y[(size_t)r * width + d] * wk;
}
// gpu.cu:521-527: out = sum of the 10 slots from 0 in router-rank order.
__global__ void moe_reduce_kernel(float *out, const float *slots, int nt, int width) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)nt * width) return;
    const size_t t = i / width, d = i % width;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < QG_TOP; k++) sum += slots[(t * QG_TOP + k) * width + d];
    out[i] = sum;
}
// gpu.cu:552-553: out += shared*sig(gate[t]) (contracted to one fma, as nvcc does).
__global__ void shared_add_kernel(float *o, const float *x, const float *g, int nt, int width) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)nt * width) o[i] = __builtin_fmaf(x[i], qg_sig(g[i / width]), o[i]);
}

unsigned blocks_for(size_t n, unsigned threads) { return (unsigned)((n + threads - 1) / threads); }

// ---- CPU handoff of flagged tokens (qwen.c:658-678) ----
// rows[i] = the i-th token, ascending, whose flag is 2 (coverage below
// 1 - threshold); count[0] = their number.  One block of 1024 threads.
__global__ __launch_bounds__(1024) void handoff_rows_kernel(int *count, int *rows, const uint8_t *flags, int nt) {
    __shared__ int s_wave[16];
    __shared__ int s_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_base = 0;
    __syncthreads();
    for (int c0 = 0; c0 < nt; c0 += 1024) {
        const int t = c0 + tid;
        const bool h = t < nt && flags[t] == 2;
        const unsigned long long b = __ballot(h);
        if (lane == 0) s_wave[wave] = __popcll(b);
        __syncthreads();
        int off = s_base;
        for (int w = 0; w < wave; w++) off += s_wave[w];
        if (h) rows[off + __popcll(b & ((1ULL << lane) - 1ULL))] = t;
        __syncthreads();
        if (tid == 0) {
            int n = 0;
            for (int w = 0; w < 16; w++) n += s_wave[w];
            s_base += n;
        }
        __syncthreads();
    }
    if (tid == 0) count[0] = s_base;
}

// Block i < count: row i of the packed arrays = token rows[i]'s input row,
// ids and weights (blocks past the count exit).
__global__ __launch_bounds__(256) void handoff_pack_kernel(float *xp, int *idp, float *wp, const int *count, const int *rows,
                                                           const float *x, const int *ids, const float *w, int width) {
    const int i = blockIdx.x;
    if (i >= count[0]) return;
    const int t = rows[i];
    const float *src = x + (size_t)t * width;
    float *dst = xp + (size_t)i * width;
    for (int d = threadIdx.x; d < width; d += 256) dst[d] = src[d];
    if (threadIdx.x < QG_TOP) {
        idp[(size_t)i * QG_TOP + threadIdx.x] = ids[(size_t)t * QG_TOP + threadIdx.x];
        wp[(size_t)i * QG_TOP + threadIdx.x] = w[(size_t)t * QG_TOP + threadIdx.x];
    }
}

// count[0] into the host word: a store at system scope, which the host
// observes by polling the word (page-locked host memory).
__global__ void handoff_notify_kernel(int *host_word, const int *count) {
    __hip_atomic_store(host_word, count[0], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Block i < count: out[rows[i]] += y[i] (the host's routed rows onto the
// device rows, which hold the shared expert's part).
__global__ __launch_bounds__(256) void handoff_merge_kernel(float *out, const float *y, const int *count, const int *rows, int width) {
    const int i = blockIdx.x;
    if (i >= count[0]) return;
    float *o = out + (size_t)rows[i] * width;
    const float *src = y + (size_t)i * width;
    for (int d = threadIdx.x; d < width; d += 256) o[d] += src[d];
}

}  // namespace

int qg_launch_matmul_exact(float *out, const uint8_t *w, int type, int rows, int cols, const float *x, int nt,
                           const uint8_t *extra, hipStream_t s) {
    const size_t stride = qg_row_bytes_host(type, cols);
    switch (type) {
    case QT_F32: launch_mm_exact<QT_F32>(out, w, type, rows, cols, x, nt, stride, extra, s); break;
    case QT_Q4_K: launch_mm_exact<QT_Q4_K>(out, w, type, rows, cols, x, nt, stride, extra, s); break;
    case QT_IQ4_NL: launch_mm_exact<QT_IQ4_NL>(out, w, type, rows, cols, x, nt, stride, extra, s); break;
    default: launch_mm_exact<-1>(out, w, type, rows, cols, x, nt, stride, extra, s); break;
    }
    return hipGetLastError();
}

extern "C" {

static bool widths_ok(int width, int ff) {
    return width >= 256 && width <= 8192 && width % 256 == 0 && ff >= 32 && ff <= 4096 && ff % 32 == 0;
}

int qg_moe_configure(int width, int ff) {
    if (!widths_ok(width, ff)) return hipErrorInvalidValue;
    g_width.store(width, std::memory_order_relaxed);
    g_ff.store(ff, std::memory_order_relaxed);
    return hipSuccess;
}

int qg_moe_configure_thread(int width, int ff) {
    if (width == 0 && ff == 0) {
        t_width = t_ff = 0;
        return hipSuccess;
    }
    if (!widths_ok(width, ff)) return hipErrorInvalidValue;
    t_width = width;
    t_ff = ff;
    return hipSuccess;
}

// gpu.cu:181-189: same validation (tokens 1..8192, block-multiple columns).
int qg_matmul(float *o, const void *w, int type, int rows, int cols, const float *x, int nt) {
    const size_t stride = qg_row_bytes_host(type, cols);
    if (!stride || rows < 1 || cols < 1 || nt < 1 || nt > QG_MAX_TOKENS || !o || !w || !x) return hipErrorInvalidValue;
    if (cols % 32) {  // only F32/F16/BF16 rows can have a partial last step
        launch_mm_exact<-1>(o, (const uint8_t *)w, type, rows, cols, x, nt, stride, nullptr, qg_stream());
        return hipGetLastError();
    }
    return qg_launch_matmul_exact(o, (const uint8_t *)w, type, rows, cols, x, nt, nullptr, qg_stream());
}

int qg_gather(float *o, const void *w, int type, int cols, int row) {  // gpu.cu:193-196
    const size_t stride = qg_row_bytes_host(type, cols);
    if (!stride || row < 0) return hipErrorInvalidValue;
    gather_kernel<<<blocks_for(cols, 256), 256, 0, qg_stream()>>>(o, (const uint8_t *)w, type, cols, stride, row);
    return hipGetLastError();
}

int qg_dequant(float *o, const void *w, int type, int rows, int cols) {  // gpu.cu:200-203
    const size_t stride = qg_row_bytes_host(type, cols);
    if (!stride || rows < 1) return hipErrorInvalidValue;
    dequant_kernel<<<blocks_for((size_t)rows * cols, 256), 256, 0, qg_stream()>>>(o, (const uint8_t *)w, type, rows, cols, stride);
    return hipGetLastError();
}

int qg_norm(float *o, const float *x, const float *w, int width, int groups, int nt, int wg, int l2, float eps) {  // gpu.cu:212-214
    if (width < 1 || groups < 1 || nt < 1) return hipErrorInvalidValue;
    norm_kernel<<<groups * nt, 256, 0, qg_stream()>>>(o, x, w, width, groups, wg, l2, eps);
    return hipGetLastError();
}

int qg_unary(float *o, const float *x, int n, int op, float s) {  // gpu.cu:219-220
    if (n < 1) return hipSuccess;
    unary_kernel<<<blocks_for(n, 256), 256, 0, qg_stream()>>>(o, x, n, op, s);
    return hipGetLastError();
}

int qg_binary(float *o, const float *a, const float *b, int n, int op) {  // gpu.cu:225-226
    if (n < 1) return hipSuccess;
    binary_kernel<<<blocks_for(n, 256), 256, 0, qg_stream()>>>(o, a, b, n, op);
    return hipGetLastError();
}

int qg_route(int *ids, float *w, const float *logits, int nt) {  // gpu.cu:466
    if (nt < 1 || nt > QG_MAX_TOKENS || !ids || !w || !logits) return hipErrorInvalidValue;
    route_kernel<<<(nt + 1) / 2, 64, 0, qg_stream()>>>(ids, w, logits, nt, QG_EXPERTS);
    return hipGetLastError();
}

int qg_prune_routes(int *ids, float *w, const unsigned char *resident, int nt, double thr, qg_prune_stats *st) {  // gpu.cu:484-488
    if (nt < 1 || nt > QG_MAX_TOKENS || thr < 0 || thr > 0.1 || !__builtin_isfinite(thr)) return hipErrorInvalidValue;
    prune_kernel<<<blocks_for(nt, 128), 128, 0, qg_stream()>>>(ids, w, resident, nt, thr, st);
    return hipGetLastError();
}

int qg_moe_map(int *map, const int *ids, int nt) {  // gpu.cu:501-505
    if (nt < 1 || nt > QG_MAX_TOKENS) return hipErrorInvalidValue;
    moe_map_kernel<<<QG_EXPERTS, 64, 0, qg_stream()>>>(map, ids, nt);
    return hipGetLastError();
}

int qg_moe_gather(float *o, const float *x, const int *map, int selected) {  // gpu.cu:509-512
    if (selected < 1) return selected ? hipErrorInvalidValue : hipSuccess;
    moe_gather_kernel<<<selected, 256, 0, qg_stream()>>>(o, x, map, qg_cfg_width());
    return hipGetLastError();
}

int qg_moe_scatter(float *o, const float *y, const float *w, const int *ids, const int *map, int expert, int selected) {  // gpu.cu:518-520
    if (selected < 1) return selected ? hipErrorInvalidValue : hipSuccess;
    moe_scatter_kernel<<<selected, 256, 0, qg_stream()>>>(o, y, w, ids, map, expert, qg_cfg_width());
    return hipGetLastError();
}

int qg_moe_reduce(float *out, const float *slots, int nt) {  // gpu.cu:525-527
    if (nt < 1) return hipErrorInvalidValue;
    moe_reduce_kernel<<<blocks_for((size_t)nt * qg_cfg_width(), 256), 256, 0, qg_stream()>>>(out, slots, nt, qg_cfg_width());
    return hipGetLastError();
}

int qg_shared_add(float *o, const float *x, const float *g, int nt) {  // gpu.cu:553
    if (nt < 1) return hipErrorInvalidValue;
    shared_add_kernel<<<blocks_for((size_t)nt * qg_cfg_width(), 256), 256, 0, qg_stream()>>>(o, x, g, nt, qg_cfg_width());
    return hipGetLastError();
}

// qwen.c:665-666 read every token's input and weights to the host when a
// selection is missing; here only the flag-2 tokens are packed for it.
int qg_moe_handoff_pack(int *count, int *rows, float *x_pack, int *ids_pack, float *w_pack, const unsigned char *flags,
                        const float *x, const int *ids, const float *weights, int nt, int width) {
    if (nt < 1 || nt > QG_MAX_TOKENS || width < 1 || !count || !rows || !x_pack || !ids_pack || !w_pack || !flags || !x ||
        !ids || !weights)
        return hipErrorInvalidValue;
    handoff_rows_kernel<<<1, 1024, 0, qg_stream()>>>(count, rows, flags, nt);
    handoff_pack_kernel<<<nt, 256, 0, qg_stream()>>>(x_pack, ids_pack, w_pack, count, rows, x, ids, weights, width);
    return hipGetLastError();
}

int qg_moe_handoff_notify(int *host_word, const int *count) {
    if (!host_word || !count) return hipErrorInvalidValue;
    handoff_notify_kernel<<<1, 1, 0, qg_stream()>>>(host_word, count);
    return hipGetLastError();
}

// qwen.c:672 writes the host's rows over the layer output; here they are
// added to the device rows of the packed tokens (the shared expert's part).
int qg_moe_handoff_merge(float *out, const float *y_pack, const int *count, const int *rows, int nt, int width) {
    if (nt < 1 || nt > QG_MAX_TOKENS || width < 1 || !out || !y_pack || !count || !rows) return hipErrorInvalidValue;
    handoff_merge_kernel<<<nt, 256, 0, qg_stream()>>>(out, y_pack, count, rows, width);
    return hipGetLastError();
}

}  // extern "C"
